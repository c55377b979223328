// The HopCuda-style hop (flyguy/fly_cuda.py:78-115) on the library's kernels: states are [rows][B] row-major
// (B contiguous), the connection weights come in per call, the caller owns every buffer (plans included).
#include "../../include/flyguy_core.h"
#include "kernels.h"

using namespace fg;

extern "C" {

void fh_spmm(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
             const int* pcol, const int* pidx, long long npos, const float* w, const float* h, float* out, int n_rows,
             int n_src, int B, void* cw, float* scratch, void* stream) {
    clear_error();
    if (B <= 0 || B % TW || n_rows <= 0 || n_src <= 0 || nwave < 0 || nseg < 0 || nseg > 8LL * nwave || npos < 0 ||
        nslot < 0 || !w || !h || !out || (nwave > 0 && (!wave || !seg || !pcol || !pidx || !cw)) ||
        (nsplit > 0 && (!split || !scratch))) {
        set_error("fh_spmm: bad argument");
        return;
    }
    hipStream_t st = (hipStream_t)stream;
    FG_CHECK(launch_pack(pcol, pidx, w, (int2*)cw, npos, st), );
    FwdEpi e;
    e.z = out;
    e.lz = plain(B);
    Plan p{(const int2*)wave, nwave, (const int4*)seg, nseg, (const int4*)split, nsplit, n_rows, nslot, npos};
    FG_CHECK(launch_fwd(p, (const int2*)cw, h, plain(B), n_src, e, scratch, tiled(nslot), B / TW, st), );
}

void fh_spmm_bwd(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                 const int* pcol, const int* pidx, long long npos, const float* w, const float* gz, const float* h,
                 float* gh, float* gw, int n_rows, int n_src, int B, void* cw, float* gwpart, float* scratch,
                 void* stream) {
    clear_error();
    if (B <= 0 || B % TW || n_rows <= 0 || n_src <= 0 || nwave < 0 || nseg < 0 || nseg > 8LL * nwave || npos < 0 ||
        nslot < 0 || !w || !gz || !h || !gh || (nwave > 0 && (!wave || !seg || !pcol || !pidx || !cw)) ||
        (gw && !gwpart) || (nsplit > 0 && (!split || !scratch))) {
        set_error("fh_spmm_bwd: bad argument");
        return;
    }
    hipStream_t st = (hipStream_t)stream;
    const int T = B / TW;
    FG_CHECK(launch_pack(pcol, pidx, w, (int2*)cw, npos, st), );
    BwdEpi e;
    e.mode = 0;
    e.gh_out = gh;
    e.lgh = plain(B);
    Plan p{(const int2*)wave, nwave, (const int4*)seg, nseg, (const int4*)split, nsplit, n_src, nslot, npos};
    FG_CHECK(launch_bwd(p, (const int2*)cw, gz, plain(B), n_rows, h, plain(B), gw ? gwpart : nullptr, npos, e, scratch,
                        tiled(nslot), T, st), );
    if (gw) FG_CHECK(launch_reduce(gwpart, npos, npos, T, pidx, nullptr, gw, st), );
}

}  // extern "C"
