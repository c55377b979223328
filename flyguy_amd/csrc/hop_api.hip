// The HopCuda-style hop (flyguy/fly_cuda.py:78-115) on the library's kernels: states are [rows][B] row-major
// (B contiguous), the connection weights come in per call, the caller owns every buffer.
#include "../../include/flyguy_core.h"
#include "kernels.h"

using namespace fg;

extern "C" {

void fh_spmm(const long long* rowptr, const int* col, const float* w, const float* h, float* out, int n_rows, int n_src,
             int B, long long E, const int* plan, int nseg, const int* split, int nsplit, int nslot, void* cw,
             float* scratch, void* stream) {
    (void)rowptr;
    clear_error();
    if (B <= 0 || B % TW || n_rows <= 0 || n_src <= 0 || E < 0 || !col || !w || !h || !out || !plan || !cw ||
        (nsplit > 0 && (!split || !scratch))) {
        set_error("fh_spmm: bad argument");
        return;
    }
    hipStream_t st = (hipStream_t)stream;
    FG_CHECK(launch_pack(col, nullptr, w, (int2*)cw, E, st), );
    FwdEpi e;
    e.z = out;
    e.lz = plain(B);
    Plan p{(const int4*)plan, nseg, (const int4*)split, nsplit, n_rows, nslot, E};
    FG_CHECK(launch_fwd(p, (const int2*)cw, h, plain(B), n_src, e, scratch, tiled(nslot), B / TW, st), );
}

void fh_spmm_bwd(const long long* tcrow, const int* tcol, const long long* tperm, const float* w, const float* gz,
                 const float* h, float* gh, float* gw, int n_rows, int n_src, int B, long long E, const int* plan,
                 int nseg, const int* split, int nsplit, int nslot, void* cw, float* gwpart, float* scratch,
                 void* stream) {
    (void)tcrow;
    (void)n_rows;
    clear_error();
    if (B <= 0 || B % TW || n_src <= 0 || E < 0 || !tcol || !tperm || !w || !gz || !h || !gh || !plan || !cw ||
        (gw && !gwpart) || (nsplit > 0 && (!split || !scratch))) {
        set_error("fh_spmm_bwd: bad argument");
        return;
    }
    hipStream_t st = (hipStream_t)stream;
    const int T = B / TW;
    FG_CHECK(launch_pack64(tcol, tperm, w, (int2*)cw, E, st), );
    BwdEpi e;
    e.mode = 0;
    e.gh_out = gh;
    e.lgh = plain(B);
    Plan p{(const int4*)plan, nseg, (const int4*)split, nsplit, n_src, nslot, E};
    FG_CHECK(launch_bwd(p, (const int2*)cw, gz, plain(B), n_rows, h, plain(B), gw ? gwpart : nullptr, E, e, scratch, tiled(nslot),
                        T, st), );
    if (gw) FG_CHECK(launch_reduce64(gwpart, E, E, T, tperm, gw, st), );
}

}  // extern "C"
