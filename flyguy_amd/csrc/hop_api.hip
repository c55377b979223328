// The HopCuda-style hop (flyguy/fly_cuda.py:78-115) on the library's kernels: states are [rows][B] row-major
// (B contiguous), the connection weights come in per call, the caller owns every buffer (plans included).
//
// fh_spmm_static is fh_spmm for callers that cannot allocate device memory (code under HIP graph capture, serving
// loops that forbid allocation): its two workspaces, the packed (source, weight) pairs and the split rows' partial
// sums, live in `scratch`, a file-scope device array of FH_STATIC_BYTES.  Every GPU the library runs on holds its
// own copy until the process ends.  Calls on one GPU share that copy, so calls that overlap on one GPU (two streams,
// two threads) race; calls in one stream are ordered.  Nothing in it needs clearing: a call packs every pair it
// reads and writes every partial sum before it reads it.
#include <mutex>

#include "../../include/flyguy_core.h"
#include "kernels.h"

using namespace fg;

static __device__ __align__(256) unsigned char scratch[FH_STATIC_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_static_mu;
void* g_static_ptr[MAX_DEVICES] = {};      // per device: the device address of its copy of `scratch`

// The device address of the current device's `scratch` (looked up once per device, with that device current).  In
// host code the array's name is only a stand-in for the symbol: kernels and copies get this address instead.
unsigned char* static_scratch() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        set_error("fh_spmm_static: no current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_static_mu);
    if (!g_static_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error(std::string("fh_spmm_static: hipGetSymbolAddress: ") + hipGetErrorString(e));
            return nullptr;
        }
        g_static_ptr[dev] = p;
    }
    return static_cast<unsigned char*>(g_static_ptr[dev]);
}

bool spmm_args_ok(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                  const int* pcol, const int* pidx, long long npos, const float* w, const float* h, const float* out,
                  int n_rows, int n_src, int B) {
    return !(B <= 0 || B % TW || n_rows <= 0 || n_src <= 0 || nwave < 0 || nseg < 0 || nseg > 8LL * nwave ||
             npos < 0 || nslot < 0 || !w || !h || !out || (nwave > 0 && (!wave || !seg || !pcol || !pidx)) ||
             (nsplit > 0 && !split));
}

// pack the pairs into cw, then the product through the plan (split rows' partial sums in `partials`); h row-major
// [n_src][B], or tiled [B/32][n_src][32] (h_tiled)
void spmm_run(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
              const int* pcol, const int* pidx, long long npos, const float* w, const float* h, float* out, int n_rows,
              int n_src, int B, int2* cw, float* partials, hipStream_t st, bool h_tiled = false) {
    FG_CHECK(launch_pack(pcol, pidx, w, cw, npos, st), );
    FwdEpi e;
    e.z = out;
    e.lz = plain(B);
    Plan p{(const int2*)wave, nwave, (const int4*)seg, nseg, (const int4*)split, nsplit, n_rows, nslot, npos};
    FG_CHECK(launch_fwd(p, cw, h, h_tiled ? tiled(n_src) : plain(B), n_src, e, partials, tiled(nslot), B / TW, st), );
}

bool spmm_bwd_args_ok(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                      const int* pcol, const int* pidx, long long npos, const float* w, const float* gz, const float* h,
                      const float* gh, const float* gw, int n_rows, int n_src, int B, const void* cw,
                      const float* gwpart, const float* scratch) {
    return !(B <= 0 || B % TW || n_rows <= 0 || n_src <= 0 || nwave < 0 || nseg < 0 || nseg > 8LL * nwave ||
             npos < 0 || nslot < 0 || !w || !gz || !h || !gh ||
             (nwave > 0 && (!wave || !seg || !pcol || !pidx || !cw)) || (gw && !gwpart) ||
             (nsplit > 0 && (!split || !scratch)));
}

// the backward through the transposed plan: gz row-major [n_rows][B] or tiled (gz_tiled); h and gh row-major
void spmm_bwd_run(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                  const int* pcol, const int* pidx, long long npos, const float* w, const float* gz, const float* h,
                  float* gh, float* gw, int n_rows, int n_src, int B, int2* cw, float* gwpart, float* scratch,
                  hipStream_t st, bool gz_tiled) {
    const int T = B / TW;
    FG_CHECK(launch_pack(pcol, pidx, w, cw, npos, st), );
    BwdEpi e;
    e.mode = 0;
    e.gh_out = gh;
    e.lgh = plain(B);
    Plan p{(const int2*)wave, nwave, (const int4*)seg, nseg, (const int4*)split, nsplit, n_src, nslot, npos};
    FG_CHECK(launch_bwd(p, cw, gz, gz_tiled ? tiled(n_rows) : plain(B), n_rows, h, plain(B), gw ? gwpart : nullptr,
                        npos, e, scratch, tiled(nslot), T, st), );
    if (gw) FG_CHECK(launch_reduce(gwpart, npos, npos, T, pidx, nullptr, gw, st), );
}

// one 8-lane group per (tile, row): a row's 128-byte line of the tile, row-major -> tiled
__global__ __launch_bounds__(WG) void k_to_tiled(const float* __restrict__ x, int rows, int B, float* __restrict__ out,
                                                 long long n) {
    const long long i = (long long)blockIdx.x * WG + threadIdx.x;
    if (i >= n) return;
    const int sub = (int)(i & 7);
    const long long rt = i >> 3;                    // tile * rows + row: the tiled layout's line, written in order
    const int row = (int)(rt % rows), tile = (int)(rt / rows);
    const float4 v = reinterpret_cast<const float4*>(x + (size_t)row * B + (size_t)tile * TW)[sub];
    reinterpret_cast<float4*>(out + (size_t)rt * TW)[sub] = v;
}

}  // namespace

extern "C" {

void fh_spmm(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
             const int* pcol, const int* pidx, long long npos, const float* w, const float* h, float* out, int n_rows,
             int n_src, int B, void* cw, float* partials, void* stream) {
    clear_error();
    if (!spmm_args_ok(wave, nwave, seg, nseg, split, nsplit, nslot, pcol, pidx, npos, w, h, out, n_rows, n_src, B) ||
        (nwave > 0 && !cw) || (nsplit > 0 && !partials)) {
        set_error("fh_spmm: bad argument");
        return;
    }
    spmm_run(wave, nwave, seg, nseg, split, nsplit, nslot, pcol, pidx, npos, w, h, out, n_rows, n_src, B, (int2*)cw,
             partials, (hipStream_t)stream);
}

void fh_spmm_static(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                    const int* pcol, const int* pidx, long long npos, const float* w, const float* h, float* out,
                    int n_rows, int n_src, int B, void* stream) {
    clear_error();
    if (!spmm_args_ok(wave, nwave, seg, nseg, split, nsplit, nslot, pcol, pidx, npos, w, h, out, n_rows, n_src, B)) {
        set_error("fh_spmm_static: bad argument");
        return;
    }
    // layout of the workspace: the npos pairs (8 bytes each), then nslot x B partial sums, each at 256 bytes
    const unsigned long long pair_bytes = ((unsigned long long)npos * 8ull + 255ull) & ~255ull;
    const unsigned long long part_bytes = (unsigned long long)nslot * (unsigned long long)B * 4ull;
    if (pair_bytes + part_bytes > FH_STATIC_BYTES) {
        set_error("fh_spmm_static: the product needs " + std::to_string(pair_bytes + part_bytes) +
                  " bytes of workspace (8 per plan position + 4 per split-row slot and sample), more than the " +
                  std::to_string((unsigned long long)FH_STATIC_BYTES) + " of the static workspace; use fh_spmm");
        return;
    }
    unsigned char* base = static_scratch();
    if (!base) return;
    spmm_run(wave, nwave, seg, nseg, split, nsplit, nslot, pcol, pidx, npos, w, h, out, n_rows, n_src, B,
             reinterpret_cast<int2*>(base), reinterpret_cast<float*>(base + pair_bytes), (hipStream_t)stream);
}

void fh_spmm_bwd(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                 const int* pcol, const int* pidx, long long npos, const float* w, const float* gz, const float* h,
                 float* gh, float* gw, int n_rows, int n_src, int B, void* cw, float* gwpart, float* scratch,
                 void* stream) {
    clear_error();
    if (!spmm_bwd_args_ok(wave, nwave, seg, nseg, split, nsplit, nslot, pcol, pidx, npos, w, gz, h, gh, gw, n_rows,
                          n_src, B, cw, gwpart, scratch)) {
        set_error("fh_spmm_bwd: bad argument");
        return;
    }
    spmm_bwd_run(wave, nwave, seg, nseg, split, nsplit, nslot, pcol, pidx, npos, w, gz, h, gh, gw, n_rows, n_src, B,
                 (int2*)cw, gwpart, scratch, (hipStream_t)stream, false);
}

void fh_to_tiled(const float* x, int rows, int B, float* out, void* stream) {
    clear_error();
    if (!x || !out || rows < 0 || B <= 0 || B % TW) {
        set_error("fh_to_tiled: bad argument");
        return;
    }
    const long long n = (long long)rows * B / 4;    // 8 lanes per 32-sample line
    if (n == 0) return;
    k_to_tiled<<<(unsigned)((n + WG - 1) / WG), WG, 0, (hipStream_t)stream>>>(x, rows, B, out, n);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) set_error(std::string("fh_to_tiled: ") + hipGetErrorString(e));
}

void fh_spmm_tiled(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                   const int* pcol, const int* pidx, long long npos, const float* w, const float* ht, float* out,
                   int n_rows, int n_src, int B, void* cw, float* scratch, void* stream) {
    clear_error();
    if (!spmm_args_ok(wave, nwave, seg, nseg, split, nsplit, nslot, pcol, pidx, npos, w, ht, out, n_rows, n_src, B) ||
        (nwave > 0 && !cw) || (nsplit > 0 && !scratch)) {
        set_error("fh_spmm_tiled: bad argument");
        return;
    }
    spmm_run(wave, nwave, seg, nseg, split, nsplit, nslot, pcol, pidx, npos, w, ht, out, n_rows, n_src, B, (int2*)cw,
             scratch, (hipStream_t)stream, true);
}

void fh_spmm_bwd_tiled(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                       const int* pcol, const int* pidx, long long npos, const float* w, const float* gzt, const float* h,
                       float* gh, float* gw, int n_rows, int n_src, int B, void* cw, float* gwpart, float* scratch,
                       void* stream) {
    clear_error();
    if (!spmm_bwd_args_ok(wave, nwave, seg, nseg, split, nsplit, nslot, pcol, pidx, npos, w, gzt, h, gh, gw, n_rows,
                          n_src, B, cw, gwpart, scratch)) {
        set_error("fh_spmm_bwd_tiled: bad argument");
        return;
    }
    spmm_bwd_run(wave, nwave, seg, nseg, split, nsplit, nslot, pcol, pidx, npos, w, gzt, h, gh, gw, n_rows, n_src, B,
                 (int2*)cw, gwpart, scratch, (hipStream_t)stream, true);
}

}  // extern "C"
