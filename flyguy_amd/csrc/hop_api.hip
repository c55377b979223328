// The HopCuda-style hop (flyguy/fly_cuda.py:78-115) on the library's kernels: states are [rows][B] row-major
// (B contiguous), the connection weights come in per call, the caller owns every buffer (plans included).
//
// fh_spmm_static is fh_spmm for callers that cannot allocate device memory (code under HIP graph capture, serving
// loops that forbid allocation): its two workspaces, the packed (source, weight) pairs and the split rows' partial
// sums, live in `g_fh_static_ws`, a file-scope device array of FH_STATIC_BYTES.  Every GPU the library runs on holds its
// own copy until the process ends.  Calls on one GPU share that copy, so calls that overlap on one GPU (two streams,
// two threads) race; calls in one stream are ordered.  Nothing in it needs clearing: a call packs every pair it
// reads and writes every partial sum before it reads it.
#include <mutex>

#include "../../include/flyguy_core.h"
#include "kernels.h"

using namespace fg;

static __device__ __align__(256) unsigned char g_fh_static_ws[FH_STATIC_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_static_mu;
void* g_static_ptr[MAX_DEVICES] = {};      // per device: the device address of its copy of g_fh_static_ws

// The device address of the current device's g_fh_static_ws (looked up once per device, with that device current:
// a runtime lookup, no allocation; a caller that captures its calls in a graph makes one call first).  In host code
// the array's name is only a stand-in for the symbol: kernels and copies get this address instead.
unsigned char* static_scratch() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        set_error("fh_spmm_static: no current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_static_mu);
    if (!g_static_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_fh_static_ws));
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

// The neuron activation of FlyActor's GPU path, h = relu(g z - t) per row of row-major [rows][B] states (g the
// gain, t softplus(theta) of the row's neuron), in one pass instead of PyTorch's three (product, difference, relu),
// rounded as PyTorch rounds them: the product, then the difference, no fused multiply-add.  relu passes a NaN on.
__device__ __forceinline__ float pre1(float g, float z, float t) {
#pragma clang fp contract(off)
    return g * z - t;                           // (two roundings: the compiler may not fuse them here)
}
__device__ __forceinline__ float fire1(float g, float z, float t) {
    const float a = pre1(g, z, t);
    return a > 0.f ? a : (a != a ? a : 0.f);
}

// I: the index type (32-bit unless the states hold 2^31 float4 or more: its division is the cheaper one)
template <class I>
__global__ __launch_bounds__(WG) void k_fire(const float4* __restrict__ z, const float* __restrict__ g,
                                             const float* __restrict__ t, I q, I n, float4* __restrict__ h) {
    const I i = (I)blockIdx.x * WG + threadIdx.x;                           // q float4 per row
    if (i >= n) return;
    const int r = (int)(i / q);
    const float gr = g[r], tr = t[r];
    const float4 v = z[i];
    h[i] = make_float4(fire1(gr, v.x, tr), fire1(gr, v.y, tr), fire1(gr, v.z, tr), fire1(gr, v.w, tr));
}

// Its backward, one workgroup per row: where g z - t is not <= 0 (positive, or NaN: PyTorch's relu passes the
// gradient of a NaN on) gz = gh g, elsewhere 0, and the row's gradients of g and t, gg = sum gh z and gt = -sum gh
// over those samples (each product rounded, as PyTorch forms them; the sums in this kernel's order)
__global__ __launch_bounds__(WG) void k_fire_bwd(const float4* __restrict__ gh, const float4* __restrict__ z,
                                                 const float* __restrict__ g, const float* __restrict__ t, int q,
                                                 float4* __restrict__ gz, float* __restrict__ gg,
                                                 float* __restrict__ gt) {
    __shared__ float red[2][WG / 64];
    const int r = blockIdx.x;
    const float gr = g[r], tr = t[r];
    float sz = 0.f, s1 = 0.f;
    for (int k = threadIdx.x; k < q; k += WG) {
        const size_t i = (size_t)r * q + k;
        const float4 v = z[i], d = gh[i];
        const float zv[4] = {v.x, v.y, v.z, v.w}, dv[4] = {d.x, d.y, d.z, d.w};
        float o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const bool on = !(pre1(gr, zv[c], tr) <= 0.f);
            o[c] = on ? __fmul_rn(dv[c], gr) : 0.f;
            sz += on ? __fmul_rn(dv[c], zv[c]) : 0.f;
            s1 += on ? dv[c] : 0.f;
        }
        gz[i] = make_float4(o[0], o[1], o[2], o[3]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        sz += __shfl_xor(sz, o, 64);
        s1 += __shfl_xor(s1, o, 64);
    }
    if ((threadIdx.x & 63) == 0) {
        red[0][threadIdx.x >> 6] = sz;
        red[1][threadIdx.x >> 6] = s1;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float a = 0.f, b = 0.f;
        for (int w = 0; w < WG / 64; ++w) {
            a += red[0][w];
            b += red[1][w];
        }
        gg[r] = a;
        gt[r] = -b;
    }
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

void fh_fire(const float* z, const float* g, const float* t, int rows, int B, float* h, void* stream) {
    clear_error();
    if (!z || !g || !t || !h || rows < 0 || B <= 0 || B % 4) {
        set_error("fh_fire: bad argument");
        return;
    }
    const long long n = (long long)rows * (B / 4);
    if (n == 0) return;
    const unsigned blocks = (unsigned)((n + WG - 1) / WG);
    if (n < (1LL << 31))
        k_fire<unsigned><<<blocks, WG, 0, (hipStream_t)stream>>>((const float4*)z, g, t, (unsigned)(B / 4), (unsigned)n,
                                                                 (float4*)h);
    else
        k_fire<unsigned long long><<<blocks, WG, 0, (hipStream_t)stream>>>(
            (const float4*)z, g, t, (unsigned long long)(B / 4), (unsigned long long)n, (float4*)h);
    FG_CHECK(hipGetLastError(), );
}

void fh_fire_bwd(const float* gh, const float* z, const float* g, const float* t, int rows, int B, float* gz, float* gg,
                 float* gt, void* stream) {
    clear_error();
    if (!gh || !z || !g || !t || !gz || !gg || !gt || rows < 0 || B <= 0 || B % 4) {
        set_error("fh_fire_bwd: bad argument");
        return;
    }
    if (rows == 0) return;
    k_fire_bwd<<<(unsigned)rows, WG, 0, (hipStream_t)stream>>>((const float4*)gh, (const float4*)z, g, t, B / 4,
                                                                (float4*)gz, gg, gt);
    FG_CHECK(hipGetLastError(), );
}

}  // extern "C"
