// 16-bit states for the HopCuda-style hop: the reference's half path (flyguy/fly_cuda.py:34-56, 93-115), where
// states and gradients are read as 16-bit numbers and every sum is accumulated in float32.
//
// A 16-bit state tensor is stored tiled, [T = ceil(B/64)][rows][64]: one 128-byte line holds 64 samples of one row,
// so a gather of a row costs one line, as in the float32 layout, for twice the samples.  Each lane of an 8-lane
// group holds 8 samples.  The row plan, the (source, weight) pairs and the gather loop are those of the float32
// kernels (kernels.hip); the epilogues write the caller's row-major float32 [rows][B] outputs.
#include <algorithm>

#include "../../include/flyguy_core.h"
#include "half.h"

namespace fg {

// ------------------------------------------------------------------------------------------------ conversions
// dst (tiled 16-bit) = x (row-major float32 [rows][B]) / (*scale if scale), rounded to nearest even; samples past
// B are zero.  One thread per 8 samples.
template <typename S>
__global__ void k_to16(const float* __restrict__ x, int rows, int B, const float* __restrict__ scale,
                       unsigned short* __restrict__ dst, long long n8) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n8) return;
    const int sub = (int)(i & 7);
    const long long rt = i >> 3;                    // (tile, row)
    const int row = (int)(rt % rows);
    const int tile = (int)(rt / rows);
    const int b0 = tile * TW16 + sub * 8;
    u32x4 o = {0u, 0u, 0u, 0u};
    if (b0 < B) {                                   // B % 32 == 0: the 8 samples are all in or all out
        const float4* p = reinterpret_cast<const float4*>(x + (size_t)row * B + b0);
        const float4 a = p[0], b = p[1];
        float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        if (scale) {
            const float sc = *scale;
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = v[k] / sc;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = Bits16<S>::from(v[2 * k]) | (Bits16<S>::from(v[2 * k + 1]) << 16);
    }
    *reinterpret_cast<u32x4*>(dst + (size_t)rt * TW16 + sub * 8) = o;
}

// *out = max(*out, max |x|) over non-negative floats (whose order is that of their bit patterns)
__global__ __launch_bounds__(WG) void k_absmax(const float* __restrict__ x, long long n, unsigned* __restrict__ out) {
    __shared__ float red[WG / 64];
    float m = 0.f;
    for (long long i = (long long)blockIdx.x * WG + threadIdx.x; i < n; i += (long long)gridDim.x * WG) m = fmaxf(m, fabsf(x[i]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < WG / 64; ++k) m = fmaxf(m, red[k]);
        atomicMax(out, __float_as_uint(m));
    }
}

// ------------------------------------------------------------------------------------------------ forward
// out[row][b] = sum over the row's edges of w * state[source][b] (float32 sums); split rows write partial sums
template <typename S>
__global__ __launch_bounds__(WG) void k_fwd16(Plan p, const int2* __restrict__ cw, const unsigned short* __restrict__ src,
                                              int src_rows, float* __restrict__ out, int B, float* __restrict__ part,
                                              int T, int RB) {
    __shared__ __align__(16) int2 slots[WG / LPR][LPR];
    int rb;
    const int tile = tile_of(blockIdx.x, RB, T, rb);
    const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7, lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(rb * (WG / 64) + (int)(threadIdx.x >> 6));
    int2 wv;
    const bool wok = load_wave(p, w, wv);
    const int2* q = cw + wv.x + lane;
    int2 nxt = (wok && wv.y > 0) ? q[0] : make_int2(NO_ROW, 0);
    int4 sg;
    const bool live = load_segment(p, w * 8 + (grp & 7), sg) && wok;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(src + (size_t)tile * src_rows * TW16), (short)0, src_rows * 128, 0x00020000);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0, left = wok ? wv.y : 0; left > 0; ++j, left -= 8) {
        int c[8];
        float wt[8];
        stage8(slots[grp], sub, nxt, c, wt);
        u32x4 raw[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) raw[s] = s < left ? gather16(rs, c[s], sub) : u32x4{0u, 0u, 0u, 0u};
        __builtin_amdgcn_sched_barrier(0);
        if (left > 8) nxt = q[64 * (j + 1)];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            float f[8];
            unpack8<S>(raw[s], f);
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[k] = fmaf(wt[s], f[k], acc[k]);
        }
    }
    if (!live) return;
    if (sg.y >= 0) {
        store8(part + ((size_t)tile * p.nslot + sg.y) * TW16 + sub * 8, acc);
        return;
    }
    const int b0 = tile * TW16 + sub * 8;
    if (b0 < B) store8(out + (size_t)sg.x * B + b0, acc);
}

// ------------------------------------------------------------------------------------------------ backward
// Over the transposed plan (rows = sources j): gh[j][b] = scale * sum_e w_e gz[col_e][b], and per (plan position,
// tile) the partial sum over the tile's samples of gz[col_e][b] * h[j][b] (the weight gradient before the scale).
template <typename S>
__global__ __launch_bounds__(WG) void k_bwd16(Plan p, const int2* __restrict__ cw, const unsigned short* __restrict__ gz,
                                              int gz_rows, const unsigned short* __restrict__ hs,
                                              float* __restrict__ gh, int B, float* __restrict__ gwpart, long long gw_ld,
                                              const float* __restrict__ scale, float* __restrict__ part, int T, int RB) {
    __shared__ __align__(16) int2 slots[WG / LPR][LPR];
    int rb;
    const int tile = tile_of(blockIdx.x, RB, T, rb);
    const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7, lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(rb * (WG / 64) + (int)(threadIdx.x >> 6));
    int2 wv;
    const bool wok = load_wave(p, w, wv);
    const int2* q = cw + wv.x + lane;
    int2 nxt = (wok && wv.y > 0) ? q[0] : make_int2(NO_ROW, 0);
    int4 sg;
    const bool live = load_segment(p, w * 8 + (grp & 7), sg) && wok;
    float hj[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (live) {
        const u32x4 hv = *reinterpret_cast<const u32x4*>(hs + ((size_t)tile * p.rows + sg.x) * TW16 + sub * 8);
        unpack8<S>(hv, hj);
    }
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(gz + (size_t)tile * gz_rows * TW16), (short)0, gz_rows * 128, 0x00020000);
    float* gwp = gwpart ? gwpart + (size_t)tile * gw_ld + wv.x + lane : nullptr;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0, left = wok ? wv.y : 0; left > 0; ++j, left -= 8) {
        int c[8];
        float wt[8];
        stage8(slots[grp], sub, nxt, c, wt);
        u32x4 raw[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) raw[s] = s < left ? gather16(rs, c[s], sub) : u32x4{0u, 0u, 0u, 0u};
        __builtin_amdgcn_sched_barrier(0);
        if (left > 8) nxt = q[64 * (j + 1)];
        __builtin_amdgcn_sched_barrier(0);
        float d[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            float f[8];
            unpack8<S>(raw[s], f);
            float dp = 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                acc[k] = fmaf(wt[s], f[k], acc[k]);
                dp = fmaf(hj[k], f[k], dp);
            }
            d[s] = dp;
        }
        if (gwp) gwp[64 * j] = rs8(d, sub);
    }
    if (!live) return;
    if (sg.y >= 0) {
        store8(part + ((size_t)tile * p.nslot + sg.y) * TW16 + sub * 8, acc);
        return;
    }
    const int b0 = tile * TW16 + sub * 8;
    if (b0 >= B) return;
    const float sc = scale ? *scale : 1.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] *= sc;
    store8(gh + (size_t)sg.x * B + b0, acc);
}

// split rows: their partial sums in segment order, times *mul (if given), into the row-major output
__global__ __launch_bounds__(WG) void k_comb16(Plan p, const float* __restrict__ part, float* __restrict__ out, int B,
                                               const float* __restrict__ mul, int T) {
    long long q = ((long long)blockIdx.x * WG + threadIdx.x);
    const int sub = (int)(q & 7);
    q >>= 3;
    const int tile = (int)(q % T);
    const long long i = q / T;
    int4 s;
    if (!load_split(p, i, s)) return;
    const int b0 = tile * TW16 + sub * 8;
    if (b0 >= B) return;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < s.z; ++k) {
        const float* src = part + ((size_t)tile * p.nslot + s.y + k) * TW16 + sub * 8;
        const float4 a = *reinterpret_cast<const float4*>(src), b = *reinterpret_cast<const float4*>(src + 4);
        acc[0] += a.x; acc[1] += a.y; acc[2] += a.z; acc[3] += a.w;
        acc[4] += b.x; acc[5] += b.y; acc[6] += b.z; acc[7] += b.w;
    }
    if (mul) {
        const float m = *mul;
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] *= m;
    }
    store8(out + (size_t)s.x * B + b0, acc);
}

// G[idx[i]] += (sum over nt tiles of part[t * ld + i]) * (*mul); idx[i] < 0 adds nothing
__global__ void k_reduce_mul(const float* __restrict__ part, long long ld, long long n, int nt, const int* __restrict__ idx,
                             const float* __restrict__ mul, float* __restrict__ G) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int o = idx[i];
    if (o < 0) return;
    float s = 0.f;
    int t = 0;
    for (; t + 8 <= nt; t += 8) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = part[(size_t)(t + k) * ld + i];
#pragma unroll
        for (int k = 0; k < 8; ++k) s += v[k];
    }
    for (; t < nt; ++t) s += part[(size_t)t * ld + i];
    G[o] += s * *mul;
}

static inline unsigned nblocks(long long n) { return (unsigned)((n + WG - 1) / WG); }

}  // namespace fg

using namespace fg;

static bool plan_args_ok(int nwave, int nseg, int nsplit, int nslot, long long npos, const int* wave, const int* seg,
                         const int* split, const int* pcol, const int* pidx, void* cw, float* scratch) {
    return nwave >= 0 && nseg >= 0 && nseg <= 8LL * nwave && npos >= 0 && nslot >= 0 && nsplit >= 0 &&
           (nwave == 0 || (wave && seg && pcol && pidx && cw)) && (nsplit == 0 || (split && scratch));
}

extern "C" {

void fh_to_half(const float* x, int rows, int B, const float* scale, void* out, void* stream) {
    clear_error();
    if (!x || !out || rows < 0 || B <= 0 || B % TW) { set_error("fh_to_half: bad argument"); return; }
    const long long n8 = (long long)((B + TW16 - 1) / TW16) * rows * 8;
    if (n8 == 0) return;
    k_to16<F16><<<nblocks(n8), WG, 0, (hipStream_t)stream>>>(x, rows, B, scale, (unsigned short*)out, n8);
    FG_CHECK(hipGetLastError(), );
}

void fh_absmax(const float* x, long long n, float* out, void* stream) {
    clear_error();
    if (!x || !out || n < 0) { set_error("fh_absmax: bad argument"); return; }
    hipStream_t st = (hipStream_t)stream;
    FG_CHECK(launch_fill(out, 1e-30f, 1, st), );
    if (n == 0) return;
    const long long nb = std::min<long long>(1024, (n + WG - 1) / WG);
    k_absmax<<<(unsigned)nb, WG, 0, st>>>(x, n, (unsigned*)out);
    FG_CHECK(hipGetLastError(), );
}

void fh_spmm_h(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
               const int* pcol, const int* pidx, long long npos, const float* w, const void* hs, float* out, int n_rows,
               int n_src, int B, void* cw, float* scratch, void* stream) {
    clear_error();
    if (B <= 0 || B % TW || n_rows <= 0 || n_src <= 0 || !w || !hs || !out ||
        !plan_args_ok(nwave, nseg, nsplit, nslot, npos, wave, seg, split, pcol, pidx, cw, scratch)) {
        set_error("fh_spmm_h: bad argument");
        return;
    }
    hipStream_t st = (hipStream_t)stream;
    const int T = (B + TW16 - 1) / TW16;
    FG_CHECK(launch_pack(pcol, pidx, w, (int2*)cw, npos, st), );
    Plan p{(const int2*)wave, nwave, (const int4*)seg, nseg, (const int4*)split, nsplit, n_rows, nslot, npos};
    if (nwave > 0) {
        const int RB = (nwave + WG / 64 - 1) / (WG / 64);
        k_fwd16<F16><<<(unsigned)((long long)T * RB), WG, 0, st>>>(p, (const int2*)cw, (const unsigned short*)hs, n_src,
                                                                  out, B, scratch, T, RB);
        FG_CHECK(hipGetLastError(), );
    }
    if (nsplit > 0) {
        k_comb16<<<nblocks((long long)nsplit * T * 8), WG, 0, st>>>(p, scratch, out, B, nullptr, T);
        FG_CHECK(hipGetLastError(), );
    }
}

void fh_spmm_bwd_h(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                   const int* pcol, const int* pidx, long long npos, const float* w, const void* gzs, const void* hs,
                   const float* scale, float* gh, float* gw, int n_rows, int n_src, int B, void* cw, float* gwpart,
                   float* scratch, void* stream) {
    clear_error();
    if (B <= 0 || B % TW || n_rows <= 0 || n_src <= 0 || !w || !gzs || !hs || !scale || !gh || (gw && !gwpart) ||
        !plan_args_ok(nwave, nseg, nsplit, nslot, npos, wave, seg, split, pcol, pidx, cw, scratch)) {
        set_error("fh_spmm_bwd_h: bad argument");
        return;
    }
    hipStream_t st = (hipStream_t)stream;
    const int T = (B + TW16 - 1) / TW16;
    FG_CHECK(launch_pack(pcol, pidx, w, (int2*)cw, npos, st), );
    Plan p{(const int2*)wave, nwave, (const int4*)seg, nseg, (const int4*)split, nsplit, n_src, nslot, npos};
    if (nwave > 0) {
        const int RB = (nwave + WG / 64 - 1) / (WG / 64);
        k_bwd16<F16><<<(unsigned)((long long)T * RB), WG, 0, st>>>(p, (const int2*)cw, (const unsigned short*)gzs, n_rows,
                                                                  (const unsigned short*)hs, gh, B, gw ? gwpart : nullptr,
                                                                  npos, scale, scratch, T, RB);
        FG_CHECK(hipGetLastError(), );
    }
    if (nsplit > 0) {
        k_comb16<<<nblocks((long long)nsplit * T * 8), WG, 0, st>>>(p, scratch, gh, B, scale, T);
        FG_CHECK(hipGetLastError(), );
    }
    if (gw && npos > 0) {
        k_reduce_mul<<<nblocks(npos), WG, 0, st>>>(gwpart, npos, npos, T, pidx, scale, gw);
        FG_CHECK(hipGetLastError(), );
    }
}

}  // extern "C"
