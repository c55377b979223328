// The library core with bfloat16 states: the observations x, the sensory layer's drive, every layer's output h and
// the gradients gz the backward gathers are stored as bfloat16 (round to nearest even).  Sums, split-row partials,
// the drive's gradient, the per-tile gradient partials, the weights and Adam stay float32.
//
// A 16-bit state tensor is [T = B/64][rows][64]: one 128-byte line per row holds 64 samples, so a gathered source
// line serves twice the samples it serves in the float32 layout ([B/32][rows][32]).  Each lane of an 8-lane group
// holds 8 samples.  Row plans, (source, weight) pairs, the gather loop and the per-edge weight gradient's
// reduce-scatter are those of the float32 kernels (kernels.hip); the epilogues do the same neuron arithmetic in float32
// on the widened values.  Quantities derived from a state use its stored (rounded) value: a hop layer's gain gradient
// uses z = (h + softplus(theta)) / gain of the stored h, the sensory layer's the stored drive, and the drive's
// gradient collects the hops' gz before their rounding.  Float32 tensors beside them (partials, the drive's gradient)
// use the same tiling, [T][rows][64] floats.
#include <initializer_list>

#include "half.h"
#include "readout.h"

namespace fg {

typedef unsigned short bf16_t;

__device__ __forceinline__ void ld8(const bf16_t* base, int rows, int tile, int row, int sub, float (&f)[8]) {
    unpack8<BF16>(*reinterpret_cast<const u32x4*>(base + ((size_t)tile * rows + row) * TW16 + sub * 8), f);
}
// two floats -> two bfloat16 in one word (low half first), rounded to nearest even by the hardware conversion
__device__ __forceinline__ unsigned pack2(float a, float b) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    const bf2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ void st8(bf16_t* base, int rows, int tile, int row, int sub, const float (&f)[8]) {
    u32x4 o;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = pack2(f[2 * k], f[2 * k + 1]);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(base + ((size_t)tile * rows + row) * TW16 + sub * 8));
}
__device__ __forceinline__ float* f8p(float* base, int rows, int tile, int row, int sub) {
    return base + ((size_t)tile * rows + row) * TW16 + sub * 8;
}
__device__ __forceinline__ void ldf8(const float* p, float (&f)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

// The products of the hop kernels: acc[k] += w_a g_a[k] + w_b g_b[k] over the lane's 8 samples, for two edges a, b
// at once on v_dot2_f32_bf16 (two exact products and the sum in float32).  The weights come packed as bfloat16
// values in float32 (low halves zero, k_pack<true>); v_perm_b32 pairs the two edges' weights, and the two gathered
// states sample by sample.
__device__ __forceinline__ void fma_pair(float wa, float wb, const u32x4& ga, const u32x4& gb, float (&acc)[8]) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    const bf2 w2 = __builtin_bit_cast(bf2, __builtin_amdgcn_perm(__float_as_uint(wb), __float_as_uint(wa), 0x07060302u));
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const unsigned a = ga[m], b = gb[m];
        const unsigned lo = __builtin_amdgcn_perm(b, a, 0x05040100u), hi = __builtin_amdgcn_perm(b, a, 0x07060302u);
        acc[2 * m] = __builtin_amdgcn_fdot2_f32_bf16(w2, __builtin_bit_cast(bf2, lo), acc[2 * m], false);
        acc[2 * m + 1] = __builtin_amdgcn_fdot2_f32_bf16(w2, __builtin_bit_cast(bf2, hi), acc[2 * m + 1], false);
    }
}

// ------------------------------------------------------------------------------------------------ forward
struct FwdIn16 {
    float dv[8];
    float g, sp, b;                             // b: the row's bias (the plug's records carry it)
};
// recs[i]: the row's record (as fwd_inputs)
__device__ __forceinline__ void fwd_inputs16(const FwdEpi16& e, const float4* recs, int i, int d, int tile, int sub,
                                             FwdIn16& in) {
#pragma unroll
    for (int k = 0; k < 8; ++k) in.dv[k] = 0.f;
    in.g = in.sp = in.b = 0.f;
    if (e.drive && d >= 0) ld8(e.drive, e.n_s, tile, d, sub, in.dv);
    if (recs) {
        const float4 r = recs[i];
        in.g = r.x;
        in.sp = r.y;
        in.b = r.w;
    }
}
__device__ __forceinline__ void fwd_finish16(const FwdEpi16& e, int t, int tile, int sub, float (&acc)[8], const FwdIn16& in) {
    if (e.drive)
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] += in.dv[k];
    if (e.z) st8(e.z, e.rows, tile, t, sub, acc);
    if (e.info) {
        float hv[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) hv[k] = fmaxf(fmaf(in.g, acc[k], -in.sp), 0.f);
        st8(e.h, e.rows, tile, t, sub, hv);
        if (e.fires) {                          // whether the row fires on some sample of the tile (a value > 0 that
            bool any = false;                   // rounds to a bfloat16 zero counts as firing: that only skips less)
#pragma unroll
            for (int k = 0; k < 8; ++k) any = any || hv[k] > 0.f;
            const bool on = !group_silent(any);
            if (sub == 0) e.fires[(size_t)tile * fires_bytes_ld(e.rows) + t] = on ? 1 : 0;
        }
    }
}

// the plug or one hop over its row plan (as k_fwd); split rows leave float32 partials [T][nslot][64]
// src_fires: the source layer's firing bitmaps (k_fires_pack, fw_ld words per tile; fw_ld 0: none)
template <int PB>
__global__ __launch_bounds__(WG) void k_cfwd16(Plan p, const int2* __restrict__ cw, const bf16_t* __restrict__ src,
                                               int src_rows, FwdEpi16 epi, float* __restrict__ part, int T, int RB,
                                               const unsigned* __restrict__ src_fires, int fw_ld) {
    __shared__ __align__(16) int2 slots[WG / LPR][LPR];
    extern __shared__ __align__(16) unsigned fires[];
    int rb;
    const int tile = tile_of(blockIdx.x, RB, T, rb);
    const bool bits = stage_fires(src_fires, fw_ld, tile, fires);     // (only for a tile with silent source rows)
    const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7, lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(rb * (WG / 64) + (int)(threadIdx.x >> 6));
    int2 wv;
    const bool wok = load_wave(p, w, wv);
    const PairLoad<PB> q(cw, wv.x, lane);
    int2 nxt = (wok && wv.y > 0) ? q.step(0) : make_int2(NO_ROW, 0);
    int4 sg;
    const bool live = load_segment(p, w * 8 + (grp & 7), sg) && wok;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(src + (size_t)tile * src_rows * TW16), (short)0, src_rows * 128, 0x00020000);
    const bool whole = live && sg.y < 0;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    FwdIn16 in{};
    for (int j = 0, left = wok ? wv.y : 0; left > 0; ++j, left -= 8) {
        int c[8];
        float wt[8];
        // (a silent source row adds zeros: its gather reads NO_ROW)
        if constexpr (PB == 8)                 // (6-byte pairs: stage_pairs drops them)
            if (bits) drop_silent(nxt, fires, src_rows);
        stage_pairs<PB>(slots, grp, sub, nxt, bits, fires, src_rows, c, wt);
        u32x4 raw[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) raw[s] = s < left ? gather16(rs, c[s], sub) : u32x4{0u, 0u, 0u, 0u};
        __builtin_amdgcn_sched_barrier(0);
        if (left > 8) nxt = q.step(j + 1);
        if (j == 0 && whole) {                 // the row's own inputs after the first gathers; the bias starts the sum
            fwd_inputs16(epi, epi.sinfo ? epi.sinfo + 8 * w : nullptr, grp & 7, sg.z, tile, sub, in);
            if (epi.bias) {
                const float b = epi.sinfo ? in.b : epi.bias[sg.x];
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[k] = b;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 8; s += 2) fma_pair(wt[s], wt[s + 1], raw[s], raw[s + 1], acc);
    }
    if (whole && !(wok && wv.y > 0)) {          // a wave without edges
        fwd_inputs16(epi, epi.sinfo ? epi.sinfo + 8 * w : nullptr, grp & 7, sg.z, tile, sub, in);
        if (epi.bias) {
            const float b = epi.sinfo ? in.b : epi.bias[sg.x];
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[k] = b;
        }
    }
    if (!live) return;
    if (sg.y >= 0) {
        store8(part + ((size_t)tile * p.nslot + sg.y) * TW16 + sub * 8, acc);
        return;
    }
    fwd_finish16(epi, sg.x, tile, sub, acc, in);
}


// The plug with the tile's observation slab (src_rows lines of 64 bfloat16 samples) staged in LDS, as k_fwd_lds:
// the same sums as k_cfwd16, plan waves walked by each wave with the next one's loads requested before the
// previous one's stores.  No re-drive rows.
template <int PB>
__global__ __launch_bounds__(FWD_LDS_NW * 64) void k_cfwd16_lds(Plan p, const int2* __restrict__ cw,
                                                               const bf16_t* __restrict__ src, int src_rows,
                                                               FwdEpi16 epi, float* __restrict__ part, int T, int S) {
    __shared__ __align__(16) int2 slots[FWD_LDS_NW * 64 / LPR][LPR];
    extern __shared__ __align__(16) u32x4 xs16[];         // the tile's slab, src_rows x 8 (16 bytes each)
    int s;
    const int tile = tile_of(blockIdx.x, S, T, s);
    const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7, lane = threadIdx.x & 63, gi = grp & 7;
    const int w0 = __builtin_amdgcn_readfirstlane(s * FWD_LDS_NW + (int)(threadIdx.x >> 6)), dw = S * FWD_LDS_NW;
    const int n = w0 < p.nwave ? (p.nwave - 1 - w0) / dw + 1 : 0;
    const int2 wrec = lane < n ? p.wave[w0 + lane * dw] : make_int2(0, 0);
    const u32x4* g = reinterpret_cast<const u32x4*>(src + (size_t)tile * src_rows * TW16);
    for (int i = threadIdx.x; i < src_rows * 8; i += FWD_LDS_NW * 64) xs16[i] = g[i];
    __syncthreads();
    struct It {
        int w;
        int2 wv, pr;
        int4 sg;
        float4 rec;
        bool wok, live;
    };
    auto plan_of = [&](int k, It& it) {         // (k_fwd_lds)
        it.w = w0 + k * dw;
        const int2 v = make_int2(__builtin_amdgcn_readlane(wrec.x, k), __builtin_amdgcn_readlane(wrec.y, k));
        it.wok = v.x >= 0 && v.y >= 0 && (long long)v.x + 64 * (((long long)v.y + 7) / 8) <= p.npos;
        it.wv = it.wok ? v : make_int2(0, 0);
        it.pr = (it.wok && it.wv.y > 0) ? PairLoad<PB>(cw, it.wv.x, lane).step(0) : make_int2(NO_ROW, 0);
        it.live = load_segment(p, it.w * 8 + gi, it.sg) && it.wok;
        it.rec = epi.sinfo && it.w * 8 + gi < p.nseg ? epi.sinfo[it.w * 8 + gi] : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    It cur{}, nx{};                            // (nx stays unused after the last plan wave)
    if (n > 0) plan_of(0, cur);
    for (int k = 0; k < n; ++k) {
        const bool whole = cur.live && cur.sg.y < 0;
        const float b = whole && epi.bias ? (epi.sinfo ? cur.rec.w : epi.bias[cur.sg.x]) : 0.f;
        float acc[8] = {b, b, b, b, b, b, b, b};            // (the bias starts the sum)
        const PairLoad<PB> q(cw, cur.wv.x, lane);
        int2 nxt = cur.pr;
        for (int j = 0, left = cur.wok ? cur.wv.y : 0; left > 0; ++j, left -= 8) {
            int c[8];
            float wt[8];
            stage_pairs<PB>(slots, grp, sub, nxt, false, nullptr, src_rows, c, wt);
            if (left > 8) nxt = q.step(j + 1);
            u32x4 raw[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                raw[u] = u < left && (unsigned)c[u] < (unsigned)src_rows ? xs16[c[u] * 8 + sub] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int u = 0; u < 8; u += 2) fma_pair(wt[u], wt[u + 1], raw[u], raw[u + 1], acc);
        }
        if (k + 1 < n) plan_of(k + 1, nx);
        if (cur.live) {
            if (cur.sg.y >= 0) {
                store8(part + ((size_t)tile * p.nslot + cur.sg.y) * TW16 + sub * 8, acc);
            } else {
                FwdIn16 in{};
                in.g = cur.rec.x;
                in.sp = cur.rec.y;
                if (!epi.sinfo) {
                    const float4 r = epi.info[cur.sg.x];
                    in.g = r.x;
                    in.sp = r.y;
                }
                fwd_finish16(epi, cur.sg.x, tile, sub, acc, in);
            }
        }
        cur = nx;
    }
}

// acc[0..8) += the n partial sums (8 samples each, slot stride TW16 floats from p) of slots y .., in slot order, 4
// slots' loads in flight
__device__ __forceinline__ void add_parts16(const float* __restrict__ p, int y, int n, float acc[8]) {
    int k = 0;
    for (; k + 4 <= n; k += 4) {
        float v[4][8];
#pragma unroll
        for (int u = 0; u < 4; ++u) ldf8(p + (size_t)(y + k + u) * TW16, v[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int m = 0; m < 8; ++m) acc[m] += v[u][m];
    }
    for (; k < n; ++k) {
        float v[8];
        ldf8(p + (size_t)(y + k) * TW16, v);
#pragma unroll
        for (int m = 0; m < 8; ++m) acc[m] += v[m];
    }
}

__global__ __launch_bounds__(WG) void k_cfwd16_combine(Plan p, const float* __restrict__ part, FwdEpi16 epi, int T) {
    long long q = ((long long)blockIdx.x * WG + threadIdx.x);
    const int sub = (int)(q & 7);
    q >>= 3;
    const int tile = (int)(q % T);
    const long long i = q / T;
    int4 s;
    if (!load_split(p, i, s)) return;
    const float b = epi.bias ? epi.bias[s.x] : 0.f;
    float acc[8] = {b, b, b, b, b, b, b, b};
    FwdIn16 in{};
    fwd_inputs16(epi, epi.info, s.x, s.w, tile, sub, in);
    add_parts16(part + (size_t)tile * p.nslot * TW16 + sub * 8, s.y, s.z, acc);
    fwd_finish16(epi, s.x, tile, sub, acc, in);
}

// ------------------------------------------------------------------------------------------------ backward
struct BwdIn16 {
    u32x4 hr;                                   // the layer's h, as stored (8 bfloat16)
    float z[8], gd[8];
    float gn, sp;
    int d;
};
__device__ __forceinline__ u32x4 ldr8(const bf16_t* base, int rows, int tile, int row, int sub) {
    return *reinterpret_cast<const u32x4*>(base + ((size_t)tile * rows + row) * TW16 + sub * 8);
}
// sum over the lane's 8 samples of a * b, both bfloat16 as stored, in float32 (v_dot2_f32_bf16: two exact products
// per instruction, samples in pairs).  The pairs are taken from a whole-vector cast with shufflevector: hipcc turns
// a bit_cast of a vector ELEMENT (a[k]) into a read of element 0 for every k.
__device__ __forceinline__ float dot8(const u32x4& a, const u32x4& b) {
    typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
    const bf8 x = __builtin_bit_cast(bf8, a), y = __builtin_bit_cast(bf8, b);
    float d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 0, 1), __builtin_shufflevector(y, y, 0, 1),
                                              0.f, false);
    d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 2, 3), __builtin_shufflevector(y, y, 2, 3), d, false);
    d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 4, 5), __builtin_shufflevector(y, y, 4, 5), d, false);
    d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 6, 7), __builtin_shufflevector(y, y, 6, 7), d, false);
    return d;
}
// MODE 1: a hop layer (d: the row's re-drive row); 2: the sensory layer
// (hr: the row's h line, already loaded by the caller)
template <int MODE>
// recs: the wave's 8 records in plan order (sinfo + 8 w; the row's is recs[i]), or null: the row's from info
__device__ __forceinline__ void bwd_inputs16(const BwdEpi16& e, int j, int d, int tile, int sub, BwdIn16& in,
                                             const u32x4* hr = nullptr, const float4* recs = nullptr, int i = 0) {
#pragma unroll
    for (int k = 0; k < 8; ++k) in.z[k] = in.gd[k] = 0.f;
    bool load;                               // (re-drive fields as in BwdEpi)
    if constexpr (MODE == 2) {
        in.d = j;
        load = d != -2;
    } else {
        in.d = d <= -3 ? -d - 3 : d;
        load = d >= 0 && !e.first;
    }
    if (load) ldf8(f8p(e.gdrive, e.n_s, tile, in.d, sub), in.gd);
    in.hr = hr ? *hr : ldr8(e.h, e.rows, tile, j, sub);
    if constexpr (MODE == 2) ld8(e.z, e.rows, tile, j, sub, in.z);
    const float2 r = *reinterpret_cast<const float2*>(recs ? recs + i : e.info + j);
    in.gn = r.x;
    in.sp = r.y;
}

// A hop layer's neuron backward for (row, tile) over the lane's 8 samples (hop_back in kernels.hip): gz = g gain with
// g = gh where the stored h > 0, the tile's sums pg = sum g z (from the stored h, see k_bwd) and ps = sum g
struct HopBack16 {
    float gz[8];
    float pg, ps;
};
__device__ __forceinline__ HopBack16 hop_back16(const float (&gh)[8], const u32x4& hr, float gn, float sp) {
    float g[8], h[8];
    float sg = 0.f, sgh = 0.f;
    unpack8<BF16>(hr, h);
    HopBack16 b;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        g[k] = h[k] > 0.f ? gh[k] : 0.f;
        b.gz[k] = g[k] * gn;
        sg += g[k];
        sgh = fmaf(g[k], h[k], sgh);
    }
    b.ps = gsum8(sg);
    b.pg = gn != 0.f ? (gsum8(sgh) + sp * b.ps) / gn : 0.f;
    return b;
}

template <int MODE>
// keep (optional): the row's gain and threshold partials of the tile are returned there instead of stored
// gcol: as in bwd_finish
__device__ __forceinline__ void bwd_finish16(const BwdEpi16& e, int j, int tile, int sub, const float (&gh)[8],
                                             const BwdIn16& in, float2* keep = nullptr, int gcol = -1) {
    float gzv[8], ps, pg;
    if constexpr (MODE == 1) {
        const HopBack16 hb = hop_back16(gh, in.hr, in.gn, in.sp);
#pragma unroll
        for (int k = 0; k < 8; ++k) gzv[k] = hb.gz[k];
        ps = hb.ps;
        pg = hb.pg;
    } else {
        float g[8], h[8];
        float sg = 0.f, sgh = 0.f;
        unpack8<BF16>(in.hr, h);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            g[k] = h[k] > 0.f ? gh[k] : 0.f;
            gzv[k] = g[k] * in.gn;
            sg += g[k];
            sgh = fmaf(g[k], in.z[k], sgh);
        }
        ps = gsum8(sg);
        pg = gsum8(sgh);
    }
    if (keep) {
        *keep = make_float2(pg, ps);
    } else if (sub == 0) {
        const int col = gcol >= 0 ? gcol : j;
        e.ggain_part[(size_t)tile * e.gp_ld + col] = pg;
        e.gsum_part[(size_t)tile * e.gp_ld + col] = ps;
    }
    if constexpr (MODE == 1) {
        st8(e.gz_out, e.rows, tile, j, sub, gzv);
        if (in.d >= 0) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = in.gd[k] + gzv[k];
            store8(f8p(e.gdrive, e.n_s, tile, in.d, sub), v);
        }
        return;
    }
    // the sensory layer: the drive's gradient is complete -> the plug's bias and per-connection gradients
    float gd[8];
    float sb = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        gd[k] = in.gd[k] + gzv[k];
        sb += gd[k];
    }
    const float pb = gsum8(sb);
    if (sub == 0) e.ginb_part[(size_t)tile * e.gb_ld + j] = pb;
    float* gwo = e.ginw_part + (size_t)tile * e.gw_ld;
    const int f0 = e.in_crow[j], f1 = e.in_crow[j + 1];
    for (int f = f0; f < f1; f += 8) {
        const int mc = f + sub < f1 ? e.in_col[f + sub] : NO_ROW;
        int c[8];
        c[0] = bcast8<0>(mc); c[1] = bcast8<1>(mc); c[2] = bcast8<2>(mc); c[3] = bcast8<3>(mc);
        c[4] = bcast8<4>(mc); c[5] = bcast8<5>(mc); c[6] = bcast8<6>(mc); c[7] = bcast8<7>(mc);
        float dd[8];
#pragma unroll
        for (int s2 = 0; s2 < 8; ++s2) {
            const bool ok = (unsigned)c[s2] < (unsigned)e.x_rows;
            float xv[8];
            ld8(e.x, e.x_rows, tile, ok ? c[s2] : 0, sub, xv);
            float dp = 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) dp = fmaf(gd[k], xv[k], dp);
            dd[s2] = ok ? dp : 0.f;
        }
        const float pw = rs8(dd, sub);
        if (f + sub < f1) gwo[f + sub] = pw;
    }
}

// over the transposed plan (rows = the layer below, j): gh_j = sum W gz (gathered), the per-edge weight gradient
// partial sum over the tile of gz * h_j, then the layer's neuron backward
template <int MODE, int PB>
__global__ __launch_bounds__(WG) void k_cbwd16(Plan p, const int2* __restrict__ cw, const bf16_t* __restrict__ gz,
                                               int gz_rows, float* __restrict__ gwpart, long long gw_ld, BwdEpi16 epi,
                                               float* __restrict__ part, int T, int RB) {
    __shared__ __align__(16) int2 slots[WG / LPR][LPR];
    int rb;
    const int tile = tile_of(blockIdx.x, RB, T, rb);
    const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7, lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(rb * (WG / 64) + (int)(threadIdx.x >> 6));
    int2 wv;
    const bool wok = load_wave(p, w, wv);
    const PairLoad<PB> q(cw, wv.x, lane);
    int2 nxt = (wok && wv.y > 0) ? q.step(0) : make_int2(NO_ROW, 0);
    int4 sg;
    const bool live = load_segment(p, w * 8 + (grp & 7), sg) && wok;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(gz + (size_t)tile * gz_rows * TW16), (short)0, gz_rows * 128, 0x00020000);
    float* gwp = gwpart ? gwpart + (size_t)tile * gw_ld + wv.x + lane : nullptr;
    // the row's h, as stored (the weight gradient's operand), first: where the row fires on no sample of the tile its
    // g is zero, and its gathers are skipped (as in k_bwd)
    u32x4 hj = {0u, 0u, 0u, 0u};
    if (live) hj = ldr8(epi.h, epi.rows, tile, sg.x, sub);
    const bool quiet = epi.skip_silent && group_silent(bf16_lane_fires(hj));
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int j = 0, left = wok ? wv.y : 0;
    float pend = 0.f;                           // (a step's partial is stored after the next step's gathers: k_bwd)
    auto step = [&](auto full) {               // (as in k_cfwd16: full steps, then the wave's last)
        constexpr bool FULL = decltype(full)::value;
        int c[8];
        float wt[8];
        stage_pairs<PB>(slots, grp, sub, nxt, false, nullptr, gz_rows, c, wt);
        u32x4 raw[8];
#pragma unroll
        for (int s = 0; s < 8; ++s)
            raw[s] = (FULL || s < left) ? gather16(rs, quiet ? NO_ROW : c[s], sub) : u32x4{0u, 0u, 0u, 0u};
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (FULL) nxt = q.step(j + 1);
        if (gwp && j > 0) gwp[64 * (j - 1)] = pend;
        __builtin_amdgcn_sched_barrier(0);
        float d[8];
#pragma unroll
        for (int s = 0; s < 8; s += 2)
            if (FULL || s < left) fma_pair(wt[s], wt[s + 1], raw[s], raw[s + 1], acc);
#pragma unroll
        for (int s = 0; s < 8; ++s) d[s] = (FULL || s < left) ? dot8(hj, raw[s]) : 0.f;   // (0: no edge there)
        if (gwp) pend = rs8(d, sub);
    };
    for (; left > 8; ++j, left -= 8) step(Full<true>{});
    if (left > 0) step(Full<false>{});
    if (gwp && left > 0) gwp[64 * j] = pend;    // (the last step's)
    if (!live) return;
    if (sg.y >= 0) {
        store8(part + ((size_t)tile * p.nslot + sg.y) * TW16 + sub * 8, acc);
        return;
    }
    BwdIn16 in{};                               // the row's other inputs, after the loop (k_bwd)
    bwd_inputs16<MODE>(epi, sg.x, sg.z, tile, sub, in, &hj, epi.sinfo ? epi.sinfo + 8 * w : nullptr, grp & 7);
    bwd_finish16<MODE>(epi, sg.x, tile, sub, acc, in, nullptr, w * 8 + (grp & 7));
}

// The same over two tiles at once, tiles 2 pr and 2 pr + 1 of a pair pr (the second may not exist): a step gathers
// the source lines of both tiles for the same (source, weight) pairs, and the weight-gradient partial of a position is
// summed over both tiles (tile 2 pr first) and stored once per pair: gwpart [ceil(T / 2)][gw_ld]
template <int MODE, int PB>
__global__ __launch_bounds__(WG) void k_cbwd16x2(Plan p, const int2* __restrict__ cw, const bf16_t* __restrict__ gz,
                                                 int gz_rows, float* __restrict__ gwpart, long long gw_ld, BwdEpi16 epi,
                                                 float* __restrict__ part, int T, int RB) {
    __shared__ __align__(16) int2 slots[WG / LPR][LPR];
    int rb;
    const int pr = tile_of(blockIdx.x, RB, (T + 1) / 2, rb);
    const int ta = 2 * pr, tb = 2 * pr + 1;
    const bool hasb = tb < T;
    const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7, lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(rb * (WG / 64) + (int)(threadIdx.x >> 6));
    int2 wv;
    const bool wok = load_wave(p, w, wv);
    const PairLoad<PB> q(cw, wv.x, lane);
    int2 nxt = (wok && wv.y > 0) ? q.step(0) : make_int2(NO_ROW, 0);
    int4 sg;
    const bool live = load_segment(p, w * 8 + (grp & 7), sg) && wok;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(gz + (size_t)ta * gz_rows * TW16), (short)0, gz_rows * 128, 0x00020000);
    const __amdgpu_buffer_rsrc_t rbs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(gz + (size_t)(hasb ? tb : ta) * gz_rows * TW16), (short)0, hasb ? gz_rows * 128 : 0, 0x00020000);
    float* gwp = gwpart ? gwpart + (size_t)pr * gw_ld + wv.x + lane : nullptr;
    // the row's h lines first, and on a tile where the row fires on no sample its gathers are skipped (k_cbwd16)
    u32x4 hja = {0u, 0u, 0u, 0u}, hjb = {0u, 0u, 0u, 0u};
    if (live) {
        hja = ldr8(epi.h, epi.rows, ta, sg.x, sub);
        if (hasb) hjb = ldr8(epi.h, epi.rows, tb, sg.x, sub);
    }
    const bool quiet_a = epi.skip_silent && group_silent(bf16_lane_fires(hja));
    const bool quiet_b = epi.skip_silent && group_silent(bf16_lane_fires(hjb));
    float acca[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, accb[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int j = 0, left = wok ? wv.y : 0;
    float pend = 0.f;                           // (a step's partial is stored after the next step's gathers: k_bwd)
    auto step = [&](auto full) {
        constexpr bool FULL = decltype(full)::value;
        int c[8];
        float wt[8];
        stage_pairs<PB>(slots, grp, sub, nxt, false, nullptr, gz_rows, c, wt);
        u32x4 va[8], vb[8];
#pragma unroll
        for (int s = 0; s < 8; ++s)
            va[s] = (FULL || s < left) ? gather16(ra, quiet_a ? NO_ROW : c[s], sub) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int s = 0; s < 8; ++s)
            vb[s] = (FULL || s < left) ? gather16(rbs, quiet_b ? NO_ROW : c[s], sub) : u32x4{0u, 0u, 0u, 0u};
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (FULL) nxt = q.step(j + 1);
        if (gwp && j > 0) gwp[64 * (j - 1)] = pend;
        __builtin_amdgcn_sched_barrier(0);
        float d[8];
#pragma unroll
        for (int s = 0; s < 8; s += 2)
            if (FULL || s < left) {
                fma_pair(wt[s], wt[s + 1], va[s], va[s + 1], acca);
                fma_pair(wt[s], wt[s + 1], vb[s], vb[s + 1], accb);
            }
#pragma unroll
        for (int s = 0; s < 8; ++s) d[s] = (FULL || s < left) ? dot8(hja, va[s]) + dot8(hjb, vb[s]) : 0.f;
        if (gwp) pend = rs8(d, sub);
    };
    for (; left > 8; ++j, left -= 8) step(Full<true>{});
    if (left > 0) step(Full<false>{});
    if (gwp && left > 0) gwp[64 * j] = pend;    // (the last step's)
    if (!live) return;
    if (sg.y >= 0) {
        store8(part + ((size_t)ta * p.nslot + sg.y) * TW16 + sub * 8, acca);
        if (hasb) store8(part + ((size_t)tb * p.nslot + sg.y) * TW16 + sub * 8, accb);
        return;
    }
    BwdIn16 ina{}, inb{};                       // the rows' other inputs, after the loop (k_bwd)
    const float4* recs = epi.sinfo ? epi.sinfo + 8 * w : nullptr;
    bwd_inputs16<MODE>(epi, sg.x, sg.z, ta, sub, ina, &hja, recs, grp & 7);
    if (hasb) bwd_inputs16<MODE>(epi, sg.x, sg.z, tb, sub, inb, &hjb, recs, grp & 7);
    float2 ka, kb = make_float2(0.f, 0.f);
    bwd_finish16<MODE>(epi, sg.x, ta, sub, acca, ina, &ka);
    if (hasb) bwd_finish16<MODE>(epi, sg.x, tb, sub, accb, inb, &kb);
    if (sub == 0) {                             // the row's gain and threshold partials, one per pair of tiles
        const int col = w * 8 + (grp & 7);      // (the plan column of the row: its segment)
        epi.ggain_part[(size_t)pr * epi.gp_ld + col] = ka.x + kb.x;
        epi.gsum_part[(size_t)pr * epi.gp_ld + col] = ka.y + kb.y;
    }
}

// PAIR: an 8-lane group finishes the split row for both tiles of a pair and stores the row's gain and threshold
// partials once per pair, as k_cbwd16x2 does
template <int MODE, bool PAIR>
__global__ __launch_bounds__(WG) void k_cbwd16_combine(Plan p, const float* __restrict__ part, BwdEpi16 epi, int T) {
    const int NT = PAIR ? (T + 1) / 2 : T;
    long long q = ((long long)blockIdx.x * WG + threadIdx.x);
    const int sub = (int)(q & 7);
    q >>= 3;
    const int u = (int)(q % NT);
    const long long i = q / NT;
    int4 s;
    if (!load_split(p, i, s)) return;
    float2 k2[2] = {make_float2(0.f, 0.f), make_float2(0.f, 0.f)};
    for (int h = 0; h < (PAIR ? 2 : 1) && (PAIR ? 2 * u + h : u) < T; ++h) {
        const int tile = PAIR ? 2 * u + h : u;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        BwdIn16 in{};
        bwd_inputs16<MODE>(epi, s.x, s.w, tile, sub, in);
        add_parts16(part + (size_t)tile * p.nslot * TW16 + sub * 8, s.y, s.z, acc);
        bwd_finish16<MODE>(epi, s.x, tile, sub, acc, in, PAIR ? &k2[h] : nullptr, (int)(p.nseg + i));
    }
    if (PAIR && sub == 0) {
        epi.ggain_part[(size_t)u * epi.gp_ld + p.nseg + i] = k2[0].x + k2[1].x;
        epi.gsum_part[(size_t)u * epi.gp_ld + p.nseg + i] = k2[0].y + k2[1].y;
    }
}

// ------------------------------------------------------------------------------------------------ x, read-out
// obs [B][obs_dim] float32 -> x [T][obs_dim][64] bfloat16; one workgroup per (tile, 64 features)
__global__ __launch_bounds__(WG) void k_obs_in16(const float* __restrict__ obs, bf16_t* __restrict__ x, int obs_dim) {
    __shared__ float s[TW16][65];
    const int tile = blockIdx.y, f0 = blockIdx.x * 64;
    for (int i = threadIdx.x; i < TW16 * 64; i += WG) {
        const int c = i / 64, f = i % 64;
        s[c][f] = (f0 + f < obs_dim) ? obs[(size_t)(tile * TW16 + c) * obs_dim + f0 + f] : 0.f;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < TW16 * 64; i += WG) {
        const int f = i / TW16, c = i % TW16;
        if (f0 + f < obs_dim) x[((size_t)tile * obs_dim + f0 + f) * TW16 + c] = __builtin_bit_cast(bf16_t, (__bf16)s[c][f]);
    }
}

// gh of the top layer from the logits' gradient on the matrix cores (readout.h): 32 rows x the tile's 64 samples
// (two 32-sample blocks), then its neuron backward
__global__ __launch_bounds__(WG) void k_rbwd_h16_mfma(const float* __restrict__ dl, const float* __restrict__ owT, int ma,
                                                      const int* __restrict__ dn_inv, int n_act, int rows, BwdEpi16 epi) {
    __shared__ float part[4 * 32 * 33];
    __shared__ float gh[32 * 65];
    const int tile = blockIdx.y, r0 = blockIdx.x * RPG;
    readout_gh_block(dl, owT, ma, dn_inv, rows, n_act, r0, tile * TW16, part, gh, 65);
    readout_gh_block(dl, owT, ma, dn_inv, rows, n_act, r0, tile * TW16 + 32, part, gh + 32, 65);
    const int r = threadIdx.x >> 3, sub = threadIdx.x & 7, t = r0 + r;
    if (t >= rows) return;                   // whole 8-lane groups
    float acc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = gh[r * 65 + sub * 8 + k];
    BwdIn16 in{};
    bwd_inputs16<1>(epi, t, epi.drow ? epi.drow[t] : -1, tile, sub, in);
    bwd_finish16<1>(epi, t, tile, sub, acc, in);
}

// a 16-bit state -> [rows][B] float32 (tests and diagnostics)
__global__ void k_export16(const bf16_t* __restrict__ src, int rows, float* __restrict__ dst, int B) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)rows * B) return;
    const int r = (int)(i / B), b = (int)(i % B);
    dst[i] = __uint_as_float((unsigned)src[((size_t)(b / TW16) * rows + r) * TW16 + (b % TW16)] << 16);
}

// ------------------------------------------------------------------------------------------------ launchers
static inline unsigned nblocks(long long n, int per = WG) { return (unsigned)((n + per - 1) / per); }

hipError_t launch_obs_in16(const float* obs, unsigned short* x, int obs_dim, int B, hipStream_t st) {
    k_obs_in16<<<dim3((unsigned)((obs_dim + 63) / 64), (unsigned)(B / TW16)), WG, 0, st>>>(obs, x, obs_dim);
    return hipGetLastError();
}

hipError_t launch_fwd16c(const Plan& p, const int2* cw, const unsigned short* src, int src_rows, const FwdEpi16& epi,
                         float* part, int T, hipStream_t st, const unsigned* src_fires) {
    // (6-byte pairs: a slab of at most PAIR6_MAX_ROWS rows, as launch_fwd)
    if ((p.pb != 8 && p.pb != 6) || (p.pb == 6 && src_rows > PAIR6_MAX_ROWS)) return hipErrorInvalidValue;
    if (p.nwave > 0) {
        const int RB = (p.nwave + WG / 64 - 1) / (WG / 64);
        const int fw = src_fires && fires_ld(src_rows) <= FIRES_LDS_WORDS ? fires_ld(src_rows) : 0;
        const dim3 grid((unsigned)((long long)T * RB));
        const size_t lds = (size_t)(fw > 0 ? fw - 4 : 0) * 4;
        if (p.pb == 6)
            k_cfwd16<6><<<grid, WG, lds, st>>>(p, cw, src, src_rows, epi, part, T, RB, src_fires, fw);
        else
            k_cfwd16<8><<<grid, WG, lds, st>>>(p, cw, src, src_rows, epi, part, T, RB, src_fires, fw);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (p.nsplit > 0) {
        k_cfwd16_combine<<<nblocks((long long)p.nsplit * T * LPR), WG, 0, st>>>(p, part, epi, T);
        return hipGetLastError();
    }
    return hipSuccess;
}

bool lds_fits(std::initializer_list<const void*> kernels);
bool lds_plug_fits16() {
    return lds_fits({reinterpret_cast<const void*>(&k_cfwd16_lds<8>), reinterpret_cast<const void*>(&k_cfwd16_lds<6>)});
}

hipError_t launch_fwd16c_lds(const Plan& p, const int2* cw, const unsigned short* src, int src_rows,
                             const FwdEpi16& epi, float* part, int T, int S, hipStream_t st) {
    const size_t lds = (size_t)src_rows * 128;
    if (S < 1 || src_rows < 1 || lds > FWD_LDS_BYTES || epi.drive || !epi.info || (p.pb != 8 && p.pb != 6) ||
        (p.pb == 6 && src_rows > PAIR6_MAX_ROWS))
        return hipErrorInvalidValue;
    S = std::max(S, (p.nwave + 64 * FWD_LDS_NW - 1) / (64 * FWD_LDS_NW));     // (at most 64 plan waves per wave)
    if (p.nwave > 0) {
        const void* k =
            p.pb == 6 ? reinterpret_cast<const void*>(&k_cfwd16_lds<6>) : reinterpret_cast<const void*>(&k_cfwd16_lds<8>);
        const hipError_t attr = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)FWD_LDS_BYTES);
        if (attr != hipSuccess) return attr;       // (k_fwd_lds)
        const dim3 grid((unsigned)((long long)T * S));
        if (p.pb == 6)
            k_cfwd16_lds<6><<<grid, FWD_LDS_NW * 64, lds, st>>>(p, cw, (const bf16_t*)src, src_rows, epi, part, T, S);
        else
            k_cfwd16_lds<8><<<grid, FWD_LDS_NW * 64, lds, st>>>(p, cw, (const bf16_t*)src, src_rows, epi, part, T, S);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (p.nsplit > 0) {
        k_cfwd16_combine<<<nblocks((long long)p.nsplit * T * LPR), WG, 0, st>>>(p, part, epi, T);
        return hipGetLastError();
    }
    return hipSuccess;
}

// The last hop's backward with the descending layer's gradient staged in LDS: k_bwd_lds (kernels.hip) over
// bfloat16 states.  The `hot` most gathered rows of the tile's gz slab (64 samples, 128 bytes a row) sit in LDS, with a
// row of zeros after them; a pair's code names an LDS row (code < hot) or a slab row (hot + row), and plan waves marked
// WLDS_COLD gather their slab rows through the vector-memory path.  The sums are k_cbwd16's (one tile per workgroup),
// term for term in the same order; every plan wave issues the same loads and stores, as in k_bwd_lds.
template <int PB, bool SKIP>
__global__ __launch_bounds__(BWD_LDS_NW * 64) void k_cbwd16_lds(Plan p, const int2* __restrict__ wlds,
                                                               const int2* __restrict__ cw, const bf16_t* __restrict__ gz,
                                                               int gz_rows, const int* __restrict__ hot_rows, int hot,
                                                               float* __restrict__ gwpart, long long gw_ld, BwdEpi16 epi,
                                                               float* __restrict__ part, int T, int S) {
    constexpr int NT = BWD_LDS_NW * 64;
    constexpr int STAGE = (BWD_LDS_MAXROWS * LPR + NT - 1) / NT;
    __shared__ __align__(16) int2 slots[NT / LPR][LPR];
    extern __shared__ __align__(16) u32x4 gs16[];          // LDS row r: slab row hot_rows[r]; row `hot`: zeros
    int s;
    const int tile = tile_of(blockIdx.x, S, T, s);
    const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7, lane = threadIdx.x & 63, gi = grp & 7;
    const int w0 = __builtin_amdgcn_readfirstlane(s * BWD_LDS_NW + (int)(threadIdx.x >> 6)), dw = S * BWD_LDS_NW;
    const int n = w0 < p.nwave ? min((p.nwave - 1 - w0) / dw + 1, 64 * BWD_LDS_WREC) : 0;
    int2 wrec[BWD_LDS_WREC];
#pragma unroll
    for (int r = 0; r < BWD_LDS_WREC; ++r)
        wrec[r] = 64 * r + lane < n ? wlds[w0 + (64 * r + lane) * dw] : make_int2(0, 0);
    const u32x4* gt = reinterpret_cast<const u32x4*>(gz + (size_t)tile * gz_rows * TW16);
    {
        int ri[STAGE];
        u32x4 lv[STAGE];
#pragma unroll
        for (int u = 0; u < STAGE; ++u) {
            const int i = (int)threadIdx.x + u * NT;
            ri[u] = i < hot * LPR ? hot_rows[i / LPR] : -1;
        }
#pragma unroll
        for (int u = 0; u < STAGE; ++u) {
            const int i = (int)threadIdx.x + u * NT;
            lv[u] = (unsigned)ri[u] < (unsigned)gz_rows ? gt[(size_t)ri[u] * LPR + (i % LPR)] : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < STAGE; ++u) {
            const int i = (int)threadIdx.x + u * NT;
            if (i < hot * LPR) gs16[i] = lv[u];
        }
        if (threadIdx.x < LPR) gs16[hot * LPR + threadIdx.x] = u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(gz + (size_t)tile * gz_rows * TW16), (short)0, gz_rows * 128, 0x00020000);
    struct Pre {
        int w;
        int2 wv;
        bool wok, cold, sok;
        int2 pr0, pr1;
        int4 sg;
        float2 rec;
    };
    auto issue = [&](int k, Pre& it) __attribute__((always_inline)) {
        const bool real = k < n;
        k = min(k, n - 1);
        it.w = w0 + k * dw;
        const int r = k >> 6, kk = k & 63;
        int vx = 0, vy = 0;
#pragma unroll
        for (int q = 0; q < BWD_LDS_WREC; ++q)
            if (q == r) {
                vx = __builtin_amdgcn_readlane(wrec[q].x, kk);
                vy = __builtin_amdgcn_readlane(wrec[q].y, kk);
            }
        it.cold = (vy & WLDS_COLD) != 0;
        vy &= ~WLDS_COLD;
        it.wok = real && vx >= 0 && vy >= 0 && (long long)vx + 64 * (((long long)vy + 7) / 8) <= p.npos;
        it.wv = it.wok ? make_int2(vx, vy) : make_int2(0, 0);
        const int2* pq;
        int ps;
        if constexpr (PB == 8) {
            pq = cw + it.wv.x + lane;
            ps = 64;
        } else {
            pq = cw + (size_t)it.wv.x / 64 * 48 + min(lane, 47);
            ps = 48;
        }
        it.pr0 = pq[0];
        it.pr1 = pq[it.wv.y > 8 ? ps : 0];
        it.sok = it.w * 8 + gi < p.nseg;
        const int si = min(it.w * 8 + gi, p.nseg - 1);
        it.sg = p.seg[si];
        it.rec = *reinterpret_cast<const float2*>(epi.sinfo + si);
    };
    auto live = [&](const Pre& it) { return it.wok && it.sok && it.sg.x >= 0 && it.sg.x < p.rows && it.sg.y < p.nslot; };
    auto hline = [&](const Pre& it) { return ldr8(epi.h, epi.rows, tile, live(it) ? it.sg.x : 0, sub); };
    // one step: gathers from LDS (every code from hot up reads the row of zeros), the sums, the step's partial
    auto step = [&](bool cold, int2 pr, bool quiet, const u32x4& hc, float (&acc)[8]) __attribute__((always_inline)) {
        int c[8];
        float wt[8];
        stage_pairs<PB>(slots, grp, sub, pr, false, nullptr, 0, c, wt);
        if (SKIP && quiet) {
#pragma unroll
            for (int u = 0; u < 8; ++u) c[u] = NO_ROW;
        }
        u32x4 raw[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) raw[u] = gs16[min((unsigned)c[u], (unsigned)hot) * LPR + sub];
        if (cold) {
            unsigned cr[8];
            bool any = false;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                cr[u] = (unsigned)c[u] - (unsigned)hot;
                any |= cr[u] < (unsigned)gz_rows;
            }
            if (__ballot(any)) {
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (cr[u] < (unsigned)gz_rows) raw[u] = gather16(rs, (int)cr[u], sub);
                asm volatile("" ::"v"(raw[0][0]), "v"(raw[1][0]), "v"(raw[2][0]), "v"(raw[3][0]), "v"(raw[4][0]),
                             "v"(raw[5][0]), "v"(raw[6][0]), "v"(raw[7][0]));   // (waited for here)
            }
        }
#pragma unroll
        for (int u = 0; u < 8; u += 2) fma_pair(wt[u], wt[u + 1], raw[u], raw[u + 1], acc);
        float d[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) d[u] = dot8(hc, raw[u]);
        return rs8(d, sub);
    };
    constexpr unsigned OFF = 0x80000000u;
    auto rsrc = [](const void* b, long long bytes) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(b), (short)0,
                                                 b ? (int)min(bytes, 0x7FFFFFFFLL) : 0, 0x00020000);
    };
    const __amdgpu_buffer_rsrc_t r_gw = rsrc(gwpart ? gwpart + (size_t)tile * gw_ld : nullptr, gw_ld * 4);
    const __amdgpu_buffer_rsrc_t r_gz = rsrc(epi.gz_out + (size_t)tile * epi.rows * TW16, (long long)epi.rows * 128);
    const __amdgpu_buffer_rsrc_t r_gd = rsrc(epi.gdrive + (size_t)tile * epi.n_s * TW16, (long long)epi.n_s * 256);
    const __amdgpu_buffer_rsrc_t r_pt = rsrc(part ? part + (size_t)tile * p.nslot * TW16 : nullptr, (long long)p.nslot * 256);
    const __amdgpu_buffer_rsrc_t r_gg = rsrc(epi.ggain_part + (size_t)tile * epi.gp_ld, epi.gp_ld * 4);
    const __amdgpu_buffer_rsrc_t r_gs = rsrc(epi.gsum_part + (size_t)tile * epi.gp_ld, epi.gp_ld * 4);
    // (the buffer stores take the values' bits; aux 2: nontemporal, as st8 and the float32 kernels' stores)
    auto st1 = [](float v, __amdgpu_buffer_rsrc_t r, unsigned off) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 0);
    };
    auto st8f = [](const float (&v)[8], __amdgpu_buffer_rsrc_t r, unsigned off) {     // 8 floats, off 32-byte aligned
        const u32x4 a = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
        const u32x4 b = {__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])};
        __builtin_amdgcn_raw_buffer_store_b128(a, r, off, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(b, r, off == OFF ? OFF : off + 16u, 0, 0);
    };
    // Plan wave k (k_bwd_lds's plan_wave): 5 loads and 10 stores whatever its rows
    auto plan_wave = [&](int k, const Pre& cur, const u32x4& hr, const Pre& nx, u32x4& hn, Pre& n2)
        __attribute__((always_inline)) {
        issue(k + 2, n2);
        hn = hline(nx);
        const bool lv = live(cur);
        const u32x4 hc = lv ? hr : u32x4{0u, 0u, 0u, 0u};
        const bool quiet = SKIP && group_silent(bf16_lane_fires(hc));
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        const int L = cur.wv.y;
        float pend0 = 0.f, pend1 = 0.f;
        if (L > 0) pend0 = step(cur.cold, cur.pr0, quiet, hc, acc);
        if (L > 8) pend1 = step(cur.cold, cur.pr1, quiet, hc, acc);
        if (L > 16) {                                 // (rare: a third step and more, their pairs loaded here)
            const PairLoad<PB> q(cw, cur.wv.x, lane);
            for (int j = 2; 8 * j < L; ++j) {
                int2 pr = q.step(j);
                asm volatile("" : "+v"(pr.x), "+v"(pr.y));
                const float pe = step(cur.cold, pr, quiet, hc, acc);
                st1(pe, r_gw, (unsigned)(cur.wv.x + 64 * j + lane) * 4u);
            }
        }
        st1(pend0, r_gw, L > 0 ? (unsigned)(cur.wv.x + lane) * 4u : OFF);
        st1(pend1, r_gw, L > 8 ? (unsigned)(cur.wv.x + 64 + lane) * 4u : OFF);
        const bool whole = lv && cur.sg.y < 0;
        const HopBack16 b = hop_back16(acc, hc, cur.rec.x, cur.rec.y);
        const int d = cur.sg.z, dr = d <= -3 ? -d - 3 : d;
        float gd[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        const bool add = whole && d >= 0 && !epi.first;
        if (__ballot(add)) {                          // (rare: a drive gradient written by a layer above)
            float g[8];
            ldf8(f8p(epi.gdrive, epi.n_s, tile, add ? dr : 0, sub), g);
#pragma unroll
            for (int m = 0; m < 8; ++m) gd[m] = add ? g[m] : 0.f;
            asm volatile("" : "+v"(gd[0]), "+v"(gd[1]), "+v"(gd[2]), "+v"(gd[3]), "+v"(gd[4]), "+v"(gd[5]), "+v"(gd[6]),
                         "+v"(gd[7]));
        }
        float v[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) v[m] = gd[m] + b.gz[m];
        u32x4 o;
#pragma unroll
        for (int m = 0; m < 4; ++m) o[m] = pack2(b.gz[2 * m], b.gz[2 * m + 1]);
        __builtin_amdgcn_raw_buffer_store_b128(o, r_gz, whole ? (unsigned)cur.sg.x * 128u + (unsigned)sub * 16u : OFF, 0, 2);
        st8f(v, r_gd, whole && dr >= 0 ? (unsigned)dr * 256u + (unsigned)sub * 32u : OFF);
        st8f(acc, r_pt, lv && cur.sg.y >= 0 ? (unsigned)cur.sg.y * 256u + (unsigned)sub * 32u : OFF);
        const unsigned col = whole && sub == 0 ? (unsigned)(cur.w * 8 + gi) * 4u : OFF;
        st1(b.pg, r_gg, col);
        st1(b.ps, r_gs, col);
    };
    if (n <= 0) return;
    Pre p0, p1, p2;
    u32x4 h0, h1;
    issue(0, p0);
    issue(1, p1);
    h0 = hline(p0);
    {                                           // (the 10 stores a plan wave ends with, all dropped: k_bwd_lds)
        const float z8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        st1(0.f, r_gw, OFF);
        st1(0.f, r_gw, OFF);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, r_gz, OFF, 0, 2);
        st8f(z8, r_gd, OFF);
        st8f(z8, r_pt, OFF);
        st1(0.f, r_gg, OFF);
        st1(0.f, r_gs, OFF);
    }
    int k = 0;
    for (; k + 6 <= n; k += 6) {
        plan_wave(k, p0, h0, p1, h1, p2);
        plan_wave(k + 1, p1, h1, p2, h0, p0);
        plan_wave(k + 2, p2, h0, p0, h1, p1);
        plan_wave(k + 3, p0, h1, p1, h0, p2);
        plan_wave(k + 4, p1, h0, p2, h1, p0);
        plan_wave(k + 5, p2, h1, p0, h0, p1);
    }
    if (k < n) plan_wave(k, p0, h0, p1, h1, p2);
    if (k + 1 < n) plan_wave(k + 1, p1, h1, p2, h0, p0);
    if (k + 2 < n) plan_wave(k + 2, p2, h0, p0, h1, p1);
    if (k + 3 < n) plan_wave(k + 3, p0, h1, p1, h0, p2);
    if (k + 4 < n) plan_wave(k + 4, p1, h0, p2, h1, p0);
}

int bwd_lds_rows16() {
    int dev = 0, cap = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cap, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return 0;
    size_t stat = 0;
    for (const void* k : {reinterpret_cast<const void*>(&k_cbwd16_lds<8, false>), reinterpret_cast<const void*>(&k_cbwd16_lds<6, false>),
                          reinterpret_cast<const void*>(&k_cbwd16_lds<8, true>), reinterpret_cast<const void*>(&k_cbwd16_lds<6, true>)}) {
        hipFuncAttributes a{};
        if (hipFuncGetAttributes(&a, k) != hipSuccess) return 0;
        stat = std::max(stat, a.sharedSizeBytes);
    }
    if ((size_t)cap <= stat) return 0;
    const size_t rows = ((size_t)cap - stat) / 128;
    return rows < 2 ? 0 : (int)std::min<size_t>(rows - 1, BWD_LDS_MAXROWS);      // (less the row of zeros)
}

hipError_t launch_bwd16c_lds(const Plan& p, const int2* wlds, const int2* cw, const unsigned short* gz, int gz_rows,
                             const int* hot_rows, int hot, float* gwpart, long long gw_ld, const BwdEpi16& epi,
                             float* part, int T, int S, hipStream_t st) {
    if (epi.mode != 1 || !epi.sinfo || !epi.h || !epi.gz_out || !epi.gdrive || !epi.ggain_part || !epi.gsum_part ||
        !wlds || !hot_rows || hot < 1 || hot > BWD_LDS_MAXROWS || hot > gz_rows || S < 1 || (p.pb != 8 && p.pb != 6) ||
        (p.pb == 6 && (long long)hot + gz_rows > PAIR6_MAX_ROWS))
        return hipErrorInvalidValue;
    if (p.nwave > 0) {
        S = std::max(S, (p.nwave + 64 * BWD_LDS_WREC * BWD_LDS_NW - 1) / (64 * BWD_LDS_WREC * BWD_LDS_NW));
        const void* k = p.pb == 6 ? (epi.skip_silent ? reinterpret_cast<const void*>(&k_cbwd16_lds<6, true>)
                                                     : reinterpret_cast<const void*>(&k_cbwd16_lds<6, false>))
                                  : (epi.skip_silent ? reinterpret_cast<const void*>(&k_cbwd16_lds<8, true>)
                                                     : reinterpret_cast<const void*>(&k_cbwd16_lds<8, false>));
        const size_t lds = (size_t)(hot + 1) * 128;           // (and a row of zeros)
        const hipError_t attr = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (attr != hipSuccess) return attr;
        const dim3 grid((unsigned)((long long)T * S));
#define FG_CBWD_LDS(P, K) k_cbwd16_lds<P, K><<<grid, BWD_LDS_NW * 64, lds, st>>>(p, wlds, cw, (const bf16_t*)gz, gz_rows, \
                                                                                   hot_rows, hot, gwpart, gw_ld, epi, part, T, S)
        if (p.pb == 6) {
            if (epi.skip_silent) FG_CBWD_LDS(6, true); else FG_CBWD_LDS(6, false);
        } else {
            if (epi.skip_silent) FG_CBWD_LDS(8, true); else FG_CBWD_LDS(8, false);
        }
#undef FG_CBWD_LDS
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (p.nsplit > 0) {
        k_cbwd16_combine<1, false><<<nblocks((long long)p.nsplit * T * LPR), WG, 0, st>>>(p, part, epi, T);
        return hipGetLastError();
    }
    return hipSuccess;
}

template <int MODE, int PB>
static void launch_bwd16c_kernel(const Plan& p, const int2* cw, const unsigned short* gz, int gz_rows, float* gwpart,
                                 long long gw_ld, const BwdEpi16& epi, float* part, int T, bool pair, hipStream_t st) {
    const int RB = (p.nwave + WG / 64 - 1) / (WG / 64);
    // a hop layer may take two tiles per workgroup; the sensory layer's epilogue leaves no VGPRs for a second
    if (MODE == 1 && pair)
        k_cbwd16x2<1, PB><<<(unsigned)((long long)((T + 1) / 2) * RB), WG, 0, st>>>(p, cw, gz, gz_rows, gwpart, gw_ld,
                                                                                   epi, part, T, RB);
    else
        k_cbwd16<MODE, PB><<<(unsigned)((long long)T * RB), WG, 0, st>>>(p, cw, gz, gz_rows, gwpart, gw_ld, epi, part, T,
                                                                        RB);
}

template <int MODE>
static hipError_t launch_bwd16c_as(const Plan& p, const int2* cw, const unsigned short* gz, int gz_rows, float* gwpart,
                                   long long gw_ld, const BwdEpi16& epi, float* part, int T, bool pair, hipStream_t st) {
    if ((p.pb != 8 && p.pb != 6) || (p.pb == 6 && gz_rows > PAIR6_MAX_ROWS)) return hipErrorInvalidValue;
    if (p.nwave > 0) {
        if (p.pb == 6)
            launch_bwd16c_kernel<MODE, 6>(p, cw, gz, gz_rows, gwpart, gw_ld, epi, part, T, pair, st);
        else
            launch_bwd16c_kernel<MODE, 8>(p, cw, gz, gz_rows, gwpart, gw_ld, epi, part, T, pair, st);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (p.nsplit > 0) {
        if (MODE == 1 && pair)
            k_cbwd16_combine<MODE, true><<<nblocks((long long)p.nsplit * ((T + 1) / 2) * LPR), WG, 0, st>>>(p, part,
                                                                                                          epi, T);
        else
            k_cbwd16_combine<MODE, false><<<nblocks((long long)p.nsplit * T * LPR), WG, 0, st>>>(p, part, epi, T);
        return hipGetLastError();
    }
    return hipSuccess;
}

hipError_t launch_bwd16c(const Plan& p, const int2* cw, const unsigned short* gz, int gz_rows, float* gwpart,
                         long long gw_ld, const BwdEpi16& epi, float* part, int T, hipStream_t st, bool pair) {
    if (epi.mode == 1) return launch_bwd16c_as<1>(p, cw, gz, gz_rows, gwpart, gw_ld, epi, part, T, pair, st);
    if (epi.mode == 2) return launch_bwd16c_as<2>(p, cw, gz, gz_rows, gwpart, gw_ld, epi, part, T, false, st);
    return hipErrorInvalidValue;
}

hipError_t launch_readout_bwd_h16_mfma(const float* dl, const float* owT, const int* dn_inv, int n_act, int rows,
                                       const BwdEpi16& epi, int B, hipStream_t st) {
    if (readout_pad(n_act) > 8 * GH_STEPS) return hipErrorInvalidValue;
    dim3 grid((unsigned)((rows + RPG - 1) / RPG), (unsigned)(B / TW16));
    k_rbwd_h16_mfma<<<grid, WG, 0, st>>>(dl, owT, readout_pad(n_act), dn_inv, n_act, rows, epi);
    return hipGetLastError();
}

hipError_t launch_export16(const unsigned short* src, int rows, float* dst, int B, hipStream_t st) {
    k_export16<<<nblocks((long long)rows * B), WG, 0, st>>>(src, rows, dst, B);
    return hipGetLastError();
}

}  // namespace fg
