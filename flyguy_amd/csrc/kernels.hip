// Kernels of the flyguy MI355X library.
//
// The hot loops are the gather SpMM of a hop (k_fwd) and the fused transposed pass of its backward (k_bwd).
// Both work on "segments": runs of at most SEG_MAX edges of one row, sorted longest first, 8 segments per
// wave.  A segment's 8 lanes each hold a float4 of the 32-sample tile and sum its edges in CSR (CSC) order,
// so a row that is not split is summed exactly as flyguy_train.cu:88 / :171 sum it.  The (source, weight)
// pairs of 8 consecutive edges are loaded by the 8 lanes at once (one coalesced 64-byte load, the next one
// already in flight) and handed round the group through LDS; the 8 source rows are then gathered as independent
// 128-byte lines of the tile's slab, with no branch per edge (slots past a segment's end read row 0 and add 0).
#include "kernels.h"

namespace fg {

__device__ __forceinline__ const float4* at4(const float* base, Lay L, int tile, int row, int sub) {
    return reinterpret_cast<const float4*>(base + (size_t)tile * L.tile + (size_t)row * L.row) + sub;
}
__device__ __forceinline__ float4* at4w(float* base, Lay L, int tile, int row, int sub) {
    return reinterpret_cast<float4*>(base + (size_t)tile * L.tile + (size_t)row * L.row) + sub;
}
__device__ __forceinline__ float4 splat(float v) { return make_float4(v, v, v, v); }

template <int C>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), C, 0xf, 0xf, true));
}
// sum over the 8 lanes of a group with DPP (quad swaps, then the half-row mirror); every lane gets the total
__device__ __forceinline__ float gsum8(float v) {
    v += dppf<0xB1>(v);      // quad_perm [1,0,3,2]
    v += dppf<0x4E>(v);      // quad_perm [2,3,0,1]
    v += dppf<0x141>(v);     // row_half_mirror
    return v;
}
__device__ __forceinline__ float dot4(const float4& a, const float4& b) {
    float p = a.x * b.x;
    p = fmaf(a.y, b.y, p);
    p = fmaf(a.z, b.z, p);
    return fmaf(a.w, b.w, p);
}
__device__ __forceinline__ float hsum4(const float4& a) { return ((a.x + a.y) + a.z) + a.w; }

// segment si of the plan, or an empty dead segment when si is past the end or the entry is out of the plan's bounds
__device__ __forceinline__ bool load_segment(const Plan& p, int si, int4& sg) {
    sg = make_int4(0, 0, 0, -1);
    if (si >= p.nseg) return false;
    const int4 v = p.seg[si];
    if (v.x < 0 || v.x >= p.rows || v.y < 0 || v.y > v.z || v.z > p.E || v.w >= p.nslot) return false;
    sg = v;
    return true;
}
__device__ __forceinline__ bool load_split(const Plan& p, long long i, int4& s) {
    if (i >= p.nsplit) return false;
    s = p.split[i];
    return s.x >= 0 && s.x < p.rows && s.y >= 0 && s.z >= 0 && (long long)s.y + s.z <= p.nslot;
}

// ------------------------------------------------------------------------------------------------ packing
__global__ void k_pack(const int* __restrict__ col, const int* __restrict__ idx, const float* __restrict__ w,
                       int2* __restrict__ cw, long long E) {
    long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    long long i = idx ? idx[e] : e;
    cw[e] = make_int2(col[e], __float_as_int(w[i]));
}

__global__ void k_pack64(const int* __restrict__ col, const long long* __restrict__ idx, const float* __restrict__ w,
                         int2* __restrict__ cw, long long E) {
    long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    cw[e] = make_int2(col[e], __float_as_int(w[idx[e]]));
}

// ------------------------------------------------------------------------------------------------ forward
// The row's own inputs of the finish (re-drive row, gain, threshold), loaded before the edge loop so that their
// latency hides behind the gathers.
struct FwdIn {
    float4 dv;
    float g, sp;
};
__device__ __forceinline__ FwdIn fwd_inputs(const FwdEpi& e, int t, int tile, int sub) {
    FwdIn in{make_float4(0.f, 0.f, 0.f, 0.f), 0.f, 0.f};
    if (e.info) {
        const float4 r = e.info[t];
        in.g = r.x;
        in.sp = r.y;
        const int d = __float_as_int(r.z);
        if (e.drive && d >= 0) in.dv = *at4(e.drive, e.ldrive, tile, d, sub);
    }
    return in;
}
__device__ __forceinline__ void fwd_finish(const FwdEpi& e, int t, int tile, int sub, float4 acc, const FwdIn& in) {
    if (e.drive) add4(in.dv, acc);              // (zero when the row has no re-drive)
    if (e.z) *at4w(e.z, e.lz, tile, t, sub) = acc;
    if (e.info) {
        const float g = in.g, sp = in.sp;
        const float4 hv = make_float4(fmaxf(fmaf(g, acc.x, -sp), 0.f), fmaxf(fmaf(g, acc.y, -sp), 0.f),
                                      fmaxf(fmaf(g, acc.z, -sp), 0.f), fmaxf(fmaf(g, acc.w, -sp), 0.f));
        *at4w(e.h, e.lh, tile, t, sub) = hv;
    }
}

// The (index, weight) pairs of a group's next 8 edges reach all 8 lanes of the group through the wave's own LDS
// slots: each lane writes the pair it loaded (one 8-byte store), then reads the group's 8 pairs back (four 16-byte
// reads the 8 lanes share).  A wave only touches its own slots and its lanes run in lockstep; wave_barrier keeps
// the compiler from moving the reads above the store or the next store above the reads.
__device__ __forceinline__ void stage8(int2* slots, int sub, int2 my, int (&c)[8], float (&w)[8]) {
    slots[sub] = my;
    __builtin_amdgcn_wave_barrier();
    const int4* q = reinterpret_cast<const int4*>(slots);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int4 v = q[i];
        c[2 * i] = v.x;
        w[2 * i] = __int_as_float(v.y);
        c[2 * i + 1] = v.z;
        w[2 * i + 1] = __int_as_float(v.w);
    }
    __builtin_amdgcn_wave_barrier();
}

// A source index that no slab reaches: as a buffer offset (index * 128 B) it lies past every slab, so the buffer load
// returns zeros without touching memory.
constexpr int NO_ROW = 0x01FFFFFF;

// the largest value over the wave (every lane gets it, in an SGPR)
__device__ __forceinline__ int wave_max(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
    return __builtin_amdgcn_readfirstlane(v);
}

// Pair of edge e of a segment ending at e1, or (NO_ROW, weight 0) past the end: loaded from a clamped index, so no
// lane branches.  e_last is the segment's last edge (0 for an empty segment; every array has one element at least).
__device__ __forceinline__ int2 pair_at(const int2* __restrict__ cw, int e, int e1, int e_last) {
    int2 v = cw[min(e, e_last)];
    const bool ok = e < e1;
    v.x = ok ? v.x : NO_ROW;
    v.y = ok ? v.y : 0;
    return v;
}

// Gathers of one tile's slab.  Tiled layout: a raw buffer over the slab (rows x 128 B), 32-bit offsets, so an offset
// past the slab (NO_ROW, or any bad index) reads zeros.  Plain layout ([rows][B], the HopCuda boundary): global
// loads with the run-time row stride; rows past the end are masked to zero.
template <bool TILED>
struct Slab {
    __amdgpu_buffer_rsrc_t rsrc;
    const float* base;
    int stride, rows;
    __device__ __forceinline__ Slab(const float* tile_base, int row_stride, int n_rows, int sub)
        : base(tile_base + sub * 4), stride(row_stride), rows(n_rows) {
        if (TILED)
            rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)tile_base, (short)0, n_rows * (TW * 4), 0x00020000);
    }
    __device__ __forceinline__ float4 get(int row, int sub) const {
        if (TILED) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (unsigned)row * (TW * 4u) + (unsigned)sub * 16u, 0, 0);
            return make_float4(__int_as_float(v[0]), __int_as_float(v[1]), __int_as_float(v[2]), __int_as_float(v[3]));
        }
        const bool ok = (unsigned)row < (unsigned)rows;
        const float4 v = *reinterpret_cast<const float4*>(base + (size_t)(ok ? row : 0) * stride);
        return ok ? v : make_float4(0.f, 0.f, 0.f, 0.f);
    }
};

template <bool TILED>
__global__ __launch_bounds__(WG) void k_fwd(Plan p, const int2* __restrict__ cw, const float* __restrict__ src, Lay ls,
                                            int src_rows, FwdEpi epi, float* __restrict__ part, Lay lp, int T, int RB) {
    __shared__ __align__(16) int2 slots[WG / LPR][LPR];
    int rb;
    const int tile = tile_of(blockIdx.x, RB, T, rb);
    const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7;
    const int si = rb * RPG + grp;
    int4 sg;
    const bool live = load_segment(p, si, sg);
    const int e1 = sg.z, e_last = max(sg.z - 1, 0);
    const Slab<TILED> slab(src + (size_t)tile * ls.tile, ls.row, src_rows, sub);
    float4 acc = (live && sg.w < 0 && epi.bias) ? splat(epi.bias[sg.x]) : splat(0.f);
    int2 nxt = pair_at(cw, sg.y + sub, e1, e_last);
    FwdIn in{};
    if (live && sg.w < 0) in = fwd_inputs(epi, sg.x, tile, sub);
    // edges left in the wave's longest segment: slots no group needs are not gathered at all
    for (int eb = sg.y, left = wave_max(sg.z - sg.y); left > 0; eb += 8, left -= 8) {
        const int2 my = nxt;
        nxt = pair_at(cw, eb + 8 + sub, e1, e_last);
        int c[8];
        float w[8];
        stage8(slots[grp], sub, my, c, w);
        float4 v[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) v[s] = s < left ? slab.get(c[s], sub) : splat(0.f);
#pragma unroll
        for (int s = 0; s < 8; ++s) fma4(w[s], v[s], acc);
    }
    if (!live) return;
    if (sg.w >= 0) {
        *at4w(part, lp, tile, sg.w, sub) = acc;
        return;
    }
    fwd_finish(epi, sg.x, tile, sub, acc, in);
}

// split rows: partial sums in segment order, then the same finish
__global__ __launch_bounds__(WG) void k_fwd_combine(Plan p, const float* __restrict__ part, Lay lp, FwdEpi epi, int T) {
    long long q = ((long long)blockIdx.x * WG + threadIdx.x);
    const int sub = (int)(q & 7);
    q >>= 3;
    const int tile = (int)(q % T);
    const long long i = q / T;
    int4 s;
    if (!load_split(p, i, s)) return;     // whole 8-lane groups leave together
    float4 acc = epi.bias ? splat(epi.bias[s.x]) : splat(0.f);
    const FwdIn in = fwd_inputs(epi, s.x, tile, sub);
    for (int k = 0; k < s.z; ++k) add4(*at4(part, lp, tile, s.y + k, sub), acc);
    fwd_finish(epi, s.x, tile, sub, acc, in);
}

// ------------------------------------------------------------------------------------------------ backward
// The source row's own inputs of the neuron backward (h, z, gain, re-drive row; for the sensory layer the drive's
// gradient so far), loaded before the edge loop so that their latency hides behind the gathers.
struct BwdIn {
    float4 h, z, gd;
    float gn, sp;
    int d;
};
__device__ __forceinline__ BwdIn bwd_inputs(const BwdEpi& e, int j, int tile, int sub) {
    BwdIn in{make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f), 0.f, 0.f, -1};
    if (e.mode == 0) return in;
    in.h = *at4(e.h, e.lh, tile, j, sub);
    if (e.z) in.z = *at4(e.z, e.lz, tile, j, sub);
    const float4 r = e.info[j];
    in.gn = r.x;
    in.sp = r.y;
    if (e.mode == 1) {
        in.d = __float_as_int(r.z);
        if (in.d >= 0) in.gd = *at4(e.gdrive, e.lgd, tile, in.d, sub);
    } else {
        in.d = j;
        in.gd = *at4(e.gdrive, e.lgd, tile, j, sub);     // complete: every hop above has added its share
    }
    return in;
}

// gh: the gradient of this layer's output h for (row j, tile); every lane of the 8-lane group calls this
__device__ __forceinline__ void bwd_finish(const BwdEpi& e, int j, int tile, int sub, float4 gh, const BwdIn& in) {
    if (e.mode == 0) {
        *at4w(e.gh_out, e.lgh, tile, j, sub) = gh;
        return;
    }
    const float4 hv = in.h;
    const float4 g = make_float4(hv.x > 0.f ? gh.x : 0.f, hv.y > 0.f ? gh.y : 0.f, hv.z > 0.f ? gh.z : 0.f,
                                 hv.w > 0.f ? gh.w : 0.f);
    const float gn = in.gn;
    const float4 gzv = make_float4(g.x * gn, g.y * gn, g.z * gn, g.w * gn);
    float4 zv = in.z;
    if (!e.z) {                                 // z where it matters (h > 0): h = gain * z - softplus(theta)
        zv.x = hv.x > 0.f ? (hv.x + in.sp) / gn : 0.f;
        zv.y = hv.y > 0.f ? (hv.y + in.sp) / gn : 0.f;
        zv.z = hv.z > 0.f ? (hv.z + in.sp) / gn : 0.f;
        zv.w = hv.w > 0.f ? (hv.w + in.sp) / gn : 0.f;
    }
    const float pg = gsum8(dot4(g, zv));
    const float ps = gsum8(hsum4(g));
    if (sub == 0) {
        e.ggain_part[(size_t)tile * e.gp_ld + j] = pg;
        e.gsum_part[(size_t)tile * e.gp_ld + j] = ps;
    }
    if (e.mode == 1) {
        *at4w(e.gz_out, e.lgz, tile, j, sub) = gzv;
        if (in.d >= 0) {
            float4 v = in.gd;
            add4(gzv, v);
            *at4w(e.gdrive, e.lgd, tile, in.d, sub) = v;
        }
        return;
    }
    // the sensory layer: the drive's gradient is complete now -> the plug's bias and per-connection gradients
    float4 gd = in.gd;
    add4(gzv, gd);
    const float pb = gsum8(hsum4(gd));
    if (sub == 0) e.ginb_part[(size_t)tile * e.gb_ld + j] = pb;
    const int f0 = e.in_crow[j], f1 = e.in_crow[j + 1];
    for (int f = f0; f < f1; ++f) {
        const int c = e.in_cw[f].x;
        const float pw = gsum8(dot4(gd, *at4(e.x, e.lx, tile, c, sub)));
        if (sub == 0) e.ginw_part[(size_t)tile * e.gw_ld + f] = pw;
    }
}

template <bool TILED>
__global__ __launch_bounds__(WG) void k_bwd(Plan p, const int2* __restrict__ cw, const float* __restrict__ gz, Lay lg,
                                            int gz_rows, const float* __restrict__ hs, Lay lhs, float* __restrict__ gwpart,
                                            long long gw_ld, BwdEpi epi, float* __restrict__ part, Lay lp, int T, int RB) {
    __shared__ __align__(16) int2 slots[WG / LPR][LPR];
    int rb;
    const int tile = tile_of(blockIdx.x, RB, T, rb);
    const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7;
    const int si = rb * RPG + grp;
    int4 sg;
    const bool live = load_segment(p, si, sg);
    const int e1 = sg.z, e_last = max(sg.z - 1, 0);
    const float4 hj = live ? *at4(hs, lhs, tile, sg.x, sub) : splat(0.f);
    const Slab<TILED> slab(gz + (size_t)tile * lg.tile, lg.row, gz_rows, sub);
    float* gwp = gwpart ? gwpart + (size_t)tile * gw_ld : nullptr;
    float4 acc = splat(0.f);
    int2 nxt = pair_at(cw, sg.y + sub, e1, e_last);
    BwdIn in{};
    if (live && sg.w < 0) in = bwd_inputs(epi, sg.x, tile, sub);
    for (int eb = sg.y, left = wave_max(sg.z - sg.y); left > 0; eb += 8, left -= 8) {
        const int2 my = nxt;
        nxt = pair_at(cw, eb + 8 + sub, e1, e_last);
        int c[8];
        float w[8];
        stage8(slots[grp], sub, my, c, w);
        const int n = e1 - eb;
        float4 v[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) v[s] = s < left ? slab.get(c[s], sub) : splat(0.f);
#pragma unroll
        for (int s = 0; s < 8; ++s) fma4(w[s], v[s], acc);
        if (gwp) {
            float mine = 0.f;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const float ps = gsum8(dot4(hj, v[s]));
                mine = sub == s ? ps : mine;
            }
            if (sub < n) gwp[eb + sub] = mine;
        }
    }
    if (!live) return;
    if (sg.w >= 0) {
        *at4w(part, lp, tile, sg.w, sub) = acc;
        return;
    }
    bwd_finish(epi, sg.x, tile, sub, acc, in);
}

__global__ __launch_bounds__(WG) void k_bwd_combine(Plan p, const float* __restrict__ part, Lay lp, BwdEpi epi, int T) {
    long long q = ((long long)blockIdx.x * WG + threadIdx.x);
    const int sub = (int)(q & 7);
    q >>= 3;
    const int tile = (int)(q % T);
    const long long i = q / T;
    int4 s;
    if (!load_split(p, i, s)) return;     // whole 8-lane groups leave together
    float4 acc = splat(0.f);
    const BwdIn in = bwd_inputs(epi, s.x, tile, sub);
    for (int k = 0; k < s.z; ++k) add4(*at4(part, lp, tile, s.y + k, sub), acc);
    bwd_finish(epi, s.x, tile, sub, acc, in);
}

// ------------------------------------------------------------------------------------------------ obs / logits
// obs [B][obs_dim] (row-major, the caller's) -> x [T][obs_dim][32]; one workgroup per (tile, 64 features)
__global__ __launch_bounds__(WG) void k_obs_in(const float* __restrict__ obs, float* __restrict__ x, int obs_dim) {
    __shared__ float s[TW][65];
    const int tile = blockIdx.y, f0 = blockIdx.x * 64;
    for (int i = threadIdx.x; i < TW * 64; i += WG) {
        const int c = i / 64, f = i % 64;
        s[c][f] = (f0 + f < obs_dim) ? obs[(size_t)(tile * TW + c) * obs_dim + f0 + f] : 0.f;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < TW * 64; i += WG) {
        const int f = i / TW, c = i % TW;
        if (f0 + f < obs_dim) x[((size_t)tile * obs_dim + f0 + f) * TW + c] = s[c][f];
    }
}

// logits[b][a] = ob[a] + sum_j ow[a][j] * hK[dn[j]][b], summed in j order (flyguy_train.cu:95-101)
__global__ __launch_bounds__(WG) void k_logits(const float* __restrict__ hK, Lay lh, const int* __restrict__ dn, int n_dn,
                                               const float* __restrict__ ow, const float* __restrict__ ob, int n_act,
                                               float* __restrict__ logits) {
    __shared__ float4 hs[64][LPR];
    __shared__ float ws[64][97];
    const int tile = blockIdx.x, c4 = threadIdx.x & 7, ag = threadIdx.x >> 3;
    for (int a0 = 0; a0 < n_act; a0 += 96) {
        float4 acc[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int a = a0 + ag + 32 * i;
            acc[i] = splat(a < n_act ? ob[a] : 0.f);
        }
        for (int j0 = 0; j0 < n_dn; j0 += 64) {
            const int nj = min(64, n_dn - j0);
            __syncthreads();
            for (int i = threadIdx.x; i < 64 * LPR; i += WG) {
                const int jj = i / LPR, q = i % LPR;
                hs[jj][q] = jj < nj ? *at4(hK, lh, tile, dn[j0 + jj], q) : splat(0.f);
            }
            for (int i = threadIdx.x; i < 64 * 96; i += WG) {
                const int aa = i / 64, jj = i % 64;
                ws[jj][aa] = (jj < nj && a0 + aa < n_act) ? ow[(size_t)(a0 + aa) * n_dn + j0 + jj] : 0.f;
            }
            __syncthreads();
            for (int jj = 0; jj < nj; ++jj) {
                const float4 h4 = hs[jj][c4];
#pragma unroll
                for (int i = 0; i < 3; ++i) fma4(ws[jj][ag + 32 * i], h4, acc[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int a = a0 + ag + 32 * i;
            if (a >= n_act) continue;
            float* o = logits + (size_t)(tile * TW + c4 * 4) * n_act + a;
            o[0] = acc[i].x;
            o[n_act] = acc[i].y;
            o[2 * n_act] = acc[i].z;
            o[3 * n_act] = acc[i].w;
        }
    }
}

// gh of the top layer from the logits' gradient, then the neuron backward (flyguy_train.cu:136-141, 143-156)
__global__ __launch_bounds__(WG) void k_readout_bwd_h(const float* __restrict__ dl, const float* __restrict__ ow,
                                                      const int* __restrict__ dn_inv, int n_dn, int n_act, int rows,
                                                      BwdEpi epi) {
    extern __shared__ float sm[];
    float* dlT = sm;                       // [n_act][32]
    float* owc = sm + (size_t)n_act * TW;  // [32][n_act]
    const int tile = blockIdx.y, r0 = blockIdx.x * RPG;
    for (int i = threadIdx.x; i < n_act * TW; i += WG) {
        const int c = i / n_act, a = i % n_act;
        dlT[a * TW + c] = dl[(size_t)(tile * TW + c) * n_act + a];
    }
    for (int i = threadIdx.x; i < RPG * n_act; i += WG) {
        const int r = i / n_act, a = i % n_act, t = r0 + r;
        const int j = t < rows ? dn_inv[t] : -1;
        owc[r * n_act + a] = j >= 0 ? ow[(size_t)a * n_dn + j] : 0.f;
    }
    __syncthreads();
    const int r = threadIdx.x >> 3, sub = threadIdx.x & 7, t = r0 + r;
    if (t >= rows) return;                 // whole 8-lane groups
    float4 acc = splat(0.f);
    if (dn_inv[t] >= 0) {
        const float4* d4 = reinterpret_cast<const float4*>(dlT) + sub;
        for (int a = 0; a < n_act; ++a) fma4(owc[r * n_act + a], d4[a * LPR], acc);
    }
    bwd_finish(epi, t, tile, sub, acc, bwd_inputs(epi, t, tile, sub));
}

// per chunk of 16 tiles: gow[a][j] partial = sum_b dl[b][a] * hK[dn[j]][b], gob[a] partial = sum_b dl[b][a]
constexpr int RO_CHUNK = 16;
int readout_chunks(int B) { return (B / TW + RO_CHUNK - 1) / RO_CHUNK; }
__global__ __launch_bounds__(WG) void k_readout_bwd_w(const float* __restrict__ dl, const float* __restrict__ hK, Lay lh,
                                                      const int* __restrict__ dn, int n_dn, int n_act, int T,
                                                      float* __restrict__ gow_part, float* __restrict__ gob_part) {
    __shared__ float hT[32][33];
    __shared__ float ds[TW][97];
    const int j0 = blockIdx.x * 32, chunk = blockIdx.y;
    const int jj = threadIdx.x & 31, ag = threadIdx.x >> 5;
    const int t0 = chunk * RO_CHUNK, t1 = min(T, t0 + RO_CHUNK);
    for (int a0 = 0; a0 < n_act; a0 += 96) {
        float acc[12];
        float accb = 0.f;
#pragma unroll
        for (int i = 0; i < 12; ++i) acc[i] = 0.f;
        for (int tile = t0; tile < t1; ++tile) {
            __syncthreads();
            for (int i = threadIdx.x; i < 32 * TW; i += WG) {
                const int j = i / TW, c = i % TW;
                hT[j][c] = (j0 + j < n_dn) ? hK[(size_t)tile * lh.tile + (size_t)dn[j0 + j] * lh.row + c] : 0.f;
            }
            for (int i = threadIdx.x; i < TW * 96; i += WG) {
                const int c = i / 96, a = i % 96;
                ds[c][a] = (a0 + a < n_act) ? dl[(size_t)(tile * TW + c) * n_act + a0 + a] : 0.f;
            }
            __syncthreads();
            for (int c = 0; c < TW; ++c) {
                const float hv = hT[jj][c];
#pragma unroll
                for (int i = 0; i < 12; ++i) acc[i] = fmaf(ds[c][ag + 8 * i], hv, acc[i]);
            }
            if (blockIdx.x == 0 && threadIdx.x < 96)
                for (int c = 0; c < TW; ++c) accb += ds[c][threadIdx.x];
        }
        const size_t base = (size_t)chunk * n_act * n_dn;
#pragma unroll
        for (int i = 0; i < 12; ++i) {
            const int a = a0 + ag + 8 * i;
            if (a < n_act && j0 + jj < n_dn) gow_part[base + (size_t)a * n_dn + j0 + jj] = acc[i];
        }
        if (blockIdx.x == 0 && threadIdx.x < 96 && a0 + threadIdx.x < n_act)
            gob_part[(size_t)chunk * n_act + a0 + threadIdx.x] = accb;
    }
}

// ------------------------------------------------------------------------------------------------ reductions
// G[idx[i]] += sum_t part[t * ld + i]  (times -sigmoid(theta[idx[i]]) when theta is given: the threshold's gradient)
__global__ void k_reduce(const float* __restrict__ part, long long ld, long long n, int nt, const int* __restrict__ idx,
                         const float* __restrict__ theta, float* __restrict__ G) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float s = 0.f;
    for (int t = 0; t < nt; ++t) s += part[(size_t)t * ld + i];
    const long long o = idx ? idx[i] : i;
    if (theta) s *= -sigmoid_f(theta[o]);
    G[o] += s;
}

__global__ void k_reduce64(const float* __restrict__ part, long long ld, long long n, int nt,
                           const long long* __restrict__ idx, float* __restrict__ G) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float s = 0.f;
    for (int t = 0; t < nt; ++t) s += part[(size_t)t * ld + i];
    G[idx[i]] += s;
}

// KL(teacher || student) per sample, dl = d(mean loss)/d logits (flyguy_train.cu:104-123); one thread per sample
__global__ __launch_bounds__(WG) void k_loss(const float* __restrict__ lg, const float* __restrict__ tl, float* __restrict__ dl,
                                             float* __restrict__ stats_part, int n_act, int B, float it) {
    __shared__ float red[2][WG];
    const int b = blockIdx.x * WG + threadIdx.x;
    float kl = 0.f, agree = 0.f;
    if (b < B) {
        const float* s = lg + (size_t)b * n_act;
        const float* t = tl + (size_t)b * n_act;
        float ms = -1e30f, mt = -1e30f;
        int as = 0, at = 0;
        for (int a = 0; a < n_act; ++a) {
            const float sv = s[a], tv = t[a] * it;
            if (sv > ms) { ms = sv; as = a; }
            if (tv > mt) { mt = tv; at = a; }
        }
        float zs = 0.f, zt = 0.f;
        for (int a = 0; a < n_act; ++a) {
            zs += expf(s[a] - ms);
            zt += expf(t[a] * it - mt);
        }
        const float ls = ms + logf(zs), lt = mt + logf(zt);
        for (int a = 0; a < n_act; ++a) {
            const float lps = s[a] - ls, lpt = t[a] * it - lt, pt = expf(lpt);
            kl += pt * (lpt - lps);
            dl[(size_t)b * n_act + a] = (expf(lps) - pt) / (float)B;
        }
        agree = as == at ? 1.f : 0.f;
    }
    red[0][threadIdx.x] = kl;
    red[1][threadIdx.x] = agree;
    __syncthreads();
    for (int s = WG / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            red[0][threadIdx.x] += red[0][threadIdx.x + s];
            red[1][threadIdx.x] += red[1][threadIdx.x + s];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        stats_part[2 * blockIdx.x] = red[0][0];
        stats_part[2 * blockIdx.x + 1] = red[1][0];
    }
}
__global__ void k_sum_pairs(const float* __restrict__ part, int n, float* __restrict__ out) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float a = 0.f, b = 0.f;
    for (int i = 0; i < n; ++i) { a += part[2 * i]; b += part[2 * i + 1]; }
    out[0] = a;
    out[1] = b;
}

__global__ void k_fill(float* __restrict__ p, float v, long long n) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ __launch_bounds__(WG) void k_sumsq(const float* __restrict__ g, long long n, float* __restrict__ part) {
    __shared__ float red[WG];
    float s = 0.f;
    for (long long i = (long long)blockIdx.x * WG + threadIdx.x; i < n; i += (long long)gridDim.x * WG) s = fmaf(g[i], g[i], s);
    red[threadIdx.x] = s;
    __syncthreads();
    for (int k = WG / 2; k > 0; k >>= 1) {
        if (threadIdx.x < k) red[threadIdx.x] += red[threadIdx.x + k];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}
__global__ void k_sum(const float* __restrict__ part, int n, float* __restrict__ out) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float a = 0.f;
    for (int i = 0; i < n; ++i) a += part[i];
    out[0] = a;
}

// one Adam step with a running average of the weights over all seven arrays (flyguy_train.cu:194-203)
__global__ void k_adam(float* __restrict__ P, const float* __restrict__ G, float* __restrict__ M, float* __restrict__ V,
                       float* __restrict__ EMA, AdamSeg s, float c1, float c2, float gs, float decay) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= s.off[7]) return;
    int k = 0;
    while (k < 6 && i >= s.off[k + 1]) ++k;
    const float lr = s.lr[k];
    const float gr = G[i] * gs;
    const float mi = fmaf(0.9f, M[i], 0.1f * gr), vi = fmaf(0.999f, V[i], 0.001f * gr * gr);
    M[i] = mi;
    V[i] = vi;
    const float pi = P[i] - lr * (mi / c1) / (sqrtf(vi / c2) + 1e-8f);
    P[i] = pi;
    EMA[i] = fmaf(decay, EMA[i], (1.f - decay) * pi);
}

// per row of a layer: {gain[nid], softplus(theta[nid]), re-drive row (int bits, -1 none), 0}
__global__ void k_rowinfo(const int* __restrict__ nid, const int* __restrict__ drow, const float* __restrict__ gain,
                          const float* __restrict__ theta, float4* __restrict__ info, int rows) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows) return;
    const int n = nid[t];
    info[t] = make_float4(gain[n], softplus_f(theta[n]), __int_as_float(drow ? drow[t] : -1), 0.f);
}

// a state tensor (tiled) -> [rows][B] (tests and diagnostics)
__global__ void k_export(const float* __restrict__ src, Lay ls, float* __restrict__ dst, int rows, int B) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)rows * B) return;
    const int r = (int)(i / B), b = (int)(i % B);
    dst[i] = src[(size_t)(b / TW) * ls.tile + (size_t)r * ls.row + (b % TW)];
}

// ------------------------------------------------------------------------------------------------ launchers
static inline unsigned blocks(long long n, int per = WG) { return (unsigned)((n + per - 1) / per); }

hipError_t launch_pack(const int* col, const int* idx, const float* w, int2* cw, long long E, hipStream_t st) {
    if (E <= 0) return hipSuccess;
    k_pack<<<blocks(E), WG, 0, st>>>(col, idx, w, cw, E);
    return hipGetLastError();
}

hipError_t launch_pack64(const int* col, const long long* idx, const float* w, int2* cw, long long E, hipStream_t st) {
    if (E <= 0) return hipSuccess;
    k_pack64<<<blocks(E), WG, 0, st>>>(col, idx, w, cw, E);
    return hipGetLastError();
}

hipError_t launch_reduce64(const float* part, long long ld, long long n, int nt, const long long* idx, float* G,
                           hipStream_t st) {
    if (n <= 0) return hipSuccess;
    k_reduce64<<<blocks(n), WG, 0, st>>>(part, ld, n, nt, idx, G);
    return hipGetLastError();
}

hipError_t launch_fwd(const Plan& p, const int2* cw, const float* src, Lay ls, int src_rows, const FwdEpi& epi,
                      float* part, Lay lp, int T, hipStream_t st) {
    if (p.nseg > 0) {
        const int RB = (p.nseg + RPG - 1) / RPG;
        if (ls.row == TW)
            k_fwd<true><<<(unsigned)((long long)T * RB), WG, 0, st>>>(p, cw, src, ls, src_rows, epi, part, lp, T, RB);
        else
            k_fwd<false><<<(unsigned)((long long)T * RB), WG, 0, st>>>(p, cw, src, ls, src_rows, epi, part, lp, T, RB);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (p.nsplit > 0) {
        k_fwd_combine<<<blocks((long long)p.nsplit * T * LPR), WG, 0, st>>>(p, part, lp, epi, T);
        return hipGetLastError();
    }
    return hipSuccess;
}

hipError_t launch_bwd(const Plan& p, const int2* cw, const float* gz, Lay lg, int gz_rows, const float* hsrc, Lay lhs,
                      float* gwpart, long long gw_ld, const BwdEpi& epi, float* part, Lay lp, int T, hipStream_t st) {
    if (p.nseg > 0) {
        const int RB = (p.nseg + RPG - 1) / RPG;
        if (lg.row == TW)
            k_bwd<true><<<(unsigned)((long long)T * RB), WG, 0, st>>>(p, cw, gz, lg, gz_rows, hsrc, lhs, gwpart, gw_ld, epi, part,
                                                                      lp, T, RB);
        else
            k_bwd<false><<<(unsigned)((long long)T * RB), WG, 0, st>>>(p, cw, gz, lg, gz_rows, hsrc, lhs, gwpart, gw_ld, epi, part,
                                                                       lp, T, RB);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (p.nsplit > 0) {
        k_bwd_combine<<<blocks((long long)p.nsplit * T * LPR), WG, 0, st>>>(p, part, lp, epi, T);
        return hipGetLastError();
    }
    return hipSuccess;
}

hipError_t launch_obs_in(const float* obs, float* x, int obs_dim, int B, hipStream_t st) {
    dim3 grid((unsigned)((obs_dim + 63) / 64), (unsigned)(B / TW));
    k_obs_in<<<grid, WG, 0, st>>>(obs, x, obs_dim);
    return hipGetLastError();
}

hipError_t launch_logits(const float* hK, Lay lh, const int* dn, int n_dn, const float* ow, const float* ob, int n_act,
                         float* logits, int B, hipStream_t st) {
    k_logits<<<(unsigned)(B / TW), WG, 0, st>>>(hK, lh, dn, n_dn, ow, ob, n_act, logits);
    return hipGetLastError();
}

hipError_t launch_readout_bwd_h(const float* dl, const float* ow, const int* dn_inv, int n_dn, int n_act, int rows,
                                const BwdEpi& epi, int B, hipStream_t st) {
    dim3 grid((unsigned)((rows + RPG - 1) / RPG), (unsigned)(B / TW));
    size_t sm = (size_t)2 * n_act * TW * sizeof(float);
    k_readout_bwd_h<<<grid, WG, sm, st>>>(dl, ow, dn_inv, n_dn, n_act, rows, epi);
    return hipGetLastError();
}

hipError_t launch_readout_bwd_w(const float* dl, const float* hK, Lay lh, const int* dn, int n_dn, int n_act,
                                float* gow_part, float* gob_part, int B, hipStream_t st) {
    const int T = B / TW;
    dim3 grid((unsigned)((n_dn + 31) / 32), (unsigned)readout_chunks(B));
    k_readout_bwd_w<<<grid, WG, 0, st>>>(dl, hK, lh, dn, n_dn, n_act, T, gow_part, gob_part);
    return hipGetLastError();
}

hipError_t launch_reduce(const float* part, long long ld, long long n, int nt, const int* idx, const float* theta,
                         float* G, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    k_reduce<<<blocks(n), WG, 0, st>>>(part, ld, n, nt, idx, theta, G);
    return hipGetLastError();
}

hipError_t launch_loss(const float* lg, const float* tl, float* dl, float* stats_part, float* stats, int n_act, int B,
                       float it, hipStream_t st) {
    const unsigned nb = blocks(B);
    k_loss<<<nb, WG, 0, st>>>(lg, tl, dl, stats_part, n_act, B, it);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_sum_pairs<<<1, 64, 0, st>>>(stats_part, (int)nb, stats);
    return hipGetLastError();
}

hipError_t launch_fill(float* p, float v, long long n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    k_fill<<<blocks(n), WG, 0, st>>>(p, v, n);
    return hipGetLastError();
}

hipError_t launch_sumsq(const float* g, long long n, float* part, float* out, hipStream_t st) {
    const int nb = 1024;
    k_sumsq<<<nb, WG, 0, st>>>(g, n, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_sum<<<1, 64, 0, st>>>(part, nb, out);
    return hipGetLastError();
}

hipError_t launch_adam(float* P, const float* G, float* M, float* V, float* EMA, const AdamSeg& s, float c1, float c2,
                       const float* gs_dev, float gs, float decay, hipStream_t st) {
    (void)gs_dev;
    k_adam<<<blocks(s.off[7]), WG, 0, st>>>(P, G, M, V, EMA, s, c1, c2, gs, decay);
    return hipGetLastError();
}

hipError_t launch_rowinfo(const int* nid, const int* drow, const float* gain, const float* theta, float4* info, int rows,
                          hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    k_rowinfo<<<blocks(rows), WG, 0, st>>>(nid, drow, gain, theta, info, rows);
    return hipGetLastError();
}

hipError_t launch_export(const float* src, Lay ls, float* dst, int rows, int B, hipStream_t st) {
    k_export<<<blocks((long long)rows * B), WG, 0, st>>>(src, ls, dst, rows, B);
    return hipGetLastError();
}

}  // namespace fg
