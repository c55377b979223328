// Kernels of the flyguy MI355X library.
//
// The hot loops are the gather SpMM of a hop (k_fwd) and the fused transposed pass of its backward (k_bwd, one tile
// per workgroup; k_bwd2, two tiles, for a layer whose gathered rows are used unevenly enough that two tiles' worth of
// the most used lines stay in the L2).
// Both follow a row plan (kernels.h): segments of at most seg_cap edges of one row, sorted longest first, 8 to a
// wave.  A segment's 8 lanes each hold a float4 of the 32-sample tile and sum its edges in CSR (CSC) order, so a row
// that is not split is summed exactly as flyguy_train.cu:88 / :171 sum it.  The (source, weight) pairs of a wave's
// next step are one contiguous 512-byte block in plan order (one 8-byte load per lane, issued a step ahead) and
// reach the 8 lanes of each group through LDS; the 8 source rows are then gathered as independent 128-byte lines
// of the tile's slab, with no branch per edge (unused positions gather NO_ROW, which reads zeros).
#include <initializer_list>

#include "device.h"
#include "readout.h"

namespace fg {

// ------------------------------------------------------------------------------------------------ packing
// Several small element-wise jobs in one launch: job k takes blocks first[k] .. first[k + 1] - 1.
template <class J, int N>
struct JobTable {
    J j[N];
    long long first[N];
    int n;
};
// the job of block b and its first block (constant indices, so the table stays in the kernel arguments)
template <class J, int N>
__device__ __forceinline__ J job_of(const JobTable<J, N>& t, long long b, long long& b0) {
    J r = t.j[0];
    b0 = 0;
#pragma unroll
    for (int k = 1; k < N; ++k)
        if (k < t.n && b >= t.first[k]) { r = t.j[k]; b0 = t.first[k]; }
    return r;
}
// fill a table from jobs[0 .. n) (those of no elements left out); nb: the launch's blocks
template <class J, int N, class Elems>
static bool fill_table(JobTable<J, N>& t, const J* jobs, int n, Elems elems, long long& nb) {
    t = JobTable<J, N>{};
    nb = 0;
    if (n < 0 || n > N || (n > 0 && !jobs)) return false;
    for (int k = 0; k < n; ++k) {
        const long long m = elems(jobs[k]);
        if (m <= 0) continue;
        t.j[t.n] = jobs[k];
        t.first[t.n] = nb;
        nb += (m + WG - 1) / WG;
        ++t.n;
    }
    return nb <= 0xFFFFFFFFLL;
}

// the (source, weight) pair of every plan position, from the current weights; BF16W: the weight rounded to bfloat16
// (nearest even), kept as the float32 of that value (low 16 bits zero)
template <bool BF16W>
__global__ __launch_bounds__(WG) void k_pack(JobTable<PackJob, PACK_JOBS> t) {
    long long b0;
    const PackJob J = job_of(t, blockIdx.x, b0);
    const long long p = ((long long)blockIdx.x - b0) * WG + threadIdx.x;
    if (p >= J.n) return;
    const int i = J.pidx[p];
    float v = i >= 0 ? J.w[i] : 0.f;
    if (BF16W) v = (float)(__bf16)v;
    if (J.pb == 6) {                            // (Plan::pb) the weight plane, then the source plane of the step
        unsigned char* blk = reinterpret_cast<unsigned char*>(J.cw) + (size_t)(p >> 6) * 384;
        reinterpret_cast<float*>(blk)[p & 63] = v;
        reinterpret_cast<unsigned short*>(blk + 256)[p & 63] = i >= 0 ? (unsigned short)J.pcol[p] : (unsigned short)0xFFFF;
        return;
    }
    J.cw[p] = i >= 0 ? make_int2(J.pcol[p], __float_as_int(v)) : make_int2(NO_ROW, 0);
}

// ------------------------------------------------------------------------------------------------ forward
// 16-byte load of a line that the pass reads once (a row's own h, re-drive or drive-gradient line, a split row's
// partial sums): not kept in the L2, so that the slab being gathered keeps its place there (float32, B=4096: hop 2
// backward 1.524 -> 1.504 ms, hop 3 backward 0.381 -> 0.370 ms; loads of the pairs with the hint made every hop slower:
// all tiles read the same pairs)
__device__ __forceinline__ float4 ld_stream(const float4* p) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v v = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
// The row's own inputs of the finish (re-drive row d, gain, threshold), loaded before the edge loop so that their
// latency hides behind the gathers.
struct FwdIn {
    float4 dv;
    float g, sp, b;                             // b: the row's bias (the plug's records carry it)
};
// recs[i]: the row's record (FwdEpi::sinfo from the wave's first segment and i its group for a whole row, info and
// the row for a split one; nullptr: none)
__device__ __forceinline__ FwdIn fwd_inputs(const FwdEpi& e, const float4* recs, int i, int d, int tile, int sub) {
    FwdIn in{make_float4(0.f, 0.f, 0.f, 0.f), 0.f, 0.f, 0.f};
    if (e.drive && d >= 0) in.dv = ld_stream(at4u(e.drive, e.ldrive, tile, d, sub));
    if (recs) {
        const float4 r = recs[i];
        in.g = r.x;
        in.sp = r.y;
        in.b = r.w;
    }
    return in;
}
// 16-byte store that does not keep the line in L2: the states and partial sums a pass writes are read by a later
// kernel, long after the L2 has moved on to other tiles, and should not push the slab being gathered out of it
// (in the float32 backward this took hop 2 from 1.626 to 1.590 ms at B=4096)
__device__ __forceinline__ void st_stream(float4* p, const float4& v) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<f4v*>(p));
}
// (the lanes of whole 8-lane groups call this together)
__device__ __forceinline__ void fwd_finish(const FwdEpi& e, int t, int tile, int sub, float4 acc, const FwdIn& in) {
    if (e.drive) add4(in.dv, acc);              // (zero when the row has no re-drive)
    if (e.z) st_stream(at4w(e.z, e.lz, tile, t, sub), acc);
    if (e.info) {
        const float g = in.g, sp = in.sp;
        const float4 hv = make_float4(fmaxf(fmaf(g, acc.x, -sp), 0.f), fmaxf(fmaf(g, acc.y, -sp), 0.f),
                                      fmaxf(fmaf(g, acc.z, -sp), 0.f), fmaxf(fmaf(g, acc.w, -sp), 0.f));
        st_stream(at4uw(e.h, e.lh, tile, t, sub), hv);
        if (e.fires) {                          // whether the row fires on some sample of the tile
            const bool on = !group_silent(hv);
            if (sub == 0) e.fires[(size_t)tile * fires_bytes_ld((int)(e.lh.tile / TW)) + t] = on ? 1 : 0;   // (tiled h)
        }
    }
}

template <bool TILED, int PB>
__global__ __launch_bounds__(WG) void k_fwd(Plan p, const int2* __restrict__ cw, const float* __restrict__ src, Lay ls,
                                            int src_rows, FwdEpi epi, float* __restrict__ part, Lay lp, int T, int RB,
                                            const unsigned* __restrict__ src_fires, int fw_ld) {
    __shared__ __align__(16) int2 slots[WG / LPR][LPR];
    extern __shared__ __align__(16) unsigned fires[];     // the source rows' firing bits of this tile
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
    const Slab<TILED> slab(src + (size_t)tile * ls.tile, ls.row, src_rows, sub);
    const bool whole = live && sg.y < 0;
    float4 acc = splat(0.f);
    FwdIn in{};
    // steps of the wave's longest segment; a step gathers only the slots some group still needs.  The row's own
    // inputs (bias, re-drive row, gain, threshold) are requested right after the first step's gathers: loads
    // complete in order, so requested earlier they would hold up the first gathers.  The bias still starts the sum
    // (flyguy_train.cu:75).
    for (int j = 0, left = wok ? wv.y : 0; left > 0; ++j, left -= 8) {
        int c[8];
        float wt[8];
        // (a silent source row adds zeros: its gather reads NO_ROW)
        if constexpr (PB == 8)                 // (6-byte pairs: stage_pairs drops them)
            if (bits) drop_silent(nxt, fires, src_rows);
        stage_pairs<PB>(slots, grp, sub, nxt, bits, fires, src_rows, c, wt);
        float4 v[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) v[s] = s < left ? slab.get(c[s], sub) : splat(0.f);
        // the next step's pairs are requested after this step's gathers, so the gathers do not wait for them
        __builtin_amdgcn_sched_barrier(0);
        if (left > 8) nxt = q.step(j + 1);
        if (j == 0 && whole) {
            in = fwd_inputs(epi, epi.sinfo ? epi.sinfo + 8 * w : nullptr, grp & 7, sg.z, tile, sub);
            if (epi.bias) acc = splat(epi.sinfo ? in.b : epi.bias[sg.x]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 8; ++s) fma4(wt[s], v[s], acc);
    }
    if (whole && !(wok && wv.y > 0)) {          // a wave without edges
        in = fwd_inputs(epi, epi.sinfo ? epi.sinfo + 8 * w : nullptr, grp & 7, sg.z, tile, sub);
        if (epi.bias) acc = splat(epi.sinfo ? in.b : epi.bias[sg.x]);
    }
    if (!live) return;
    if (sg.y >= 0) {
        *at4w(part, lp, tile, sg.y, sub) = acc;
        return;
    }
    fwd_finish(epi, sg.x, tile, sub, acc, in);
}

// The same product for a source slab small enough for the LDS (the plug: each sensory row reads 16 of the 517
// observation rows, so each observation line of a tile is gathered about 500 times).  A workgroup copies the tile's
// slab (src_rows lines of 128 bytes) into LDS once and then walks its share of the row plan, gathering from the LDS
// instead of through the vector-memory path.  The sums are k_fwd's, term for term in the same order.  S workgroups
// per tile; a wave takes plan waves w0 + k dw (w0 = s FWD_LDS_NW + its index, dw = S FWD_LDS_NW), k < n <= 64.
// Stores count in the same vector-memory counter as loads, so a load issued after a store is waited for only
// once the store is done: each plan wave's records and first pairs are therefore requested before the previous
// plan wave's stores.  No re-drive rows (the plug has none).
template <int PB>
__global__ __launch_bounds__(FWD_LDS_NW * 64) void k_fwd_lds(Plan p, const int2* __restrict__ cw,
                                                            const float* __restrict__ src, int src_rows, FwdEpi epi,
                                                            float* __restrict__ part, Lay lp, int T, int S) {
    __shared__ __align__(16) int2 slots[FWD_LDS_NW * 64 / LPR][LPR];
    extern __shared__ __align__(16) float4 xs[];          // the tile's slab, src_rows x LPR float4
    int s;
    const int tile = tile_of(blockIdx.x, S, T, s);
    const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7, lane = threadIdx.x & 63, gi = grp & 7;
    const int w0 = __builtin_amdgcn_readfirstlane(s * FWD_LDS_NW + (int)(threadIdx.x >> 6)), dw = S * FWD_LDS_NW;
    const int n = w0 < p.nwave ? (p.nwave - 1 - w0) / dw + 1 : 0;
    // lane k holds the record of the wave's k-th plan wave (a vector load: waiting for it waits for no LDS read)
    const int2 wrec = lane < n ? p.wave[w0 + lane * dw] : make_int2(0, 0);
    const float4* g = reinterpret_cast<const float4*>(src + (size_t)tile * src_rows * TW);
    for (int i = threadIdx.x; i < src_rows * LPR; i += FWD_LDS_NW * 64) xs[i] = g[i];
    __syncthreads();
    struct It {
        int w;
        int2 wv, pr;
        int4 sg;
        float4 rec;
        bool wok, live;
    };
    // the loads of plan wave k: its record (from wrec), first pairs, segment and row record (by plan position)
    auto plan_of = [&](int k, It& it) {
        it.w = w0 + k * dw;
        const int2 v = make_int2(__builtin_amdgcn_readlane(wrec.x, k), __builtin_amdgcn_readlane(wrec.y, k));
        it.wok = v.x >= 0 && v.y >= 0 && (long long)v.x + 64 * (((long long)v.y + 7) / 8) <= p.npos;
        it.wv = it.wok ? v : make_int2(0, 0);
        it.pr = (it.wok && it.wv.y > 0) ? PairLoad<PB>(cw, it.wv.x, lane).step(0) : make_int2(NO_ROW, 0);
        it.live = load_segment(p, it.w * 8 + gi, it.sg) && it.wok;
        it.rec = epi.sinfo && it.w * 8 + gi < p.nseg ? epi.sinfo[it.w * 8 + gi] : splat(0.f);
    };
    It cur{}, nx{};                            // (nx stays unused after the last plan wave)
    if (n > 0) plan_of(0, cur);
    for (int k = 0; k < n; ++k) {
        const bool whole = cur.live && cur.sg.y < 0;
        float4 acc = splat(0.f);
        if (whole && epi.bias) acc = splat(epi.sinfo ? cur.rec.w : epi.bias[cur.sg.x]);   // (the bias starts the sum)
        const PairLoad<PB> q(cw, cur.wv.x, lane);
        int2 nxt = cur.pr;
        for (int j = 0, left = cur.wok ? cur.wv.y : 0; left > 0; ++j, left -= 8) {
            int c[8];
            float wt[8];
            stage_pairs<PB>(slots, grp, sub, nxt, false, nullptr, src_rows, c, wt);
            if (left > 8) nxt = q.step(j + 1);
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                v[u] = u < left && (unsigned)c[u] < (unsigned)src_rows ? xs[c[u] * LPR + sub] : splat(0.f);
#pragma unroll
            for (int u = 0; u < 8; ++u) fma4(wt[u], v[u], acc);
        }
        if (k + 1 < n) plan_of(k + 1, nx);
        if (cur.live) {
            if (cur.sg.y >= 0) {
                *at4w(part, lp, tile, cur.sg.y, sub) = acc;
            } else {
                FwdIn in{make_float4(0.f, 0.f, 0.f, 0.f), cur.rec.x, cur.rec.y, 0.f};
                if (!epi.sinfo) {
                    const float4 r = epi.info[cur.sg.x];
                    in.g = r.x;
                    in.sp = r.y;
                }
                fwd_finish(epi, cur.sg.x, tile, sub, acc, in);
            }
        }
        cur = nx;
    }
}

// The plug's gradients (flyguy_train.cu:158-167 and 174-179 on the plug's CSR) from the drive's complete gradient gd
// [T][n_s][32], which the sensory layer's backward leaves in place of the drive's gradient: per (tile, sensory row j)
// the bias partial ginb[tile][j] = the tile's sum of gd, and per connection f of the row ginw[tile][f] = the tile's
// sum of gd x[in_col[f]].  These are the sums the sensory finish of k_bwd forms (a dot of 4 per lane, then rs8 over
// the row's 8 lanes), term for term, with the tile's observation slab read from LDS (staged as in k_fwd_lds)
// instead of gathered through the vector-memory path.  S workgroups per tile; 8-lane group g of workgroup s takes
// rows s G + g, (S + s) G + g, ... (G groups per workgroup).  A row's gradient line and connection range are
// requested two rows ahead and its first 16 columns one row ahead, all before the current row's stores.
__global__ __launch_bounds__(FWD_LDS_NW * 64) void k_plug_bwd_lds(const float* __restrict__ gd,
                                                                 const float* __restrict__ x, int x_rows,
                                                                 const int* __restrict__ in_crow,
                                                                 const int* __restrict__ in_col, int n_s,
                                                                 float* __restrict__ ginb, long long gb_ld,
                                                                 float* __restrict__ ginw, long long gw_ld, int T,
                                                                 int S) {
    extern __shared__ __align__(16) float4 xs[];          // the tile's observation slab, x_rows x LPR float4
    constexpr int G = FWD_LDS_NW * 64 / LPR;
    int s;
    const int tile = tile_of(blockIdx.x, S, T, s);
    const float4* gx = reinterpret_cast<const float4*>(x + (size_t)tile * x_rows * TW);
    for (int i = threadIdx.x; i < x_rows * LPR; i += FWD_LDS_NW * 64) xs[i] = gx[i];
    __syncthreads();
    const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7;
    const float4* gdt = reinterpret_cast<const float4*>(gd + (size_t)tile * n_s * TW);
    float* wo = ginw + (size_t)tile * gw_ld;
    struct Row {
        float4 g;
        int f0, f1, c0, c1;
    };
    auto fetch = [&](int j, Row& r) {          // its gradient line and connection range
        const bool ok = j < n_s;
        // (a cached load: the sensory finish has just written these lines, and reading them with the streaming
        // hint made hop 1's backward slower, 1.385 -> 1.412 ms at B=4096)
        r.g = ok ? gdt[(size_t)j * LPR + sub] : splat(0.f);
        r.f0 = ok ? in_crow[j] : 0;
        r.f1 = ok ? in_crow[j + 1] : 0;
    };
    auto cols = [&](Row& r) {                  // its first 16 columns (NO_ROW past the row's end)
        r.c0 = r.f0 + sub < r.f1 ? in_col[r.f0 + sub] : NO_ROW;
        r.c1 = r.f0 + 8 + sub < r.f1 ? in_col[r.f0 + 8 + sub] : NO_ROW;
    };
    // the connections of 8 columns (one per lane) against the row's line: lane l ends with column l's sum
    auto chunk = [&](const float4& g, int mc) {
        int c[8];
        c[0] = bcast8<0>(mc); c[1] = bcast8<1>(mc); c[2] = bcast8<2>(mc); c[3] = bcast8<3>(mc);
        c[4] = bcast8<4>(mc); c[5] = bcast8<5>(mc); c[6] = bcast8<6>(mc); c[7] = bcast8<7>(mc);
        float dd[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            dd[u] = (unsigned)c[u] < (unsigned)x_rows ? dot4(g, xs[c[u] * LPR + sub]) : 0.f;
        return rs8(dd, sub);
    };
    const int step = S * G;
    int j = s * G + grp;
    Row cur, nx, nn;
    fetch(j, cur);
    cols(cur);
    fetch(j + step, nx);
    for (; j < n_s; j += step) {
        fetch(j + 2 * step, nn);
        cols(nx);
        const float pb = gsum8(hsum4(cur.g));
        const float p0 = chunk(cur.g, cur.c0), p1 = chunk(cur.g, cur.c1);
        if (sub == 0) ginb[(size_t)tile * gb_ld + j] = pb;
        if (cur.f0 + sub < cur.f1) wo[cur.f0 + sub] = p0;
        if (cur.f0 + 8 + sub < cur.f1) wo[cur.f0 + 8 + sub] = p1;
        for (int f = cur.f0 + 16; f < cur.f1; f += 8) {    // (rows of more than 16 connections)
            const float p = chunk(cur.g, f + sub < cur.f1 ? in_col[f + sub] : NO_ROW);
            if (f + sub < cur.f1) wo[f + sub] = p;
        }
        cur = nx;
        nx = nn;
    }
}

// Reads the given tables (16-byte words) and keeps nothing: brings them into the L2 of every XCD before a kernel
// whose workgroups all start by reading them.  Block b reads for XCD b & 7 (the hardware deals blocks to the XCDs in
// turn), so each XCD's blocks together read every table once.
__global__ __launch_bounds__(WG) void k_touch(TouchJob j) {
    const long long per = ((long long)gridDim.x / 8) * WG;        // threads per XCD
    const long long i0 = (long long)(blockIdx.x >> 3) * WG + threadIdx.x;
    unsigned acc = 0;
#pragma unroll
    for (int k = 0; k < TOUCH_JOBS; ++k)
        for (long long i = i0; i < j.n[k]; i += per) acc ^= j.p[k][i].x;
    asm volatile("" ::"v"(acc));                                   // (the loads are kept; nothing is stored)
}

// split rows: partial sums in segment order, then the same finish
// acc += the n partial sums of (slots y .., tile), in slot order, 8 loads in flight
__device__ __forceinline__ void add_parts(const float* __restrict__ part, Lay lp, int tile, int y, int n, int sub,
                                          float4& acc) {
    int k = 0;
    for (; k + 8 <= n; k += 8) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = ld_stream(at4(part, lp, tile, y + k + u, sub));
#pragma unroll
        for (int u = 0; u < 8; ++u) add4(v[u], acc);
    }
    for (; k < n; ++k) add4(ld_stream(at4(part, lp, tile, y + k, sub)), acc);
}

__global__ __launch_bounds__(WG) void k_fwd_combine(Plan p, const float* __restrict__ part, Lay lp, FwdEpi epi, int T) {
    long long q = ((long long)blockIdx.x * WG + threadIdx.x);
    const int sub = (int)(q & 7);
    q >>= 3;
    const int tile = (int)(q % T);
    const long long i = q / T;
    int4 s;
    if (!load_split(p, i, s)) return;     // whole 8-lane groups leave together
    float4 acc = epi.bias ? splat(epi.bias[s.x]) : splat(0.f);
    const FwdIn in = fwd_inputs(epi, epi.info, s.x, s.w, tile, sub);
    add_parts(part, lp, tile, s.y, s.z, sub, acc);
    fwd_finish(epi, s.x, tile, sub, acc, in);
}

// One workgroup per tile: the tile's firing bytes -> its bitmap (bits, then the count of silent rows in the header)
__global__ __launch_bounds__(WG) void k_fires_pack(const unsigned char* __restrict__ bytes, int rows,
                                                   unsigned* __restrict__ bits, int ld) {
    __shared__ unsigned silent[WG / 64];
    const int tile = blockIdx.x;
    const unsigned char* b = bytes + (size_t)tile * fires_bytes_ld(rows);
    unsigned* out = bits + (size_t)tile * ld;
    unsigned quiet = 0;
    for (int w = threadIdx.x; w < ld - 4; w += WG) {
        // the word's 32 bytes as two aligned 16-byte loads (rows of a tile are fires_bytes_ld(rows) bytes apart);
        // each byte is 0 or 1, so bit 8 j of a 32-bit piece is row 4 i + j of the piece's 4 rows
        unsigned m = 0;
        if (32 * w < rows) {
            const uint4 lo = reinterpret_cast<const uint4*>(b)[2 * w], hi = reinterpret_cast<const uint4*>(b)[2 * w + 1];
            const unsigned v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const unsigned x = v[i] & 0x01010101u;
                m |= ((x | (x >> 7) | (x >> 14) | (x >> 21)) & 0xFu) << (4 * i);
            }
            const int valid = min(32, rows - 32 * w);
            if (valid < 32) m &= (1u << valid) - 1u;
            quiet += (unsigned)(valid - __popc(m));
        }
        out[4 + w] = m;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) quiet += __shfl_xor(quiet, o, 64);
    if ((threadIdx.x & 63) == 0) silent[threadIdx.x >> 6] = quiet;
    __syncthreads();
    if (threadIdx.x < 4) out[threadIdx.x] = threadIdx.x == 0 ? ((silent[0] + silent[1]) + silent[2]) + silent[3] : 0u;
}

// ------------------------------------------------------------------------------------------------ backward
// The source row's own inputs of the neuron backward (h, z, gain, re-drive row; for the sensory layer the drive's
// gradient so far), loaded before the edge loop so that their latency hides behind the gathers.
struct BwdIn {
    float4 h, z, gd;
    float gn, sp;
    int d;
};
// MODE (the epilogue's kind, a compile-time constant so that each kernel is straight-line code for its own case):
// 0 the raw product, 1 a hop layer (d: the row's re-drive row), 2 the sensory layer
// (the row's h given: a kernel that has loaded it already, from the same layer, hands it over)
// recs: the wave's 8 records in plan order (sinfo + 8 w; the row's is recs[i]), or null: the row's from info
template <int MODE>
__device__ __forceinline__ BwdIn bwd_inputs_h(const BwdEpi& e, int j, int d, int tile, int sub, float4 h,
                                              const float4* recs = nullptr, int i = 0) {
    BwdIn in{make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f), 0.f, 0.f, -1};
    if constexpr (MODE == 0) return in;
    // the row's drive gradient so far (see BwdEpi): a first write starts from zero; the sensory layer's own is
    // complete now (every hop above has added its share), or zero where no hop re-drives the row
    bool load;
    if constexpr (MODE == 2) {
        in.d = j;
        load = d != -2;
    } else {
        in.d = d <= -3 ? -d - 3 : d;
        load = d >= 0 && !e.first;
    }
    if (load) in.gd = ld_stream(at4u(e.gdrive, e.lgd, tile, in.d, sub));
    in.h = h;
    if constexpr (MODE == 2) in.z = ld_stream(at4u(e.z, e.lz, tile, j, sub));
    const float2 r = *reinterpret_cast<const float2*>(recs ? recs + i : e.info + j);
    in.gn = r.x;
    in.sp = r.y;
    return in;
}
template <int MODE>
__device__ __forceinline__ BwdIn bwd_inputs(const BwdEpi& e, int j, int d, int tile, int sub) {
    if constexpr (MODE == 0) return bwd_inputs_h<0>(e, j, d, tile, sub, splat(0.f));
    return bwd_inputs_h<MODE>(e, j, d, tile, sub, ld_stream(at4u(e.h, e.lh, tile, j, sub)));
}

// A hop layer's neuron backward for (row, tile) from gh, the gradient of its output: gz = g gain with g = gh where the
// row fired (h > 0) and 0 elsewhere, and the tile's gain and threshold partials pg = sum g z, ps = sum g (every lane of
// the 8-lane group calls this; each gets the group's sums).  The sum of g z needs no z: where h > 0, z = (h +
// softplus(theta)) / gain, and elsewhere g = 0, so it is (sum g h + softplus(theta) sum g) / gain.  A neuron of gain 0
// never fires (h = relu(-sp)): its g and so its sum are 0.
struct HopBack {
    float4 gz;
    float pg, ps;
};
__device__ __forceinline__ HopBack hop_back(const float4& gh, const float4& hv, float gn, float sp) {
    const float4 g = make_float4(hv.x > 0.f ? gh.x : 0.f, hv.y > 0.f ? gh.y : 0.f, hv.z > 0.f ? gh.z : 0.f,
                                 hv.w > 0.f ? gh.w : 0.f);
    HopBack b;
    b.gz = make_float4(g.x * gn, g.y * gn, g.z * gn, g.w * gn);
    b.ps = gsum8(hsum4(g));
    b.pg = gn != 0.f ? (gsum8(dot4(g, hv)) + sp * b.ps) / gn : 0.f;
    return b;
}

// gh: the gradient of this layer's output h for (row j, tile); every lane of the 8-lane group calls this
template <int MODE>
// keep (optional): the row's gain and threshold partials of the tile are returned there instead of stored (a kernel
// that sums them over two tiles first)
// gcol: the column of the row's gain and threshold partials (its plan column, see BwdEpi; -1: the row itself)
__device__ __forceinline__ void bwd_finish(const BwdEpi& e, int j, int tile, int sub, float4 gh, const BwdIn& in,
                                           float2* keep = nullptr, int gcol = -1) {
    if constexpr (MODE == 0) {
        *at4w(e.gh_out, e.lgh, tile, j, sub) = gh;
        return;
    }
    float4 gzv;
    float ps, pg;
    if constexpr (MODE == 1) {
        const HopBack b = hop_back(gh, in.h, in.gn, in.sp);
        gzv = b.gz;
        ps = b.ps;
        pg = b.pg;
    } else {
        const float4 hv = in.h;
        const float4 g = make_float4(hv.x > 0.f ? gh.x : 0.f, hv.y > 0.f ? gh.y : 0.f, hv.z > 0.f ? gh.z : 0.f,
                                     hv.w > 0.f ? gh.w : 0.f);
        const float gn = in.gn;
        gzv = make_float4(g.x * gn, g.y * gn, g.z * gn, g.w * gn);
        ps = gsum8(hsum4(g));
        pg = gsum8(dot4(g, in.z));              // the sensory layer keeps its pre-activation (the drive)
    }
    if (keep) {
        *keep = make_float2(pg, ps);
    } else if (sub == 0) {
        const int col = gcol >= 0 ? gcol : j;
        e.ggain_part[(size_t)tile * e.gp_ld + col] = pg;
        e.gsum_part[(size_t)tile * e.gp_ld + col] = ps;
    }
    if constexpr (MODE == 1) {
        st_stream(at4uw(e.gz_out, e.lgz, tile, j, sub), gzv);
        if (in.d >= 0) {
            float4 v = in.gd;
            add4(gzv, v);
            st_stream(at4uw(e.gdrive, e.lgd, tile, in.d, sub), v);
        }
        return;
    }
    // the sensory layer: the drive's gradient is complete now -> the plug's bias and per-connection gradients
    float4 gd = in.gd;
    add4(gzv, gd);
    if (!e.in_crow) {                           // (they come from k_plug_bwd_lds, which reads gd back from here)
        st_stream(at4uw(e.gdrive, e.lgd, tile, j, sub), gd);
        return;
    }
    const float pb = gsum8(hsum4(gd));
    if (sub == 0) e.ginb_part[(size_t)tile * e.gb_ld + j] = pb;
    // connections 8 at a time: each lane fetches one column, the group shares them, gathers the 8 observation rows
    // (a column outside the observations reads zeros) and lane s keeps connection s's sum over the tile
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
            const float4 xv = *at4u(e.x, e.lx, tile, ok ? c[s2] : 0, sub);
            dd[s2] = ok ? dot4(gd, xv) : 0.f;
        }
        const float pw = rs8(dd, sub);
        if (f + sub < f1) gwo[f + sub] = pw;
    }
}

template <bool TILED, int MODE, int PB>
__global__ __launch_bounds__(WG) void k_bwd(Plan p, const int2* __restrict__ cw, const float* __restrict__ gz, Lay lg,
                                            int gz_rows, const float* __restrict__ hs, Lay lhs, float* __restrict__ gwpart,
                                            long long gw_ld, BwdEpi epi, float* __restrict__ part, Lay lp, int T, int RB) {
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
    // The source row's own line (the per-edge gradient's operand) comes first, with the wave's first pairs: with a
    // neuron backward (MODE 1, 2) a row that fires on none of the tile's samples has g = 0 there, so its gathers are
    // skipped (NO_ROW reads zeros without touching memory); its sums and partials are zero either way.
    float4 hj = splat(0.f);
    if (live) hj = MODE == 0 ? *at4(hs, lhs, tile, sg.x, sub) : ld_stream(at4u(hs, lhs, tile, sg.x, sub));
    const bool quiet = MODE != 0 && epi.skip_silent && group_silent(hj);
    const Slab<TILED> slab(gz + (size_t)tile * lg.tile, lg.row, gz_rows, sub);
    // the partial of (position, tile) of this lane's slot: one contiguous 256-byte block per wave and step
    float* gwp = gwpart ? gwpart + (size_t)tile * gw_ld + wv.x + lane : nullptr;
    float4 acc = splat(0.f);
    const bool whole = live && sg.y < 0;
    // A step's weight-gradient partial is stored after the next step's gathers have gone out: loads and stores count
    // in one vector-memory counter, so gathers issued after a store are waited for only once the store is done.
    float pend = 0.f;
    int j = 0;
    for (int left = wok ? wv.y : 0; left > 0; ++j, left -= 8) {
        int c[8];
        float wt[8];
        stage_pairs<PB>(slots, grp, sub, nxt, false, nullptr, gz_rows, c, wt);
        float4 v[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) v[s] = s < left ? slab.get(quiet ? NO_ROW : c[s], sub) : splat(0.f);
        __builtin_amdgcn_sched_barrier(0);
        if (left > 8) nxt = q.step(j + 1);
        if (gwp && j > 0) __builtin_nontemporal_store(pend, gwp + 64 * (j - 1));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 8; ++s) fma4(wt[s], v[s], acc);
        if (gwp) {
            float d[8];
#pragma unroll
            for (int s = 0; s < 8; ++s) d[s] = dot4(hj, v[s]);
            pend = rs8(d, sub);
        }
    }
    if (gwp && j > 0) __builtin_nontemporal_store(pend, gwp + 64 * (j - 1));
    if (!live) return;
    // the row's other inputs of the neuron backward, after the loop: live across it they would cost registers, and
    // with them waves per SIMD
    BwdIn in{};
    if (whole) in = bwd_inputs_h<MODE>(epi, sg.x, sg.z, tile, sub, hj, epi.sinfo ? epi.sinfo + 8 * w : nullptr, grp & 7);
    if (sg.y >= 0) {
        st_stream(at4w(part, lp, tile, sg.y, sub), acc);
        return;
    }
    bwd_finish<MODE>(epi, sg.x, tile, sub, acc, in, nullptr, w * 8 + (grp & 7));
}

// The same over two tiles at once, tiles 2 pr and 2 pr + 1 of a pair pr (the second may not exist): a step gathers
// the source lines of both tiles for the same (source, weight) pairs, and the weight-gradient partial of a position is
// summed over both tiles (tile 2 pr first) and stored once per pair: gwpart [ceil(T / 2)][gw_ld]
template <int MODE, int PB>
__global__ __launch_bounds__(WG) void k_bwd2(Plan p, const int2* __restrict__ cw, const float* __restrict__ gz, Lay lg,
                                             int gz_rows, const float* __restrict__ hs, Lay lhs, float* __restrict__ gwpart,
                                             long long gw_ld, BwdEpi epi, float* __restrict__ part, Lay lp, int T, int RB) {
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
    // the source row's own lines first, and on a tile where the row fires on no sample its gathers are skipped (k_bwd)
    float4 hja = splat(0.f), hjb = splat(0.f);
    if (live) {
        hja = ld_stream(at4u(hs, lhs, ta, sg.x, sub));
        if (hasb) hjb = ld_stream(at4u(hs, lhs, tb, sg.x, sub));
    }
    const bool quiet_a = epi.skip_silent && group_silent(hja), quiet_b = epi.skip_silent && group_silent(hjb);
    const Slab<true> sa(gz + (size_t)ta * lg.tile, lg.row, gz_rows, sub);
    const Slab<true> sb(gz + (size_t)(hasb ? tb : ta) * lg.tile, lg.row, gz_rows, sub);
    float* gwp = gwpart ? gwpart + (size_t)pr * gw_ld + wv.x + lane : nullptr;
    float4 acca = splat(0.f), accb = splat(0.f);
    const bool whole = live && sg.y < 0;
    float pend = 0.f;                           // (a step's partial is stored after the next step's gathers: k_bwd)
    int j = 0;
    for (int left = wok ? wv.y : 0; left > 0; ++j, left -= 8) {
        int c[8];
        float wt[8];
        stage_pairs<PB>(slots, grp, sub, nxt, false, nullptr, gz_rows, c, wt);
        float4 va[8], vb[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) va[s] = s < left ? sa.get(quiet_a ? NO_ROW : c[s], sub) : splat(0.f);
#pragma unroll
        for (int s = 0; s < 8; ++s) vb[s] = (hasb && s < left) ? sb.get(quiet_b ? NO_ROW : c[s], sub) : splat(0.f);
        __builtin_amdgcn_sched_barrier(0);
        if (left > 8) nxt = q.step(j + 1);
        if (gwp && j > 0) __builtin_nontemporal_store(pend, gwp + 64 * (j - 1));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            fma4(wt[s], va[s], acca);
            fma4(wt[s], vb[s], accb);
        }
        if (gwp) {
            float d[8];
#pragma unroll
            for (int s = 0; s < 8; ++s) d[s] = dot4(hja, va[s]) + dot4(hjb, vb[s]);
            pend = rs8(d, sub);
        }
    }
    if (gwp && j > 0) __builtin_nontemporal_store(pend, gwp + 64 * (j - 1));
    if (!live) return;
    BwdIn ina{}, inb{};                         // the rows' other inputs, after the loop (k_bwd)
    if (whole) {                                // (hs is the layer's h: the core's launches hand over e.h)
        const float4* recs = epi.sinfo ? epi.sinfo + 8 * w : nullptr;
        ina = bwd_inputs_h<MODE>(epi, sg.x, sg.z, ta, sub, hja, recs, grp & 7);
        if (hasb) inb = bwd_inputs_h<MODE>(epi, sg.x, sg.z, tb, sub, hjb, recs, grp & 7);
    }
    if (sg.y >= 0) {
        st_stream(at4w(part, lp, ta, sg.y, sub), acca);
        if (hasb) st_stream(at4w(part, lp, tb, sg.y, sub), accb);
        return;
    }
    float2 ka, kb = make_float2(0.f, 0.f);
    bwd_finish<MODE>(epi, sg.x, ta, sub, acca, ina, &ka);
    if (hasb) bwd_finish<MODE>(epi, sg.x, tb, sub, accb, inb, &kb);
    if (sub == 0) {                             // the row's gain and threshold partials, one per pair of tiles
        const int col = w * 8 + (grp & 7);      // (the plan column of the row: its segment)
        epi.ggain_part[(size_t)pr * epi.gp_ld + col] = ka.x + kb.x;
        epi.gsum_part[(size_t)pr * epi.gp_ld + col] = ka.y + kb.y;
    }
}

// PAIR: an 8-lane group finishes the split row for both tiles of a pair (tiles 2 q and 2 q + 1, the second may not
// exist) and stores the row's gain and threshold partials once per pair, as k_bwd2 does
template <int MODE, bool PAIR>
__global__ __launch_bounds__(WG) void k_bwd_combine(Plan p, const float* __restrict__ part, Lay lp, BwdEpi epi, int T) {
    const int NT = PAIR ? (T + 1) / 2 : T;
    long long q = ((long long)blockIdx.x * WG + threadIdx.x);
    const int sub = (int)(q & 7);
    q >>= 3;
    const int u = (int)(q % NT);
    const long long i = q / NT;
    int4 s;
    if (!load_split(p, i, s)) return;     // whole 8-lane groups leave together
    if constexpr (!PAIR) {
        float4 acc = splat(0.f);
        const BwdIn in = bwd_inputs<MODE>(epi, s.x, s.w, u, sub);
        add_parts(part, lp, u, s.y, s.z, sub, acc);
        bwd_finish<MODE>(epi, s.x, u, sub, acc, in, nullptr, (int)(p.nseg + i));
    } else {
        float2 k2[2] = {make_float2(0.f, 0.f), make_float2(0.f, 0.f)};
        for (int h = 0; h < 2 && 2 * u + h < T; ++h) {
            const int tile = 2 * u + h;
            float4 acc = splat(0.f);
            const BwdIn in = bwd_inputs<MODE>(epi, s.x, s.w, tile, sub);
            add_parts(part, lp, tile, s.y, s.z, sub, acc);
            bwd_finish<MODE>(epi, s.x, tile, sub, acc, in, &k2[h]);
        }
        if (sub == 0) {
            epi.ggain_part[(size_t)u * epi.gp_ld + p.nseg + i] = k2[0].x + k2[1].x;
            epi.gsum_part[(size_t)u * epi.gp_ld + p.nseg + i] = k2[0].y + k2[1].y;
        }
    }
}

// ------------------------------------------------------------------------------------------------ backward, LDS
// The backward of a hop layer (mode 1) for a gathered slab that mostly fits the LDS: the hop into the descending
// layer gathers 1,332 rows of gradient, 170 kB a tile, against the 160 kB of LDS a workgroup may hold.  Each workgroup
// stages the `hot` most gathered rows of its tile's slab in LDS once and walks its share of the transposed plan,
// gathering from the LDS.  A pair's code names an LDS row (code < hot) or a slab row (hot + row); a step issues
// vector-memory gathers only for slots that some group needs from the slab.  With the gathers off the vector-memory
// path, that path carries only the loads that come from HBM (each row's own h line, the plan's records and pairs),
// and those no longer hold up the return of gathered lines behind them.  The sums are k_bwd's (one tile per
// workgroup), term for term in the same order.
// S workgroups per tile, one per CU; a wave walks plan waves w0 + k dw, k < n <= 64 BWD_LDS_WREC, with lane l of
// wrec[r] holding plan wave 64 r + l's record.  A plan wave's segment, records and first pairs are requested two plan
// waves ahead and its rows' h lines one plan wave ahead (they need the segment's row), so that waiting for them does
// not wait for the stores issued in between.
// a ? x : y, element by element (a select of whole vector structs can turn into a select of their addresses,
// which puts arrays of them in scratch memory)
__device__ __forceinline__ float4 sel4(bool a, const float4& x, const float4& y) {
    return make_float4(a ? x.x : y.x, a ? x.y : y.y, a ? x.z : y.z, a ? x.w : y.w);
}
constexpr int BWD_LDS_STAGE = (BWD_LDS_MAXROWS * LPR + BWD_LDS_NW * 64 - 1) / (BWD_LDS_NW * 64);
template <int PB, bool SKIP>
__global__ __launch_bounds__(BWD_LDS_NW * 64) void k_bwd_lds(Plan p, const int2* __restrict__ wlds,
                                                            const int2* __restrict__ cw,
                                                            const float* __restrict__ gz, int gz_rows,
                                                            const int* __restrict__ hot_rows, int hot,
                                                            const float* __restrict__ hs, Lay lhs,
                                                            float* __restrict__ gwpart, long long gw_ld, BwdEpi epi,
                                                            float* __restrict__ part, Lay lp, int T, int S) {
    constexpr int NT = BWD_LDS_NW * 64;
    __shared__ __align__(16) int2 slots[NT / LPR][LPR];
    extern __shared__ __align__(16) float4 gs[];          // LDS row r: slab row hot_rows[r], LPR float4
    int s;
    const int tile = tile_of(blockIdx.x, S, T, s);
    const int grp = threadIdx.x >> 3, sub = threadIdx.x & 7, lane = threadIdx.x & 63, gi = grp & 7;
    const int w0 = __builtin_amdgcn_readfirstlane(s * BWD_LDS_NW + (int)(threadIdx.x >> 6)), dw = S * BWD_LDS_NW;
    const int n = w0 < p.nwave ? min((p.nwave - 1 - w0) / dw + 1, 64 * BWD_LDS_WREC) : 0;
    int2 wrec[BWD_LDS_WREC];
#pragma unroll
    for (int r = 0; r < BWD_LDS_WREC; ++r)
        wrec[r] = 64 * r + lane < n ? wlds[w0 + (64 * r + lane) * dw] : make_int2(0, 0);
    // the hot rows: every row index first, then every line, then the LDS stores (so the loads overlap)
    const float4* gt = reinterpret_cast<const float4*>(gz + (size_t)tile * gz_rows * TW);
    {
        int ri[BWD_LDS_STAGE];
        float4 lv[BWD_LDS_STAGE];
#pragma unroll
        for (int u = 0; u < BWD_LDS_STAGE; ++u) {
            const int i = (int)threadIdx.x + u * NT;
            ri[u] = i < hot * LPR ? hot_rows[i / LPR] : -1;
        }
#pragma unroll
        for (int u = 0; u < BWD_LDS_STAGE; ++u) {
            const int i = (int)threadIdx.x + u * NT;
            lv[u] = (unsigned)ri[u] < (unsigned)gz_rows ? gt[(size_t)ri[u] * LPR + (i % LPR)] : splat(0.f);
        }
#pragma unroll
        for (int u = 0; u < BWD_LDS_STAGE; ++u) {
            const int i = (int)threadIdx.x + u * NT;
            if (i < hot * LPR) gs[i] = lv[u];
        }
        if (threadIdx.x < LPR) gs[hot * LPR + threadIdx.x] = splat(0.f);     // row `hot`: zeros
    }
    __syncthreads();
    const Slab<true> slab(gz + (size_t)tile * gz_rows * TW, TW, gz_rows, sub);
    // The loads of plan waves still to come are issued on every path, at addresses clamped into their arrays, and
    // the rare loads of a step (a slab row outside the LDS, a third step's pairs, a drive gradient to add to) are
    // waited for inside their own branches.  The compiler then knows how many loads follow each prefetched one, and
    // waiting for it does not wait for those issued after it.
    // A plan wave's loads as they arrive: nothing derived from a loaded value is computed before it is needed
    struct Pre {
        int w;
        int2 wv;                                // its record {woff, longest segment} (wave-uniform)
        bool cold;                              // some pair of it names a slab row outside the LDS (wave-uniform)
        bool wok;                               // the record is real and inside the plan (wave-uniform)
        bool sok;                               // the group has a segment (w * 8 + gi < nseg)
        int2 pr0, pr1;                          // the pairs of its first two steps as loaded
        int4 sg;                                // the group's segment as loaded
        float2 rec;                             // the row's gain and softplus(theta) as loaded
    };
    // the loads of plan wave k that need only its number (k >= n: the last plan wave's again, marked empty)
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
        // (a step past the wave's last reads the first step's block again; with 6-byte pairs lanes 48-63 load a
        // lane's below, which the staging never reads)
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
    // whether the group's segment is real (load_segment's test)
    auto live = [&](const Pre& it) { return it.wok && it.sok && it.sg.x >= 0 && it.sg.x < p.rows && it.sg.y < p.nslot; };
    // the h lines of a plan wave's rows (row 0's where a group has none: the reader masks them)
    auto hline = [&](const Pre& it) { return ld_stream(at4u(hs, lhs, tile, live(it) ? it.sg.x : 0, sub)); };
    // one step of plan wave `cur`: the gathers of its pairs `pr` (8 slots of each group) and the sums; returns the step's
    // weight-gradient partial of the lane's position
    // (slots past a segment's end hold the pair (no row, 0), which gathers zeros, as does a silent row's: every code
    // from hot up reads LDS row `hot`, which holds zeros, so that no slot's read is conditional)
    auto step = [&](bool cold, int2 pr, bool quiet, const float4& hc, float4& acc) __attribute__((always_inline)) {
        int c[8];
        float wt[8];
        stage_pairs<PB>(slots, grp, sub, pr, false, nullptr, 0, c, wt);
        if (SKIP && quiet) {
#pragma unroll
            for (int u = 0; u < 8; ++u) c[u] = NO_ROW;
        }
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = gs[min((unsigned)c[u], (unsigned)hot) * LPR + sub];
        if (cold) {                                   // (the plan waves with a pair outside the LDS: 1 in 8)
            unsigned cr[8];
            bool any = false;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                cr[u] = (unsigned)c[u] - (unsigned)hot;
                any |= cr[u] < (unsigned)gz_rows;
            }
            if (__ballot(any)) {                      // (the loads go out together)
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    if (cr[u] < (unsigned)gz_rows) v[u] = slab.get((int)cr[u], sub);
                asm volatile("" ::"v"(v[0].x), "v"(v[1].x), "v"(v[2].x), "v"(v[3].x), "v"(v[4].x), "v"(v[5].x),
                             "v"(v[6].x), "v"(v[7].x));   // (waited for here)
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) fma4(wt[u], v[u], acc);
        float d[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) d[u] = dot4(hc, v[u]);
        return rs8(d, sub);
    };
    // Every plan wave issues the same vector-memory operations whatever its rows: 5 loads (plan wave k + 2's four,
    // plan wave k + 1's h lines) and 7 stores (two steps' weight-gradient partials, the row's gz, drive gradient,
    // split-row sum, gain and threshold partials).  A store that does not apply gets an offset past its buffer, which
    // the hardware drops.  Stores count in the same counter as loads: with their number fixed, waiting for a
    // prefetched load does not wait for the stores issued after it.
    constexpr unsigned OFF = 0x80000000u;
    auto rsrc = [](const void* b, long long bytes) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(b), (short)0,
                                                 b ? (int)min(bytes, 0x7FFFFFFFLL) : 0, 0x00020000);
    };
    const __amdgpu_buffer_rsrc_t r_gw = rsrc(gwpart ? gwpart + (size_t)tile * gw_ld : nullptr, gw_ld * 4);
    const __amdgpu_buffer_rsrc_t r_gz = rsrc(epi.gz_out + (size_t)tile * epi.lgz.tile, epi.lgz.tile * 4);
    const __amdgpu_buffer_rsrc_t r_gd = rsrc(epi.gdrive + (size_t)tile * epi.lgd.tile, epi.lgd.tile * 4);
    const __amdgpu_buffer_rsrc_t r_pt = rsrc(part ? part + (size_t)tile * lp.tile : nullptr, lp.tile * 4);
    const __amdgpu_buffer_rsrc_t r_gg = rsrc(epi.ggain_part + (size_t)tile * epi.gp_ld, epi.gp_ld * 4);
    const __amdgpu_buffer_rsrc_t r_gs = rsrc(epi.gsum_part + (size_t)tile * epi.gp_ld, epi.gp_ld * 4);
    // (the buffer stores take the values' bits: a float handed over as it is would be converted to an integer)
    auto st4 = [](const float4& v, __amdgpu_buffer_rsrc_t r, unsigned off) {
        const u32x4 t = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
        __builtin_amdgcn_raw_buffer_store_b128(t, r, off, 0, 2);        // (nontemporal)
    };
    auto st1 = [](float v, __amdgpu_buffer_rsrc_t r, unsigned off, int nt) {
        if (nt)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 2);
        else
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 0);
    };
    // Plan wave k with its loads in flight: cur (its own, issued two plan waves ago) and hr (its rows' h lines, one
    // plan wave ago); it issues nx's h lines (plan wave k + 1) into hn and plan wave k + 2's loads into n2.  The caller
    // rotates three Pre and two h slots by unrolling (below) instead of copying them: a copy of a register whose load
    // is still in flight would wait for it.
    auto plan_wave = [&](int k, const Pre& cur, const float4& hr, const Pre& nx, float4& hn, Pre& n2)
        __attribute__((always_inline)) {
        issue(k + 2, n2);
        hn = hline(nx);
        const bool lv = live(cur);
        const float4 hc = sel4(lv, hr, splat(0.f));
        // a row that fires on none of the tile's samples gathers nothing (k_bwd)
        const bool quiet = SKIP && group_silent(hc);
        float4 acc = splat(0.f);
        const int L = cur.wv.y;                       // (0 unless the record is real)
        float pend0 = 0.f, pend1 = 0.f;
        if (L > 0) pend0 = step(cur.cold, cur.pr0, quiet, hc, acc);
        if (L > 8) pend1 = step(cur.cold, cur.pr1, quiet, hc, acc);
        if (L > 16) {                                 // (rare: a third step and more, their pairs loaded here)
            const PairLoad<PB> q(cw, cur.wv.x, lane);
            for (int j = 2; 8 * j < L; ++j) {
                int2 pr = q.step(j);
                asm volatile("" : "+v"(pr.x), "+v"(pr.y));
                const float pe = step(cur.cold, pr, quiet, hc, acc);
                st1(pe, r_gw, (unsigned)(cur.wv.x + 64 * j + lane) * 4u, 1);
            }
        }
        st1(pend0, r_gw, L > 0 ? (unsigned)(cur.wv.x + lane) * 4u : OFF, 1);
        st1(pend1, r_gw, L > 8 ? (unsigned)(cur.wv.x + 64 + lane) * 4u : OFF, 1);
        // the row's neuron backward (bwd_finish, MODE 1), or a split row's partial sum
        const bool whole = lv && cur.sg.y < 0;
        const HopBack b = hop_back(acc, hc, cur.rec.x, cur.rec.y);
        const int d = cur.sg.z, dr = d <= -3 ? -d - 3 : d;
        float4 gdv = splat(0.f);
        const bool add = whole && d >= 0 && !epi.first;
        if (__ballot(add)) {                          // (rare: a drive gradient written by a layer above)
            const float4 g = ld_stream(at4u(epi.gdrive, epi.lgd, tile, add ? dr : 0, sub));
            gdv = sel4(add, g, gdv);
            asm volatile("" : "+v"(gdv.x), "+v"(gdv.y), "+v"(gdv.z), "+v"(gdv.w));
        }
        add4(b.gz, gdv);
        const unsigned line = (unsigned)sub * 16u;
        st4(b.gz, r_gz, whole ? (unsigned)cur.sg.x * (TW * 4u) + line : OFF);
        st4(gdv, r_gd, whole && dr >= 0 ? (unsigned)dr * (TW * 4u) + line : OFF);
        st4(acc, r_pt, lv && cur.sg.y >= 0 ? (unsigned)cur.sg.y * (TW * 4u) + line : OFF);
        const unsigned col = whole && sub == 0 ? (unsigned)(cur.w * 8 + gi) * 4u : OFF;
        st1(b.pg, r_gg, col, 0);
        st1(b.ps, r_gs, col, 0);
    };
    if (n <= 0) return;
    Pre p0, p1, p2;                             // plan wave k's loads in slot k % 3
    float4 h0, h1;                              // its rows' h lines in slot k % 2
    issue(0, p0);
    issue(1, p1);
    h0 = hline(p0);
    // the 7 stores a plan wave ends with, all dropped: the first plan wave then finds the operations in flight in the
    // same order as every later one, and its waits are counted as theirs
    st1(0.f, r_gw, OFF, 1);
    st1(0.f, r_gw, OFF, 1);
    st4(splat(0.f), r_gz, OFF);
    st4(splat(0.f), r_gd, OFF);
    st4(splat(0.f), r_pt, OFF);
    st1(0.f, r_gg, OFF, 0);
    st1(0.f, r_gs, OFF, 0);
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

// gh of the top layer from the logits' gradient (flyguy_train.cu:136-141) on the matrix cores (readout.h): 32 rows x
// 32 samples per workgroup, then the neuron backward (:143-156) per row and lane
__global__ __launch_bounds__(WG) void k_readout_bwd_h_mfma(const float* __restrict__ dl, const float* __restrict__ owT,
                                                           int ma, const int* __restrict__ dn_inv, int n_act, int rows,
                                                           BwdEpi epi) {
    __shared__ float part[4 * 32 * 33];
    __shared__ float gh[32 * 33];
    const int tile = blockIdx.y, r0 = blockIdx.x * RPG;
    readout_gh_block(dl, owT, ma, dn_inv, rows, n_act, r0, tile * TW, part, gh, 33);
    const int r = threadIdx.x >> 3, sub = threadIdx.x & 7, t = r0 + r;
    if (t >= rows) return;                 // whole 8-lane groups
    const float* g = gh + r * 33 + sub * 4;
    const float4 acc = make_float4(g[0], g[1], g[2], g[3]);
    bwd_finish<1>(epi, t, tile, sub, acc, bwd_inputs<1>(epi, t, epi.drow ? epi.drow[t] : -1, tile, sub));
}

// per chunk of RO_CHUNK_S samples: the read-out weights' gradient partials (readout.hip)
int readout_chunks(int B) { return (B + RO_CHUNK_S - 1) / RO_CHUNK_S; }

// ------------------------------------------------------------------------------------------------ reductions
// G[idx[i]] += sum_t part[t * ld + i]  (times -sigmoid(theta[idx[i]]) when theta is given: the threshold's gradient);
// idx[i] = -1 (a plan position no edge uses) adds nothing; idx[i] <= -2 marks entry -idx[i] - 2's first sum, which a
// fresh job stores (kernels.h, RedJob)
__global__ __launch_bounds__(WG) void k_reduce(JobTable<RedJob, RED_JOBS> jt) {
    long long b0;
    const RedJob r = job_of(jt, blockIdx.x, b0);
    const long long i = ((long long)blockIdx.x - b0) * WG + threadIdx.x;
    if (i >= r.n) return;
    const int v = r.idx ? r.idx[i] : -1;
    if (r.idx && v == -1) return;
    const bool first = !r.idx || v < -1;
    const long long o = !r.idx ? i : (v < -1 ? -(long long)v - 2 : (long long)v);
    const float* __restrict__ part = r.part;
    float s = 0.f;
    int t = 0;
    for (; t + 8 <= r.nt; t += 8) {          // 8 loads in flight, added in tile order
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = part[(size_t)(t + k) * r.ld + i];
#pragma unroll
        for (int k = 0; k < 8; ++k) s += v[k];
    }
    for (; t < r.nt; ++t) s += part[(size_t)t * r.ld + i];
    if (r.theta) s *= -sigmoid_f(r.theta[o]);
    if (r.fresh && first)
        r.G[o] = s + 0.f;                       // (= 0 + s, -0 included, without reading the entry)
    else
        r.G[o] += s;
}

// KL(teacher || student) per sample, dl = d(mean loss)/d logits (flyguy_train.cu:104-123).  Eight lanes per sample,
// a workgroup of 256 threads per 32 samples: the samples' logits are staged through LDS with coalesced loads (and dl
// leaves the same way).  Lane k of a sample's group takes actions k, k + 8, ...; the group then combines its maxima
// (the larger value, on equal values the smaller action: the first maximum wins, as the reference's strict > does),
// its sums of exponentials and its KL terms over the 8 lanes.  Per-block sums of KL and argmax agreement go to
// stats_part.
constexpr int LOSS_S = 32;
__global__ __launch_bounds__(256) void k_loss(const float* __restrict__ lg, const float* __restrict__ tl,
                                              float* __restrict__ dl, float* __restrict__ stats_part, int n_act, int B,
                                              float it) {
    extern __shared__ float sm[];
    float* S = sm;                              // [LOSS_S][n_act] student logits, then dl
    float* Tt = sm + (size_t)LOSS_S * n_act;    // [LOSS_S][n_act] teacher logits * (1 / temperature)
    __shared__ float red[2][4];
    const int b0 = blockIdx.x * LOSS_S, nb = min(LOSS_S, B - b0);
    const size_t base = (size_t)b0 * n_act;
    for (int i = threadIdx.x; i < nb * n_act; i += 256) {
        S[i] = lg[base + i];
        Tt[i] = tl[base + i] * it;
    }
    __syncthreads();
    const int smp = threadIdx.x >> 3, sub = threadIdx.x & 7;
    float kl = 0.f, agree = 0.f;
    if (smp < nb) {                             // (whole 8-lane groups)
        float* s = S + (size_t)smp * n_act;
        const float* t = Tt + (size_t)smp * n_act;
        float ms = -1e30f, mt = -1e30f;
        int as = n_act, at = n_act;
        for (int a = sub; a < n_act; a += 8) {
            const float sv = s[a], tv = t[a];
            if (sv > ms) { ms = sv; as = a; }
            if (tv > mt) { mt = tv; at = a; }
        }
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) {
            const float vs = __shfl_xor(ms, o, 8), vt = __shfl_xor(mt, o, 8);
            const int is = __shfl_xor(as, o, 8), jt = __shfl_xor(at, o, 8);
            if (vs > ms || (vs == ms && is < as)) { ms = vs; as = is; }
            if (vt > mt || (vt == mt && jt < at)) { mt = vt; at = jt; }
        }
        if (as == n_act) as = 0;                // (no logit above -1e30: the reference keeps action 0)
        if (at == n_act) at = 0;
        float zs = 0.f, zt = 0.f;
        for (int a = sub; a < n_act; a += 8) {
            zs += expf(s[a] - ms);
            zt += expf(t[a] - mt);
        }
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) {
            zs += __shfl_xor(zs, o, 8);
            zt += __shfl_xor(zt, o, 8);
        }
        const float ls = ms + logf(zs), lt = mt + logf(zt);
        for (int a = sub; a < n_act; a += 8) {
            const float lps = s[a] - ls, lpt = t[a] - lt, pt = expf(lpt);
            kl += pt * (lpt - lps);
            s[a] = (expf(lps) - pt) / (float)B;
        }
        agree = (sub == 0 && as == at) ? 1.f : 0.f;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nb * n_act; i += 256) dl[base + i] = S[i];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        kl += __shfl_xor(kl, o, 64);
        agree += __shfl_xor(agree, o, 64);
    }
    if ((threadIdx.x & 63) == 0) {
        red[0][threadIdx.x >> 6] = kl;
        red[1][threadIdx.x >> 6] = agree;
    }
    __syncthreads();
    if (threadIdx.x == 0) {                     // the 4 waves' sums in wave order
        stats_part[2 * blockIdx.x] = ((red[0][0] + red[0][1]) + red[0][2]) + red[0][3];
        stats_part[2 * blockIdx.x + 1] = ((red[1][0] + red[1][1]) + red[1][2]) + red[1][3];
    }
}
__global__ void k_sum_pairs(const float* __restrict__ part, int n, float* __restrict__ out, int acc) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float a = 0.f, b = 0.f;
    for (int i = 0; i < n; ++i) { a += part[2 * i]; b += part[2 * i + 1]; }
    out[0] = acc ? out[0] + a : a;
    out[1] = acc ? out[1] + b : b;
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

// per row of a layer: {gain[nid], softplus(theta[nid]), re-drive row (int bits, -1 none), bias of the row or 0}
__global__ __launch_bounds__(WG) void k_rowinfo(JobTable<RowJob, ROW_JOBS> t, const float* __restrict__ gain,
                                                const float* __restrict__ theta) {
    long long b0;
    const RowJob J = job_of(t, blockIdx.x, b0);
    const long long r = ((long long)blockIdx.x - b0) * WG + threadIdx.x;
    if (r >= J.rows) return;
    const int row = J.seg ? J.seg[r].x : (int)r;
    const int n = J.nid[row];
    J.info[r] = make_float4(gain[n], softplus_f(theta[n]), __int_as_float(J.drow ? J.drow[row] : -1),
                            J.bias ? J.bias[row] : 0.f);
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

hipError_t launch_pack_n(const PackJob* jobs, int n, hipStream_t st, bool bf16w) {
    JobTable<PackJob, PACK_JOBS> t;
    long long nb;
    if (!fill_table(t, jobs, n, [](const PackJob& j) { return j.n; }, nb)) return hipErrorInvalidValue;
    for (int k = 0; k < t.n; ++k)
        if (!t.j[k].pcol || !t.j[k].pidx || !t.j[k].w || !t.j[k].cw || (t.j[k].pb != 8 && t.j[k].pb != 6) ||
            (t.j[k].pb == 6 && t.j[k].n % 64))
            return hipErrorInvalidValue;
    if (nb == 0) return hipSuccess;
    if (bf16w)
        k_pack<true><<<(unsigned)nb, WG, 0, st>>>(t);
    else
        k_pack<false><<<(unsigned)nb, WG, 0, st>>>(t);
    return hipGetLastError();
}

hipError_t launch_pack(const int* pcol, const int* pidx, const float* w, int2* cw, long long npos, hipStream_t st,
                       bool bf16w) {
    const PackJob j{pcol, pidx, w, cw, npos};
    return launch_pack_n(&j, 1, st, bf16w);
}

hipError_t launch_fwd(const Plan& p, const int2* cw, const float* src, Lay ls, int src_rows, const FwdEpi& epi,
                      float* part, Lay lp, int T, hipStream_t st, const unsigned* src_fires) {
    // 6-byte pairs name rows by 16 bits: only a tiled slab of at most PAIR6_MAX_ROWS rows reads 0xFFFF as past its end
    if ((p.pb != 8 && p.pb != 6) || (p.pb == 6 && (ls.row != TW || src_rows > PAIR6_MAX_ROWS)))
        return hipErrorInvalidValue;
    if (p.nwave > 0) {
        const int RB = (p.nwave + WG / 64 - 1) / (WG / 64);
        const int fw = src_fires && ls.row == TW && fires_ld(src_rows) <= FIRES_LDS_WORDS ? fires_ld(src_rows) : 0;
        const dim3 grid((unsigned)((long long)T * RB));
        const size_t lds = (size_t)(fw > 0 ? fw - 4 : 0) * 4;
        if (ls.row != TW)
            k_fwd<false, 8><<<grid, WG, 0, st>>>(p, cw, src, ls, src_rows, epi, part, lp, T, RB, nullptr, 0);
        else if (p.pb == 6)
            k_fwd<true, 6><<<grid, WG, lds, st>>>(p, cw, src, ls, src_rows, epi, part, lp, T, RB, src_fires, fw);
        else
            k_fwd<true, 8><<<grid, WG, lds, st>>>(p, cw, src, ls, src_rows, epi, part, lp, T, RB, src_fires, fw);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (p.nsplit > 0) {
        k_fwd_combine<<<blocks((long long)p.nsplit * T * LPR), WG, 0, st>>>(p, part, lp, epi, T);
        return hipGetLastError();
    }
    return hipSuccess;
}

hipError_t launch_fwd_lds(const Plan& p, const int2* cw, const float* src, int src_rows, const FwdEpi& epi, float* part,
                          Lay lp, int T, int S, hipStream_t st) {
    const size_t lds = (size_t)src_rows * TW * 4;
    if (S < 1 || src_rows < 1 || lds > FWD_LDS_BYTES || epi.drive || !epi.info || (p.pb != 8 && p.pb != 6) ||
        (p.pb == 6 && src_rows > PAIR6_MAX_ROWS))
        return hipErrorInvalidValue;
    S = std::max(S, (p.nwave + 64 * FWD_LDS_NW - 1) / (64 * FWD_LDS_NW));     // (at most 64 plan waves per wave)
    if (p.nwave > 0) {
        // (above 64 kB of dynamic LDS the kernel must be told its size; set on every launch, so that it holds on
        // whichever device is current)
        const void* k = p.pb == 6 ? reinterpret_cast<const void*>(&k_fwd_lds<6>) : reinterpret_cast<const void*>(&k_fwd_lds<8>);
        const hipError_t attr = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)FWD_LDS_BYTES);
        if (attr != hipSuccess) return attr;
        const dim3 grid((unsigned)((long long)T * S));
        if (p.pb == 6)
            k_fwd_lds<6><<<grid, FWD_LDS_NW * 64, lds, st>>>(p, cw, src, src_rows, epi, part, lp, T, S);
        else
            k_fwd_lds<8><<<grid, FWD_LDS_NW * 64, lds, st>>>(p, cw, src, src_rows, epi, part, lp, T, S);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (p.nsplit > 0) {
        k_fwd_combine<<<blocks((long long)p.nsplit * T * LPR), WG, 0, st>>>(p, part, lp, epi, T);
        return hipGetLastError();
    }
    return hipSuccess;
}

// the LDS a workgroup may use on the current device against FWD_LDS_BYTES + each kernel's static LDS
bool lds_fits(std::initializer_list<const void*> kernels) {
    int dev = 0, cap = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cap, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return false;
    for (const void* k : kernels) {
        hipFuncAttributes a{};
        if (hipFuncGetAttributes(&a, k) != hipSuccess || FWD_LDS_BYTES + a.sharedSizeBytes > (size_t)cap) return false;
    }
    return true;
}

bool lds_plug_fits() {
    return lds_fits({reinterpret_cast<const void*>(&k_fwd_lds<8>), reinterpret_cast<const void*>(&k_fwd_lds<6>),
                     reinterpret_cast<const void*>(&k_plug_bwd_lds)});
}

hipError_t launch_plug_bwd_lds(const float* gd, const float* x, int x_rows, const int* in_crow, const int* in_col,
                               int n_s, float* ginb, long long gb_ld, float* ginw, long long gw_ld, int T, int S,
                               hipStream_t st) {
    const size_t lds = (size_t)x_rows * TW * 4;
    if (S < 1 || x_rows < 1 || lds > FWD_LDS_BYTES || !gd || !x || !in_crow || !in_col || !ginb || !ginw)
        return hipErrorInvalidValue;
    if (n_s <= 0 || T <= 0) return hipSuccess;
    const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_plug_bwd_lds),    // (k_fwd_lds)
                                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)FWD_LDS_BYTES);
    if (attr != hipSuccess) return attr;
    k_plug_bwd_lds<<<(unsigned)((long long)T * S), FWD_LDS_NW * 64, lds, st>>>(gd, x, x_rows, in_crow, in_col, n_s, ginb,
                                                                               gb_ld, ginw, gw_ld, T, S);
    return hipGetLastError();
}

hipError_t launch_touch(const TouchJob& j, hipStream_t st) {
    long long most = 0;
    for (int k = 0; k < TOUCH_JOBS; ++k) {
        if (j.n[k] > 0 && !j.p[k]) return hipErrorInvalidValue;
        most = std::max(most, j.n[k]);
    }
    if (most == 0) return hipSuccess;
    const long long per_xcd = std::min<long long>((most + WG - 1) / WG, 32);      // blocks per XCD
    k_touch<<<(unsigned)(8 * per_xcd), WG, 0, st>>>(j);
    return hipGetLastError();
}

template <bool TILED, int MODE, int PB>
static void launch_bwd_kernel(const Plan& p, const int2* cw, const float* gz, Lay lg, int gz_rows, const float* hsrc,
                              Lay lhs, float* gwpart, long long gw_ld, const BwdEpi& epi, float* part, Lay lp, int T,
                              bool pair, hipStream_t st) {
    const int RB = (p.nwave + WG / 64 - 1) / (WG / 64);
    if constexpr (TILED && MODE != 0) {
        if (pair) {                             // two tiles per workgroup
            k_bwd2<MODE, PB><<<(unsigned)((long long)((T + 1) / 2) * RB), WG, 0, st>>>(p, cw, gz, lg, gz_rows, hsrc, lhs,
                                                                                     gwpart, gw_ld, epi, part, lp, T, RB);
            return;
        }
    }
    k_bwd<TILED, MODE, PB><<<(unsigned)((long long)T * RB), WG, 0, st>>>(p, cw, gz, lg, gz_rows, hsrc, lhs, gwpart, gw_ld,
                                                                         epi, part, lp, T, RB);
}

template <bool TILED, int MODE>
static hipError_t launch_bwd_as(const Plan& p, const int2* cw, const float* gz, Lay lg, int gz_rows, const float* hsrc,
                                Lay lhs, float* gwpart, long long gw_ld, const BwdEpi& epi, float* part, Lay lp, int T,
                                bool pair, hipStream_t st) {
    // (6-byte pairs: a tiled slab of at most PAIR6_MAX_ROWS rows, as launch_fwd)
    if ((p.pb != 8 && p.pb != 6) || (p.pb == 6 && (!TILED || gz_rows > PAIR6_MAX_ROWS))) return hipErrorInvalidValue;
    if (p.nwave > 0) {
        if constexpr (TILED) {
            if (p.pb == 6)
                launch_bwd_kernel<true, MODE, 6>(p, cw, gz, lg, gz_rows, hsrc, lhs, gwpart, gw_ld, epi, part, lp, T, pair, st);
            else
                launch_bwd_kernel<true, MODE, 8>(p, cw, gz, lg, gz_rows, hsrc, lhs, gwpart, gw_ld, epi, part, lp, T, pair, st);
        } else {
            launch_bwd_kernel<false, MODE, 8>(p, cw, gz, lg, gz_rows, hsrc, lhs, gwpart, gw_ld, epi, part, lp, T, pair, st);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (p.nsplit > 0) {
        if constexpr (TILED && MODE != 0) {
            if (pair) {
                k_bwd_combine<MODE, true><<<blocks((long long)p.nsplit * ((T + 1) / 2) * LPR), WG, 0, st>>>(p, part, lp,
                                                                                                            epi, T);
                return hipGetLastError();
            }
        }
        k_bwd_combine<MODE, false><<<blocks((long long)p.nsplit * T * LPR), WG, 0, st>>>(p, part, lp, epi, T);
        return hipGetLastError();
    }
    return hipSuccess;
}

hipError_t launch_bwd(const Plan& p, const int2* cw, const float* gz, Lay lg, int gz_rows, const float* hsrc, Lay lhs,
                      float* gwpart, long long gw_ld, const BwdEpi& epi, float* part, Lay lp, int T, hipStream_t st,
                      bool pair) {
    const bool tiled_ = lg.row == TW;
    switch (epi.mode) {
        case 0:
            return tiled_ ? launch_bwd_as<true, 0>(p, cw, gz, lg, gz_rows, hsrc, lhs, gwpart, gw_ld, epi, part, lp, T,
                                                   false, st)
                          : launch_bwd_as<false, 0>(p, cw, gz, lg, gz_rows, hsrc, lhs, gwpart, gw_ld, epi, part, lp, T,
                                                    false, st);
        case 1:
            if (!tiled_) return hipErrorInvalidValue;
            return launch_bwd_as<true, 1>(p, cw, gz, lg, gz_rows, hsrc, lhs, gwpart, gw_ld, epi, part, lp, T, pair, st);
        case 2:
            if (!tiled_) return hipErrorInvalidValue;
            return launch_bwd_as<true, 2>(p, cw, gz, lg, gz_rows, hsrc, lhs, gwpart, gw_ld, epi, part, lp, T, pair, st);
        default:
            return hipErrorInvalidValue;
    }
}

int bwd_lds_rows() {
    int dev = 0, cap = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cap, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return 0;
    size_t stat = 0;
    for (const void* k : {reinterpret_cast<const void*>(&k_bwd_lds<8, false>), reinterpret_cast<const void*>(&k_bwd_lds<6, false>),
                          reinterpret_cast<const void*>(&k_bwd_lds<8, true>), reinterpret_cast<const void*>(&k_bwd_lds<6, true>)}) {
        hipFuncAttributes a{};
        if (hipFuncGetAttributes(&a, k) != hipSuccess) return 0;
        stat = std::max(stat, a.sharedSizeBytes);
    }
    if ((size_t)cap <= stat) return 0;
    const size_t rows = ((size_t)cap - stat) / (TW * 4);
    return rows < 2 ? 0 : (int)std::min<size_t>(rows - 1, BWD_LDS_MAXROWS);      // (less the row of zeros)
}

hipError_t launch_bwd_lds(const Plan& p, const int2* wlds, const int2* cw, const float* gz, int gz_rows,
                          const int* hot_rows, int hot, const float* hsrc, Lay lhs, float* gwpart, long long gw_ld,
                          const BwdEpi& epi, float* part, Lay lp, int T, int S, hipStream_t st) {
    // (codes name rows below hot + gz_rows: with 6-byte pairs that must stay below 0xFFFF, which names no row)
    if (epi.mode != 1 || !epi.sinfo || !epi.h || !epi.gz_out || !epi.gdrive || !epi.ggain_part || !epi.gsum_part ||
        !wlds || !hot_rows || hot < 1 || hot > BWD_LDS_MAXROWS || hot > gz_rows || S < 1 || lhs.row != TW ||
        lp.row != TW || epi.lgz.row != TW || epi.lgd.row != TW || (p.pb != 8 && p.pb != 6) ||
        (p.pb == 6 && (long long)hot + gz_rows > PAIR6_MAX_ROWS))
        return hipErrorInvalidValue;
    if (p.nwave > 0) {
        S = std::max(S, (p.nwave + 64 * BWD_LDS_WREC * BWD_LDS_NW - 1) / (64 * BWD_LDS_WREC * BWD_LDS_NW));
        const void* k = p.pb == 6 ? (epi.skip_silent ? reinterpret_cast<const void*>(&k_bwd_lds<6, true>)
                                                     : reinterpret_cast<const void*>(&k_bwd_lds<6, false>))
                                  : (epi.skip_silent ? reinterpret_cast<const void*>(&k_bwd_lds<8, true>)
                                                     : reinterpret_cast<const void*>(&k_bwd_lds<8, false>));
        const size_t lds = (size_t)(hot + 1) * TW * 4;        // (and a row of zeros)
        const hipError_t attr = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (attr != hipSuccess) return attr;
        const dim3 grid((unsigned)((long long)T * S));
#define FG_BWD_LDS(P, K) k_bwd_lds<P, K><<<grid, BWD_LDS_NW * 64, lds, st>>>(p, wlds, cw, gz, gz_rows, hot_rows, hot, \
                                                                               hsrc, lhs, gwpart, gw_ld, epi, part, lp, T, S)
        if (p.pb == 6) {
            if (epi.skip_silent) FG_BWD_LDS(6, true); else FG_BWD_LDS(6, false);
        } else {
            if (epi.skip_silent) FG_BWD_LDS(8, true); else FG_BWD_LDS(8, false);
        }
#undef FG_BWD_LDS
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (p.nsplit > 0) {
        k_bwd_combine<1, false><<<blocks((long long)p.nsplit * T * LPR), WG, 0, st>>>(p, part, lp, epi, T);
        return hipGetLastError();
    }
    return hipSuccess;
}

hipError_t launch_fires_pack(const unsigned char* bytes, int rows, unsigned* bits, int T, hipStream_t st) {
    if (rows <= 0 || T <= 0) return hipSuccess;
    k_fires_pack<<<(unsigned)T, WG, 0, st>>>(bytes, rows, bits, fires_ld(rows));
    return hipGetLastError();
}

hipError_t launch_obs_in(const float* obs, float* x, int obs_dim, int B, hipStream_t st) {
    dim3 grid((unsigned)((obs_dim + 63) / 64), (unsigned)(B / TW));
    k_obs_in<<<grid, WG, 0, st>>>(obs, x, obs_dim);
    return hipGetLastError();
}

hipError_t launch_readout_bwd_h_mfma(const float* dl, const float* owT, const int* dn_inv, int n_act, int rows,
                                     const BwdEpi& epi, int B, hipStream_t st) {
    if (readout_pad(n_act) > 8 * GH_STEPS) return hipErrorInvalidValue;
    dim3 grid((unsigned)((rows + RPG - 1) / RPG), (unsigned)(B / TW));
    k_readout_bwd_h_mfma<<<grid, WG, 0, st>>>(dl, owT, readout_pad(n_act), dn_inv, n_act, rows, epi);
    return hipGetLastError();
}

hipError_t launch_reduce_n(const RedJob* jobs, int n, hipStream_t st) {
    JobTable<RedJob, RED_JOBS> t;
    long long nb;
    if (!fill_table(t, jobs, n, [](const RedJob& j) { return j.n; }, nb)) return hipErrorInvalidValue;
    for (int k = 0; k < t.n; ++k)
        if (!t.j[k].part || !t.j[k].G || t.j[k].nt < 0 || t.j[k].ld < t.j[k].n) return hipErrorInvalidValue;
    if (nb == 0) return hipSuccess;
    k_reduce<<<(unsigned)nb, WG, 0, st>>>(t);
    return hipGetLastError();
}

hipError_t launch_reduce(const float* part, long long ld, long long n, int nt, const int* idx, const float* theta,
                         float* G, hipStream_t st) {
    const RedJob j{part, ld, n, nt, idx, theta, G};
    return launch_reduce_n(&j, 1, st);
}

hipError_t launch_loss(const float* lg, const float* tl, float* dl, float* stats_part, float* stats, int n_act, int B,
                       float it, hipStream_t st, bool accumulate) {
    if (n_act > 128) return hipErrorInvalidValue;       // the staged logits must fit the LDS
    const unsigned nb = blocks(B, LOSS_S);
    k_loss<<<nb, 256, (size_t)2 * LOSS_S * n_act * sizeof(float), st>>>(lg, tl, dl, stats_part, n_act, B, it);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_sum_pairs<<<1, 64, 0, st>>>(stats_part, (int)nb, stats, accumulate ? 1 : 0);
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

hipError_t launch_rowinfo_n(const RowJob* jobs, int n, const float* gain, const float* theta, hipStream_t st) {
    JobTable<RowJob, ROW_JOBS> t;
    long long nb;
    if (!fill_table(t, jobs, n, [](const RowJob& j) { return (long long)j.rows; }, nb)) return hipErrorInvalidValue;
    for (int k = 0; k < t.n; ++k)
        if (!t.j[k].nid || !t.j[k].info) return hipErrorInvalidValue;
    if (nb == 0) return hipSuccess;
    k_rowinfo<<<(unsigned)nb, WG, 0, st>>>(t, gain, theta);
    return hipGetLastError();
}

hipError_t launch_export(const float* src, Lay ls, float* dst, int rows, int B, hipStream_t st) {
    k_export<<<blocks((long long)rows * B), WG, 0, st>>>(src, ls, dst, rows, B);
    return hipGetLastError();
}

}  // namespace fg
