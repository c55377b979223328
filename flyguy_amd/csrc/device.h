// Device helpers shared by the kernels of the flyguy MI355X library: state addressing, the row plan, the hand-round
// of (source, weight) pairs through LDS, the slab gathers and the lane-group reductions.
#pragma once
#include "kernels.h"

namespace fg {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));     // 8 16-bit states of a lane

__device__ __forceinline__ const float4* at4(const float* base, Lay L, int tile, int row, int sub) {
    return reinterpret_cast<const float4*>(base + (size_t)tile * L.tile + (size_t)row * L.row) + sub;
}
__device__ __forceinline__ float4* at4w(float* base, Lay L, int tile, int row, int sub) {
    return reinterpret_cast<float4*>(base + (size_t)tile * L.tile + (size_t)row * L.row) + sub;
}
__device__ __forceinline__ float4 splat(float v) { return make_float4(v, v, v, v); }
// The same element of a tiled state ([T][rows][32]) as a wave-uniform tile base plus a 32-bit element offset (cheaper
// addressing than at4's 64-bit products; a tiled slab is far below 2^32 elements)
__device__ __forceinline__ const float4* at4u(const float* base, Lay L, int tile, int row, int sub) {
    return reinterpret_cast<const float4*>(base + (size_t)tile * L.tile + (unsigned)(row * L.row + sub * 4));
}
__device__ __forceinline__ float4* at4uw(float* base, Lay L, int tile, int row, int sub) {
    return reinterpret_cast<float4*>(base + (size_t)tile * L.tile + (unsigned)(row * L.row + sub * 4));
}

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

// wave w of the plan ({woff, longest segment}); false when w is past the end or names positions outside the plan
__device__ __forceinline__ bool load_wave(const Plan& p, int w, int2& wv) {
    wv = make_int2(0, 0);
    if (w >= p.nwave) return false;
    const int2 v = p.wave[w];
    if (v.x < 0 || v.y < 0 || (long long)v.x + 64 * (((long long)v.y + 7) / 8) > p.npos) return false;
    wv = v;
    return true;
}
// segment si ({row, slot, re-drive row, 0}); false when si is past the end or names a row or slot outside the plan
__device__ __forceinline__ bool load_segment(const Plan& p, int si, int4& sg) {
    sg = make_int4(0, -1, -1, 0);
    if (si >= p.nseg) return false;
    const int4 v = p.seg[si];
    if (v.x < 0 || v.x >= p.rows || v.y >= p.nslot) return false;
    sg = v;
    return true;
}
__device__ __forceinline__ bool load_split(const Plan& p, long long i, int4& s) {
    if (i >= p.nsplit) return false;
    s = p.split[i];
    return s.x >= 0 && s.x < p.rows && s.y >= 0 && s.z >= 0 && (long long)s.y + s.z <= p.nslot;
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

// Whether the 8-lane group's line of a state is zero on all of its samples (every lane of the wave must call this).  A
// neuron's output is relu(...) >= 0, so a line of h with no sample > 0 is a neuron that fires on none of the tile's
// samples: its gradient g = (h > 0 ? gh : 0) is zero there whatever gh is.
// (lane_fires: whether the lane's own samples hold a value > 0)
__device__ __forceinline__ bool group_silent(bool lane_fires) {
    const unsigned long long fires = __ballot(lane_fires);
    return ((fires >> (threadIdx.x & 56)) & 0xFFull) == 0;
}
__device__ __forceinline__ bool group_silent(const float4& h) {
    return group_silent(h.x > 0.f || h.y > 0.f || h.z > 0.f || h.w > 0.f);
}
// The 8 stored bfloat16 values of a lane: whether one may be > 0 (any with a nonzero magnitude; a negative value,
// which a neuron's output never is, counts as firing too, which only turns a skip off)
__device__ __forceinline__ bool bf16_lane_fires(const u32x4& h) {
    return ((h[0] | h[1] | h[2] | h[3]) & 0x7FFF7FFFu) != 0u;
}
// Stage the firing bitmap of a tile (k_fires_pack) in LDS when the tile has silent rows; every thread of the
// workgroup calls this.  Returns whether it did (then the hop skips the silent rows' gathers).
__device__ __forceinline__ bool stage_fires(const unsigned* src_fires, int fw_ld, int tile, unsigned* lds) {
    if (fw_ld <= 0) return false;
    const unsigned* b = src_fires + (size_t)tile * fw_ld;
    if (__builtin_amdgcn_readfirstlane(b[0]) == 0) return false;     // (uniform: one word for the whole workgroup)
    const uint4* b4 = reinterpret_cast<const uint4*>(b + 4);
    for (int i = threadIdx.x; i < (fw_ld - 4) / 4; i += WG) reinterpret_cast<uint4*>(lds)[i] = b4[i];
    __syncthreads();
    return true;
}
// A pair whose source row is silent on the tile (its bit clear, or outside the source layer) gathers NO_ROW instead
__device__ __forceinline__ void drop_silent(int2& pair, const unsigned* lds, int src_rows) {
    const unsigned r = (unsigned)pair.x;
    if (r >= (unsigned)src_rows || !((lds[r >> 5] >> (r & 31)) & 1u)) pair.x = NO_ROW;
}

// The 8 bytes a lane loads of each step's pairs (Plan::pb).  PB 8: the pair of its own slot (position woff + 64 j +
// lane).  PB 6: bytes 8 lane .. 8 lane + 7 of the step's 384-byte block (lanes 0-31 two weights each, lanes 32-47
// four sources each; lanes 48-63 load nothing).  woff is a multiple of 64, so a block starts on a 128-byte boundary.
template <int PB>
struct PairLoad {
    const int2* q;
    bool on;
    __device__ __forceinline__ PairLoad(const int2* cw, int woff, int lane) {
        if constexpr (PB == 8) {
            q = cw + woff + lane;
            on = true;
        } else {
            q = cw + (size_t)woff / 64 * 48 + lane;
            on = lane < 48;
        }
    }
    __device__ __forceinline__ int2 step(int j) const {
        if constexpr (PB == 8) return q[64 * j];
        return on ? q[48 * j] : make_int2(0, 0);
    }
};

// A step's pairs from the lanes' loads to each 8-lane group: c[s], w[s] = source and weight of the group's slot s.
// slots: the workgroup's staging, 64 int2 per wave (slots[grp] is group grp's 8).  bits: fires holds the source
// layer's firing bits of the tile (in LDS); then a silent source (or one outside src_rows) becomes NO_ROW (PB 6; with
// 8-byte pairs the caller drops it from the lane's own pair before, drop_silent).
// PB 8 hands the pairs round within each group (stage8).  PB 6 writes the lanes' 8-byte pieces of the block to the
// wave's 512 bytes of staging, and each group reads its 8 weights (two 16-byte reads) and 8 sources (one); an unused
// slot's source reads 0xFFFF, which lies past every slab of at most PAIR6_MAX_ROWS rows.  Silent sources are found
// after the staging there: lane s of a group tests the group's slot s and a ballot shares the 8 answers.
template <int PB>
__device__ __forceinline__ void stage_pairs(int2 (*slots)[LPR], int grp, int sub, int2 my, bool bits,
                                            const unsigned* fires, int src_rows, int (&c)[8], float (&w)[8]) {
    if constexpr (PB == 8) {
        stage8(slots[grp], sub, my, c, w);
    } else {
        int2* wb = slots[grp & ~7];
        const int g = grp & 7, lane = (g << 3) | sub;
        wb[lane] = my;
        __builtin_amdgcn_wave_barrier();
        const int4* q = reinterpret_cast<const int4*>(wb);
        const int4 a = q[2 * g], b = q[2 * g + 1], s = q[16 + g];
        w[0] = __int_as_float(a.x); w[1] = __int_as_float(a.y); w[2] = __int_as_float(a.z); w[3] = __int_as_float(a.w);
        w[4] = __int_as_float(b.x); w[5] = __int_as_float(b.y); w[6] = __int_as_float(b.z); w[7] = __int_as_float(b.w);
        c[0] = s.x & 0xFFFF; c[1] = (int)((unsigned)s.x >> 16);
        c[2] = s.y & 0xFFFF; c[3] = (int)((unsigned)s.y >> 16);
        c[4] = s.z & 0xFFFF; c[5] = (int)((unsigned)s.z >> 16);
        c[6] = s.w & 0xFFFF; c[7] = (int)((unsigned)s.w >> 16);
        if (bits) {
            const unsigned r = reinterpret_cast<const unsigned short*>(wb)[128 + lane];     // the lane's own slot
            const bool alive = r < (unsigned)src_rows && ((fires[r >> 5] >> (r & 31)) & 1u);
            const unsigned gm = (unsigned)(__ballot(alive) >> (lane & 56)) & 0xFFu;
#pragma unroll
            for (int k = 0; k < 8; ++k)
                if (!((gm >> k) & 1u)) c[k] = NO_ROW;
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// Reduce-scatter over the 8 lanes of a group: lane s ends with the sum over the group's lanes of d[s].  Three
// butterfly steps, each pairing lanes that hold the same set of slots and keeping the half named by a lane bit:
// lanes i and 7-i (row_half_mirror) split the slots by bit 2, then i and i^2, then i and i^1 (quad perms).
__device__ __forceinline__ float rs8(const float (&d)[8], int sub) {
    const bool b2 = sub & 4, b1 = sub & 2, b0 = sub & 1;
    float a[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) a[t] = (b2 ? d[4 + t] : d[t]) + dppf<0x141>(b2 ? d[t] : d[4 + t]);
    float b[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) b[u] = (b1 ? a[2 + u] : a[u]) + dppf<0x4E>(b1 ? a[u] : a[2 + u]);
    return (b0 ? b[1] : b[0]) + dppf<0xB1>(b0 ? b[0] : b[1]);
}

}  // namespace fg
