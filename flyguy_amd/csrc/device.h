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
