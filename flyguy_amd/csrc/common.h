// Shared definitions of the flyguy MI355X library: error state, launch helpers, tile layout, lane helpers.
//
// Activation layout ("tiled"): a state tensor of N rows and B columns (B = batch, a multiple of 32) is stored
// as [T = B/32][N][32] fp32: one 128-byte line holds 32 samples of one row, and the N x 128 B "slab" of one
// tile is contiguous.  A workgroup works on one tile at a time, so the source slab it gathers from stays in
// the L2 of its XCD.  Kernels that serve the row-major [N][B] layout of the HopCuda-style boundary use the same
// code with different strides (row stride B, tile stride 32).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#include <string>

namespace fg {

constexpr int TW = 32;          // columns (samples) per tile
constexpr int TW16 = 64;        // samples per tile of 16-bit states (one 128-byte line)
constexpr int LPR = TW / 4;     // lanes per row: each lane holds a float4 of the tile
constexpr int RPW = 64 / LPR;   // rows per wave (8)
constexpr int WG = 256;         // threads per workgroup
constexpr int RPG = WG / LPR;   // rows per workgroup (32)
constexpr int SEG_MAX = 512;    // longest run of edges one lane group sums before a row is split into segments
constexpr int SEG_MIN_PER_TILE = 4096;   // segments a product should have per tile: >= 128 workgroups, so that the
                                         // workgroups resident on an XCD work on one or two tiles at a time (4096
                                         // measured 2-4% faster than 8192 and 2048 on the 3-hop benchmark network:
                                         // fewer split rows to combine, segments still short enough to balance)

// the segment cap of a product of E edges: SEG_MAX, lowered (not below 16) until there are SEG_MIN_PER_TILE segments
inline int seg_cap(long long E) {
    long long c = (E + SEG_MIN_PER_TILE - 1) / SEG_MIN_PER_TILE;
    return (int)(c < 16 ? 16 : (c > SEG_MAX ? SEG_MAX : c));
}

// Last error of this thread (set by a failing entry point, read by fc_last_error).
void set_error(const std::string& msg);
const char* last_error();
void clear_error();

// XCD-aware tile mapping: the hardware deals workgroups to the 8 XCDs round robin (block i -> XCD i % 8).
// With T % 8 == 0 each XCD works through its own tiles x, x+8, ... one after another, row blocks inner, so its
// L2 holds one tile's source slab at a time.  Otherwise tiles are walked in plain order.
__device__ __forceinline__ int tile_of(int bid, int RB, int T, int& rb) {
    if ((T & 7) == 0) {
        int x = bid & 7, s = bid >> 3;
        rb = s % RB;
        return x + 8 * (s / RB);
    }
    rb = bid % RB;
    return bid / RB;
}

// a compile-time flag as a type (the hop kernels' step bodies take it: Full<true> for a step whose 8 slots are all
// needed, Full<false> for a wave's last step)
template <bool B>
struct Full {
    static constexpr bool value = B;
};

// broadcast lane (group_base + S) of each 8-lane group (ds_swizzle bit mode inside each 32-lane half)
template <int S>
__device__ __forceinline__ int bcast8(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x18 | (S << 5)); }
template <int S>
__device__ __forceinline__ float bcast8f(float v) { return __int_as_float(bcast8<S>(__float_as_int(v))); }

// sum over the 8 lanes of a group (xor butterfly; every lane ends with the same value)
__device__ __forceinline__ float sum8(float v) {
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (1 << 10)));
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (2 << 10)));
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (4 << 10)));
    return v;
}

__device__ __forceinline__ float softplus_f(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }

__device__ __forceinline__ void fma4(float w, const float4& v, float4& a) {
    a.x = fmaf(w, v.x, a.x); a.y = fmaf(w, v.y, a.y); a.z = fmaf(w, v.z, a.z); a.w = fmaf(w, v.w, a.w);
}
__device__ __forceinline__ void add4(const float4& v, float4& a) { a.x += v.x; a.y += v.y; a.z += v.z; a.w += v.w; }

}  // namespace fg

#define FG_CHECK(call, ret)                                                                  \
    do {                                                                                     \
        hipError_t e_ = (call);                                                              \
        if (e_ != hipSuccess) {                                                              \
            char b_[256];                                                                    \
            snprintf(b_, sizeof b_, "HIP error %s at %s:%d", hipGetErrorString(e_), __FILE__, __LINE__); \
            fg::set_error(b_);                                                               \
            return ret;                                                                      \
        }                                                                                    \
    } while (0)
