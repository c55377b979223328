// 16-bit numbers in 128-byte lines: the binary16 / bfloat16 conversions and the gathers and stores of 8 samples per
// lane shared by the 16-bit kernels (half.hip: the HopCuda-style hop; core16.hip: the library core's bf16 states).
#pragma once
#include "device.h"

namespace fg {

struct F16 {};                            // IEEE binary16
struct BF16 {};                           // bfloat16
template <typename S> struct Bits16;
template <> struct Bits16<F16> {
    static __device__ __forceinline__ float lo(unsigned w) {
        return (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xffffu));
    }
    static __device__ __forceinline__ float hi(unsigned w) {
        return (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
    }
    static __device__ __forceinline__ unsigned from(float x) {   // round to nearest even
        return (unsigned)__builtin_bit_cast(unsigned short, (_Float16)x);
    }
};
template <> struct Bits16<BF16> {
    static __device__ __forceinline__ float lo(unsigned w) { return __uint_as_float(w << 16); }
    static __device__ __forceinline__ float hi(unsigned w) { return __uint_as_float(w & 0xffff0000u); }
    static __device__ __forceinline__ unsigned from(float x) {   // round to nearest even; a NaN stays a (quiet) NaN
        const unsigned u = __float_as_uint(x);
        if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
        return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    }
};

// the 8 samples of (row, lane) of a 16-bit tile slab: a 16-byte buffer load, zeros past the slab
__device__ __forceinline__ u32x4 gather16(__amdgpu_buffer_rsrc_t r, int row, int sub) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (unsigned)row * 128u + (unsigned)sub * 16u, 0, 0));
}
template <typename S>
__device__ __forceinline__ void unpack8(const u32x4& v, float (&f)[8]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        f[2 * k] = Bits16<S>::lo(v[k]);
        f[2 * k + 1] = Bits16<S>::hi(v[k]);
    }
}
__device__ __forceinline__ void store8(float* dst, const float (&a)[8]) {
    *reinterpret_cast<float4*>(dst) = make_float4(a[0], a[1], a[2], a[3]);
    *reinterpret_cast<float4*>(dst + 4) = make_float4(a[4], a[5], a[6], a[7]);
}

}  // namespace fg
