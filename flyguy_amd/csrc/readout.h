// The read-out's backward products on the matrix cores (float32 MFMA, v_mfma_f32_32x32x2_f32), shared by the
// float32 and bfloat16-state kernels.
#pragma once
#include "device.h"

namespace fg {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// A 32 x 32 output block of an MFMA (lane l, register r) holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
__device__ __forceinline__ int mfma_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

constexpr int GH_STEPS = 16;     // MFMA steps per wave of readout_gh_block at most: 4 waves x 16 x 2 = 128 actions
// gh of 32 rows (r0 ..) of the top layer for 32 samples (s0 ..): gh[t][c] = sum_a ow[a][j(t)] dl[s0 + c][a] with
// j(t) = dn_inv[t] (rows without a read-out column: 0), summed over the actions on the matrix cores, the 4 waves of
// the workgroup taking a quarter of the (padded) actions each; their partials are added in wave order into out[t][c].
// owT[j][a]: the read-out weights transposed (ma columns, zero past n_act).  Every thread of the (256-thread)
// workgroup calls it; part is LDS of 4 x 32 x 33 floats, out of 32 x ld floats.
__device__ __forceinline__ void readout_gh_block(const float* __restrict__ dl, const float* __restrict__ owT, int ma,
                                                 const int* __restrict__ dn_inv, int rows, int n_act, int r0, int s0,
                                                 float* part, float* out, int ld) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane & 31, kk = lane >> 5;
    const int t = r0 + i;
    const int j = t < rows ? dn_inv[t] : -1;
    const int steps = ma / 2, per = (steps + 3) / 4;                 // MFMA steps (2 actions each) per wave: <= 16
    const int k0 = wave * per, k1 = min(steps, k0 + per);
    float av[GH_STEPS], bv[GH_STEPS];
#pragma unroll
    for (int u = 0; u < GH_STEPS; ++u) {                              // every load first: their latencies overlap
        const int a = 2 * (k0 + u) + kk;
        const bool ok = k0 + u < k1 && a < n_act;
        av[u] = (ok && j >= 0) ? owT[(size_t)j * ma + a] : 0.f;
        bv[u] = ok ? dl[(size_t)(s0 + i) * n_act + a] : 0.f;
    }
    f32x16 acc = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < GH_STEPS; ++u)
        if (k0 + u < k1) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u], bv[u], acc, 0, 0, 0);
    float* pw = part + (size_t)wave * 32 * 33;
#pragma unroll
    for (int r = 0; r < 16; ++r) pw[mfma_row(r, lane) * 33 + i] = acc[r];
    __syncthreads();
    for (int e = threadIdx.x; e < 32 * 32; e += 256) {
        const int tr = e >> 5, c = e & 31;
        out[tr * ld + c] = ((part[tr * 33 + c] + part[32 * 33 + tr * 33 + c]) + part[2 * 32 * 33 + tr * 33 + c]) +
                           part[3 * 32 * 33 + tr * 33 + c];
    }
    __syncthreads();
}

}  // namespace fg
