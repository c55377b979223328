// The read-out on the matrix cores: logits[b][a] = ob[a] + sum_j ow[a][j] * hK[dn[j]][b] (flyguy_train.cu:95-101) as
// float32 MFMA products (v_mfma_f32_32x32x2_f32: a 32 x 32 block of the output, two read-out rows per instruction).
// A workgroup owns 32 samples and every action; its 8 waves each take an eighth of the 1,332 read-out rows, and their
// partial blocks are added through LDS in wave order, then the bias: the sums do not depend on scheduling.  The
// weights are read from a transposed copy owT[j][a] (actions padded to a multiple of 32 with zeros) so that a
// half-wave's operand is one 128-byte line; the read-out rows are gathered from the tiled states (float32 tiles of 32
// samples, or bfloat16 tiles of 64).
#include "readout.h"

namespace fg {

// owT[j][a] = ow[a][j] for a < n_act, 0 up to ma (a multiple of 32)
__global__ void k_owT(const float* __restrict__ ow, int n_act, int n_dn, int ma, float* __restrict__ owT) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)n_dn * ma) return;
    const int j = (int)(i / ma), a = (int)(i % ma);
    owT[i] = a < n_act ? ow[(size_t)a * n_dn + j] : 0.f;
}

template <bool BF16S>
__device__ __forceinline__ float state_at(const void* hK, size_t i) {
    if (BF16S) return __uint_as_float((unsigned)reinterpret_cast<const unsigned short*>(hK)[i] << 16);
    return reinterpret_cast<const float*>(hK)[i];
}

// grid (B / 32, RO_SPLIT), 512 threads (8 waves).  hK: the top layer's states, tiles of tw samples ([T][rows][tw]).
// Workgroup (b, s) takes the s-th of RO_SPLIT equal (even) ranges of the read-out rows for samples 32 b ..; wave w
// sums the w-th eighth of that range for every action block (a gathered state value feeds the ma / 32 blocks), so a
// wave walks about 21 rows: its chain of dependent loads stays short.  The split is fixed, so a sample's sums do not
// depend on the batch.  lpart[s][B][n_act]: the workgroup's sum (no bias), added up by k_logits_sum.
constexpr int RO_WAVES = 8;
constexpr int RO_MAXB = 4;                   // action blocks of 32 a workgroup holds (n_act <= 128)
template <bool BF16S>
__global__ __launch_bounds__(64 * RO_WAVES) void k_logits_mfma(const void* __restrict__ hK, int rows, int tw,
                                                             const int* __restrict__ dn, int n_dn,
                                                             const float* __restrict__ owT, int ma, int n_act,
                                                             float* __restrict__ lpart) {
    extern __shared__ int sm_dn[];                          // dn, then the partial blocks [RO_WAVES][32][33]
    float* part = reinterpret_cast<float*>(sm_dn + ((n_dn + 3) & ~3));
    const int sb = blockIdx.x, sp = blockIdx.y, B = gridDim.x * 32;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int tile = sb * 32 / tw, col = sb * 32 % tw + (lane & 31);
    const int i = lane & 31, kk = lane >> 5;
    const int nb = ma / 32;
    for (int j = threadIdx.x; j < n_dn; j += 64 * RO_WAVES) sm_dn[j] = dn[j];
    __syncthreads();
    const int ps = ((n_dn + RO_SPLIT - 1) / RO_SPLIT + 1) & ~1;     // read-out rows per workgroup (even)
    const int s0 = min(n_dn, sp * ps), s1 = min(n_dn, s0 + ps);
    const int per = ((s1 - s0 + RO_WAVES - 1) / RO_WAVES + 1) & ~1; // ... per wave (even)
    const int j0 = min(s1, s0 + wave * per), j1 = min(s1, j0 + per);
    const size_t base = (size_t)tile * rows * tw + col;
    f32x16 acc[RO_MAXB];
#pragma unroll
    for (int m = 0; m < RO_MAXB; ++m)
        acc[m] = f32x16{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = j0; j < j1; j += 8) {
        float bv[4], av[4][RO_MAXB];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int jj = j + 2 * u + kk;
            const bool ok = jj < j1;
            bv[u] = ok ? state_at<BF16S>(hK, base + (size_t)sm_dn[jj] * tw) : 0.f;
#pragma unroll
            for (int m = 0; m < RO_MAXB; ++m) av[u][m] = (ok && m < nb) ? owT[(size_t)jj * ma + m * 32 + i] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int m = 0; m < RO_MAXB; ++m)
                if (m < nb) acc[m] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u][m], bv[u], acc[m], 0, 0, 0);
    }
    // per action block: the waves' partial blocks through LDS (lane l, register r holds action 8 (r / 4) + 4 (l / 32)
    // + r % 4 of the block, sample l % 32), added in wave order
    float* out = lpart + (size_t)sp * B * n_act;
#pragma unroll
    for (int m = 0; m < RO_MAXB; ++m) {
        if (m >= nb) break;
        float* pw = part + (size_t)wave * 32 * 33;
#pragma unroll
        for (int r = 0; r < 16; ++r) pw[(8 * (r >> 2) + 4 * kk + (r & 3)) * 33 + i] = acc[m][r];
        __syncthreads();
        for (int e = threadIdx.x; e < 32 * 32; e += 64 * RO_WAVES) {
            const int ai = e & 31, c = e >> 5, a = m * 32 + ai;
            if (a < n_act) {
                float v = part[ai * 33 + c];
                for (int w = 1; w < RO_WAVES; ++w) v += part[(size_t)w * 32 * 33 + ai * 33 + c];
                out[(size_t)(sb * 32 + c) * n_act + a] = v;
            }
        }
        __syncthreads();
    }
}

// logits[b][a] = ob[a] + the RO_SPLIT partial sums of k_logits_mfma, added in split order
__global__ __launch_bounds__(WG) void k_logits_sum(const float* __restrict__ lpart, const float* __restrict__ ob,
                                                   int n_act, long long n, float* __restrict__ logits) {
    const long long i = (long long)blockIdx.x * WG + threadIdx.x;
    if (i >= n) return;
    float v = lpart[i];
#pragma unroll
    for (int s = 1; s < RO_SPLIT; ++s) v += lpart[(size_t)s * n + i];
    logits[i] = ob[i % n_act] + v;
}

// The read-out weights' gradient per chunk of RO_CHUNK_S samples (flyguy_train.cu:125-135):
//   gow_part[chunk][a][j] = sum_b dl[b][a] hK[dn[j]][b],  gob_part[chunk][a] = sum_b dl[b][a]  (b in the chunk)
// Grid (n_dn / 32 blocks of read-out rows, chunks), 256 threads: the 4 waves each take a quarter of the chunk's
// samples for every block of 32 actions (M = actions, N = read-out rows, K = samples); partials added through LDS in
// wave order.  Short chunks keep each wave's chain of dependent loads short (4 steps of 8 samples).
template <bool BF16S>
__global__ __launch_bounds__(WG) void k_readout_bwd_w_mfma(const float* __restrict__ dl, const void* __restrict__ hK,
                                                           int rows, int tw, const int* __restrict__ dn, int n_dn,
                                                           int n_act, int B, float* __restrict__ gow_part,
                                                           float* __restrict__ gob_part) {
    __shared__ float part[4 * 32 * 33];
    const int j0 = blockIdx.x * 32, chunk = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane & 31, kk = lane >> 5;
    const int nb = (n_act + 31) / 32;
    const int row = j0 + i < n_dn ? dn[j0 + i] : -1;
    const int bs = min(B, chunk * RO_CHUNK_S + wave * (RO_CHUNK_S / 4)), be = min(B, bs + RO_CHUNK_S / 4);
    f32x16 acc[RO_MAXB];
#pragma unroll
    for (int m = 0; m < RO_MAXB; ++m)
        acc[m] = f32x16{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int b = bs; b < be; b += 8) {
        float bv[4], av[4][RO_MAXB];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int sm = b + 2 * u + kk;
            const bool ok = sm < be;
            bv[u] = (ok && row >= 0) ? state_at<BF16S>(hK, ((size_t)(sm / tw) * rows + row) * tw + sm % tw) : 0.f;
#pragma unroll
            for (int m = 0; m < RO_MAXB; ++m)
                av[u][m] = (ok && m < nb && m * 32 + i < n_act) ? dl[(size_t)sm * n_act + m * 32 + i] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int m = 0; m < RO_MAXB; ++m)
                if (m < nb) acc[m] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u][m], bv[u], acc[m], 0, 0, 0);
    }
    const size_t base = (size_t)chunk * n_act * n_dn;
#pragma unroll
    for (int m = 0; m < RO_MAXB; ++m) {
        if (m >= nb) break;
        float* pw = part + (size_t)wave * 32 * 33;
#pragma unroll
        for (int r = 0; r < 16; ++r) pw[mfma_row(r, lane) * 33 + i] = acc[m][r];
        __syncthreads();
        for (int e = threadIdx.x; e < 32 * 32; e += WG) {
            const int ai = e >> 5, jc = e & 31, a = m * 32 + ai;
            if (a < n_act && j0 + jc < n_dn)
                gow_part[base + (size_t)a * n_dn + j0 + jc] =
                    ((part[ai * 33 + jc] + part[32 * 33 + ai * 33 + jc]) + part[2 * 32 * 33 + ai * 33 + jc]) +
                    part[3 * 32 * 33 + ai * 33 + jc];
        }
        __syncthreads();
    }
    if (blockIdx.x == 0 && (int)threadIdx.x < n_act) {
        float sb = 0.f;
        for (int b = min(B, chunk * RO_CHUNK_S); b < min(B, (chunk + 1) * RO_CHUNK_S); ++b)
            sb += dl[(size_t)b * n_act + threadIdx.x];
        gob_part[(size_t)chunk * n_act + threadIdx.x] = sb;
    }
}

int readout_pad(int n_act) { return (n_act + 31) / 32 * 32; }

hipError_t launch_owT(const float* ow, int n_act, int n_dn, float* owT, hipStream_t st) {
    const int ma = readout_pad(n_act);
    const long long n = (long long)n_dn * ma;
    k_owT<<<(unsigned)((n + WG - 1) / WG), WG, 0, st>>>(ow, n_act, n_dn, ma, owT);
    return hipGetLastError();
}

hipError_t launch_readout_bwd_w_mfma(const float* dl, const void* hK, bool bf16_states, int rows, const int* dn,
                                     int n_dn, int n_act, float* gow_part, float* gob_part, int B, hipStream_t st) {
    if (readout_pad(n_act) > 32 * RO_MAXB || n_act > WG) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((n_dn + 31) / 32), (unsigned)readout_chunks(B));
    if (bf16_states)
        k_readout_bwd_w_mfma<true><<<grid, WG, 0, st>>>(dl, hK, rows, TW16, dn, n_dn, n_act, B, gow_part, gob_part);
    else
        k_readout_bwd_w_mfma<false><<<grid, WG, 0, st>>>(dl, hK, rows, TW, dn, n_dn, n_act, B, gow_part, gob_part);
    return hipGetLastError();
}

hipError_t launch_logits_mfma(const void* hK, bool bf16_states, int rows, const int* dn, int n_dn, const float* ow,
                              const float* ob, int n_act, float* owT, float* lpart, float* logits, int B,
                              hipStream_t st, bool owT_current) {
    const int ma = readout_pad(n_act);
    if (ma > 32 * RO_MAXB || B % 32 != 0) return hipErrorInvalidValue;
    const size_t sm = (size_t)((n_dn + 3) & ~3) * sizeof(int) + (size_t)RO_WAVES * 32 * 33 * sizeof(float);
    if (sm > 64 * 1024) return hipErrorInvalidValue;
    const long long n = (long long)n_dn * ma;
    if (!owT_current) k_owT<<<(unsigned)((n + WG - 1) / WG), WG, 0, st>>>(ow, n_act, n_dn, ma, owT);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || B == 0) return e;
    const dim3 grid((unsigned)(B / 32), RO_SPLIT);
    const unsigned threads = 64 * RO_WAVES;
    if (bf16_states)
        k_logits_mfma<true><<<grid, threads, sm, st>>>(hK, rows, TW16, dn, n_dn, owT, ma, n_act, lpart);
    else
        k_logits_mfma<false><<<grid, threads, sm, st>>>(hK, rows, TW, dn, n_dn, owT, ma, n_act, lpart);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const long long nl = (long long)B * n_act;
    k_logits_sum<<<(unsigned)((nl + WG - 1) / WG), WG, 0, st>>>(lpart, ob, n_act, nl, logits);
    return hipGetLastError();
}

}  // namespace fg
