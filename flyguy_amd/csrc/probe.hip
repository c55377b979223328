// The gather ceiling: the rate at which the device's vector-memory path gathers 128-byte lines of a tile's slab,
// measured the way the hop kernels gather (an 8-lane group loads one line, 16 bytes a lane, so a wave instruction
// reads 8 lines; each step's 8 row indices are read by the group's lanes, one each, from a stream in the lanes' order,
// and shared within the group).
// The hop kernels are bound by this path rather than by HBM bandwidth: a wave instruction costs about the same number
// of CU cycles whatever its width, so the rate is lines per instruction times instructions per cycle, and a slab
// larger than an XCD's L2 lowers it through misses.  bench.py reports each dominant hop kernel's time against this
// ceiling, with the rows drawn as that kernel's connections draw them.
#include "../../include/flyguy_core.h"
#include "kernels.h"

namespace fg {

__device__ __forceinline__ unsigned mix32(unsigned x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

constexpr int CEIL_STEPS = 16;     // steps per group and launch, 8 rows each

// The rows a launch gathers, in the order its lanes read them: entry i is the row of a connection drawn at random (a
// hash of i), row_of[e], or a row drawn uniformly when row_of is null (untimed set-up)
__global__ __launch_bounds__(WG) void k_ceiling_rows(const int* __restrict__ row_of, unsigned n_edges, unsigned rows,
                                                     int* __restrict__ seq, unsigned n) {
    const unsigned i = blockIdx.x * WG + threadIdx.x;
    if (i >= n) return;
    const unsigned h = mix32(i * 2654435761u + 12345u);
    seq[i] = row_of ? row_of[h % n_edges] : (int)(h % rows);
}

// Every 8-lane group takes CEIL_STEPS steps of 8 rows: each lane reads one entry of seq (a wave's 64 lanes read 64
// consecutive entries, as the hop kernels read a step's pairs), the 8 rows reach the group's lanes by swizzles, and
// the group gathers each row's line from each of the TILES slabs (rows x 128 bytes apiece, one after the other).
// The lines are summed so that the loads stay.
template <int TILES>
__global__ __launch_bounds__(WG) void k_gather_ceiling(const float* __restrict__ slab, unsigned rows,
                                                       const int* __restrict__ seq, float* __restrict__ out) {
    const unsigned grp = (blockIdx.x * WG + threadIdx.x) >> 3, sub = threadIdx.x & 7, groups = gridDim.x * (WG / LPR);
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void*)slab, (short)0, rows * TILES * (TW * 4u), 0x00020000);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = 0; j < CEIL_STEPS; ++j) {
        const int mine = seq[((size_t)j * groups + grp) * 8 + sub];
        int c[8];
        c[0] = bcast8<0>(mine); c[1] = bcast8<1>(mine); c[2] = bcast8<2>(mine); c[3] = bcast8<3>(mine);
        c[4] = bcast8<4>(mine); c[5] = bcast8<5>(mine); c[6] = bcast8<6>(mine); c[7] = bcast8<7>(mine);
        float4 v[8 * TILES];
#pragma unroll
        for (int t = 0; t < TILES; ++t)
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const unsigned off = ((unsigned)t * rows + (unsigned)c[s]) * (TW * 4u) + sub * 16u;
                const auto x = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
                v[t * 8 + s] = make_float4(__int_as_float(x[0]), __int_as_float(x[1]), __int_as_float(x[2]),
                                           __int_as_float(x[3]));
            }
#pragma unroll
        for (int s = 0; s < 8 * TILES; ++s) add4(v[s], acc);
    }
    reinterpret_cast<float4*>(out)[(size_t)blockIdx.x * WG + threadIdx.x] = acc;
}

}  // namespace fg

using namespace fg;

extern "C" int fc_gather_ceiling(int rows, int tiles, const int* row_of, long long n_edges, int reps, void* stream,
                                 double* ns_per_line) {
    clear_error();
    if (rows < 1 || (long long)rows * tiles > (1 << 24) || (tiles != 1 && tiles != 2) || reps < 1 || !ns_per_line ||
        (row_of && (n_edges < 1 || n_edges > 0x7fffffffLL))) {
        set_error("fc_gather_ceiling: rows 1 .. 2^24 in all, tiles 1 or 2, reps >= 1, ns_per_line given, and with "
                  "row_of 1 .. 2^31 - 1 connections");
        return -1;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    int dev = 0, cus = 0;
    FG_CHECK(hipGetDevice(&dev), -1);
    FG_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), -1);
    const long long blocks = 32LL * (cus > 0 ? cus : 1);          // several waves per SIMD on every CU
    const long long n_seq = blocks * (WG / LPR) * CEIL_STEPS * 8;  // the row entries one launch reads
    const size_t slab_bytes = (size_t)rows * tiles * TW * 4, out_bytes = (size_t)blocks * WG * 16;
    void *slab = nullptr, *out = nullptr, *seq = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    int rc = -1;
    float ms = 0.f;
    auto launch = [&]() {
        if (tiles == 2)
            k_gather_ceiling<2><<<(unsigned)blocks, WG, 0, st>>>((const float*)slab, (unsigned)rows, (const int*)seq,
                                                                 (float*)out);
        else
            k_gather_ceiling<1><<<(unsigned)blocks, WG, 0, st>>>((const float*)slab, (unsigned)rows, (const int*)seq,
                                                                 (float*)out);
    };
    do {
        if (hipMalloc(&slab, slab_bytes) != hipSuccess || hipMalloc(&out, out_bytes) != hipSuccess ||
            hipMalloc(&seq, (size_t)n_seq * sizeof(int)) != hipSuccess) {
            set_error("fc_gather_ceiling: out of device memory");
            break;
        }
        k_ceiling_rows<<<(unsigned)((n_seq + WG - 1) / WG), WG, 0, st>>>(row_of, (unsigned)(row_of ? n_edges : 1),
                                                                          (unsigned)rows, (int*)seq, (unsigned)n_seq);
        if (hipMemsetAsync(slab, 0x3f, slab_bytes, st) != hipSuccess || hipEventCreate(&a) != hipSuccess ||
            hipEventCreate(&b) != hipSuccess) {
            set_error("fc_gather_ceiling: set-up failed");
            break;
        }
        launch();                                   // (untimed)
        if (hipEventRecord(a, st) != hipSuccess) { set_error("fc_gather_ceiling: event"); break; }
        for (int i = 0; i < reps; ++i) launch();
        if (hipGetLastError() != hipSuccess || hipEventRecord(b, st) != hipSuccess ||
            hipEventSynchronize(b) != hipSuccess || hipEventElapsedTime(&ms, a, b) != hipSuccess) {
            set_error("fc_gather_ceiling: launch or timing failed");
            break;
        }
        const double lines = (double)blocks * (WG / LPR) * CEIL_STEPS * 8 * tiles * reps;
        *ns_per_line = (double)ms * 1e6 / lines;
        rc = 0;
    } while (false);
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (slab || out || seq) (void)hipStreamSynchronize(st);
    if (slab) (void)hipFree(slab);
    if (out) (void)hipFree(out);
    if (seq) (void)hipFree(seq);
    return rc;
}
