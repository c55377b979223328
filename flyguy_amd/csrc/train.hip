// The standalone teaching trainer over the library's core (flyguy/native/flyguy_train.cu:368-787), with the survey of
// firing neurons (:181-187, :436-478) and the revive surgery (:479-551).
//
// Data path: the chunks of the ring live in device memory as binary16, uploaded once when a chunk enters the ring
// (the reference keeps them in host memory and copies every batch over PCIe).  A step's batch is drawn on the host
// exactly as the reference draws it (std::mt19937_64 + std::uniform_int_distribution over the ring's samples), sent
// as B (chunk, sample) pairs through a pinned double buffer, and gathered and widened to float32 on the device.
//
// Surveys are ordinary forward passes that also store every hop layer's pre-activation, followed by one counting
// pass per layer (one 8-lane group per row, tiles in order: the sums do not depend on scheduling).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <filesystem>
#include <functional>
#include <iterator>
#include <map>
#include <memory>
#include <mutex>
#include <numeric>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "../../include/flyguy_core.h"
#include "../../include/flyguy_train.h"
#include "core.h"

namespace fs = std::filesystem;

namespace fg {

// ================================================================================================ device
__device__ __forceinline__ float from_half(unsigned short u) { return (float)__builtin_bit_cast(_Float16, u); }

// one workgroup per sample: its obs and teacher rows, binary16 -> float32 (exact)
__global__ __launch_bounds__(256) void k_gather16(const unsigned short* const* __restrict__ obs_tab,
                                                  const unsigned short* const* __restrict__ lg_tab,
                                                  const long long* __restrict__ n_tab, int n_chunks,
                                                  const int2* __restrict__ sel, int od, int na, float* __restrict__ obs,
                                                  float* __restrict__ tl) {
    const int b = blockIdx.x;
    const int2 s = sel[b];
    const bool ok = s.x >= 0 && s.x < n_chunks && s.y >= 0 && (long long)s.y < n_tab[s.x];
    float* xo = obs + (size_t)b * od;
    float* to = tl + (size_t)b * na;
    if (!ok) {
        for (int i = threadIdx.x; i < od; i += 256) xo[i] = __builtin_nanf("");
        for (int i = threadIdx.x; i < na; i += 256) to[i] = __builtin_nanf("");
        return;
    }
    const unsigned short* xi = obs_tab[s.x] + (size_t)s.y * od;
    const unsigned short* ti = lg_tab[s.x] + (size_t)s.y * na;
    for (int i = threadIdx.x; i < od; i += 256) xo[i] = from_half(xi[i]);
    for (int i = threadIdx.x; i < na; i += 256) to[i] = from_half(ti[i]);
}

__global__ __launch_bounds__(256) void k_unpack16(const unsigned short* __restrict__ st, int od, int na,
                                                  float* __restrict__ obs, float* __restrict__ tl) {
    const int b = blockIdx.x, w = od + na;
    const unsigned short* r = st + (size_t)b * w;
    for (int i = threadIdx.x; i < w; i += 256) {
        const float v = from_half(r[i]);
        if (i < od) obs[(size_t)b * od + i] = v;
        else tl[(size_t)b * na + (i - od)] = v;
    }
}

__device__ __forceinline__ int isum8(int v) {
    v += __builtin_amdgcn_ds_swizzle(v, 0x1f | (1 << 10));
    v += __builtin_amdgcn_ds_swizzle(v, 0x1f | (2 << 10));
    v += __builtin_amdgcn_ds_swizzle(v, 0x1f | (4 << 10));
    return v;
}

// per row of a tiled [T][rows][32] layer: cnt[row] += samples with h > 0, sq[row] += sum of z^2 (z nullable).
// 8 lanes per row, each over its float4 of every tile in tile order, then summed over the 8 lanes.
__global__ __launch_bounds__(256) void k_fired(const float* __restrict__ h, const float* __restrict__ z, int rows,
                                               int T, int* __restrict__ cnt, float* __restrict__ sq) {
    const int row = blockIdx.x * 32 + (int)(threadIdx.x >> 3), sub = threadIdx.x & 7;
    int c = 0;
    float v = 0.f;
    if (row < rows) {
        for (int t = 0; t < T; ++t) {
            const size_t o = ((size_t)t * rows + row) * TW + 4 * sub;
            const float4 hv = *reinterpret_cast<const float4*>(h + o);
            c += (hv.x > 0.f) + (hv.y > 0.f) + (hv.z > 0.f) + (hv.w > 0.f);
            if (z) {
                const float4 zv = *reinterpret_cast<const float4*>(z + o);
                v += zv.x * zv.x + zv.y * zv.y + zv.z * zv.z + zv.w * zv.w;
            }
        }
    }
    c = isum8(c);
    v = sum8(v);
    if (row < rows && sub == 0) {
        cnt[row] += c;
        sq[row] += v;
    }
}

// the same over a bfloat16 layer [T][rows][64]: each of the 8 lanes of a row takes 8 samples of every tile
__global__ __launch_bounds__(256) void k_fired16(const unsigned short* __restrict__ h, const unsigned short* __restrict__ z,
                                                 int rows, int T, int* __restrict__ cnt, float* __restrict__ sq) {
    const int row = blockIdx.x * 32 + (int)(threadIdx.x >> 3), sub = threadIdx.x & 7;
    int c = 0;
    float v = 0.f;
    if (row < rows) {
        for (int t = 0; t < T; ++t) {
            const size_t o = ((size_t)t * rows + row) * TW16 + 8 * sub;
            const uint4 hv = *reinterpret_cast<const uint4*>(h + o);
            const unsigned hw[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                c += (__uint_as_float(hw[k] << 16) > 0.f) + (__uint_as_float(hw[k] & 0xffff0000u) > 0.f);
            if (z) {
                const uint4 zv = *reinterpret_cast<const uint4*>(z + o);
                const unsigned zw[4] = {zv.x, zv.y, zv.z, zv.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float a = __uint_as_float(zw[k] << 16), b = __uint_as_float(zw[k] & 0xffff0000u);
                    v += a * a + b * b;
                }
            }
        }
    }
    c = isum8(c);
    v = sum8(v);
    if (row < rows && sub == 0) {
        cnt[row] += c;
        sq[row] += v;
    }
}

// the survey sums of one layer's states (float32 [T][rows][32] or, bf16, bfloat16 [T][rows][64]; z nullable) over
// B samples
static hipError_t launch_fired(const void* h, const void* z, bool bf16, int rows, int B, int* cnt, float* sq,
                               hipStream_t st) {
    const int T = B / (bf16 ? TW16 : TW);
    if (rows <= 0 || T <= 0) return hipSuccess;
    if (bf16)
        k_fired16<<<(unsigned)((rows + 31) / 32), 256, 0, st>>>((const unsigned short*)h, (const unsigned short*)z, rows,
                                                                 T, cnt, sq);
    else
        k_fired<<<(unsigned)((rows + 31) / 32), 256, 0, st>>>((const float*)h, (const float*)z, rows, T, cnt, sq);
    return hipGetLastError();
}

// ================================================================================================ host: device copies
// One parameter array of one set, copied to the host for an edit and written back.  A write to the weights or to the
// running average makes the handle's derived tables (packed pairs, row records) stale: weights_written says so.
struct HostArray {
    Core& c;
    int set, array;
    std::vector<float> v;
    HostArray(Core& core, int s, int i) : c(core), set(s), array(i) {}
    float& operator[](size_t i) { return v[i]; }
    bool load() {
        v.resize((size_t)c.psize[array]);
        if (!v.empty() &&
            hipMemcpyAsync(v.data(), c.arr(set, array), v.size() * 4, hipMemcpyDeviceToHost, c.st) != hipSuccess)
            return false;
        return hipStreamSynchronize(c.st) == hipSuccess;
    }
    bool store() {
        c.weights_written(set);
        if (!v.empty() &&
            hipMemcpyAsync(c.arr(set, array), v.data(), v.size() * 4, hipMemcpyHostToDevice, c.st) != hipSuccess)
            return false;
        return hipStreamSynchronize(c.st) == hipSuccess;
    }
};

static bool copy_in(Core& c, void* dst, const void* src, size_t bytes) {
    if (bytes && hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c.st) != hipSuccess) return false;
    return hipStreamSynchronize(c.st) == hipSuccess;
}
static bool copy_out(Core& c, void* dst, const void* src, size_t bytes) {
    if (bytes && hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c.st) != hipSuccess) return false;
    return hipStreamSynchronize(c.st) == hipSuccess;
}

// ================================================================================================ survey
static bool ensure_survey(Core& c) {
    if (c.scnt) return true;
    c.scnt = dalloc<int>(c, (size_t)c.rows_total);
    c.ssq = dalloc<float>(c, (size_t)c.rows_total);
    c.sstats = dalloc<float>(c, 4);
    bool ok = c.scnt && c.ssq && c.sstats;
    for (auto& d : c.hop) {                     // the pre-activation, stored like the layer's states
        d.zk = c.prec ? reinterpret_cast<float*>(dalloc<unsigned short>(c, (size_t)c.maxB * d.rows))
                      : dalloc<float>(c, (size_t)c.maxB * d.rows);
        ok = ok && d.zk;
    }
    return ok;
}

static bool survey_reset(Core& c) {
    if (!ensure_survey(c)) return false;
    FG_CHECK(launch_fill(reinterpret_cast<float*>(c.scnt), 0.f, c.rows_total, c.st), false);   // (0.0f: all bits 0)
    FG_CHECK(launch_fill(c.ssq, 0.f, c.rows_total, c.st), false);
    FG_CHECK(launch_fill(c.sstats, 0.f, 4, c.st), false);
    c.s_samples = 0;
    return true;
}

static bool survey_batch(Core& c, const float* obs, const float* teacher, int B, int set, float it) {
    if (!ensure_survey(c)) return false;
    c.keep_z = true;
    const bool ok = forward(c, obs, B, c.lg, set);
    c.keep_z = false;
    if (!ok) return false;
    FG_CHECK(launch_loss(c.lg, teacher, c.dl, c.stats_part, c.sstats, c.n_act, B, it, c.st, true), false);
    const bool b16 = c.prec != 0;
    FG_CHECK(launch_fired(c.h0, nullptr, b16, c.n_s, B, c.scnt, c.ssq, c.st), false);
    long long off = c.n_s;
    for (auto& d : c.hop) {
        FG_CHECK(launch_fired(d.h, d.zk, b16, d.rows, B, c.scnt + off, c.ssq + off, c.st), false);
        off += d.rows;
    }
    c.s_samples += B;
    return true;
}

// The sums of a survey on the host: per row of every layer (sensory rows first, then each hop's), the samples it
// fired for and the sum of its squared pre-activation; the loss sums and their per-sample means.
struct Survey {
    std::vector<int> cnt;
    std::vector<float> sq;
    float kl_sum = 0, agree_sum = 0;
    double kl = 0, agree = 0, samples = 0;
};

static bool survey_read(Core& c, Survey& s) {
    if (!ensure_survey(c)) return false;
    s.cnt.resize((size_t)c.rows_total);
    s.sq.resize((size_t)c.rows_total);
    float sums[4] = {0, 0, 0, 0};
    if (!copy_out(c, s.cnt.data(), c.scnt, s.cnt.size() * 4) || !copy_out(c, s.sq.data(), c.ssq, s.sq.size() * 4) ||
        !copy_out(c, sums, c.sstats, sizeof sums)) {
        set_error("survey: copy from the device");
        return false;
    }
    s.samples = c.s_samples;
    s.kl_sum = sums[0];
    s.agree_sum = sums[1];
    s.kl = s.samples > 0 ? sums[0] / s.samples : 0;
    s.agree = s.samples > 0 ? sums[1] / s.samples : 0;
    return true;
}

// a survey of the weights (set) over `batches` staged batches of B samples (obs [batches * B][obs_dim]) at
// temperature 1
static bool survey_staged(Core& c, const float* obs, const float* tl, int B, int batches, int set, Survey& s) {
    if (!survey_reset(c)) return false;
    for (int i = 0; i < batches; ++i)
        if (!survey_batch(c, obs + (size_t)i * B * c.obs_dim, tl + (size_t)i * B * c.n_act, B, set, 1.f)) return false;
    return survey_read(c, s);
}

// Where the neurons sit in a survey's rows.  A neuron can be a row of several hop layers; the sensory layer is not
// "past the sensory layer", and neither is a sensory neuron that a hop re-uses.
struct Census {
    int n_neurons = 0;
    std::vector<int> layer_rows;                         // rows per layer, sensory first
    std::vector<char> sensory;                           // per neuron
    std::vector<std::pair<size_t, int>> hop_rows;        // (survey row, neuron) of every hop layer's row

    explicit Census(const Core& c) : n_neurons(c.n_neurons), sensory((size_t)c.n_neurons, 0) {
        layer_rows.push_back(c.n_s);
        for (int g : c.h_n0) sensory[(size_t)g] = 1;
        size_t row = (size_t)c.n_s;
        for (const HopD& h : c.hop) {
            layer_rows.push_back(h.rows);
            for (int g : h.h_nid) hop_rows.push_back({row++, g});
        }
    }
    // per neuron past the sensory layer: the samples it fired for, over all its hop rows; -1 for every other neuron
    std::vector<long long> fired(const Survey& s) const {
        std::vector<long long> f((size_t)n_neurons, -1);
        for (const auto& rg : hop_rows)
            if (!sensory[(size_t)rg.second]) f[(size_t)rg.second] = std::max(f[(size_t)rg.second], 0LL) + s.cnt[rg.first];
        return f;
    }
    // per neuron: the largest rms of its pre-activation over its hop rows (0 where it is in no hop)
    std::vector<float> input_rms(const Survey& s) const {
        std::vector<float> r((size_t)n_neurons, 0.f);
        for (const auto& rg : hop_rows)
            r[(size_t)rg.second] = std::max(r[(size_t)rg.second], (float)std::sqrt(s.sq[rg.first] / s.samples));
        return r;
    }
    // " f0 f1 ...": per layer the share of (row, sample) pairs that fired
    std::string layer_shares(const Survey& s) const {
        std::string out;
        size_t row = 0;
        for (int rows : layer_rows) {
            double n = 0;
            for (int t = 0; t < rows; ++t) n += s.cnt[row++];
            char b[32];
            snprintf(b, sizeof b, " %.3f", n / (rows * s.samples));
            out += b;
        }
        return out;
    }
};

// the value of rank floor(n / 2) among the n positive entries of v (0 when there is none)
static float positive_median(const std::vector<float>& v) {
    std::vector<float> pos;
    std::copy_if(v.begin(), v.end(), std::back_inserter(pos), [](float x) { return x > 0.f; });
    if (pos.empty()) return 0.f;
    const auto mid = pos.begin() + (std::ptrdiff_t)(pos.size() / 2);
    std::nth_element(pos.begin(), mid, pos.end());
    return *mid;
}

// ================================================================================================ revive
// Per strength in play: the neuron it feeds and the neuron it comes from (the same in every hop that uses it), and
// the strengths in the order they first appear walking the hops in turn, each hop in CSR order (rows, then their
// connections): the order in which a revive draws the new signs.
struct Wiring {
    std::vector<int> post, pre, order;
    explicit Wiring(const Core& c) : post((size_t)c.n_w, -1), pre((size_t)c.n_w, -1) {
        for (size_t k = 0; k < c.hop.size(); ++k) {
            const HopD& h = c.hop[k];
            const std::vector<int>& below = k ? c.hop[k - 1].h_nid : c.h_n0;
            for (int t = 0; t < h.rows; ++t)
                for (int e = h.h_crow[(size_t)t]; e < h.h_crow[(size_t)t + 1]; ++e) {
                    const int wi = h.h_widx[(size_t)e];
                    if (post[(size_t)wi] >= 0) continue;
                    post[(size_t)wi] = h.h_nid[(size_t)t];
                    pre[(size_t)wi] = below[(size_t)h.h_col[(size_t)e]];
                    order.push_back(wi);
                }
        }
    }
};

// Silent neurons back to work, the network's output unchanged (the rules of flyguy_train.cu:479-551).  Every
// neuron past the sensory layer that fires for none of the surveyed samples: its incoming strengths keep their sizes
// (at least 1e-4) with a new random sign, its gain and threshold go back to 1 and -4, its strengths onto live
// neurons and its read-out weights become 0 (it sent nothing before and sends nothing after), and three surveys scale
// its incoming strengths until its input's rms over the samples is `target`.  The running average takes the new
// values and Adam restarts for them at the median of its positive second moments.  The surveys all see the same
// staged batches (obs, tl: `batches` batches of B).  Returns the number of silent neurons, or -1.
static int revive(Core& c, const float* obs, const float* tl, int B, int batches, float target, unsigned long long seed,
                  long long step, std::string& report) {
    const Census census(c);
    auto survey = [&](Survey& s) { return survey_staged(c, obs, tl, B, batches, SET_P, s); };
    auto failed = [](const char* what) {
        if (!*last_error()) set_error(std::string("revive: ") + what);
        return -1;
    };
    char line[512];
    Survey first;
    if (!survey(first)) return -1;
    const std::vector<long long> fired = census.fired(first);
    std::vector<char> silent((size_t)c.n_neurons, 0);
    int n_silent = 0, n_play = 0;
    for (size_t g = 0; g < fired.size(); ++g) {
        n_play += fired[g] >= 0;
        if (fired[g] == 0) { silent[g] = 1; ++n_silent; }
    }
    if (n_silent == 0) {
        snprintf(line, sizeof line, "revive step %lld | no silent neuron among %d over %.0f samples", step, n_play,
                 first.samples);
        report = line;
        return 0;
    }
    HostArray W(c, SET_P, 0), gain(c, SET_P, 1), theta(c, SET_P, 2), ro(c, SET_P, 5);
    if (!W.load() || !gain.load() || !theta.load() || !ro.load()) return failed("copy from the device");

    // the strengths the surgery sets: a new sign into a silent neuron, zero from a silent neuron into a live one
    enum : char { KEPT = 0, RESIGNED = 1, CUT = 2 };
    const Wiring wiring(c);
    std::vector<char> fate((size_t)c.n_w, KEPT);
    std::mt19937_64 signs(seed * 7919ULL + 17);
    long long n_in = 0, n_out = 0;
    for (int wi : wiring.order) {
        if (silent[(size_t)wiring.post[(size_t)wi]]) {
            const float size = std::max(std::fabs(W[(size_t)wi]), 1e-4f);
            W[(size_t)wi] = (signs() & 1) ? size : -size;
            fate[(size_t)wi] = RESIGNED;
            ++n_in;
        } else if (silent[(size_t)wiring.pre[(size_t)wi]]) {
            W[(size_t)wi] = 0.f;
            fate[(size_t)wi] = CUT;
            ++n_out;
        }
    }
    for (size_t g = 0; g < silent.size(); ++g)
        if (silent[g]) { gain[g] = 1.f; theta[g] = -4.f; }
    // read-out columns of silent descending neurons
    std::vector<int> quiet_cols;
    const std::vector<int>& top_nid = c.hop.back().h_nid;
    for (int j = 0; j < c.n_dn; ++j)
        if (silent[(size_t)top_nid[(size_t)c.h_dn[(size_t)j]]]) quiet_cols.push_back(j);
    for (int j : quiet_cols)
        for (int a = 0; a < c.n_act; ++a) ro[(size_t)a * c.n_dn + j] = 0.f;
    if (!W.store() || !gain.store() || !theta.store() || !ro.store()) return failed("copy to the device");

    // three rounds: survey, then every strength into a revived neuron scaled by target / that neuron's input rms
    // (within [0.02, 200]), so that hop after hop the inputs come to size
    for (int round = 0; round < 3; ++round) {
        Survey s;
        if (!survey(s)) return -1;
        const std::vector<float> rms = census.input_rms(s);
        for (size_t wi = 0; wi < (size_t)c.n_w; ++wi) {
            const int g = wiring.post[wi];
            if (g < 0 || !silent[(size_t)g] || rms[(size_t)g] <= 0.f) continue;
            W[wi] *= std::min(200.f, std::max(0.02f, target / rms[(size_t)g]));
        }
        if (!W.store()) return failed("copy to the device");
    }
    Survey last;
    if (!survey(last)) return -1;
    const std::vector<long long> fired_after = census.fired(last);
    int still = 0;
    for (size_t g = 0; g < silent.size(); ++g) still += silent[g] && fired_after[g] == 0;

    // the running average takes the new values; Adam restarts for them
    {
        HostArray avg(c, SET_EMA, 0), m(c, SET_M, 0), v(c, SET_V, 0);
        if (!avg.load() || !m.load() || !v.load()) return failed("copy from the device");
        const float v_typ = positive_median(v.v);
        for (size_t wi = 0; wi < fate.size(); ++wi)
            if (fate[wi] != KEPT) { avg[wi] = W[wi]; m[wi] = 0.f; v[wi] = v_typ; }
        if (!avg.store() || !m.store() || !v.store()) return failed("copy to the device");
    }
    for (int array = 1; array <= 2; ++array) {            // gains, thresholds
        HostArray avg(c, SET_EMA, array), m(c, SET_M, array), v(c, SET_V, array);
        if (!avg.load() || !m.load() || !v.load()) return failed("copy from the device");
        const float v_typ = positive_median(v.v), start = array == 1 ? 1.f : -4.f;
        for (size_t g = 0; g < silent.size(); ++g)
            if (silent[g]) { avg[g] = start; m[g] = 0.f; v[g] = v_typ; }
        if (!avg.store() || !m.store() || !v.store()) return failed("copy to the device");
    }
    {
        HostArray avg(c, SET_EMA, 5), m(c, SET_M, 5);
        if (!avg.load() || !m.load()) return failed("copy from the device");
        for (int j : quiet_cols)
            for (int a = 0; a < c.n_act; ++a) avg[(size_t)a * c.n_dn + j] = m[(size_t)a * c.n_dn + j] = 0.f;
        if (!avg.store() || !m.store()) return failed("copy to the device");
    }
    snprintf(line, sizeof line,
             "revive step %lld | %d of %d neurons past the sensory layer silent over %.0f samples | new sign for %lld "
             "incoming strengths, zero for %lld outgoing and for %d descending neurons' action weights | %d still silent "
             "| kl %.5f -> %.5f (must be equal)",
             step, n_silent, n_play, first.samples, n_in, n_out, (int)quiet_cols.size(), still, first.kl, last.kl);
    report = line;
    return n_silent;
}

// ================================================================================================ files
// A file read or written in whole records, closed when it goes out of scope.
class BinFile {
public:
    BinFile(const std::string& path, const char* mode) : f_(std::fopen(path.c_str(), mode)) {}
    ~BinFile() {
        if (f_) std::fclose(f_);
    }
    BinFile(const BinFile&) = delete;
    BinFile& operator=(const BinFile&) = delete;
    bool is_open() const { return f_ != nullptr; }
    template <class T> bool get(T* p, size_t n = 1) { return f_ && std::fread(p, sizeof(T), n, f_) == n; }
    template <class T> bool put(const T* p, size_t n = 1) { return f_ && std::fwrite(p, sizeof(T), n, f_) == n; }
    bool expect(const char* tag4) {
        char t[4];
        return get(t, 4) && std::memcmp(t, tag4, 4) == 0;
    }
    bool close() {                                         // (flushes; false if anything failed)
        const bool ok = f_ && std::fflush(f_) == 0 && !std::ferror(f_);
        if (f_) std::fclose(f_);
        f_ = nullptr;
        return ok;
    }

private:
    FILE* f_;
};

// A file written under a temporary name and renamed into place once whole, so a reader never sees half of it.
static bool write_whole(const std::string& path, const std::function<bool(BinFile&)>& body) {
    const std::string tmp = path + ".tmp";
    bool ok;
    {
        BinFile f(tmp, "wb");
        ok = f.is_open() && body(f);
        ok = f.close() && ok;
    }
    std::error_code ec;
    if (ok) {
        fs::rename(tmp, path, ec);
        if (ec) {                                           // (a target some systems will not replace)
            fs::remove(path, ec);
            fs::rename(tmp, path, ec);
        }
    }
    return ok && !ec;
}

static std::vector<unsigned char> slurp(const std::string& path) {
    std::error_code ec;
    const auto size = fs::file_size(path, ec);
    std::vector<unsigned char> bytes;
    if (ec) return bytes;
    BinFile f(path, "rb");
    bytes.resize((size_t)size);
    if (!f.get(bytes.data(), bytes.size())) bytes.clear();
    return bytes;
}

// A FLYD chunk of (obs_dim, n_act): its sample count if the file holds the header and every sample, else -1.  With
// payload, the samples too: n x obs_dim observations then n x n_act teacher logits, binary16, as in the file.
static long long read_flyd(const std::string& path, int od, int na, std::vector<unsigned short>* payload) {
    BinFile f(path, "rb");
    long long n = 0;
    int dims[2] = {0, 0};
    if (!f.expect("FLYD") || !f.get(&n) || !f.get(dims, 2) || dims[0] != od || dims[1] != na || n <= 0 ||
        n > 0x7fffffffLL)
        return -1;
    const size_t words = (size_t)n * (size_t)(od + na);
    if (!payload) {
        std::error_code ec;
        const auto size = fs::file_size(path, ec);
        return !ec && size >= 20 + 2 * words ? n : -1;
    }
    payload->resize(words);
    return f.get(payload->data(), words) ? n : -1;
}

// ---- FLYP / FLYO parameter files
static const char* const kArrays[7] = {"W", "gain", "theta", "in_w", "in_b", "out_w", "out_b"};

// the seven arrays of one set from a stream (host buffer, then the device)
static bool read_set(Core& c, BinFile& f, int set) {
    for (int i = 0; i < 7; ++i) {
        HostArray a(c, set, i);
        a.v.resize((size_t)c.psize[i]);
        if (!f.get(a.v.data(), a.v.size()) || !a.store()) return false;
    }
    return true;
}

// FLYP weights from `path` into the weights, and from avg_path (or `path` again) into the running average; the
// step stored in `path`.  Messages on stderr.
static bool load_weights(Core& c, const std::string& path, const std::string& avg_path, long long& step) {
    const std::string sources[2] = {path, avg_path.empty() ? path : avg_path};
    for (int set = SET_P; set <= SET_EMA; ++set) {
        BinFile f(sources[set], "rb");
        if (!f.is_open()) { fprintf(stderr, "cannot open %s\n", sources[set].c_str()); return false; }
        long long st = 0;
        if (!f.expect("FLYP") || !f.get(&st)) { fprintf(stderr, "%s: not a FLYP parameter file\n", sources[set].c_str()); return false; }
        if (set == SET_P) step = st;
        if (!read_set(c, f, set)) { fprintf(stderr, "short params file\n"); return false; }
    }
    return true;
}

static bool save_weights(Core& c, const std::string& path, long long step, int set) {
    return write_whole(path, [&](BinFile& f) {
        if (!f.put("FLYP", 4) || !f.put(&step)) return false;
        for (int i = 0; i < 7; ++i) {
            HostArray a(c, set, i);
            if (!a.load() || !f.put(a.v.data(), a.v.size())) return false;
        }
        return true;
    });
}

static bool save_moments(Core& c, const std::string& path, long long step) {
    return write_whole(path, [&](BinFile& f) {
        if (!f.put("FLYO", 4) || !f.put(&step) || !f.put(&c.adam_t)) return false;
        for (int i = 0; i < 7; ++i) {
            HostArray m(c, SET_M, i), v(c, SET_V, i);
            if (!m.load() || !v.load() || !f.put(m.v.data(), m.v.size()) || !f.put(v.v.data(), v.v.size())) return false;
        }
        return true;
    });
}

// Adam's moments and step count from a FLYO file written at `step` (a file of another step restores nothing)
static bool load_moments(Core& c, const std::string& path, long long step) {
    BinFile f(path, "rb");
    long long st = -1, t = 0;
    if (!f.expect("FLYO") || !f.get(&st) || !f.get(&t) || st != step) return false;
    std::vector<HostArray> m, v;
    for (int i = 0; i < 7; ++i) {
        m.emplace_back(c, SET_M, i);
        v.emplace_back(c, SET_V, i);
        m[i].v.resize((size_t)c.psize[i]);
        v[i].v.resize((size_t)c.psize[i]);
        if (!f.get(m[i].v.data(), m[i].v.size()) || !f.get(v[i].v.data(), v[i].v.size())) return false;
    }
    for (int i = 0; i < 7; ++i)
        if (!m[i].store() || !v[i].store()) return false;
    c.adam_t = t;
    return true;
}

// ================================================================================================ data
// B samples, each uniform over the concatenation of chunks of these sizes, as (chunk, sample): one draw of
// uniform_int_distribution<long long>(0, total - 1) per sample from the engine g (the trainer's draw contract).
static void draw_samples(std::mt19937_64& g, const std::vector<long long>& sizes, int B, int2* out) {
    std::vector<long long> ends(sizes.size());
    std::partial_sum(sizes.begin(), sizes.end(), ends.begin());
    std::uniform_int_distribution<long long> pick(0, ends.back() - 1);
    for (int i = 0; i < B; ++i) {
        const long long s = pick(g);
        const size_t k = (size_t)(std::upper_bound(ends.begin(), ends.end(), s) - ends.begin());
        out[i] = make_int2((int)k, (int)(s - (k ? ends[k - 1] : 0)));
    }
}

// A chunk file's version: its modification time, then its path (the order in which chunks are taken).
struct FileVersion {
    fs::file_time_type mtime{};
    std::string path;
    bool operator<(const FileVersion& o) const { return mtime != o.mtime ? mtime < o.mtime : path < o.path; }
    std::string name() const { return fs::path(path).filename().string(); }
};

// The chunk files of a directory (chunk_*.bin) that are new or rewritten since they were last taken.  Of more than
// `newest` such files only the newest are offered; the older ones are passed over for good.
class ChunkWatch {
public:
    ChunkWatch(std::string dir, size_t newest) : dir_(std::move(dir)), newest_(newest) {}
    std::vector<FileVersion> fresh() {
        std::vector<FileVersion> out;
        std::error_code ec;
        for (const auto& e : fs::directory_iterator(dir_, ec)) {
            const std::string name = e.path().filename().string();
            if (name.compare(0, 6, "chunk_") != 0 || e.path().extension() != ".bin") continue;
            std::error_code e2;
            const auto mt = fs::last_write_time(e.path(), e2);
            if (e2) continue;
            const auto had = taken_.find(name);
            if (had == taken_.end() || had->second != mt) out.push_back({mt, e.path().string()});
        }
        std::sort(out.begin(), out.end());
        const size_t over = out.size() > newest_ ? out.size() - newest_ : 0;
        for (size_t i = 0; i < over; ++i) taken(out[i]);
        out.erase(out.begin(), out.begin() + (std::ptrdiff_t)over);
        return out;
    }
    void taken(const FileVersion& f) { taken_[f.name()] = f.mtime; }

private:
    std::string dir_;
    size_t newest_;
    std::map<std::string, fs::file_time_type> taken_;
};

// A chunk read into host memory, on its way to the device.
struct HostChunk {
    FileVersion file;
    long long n = 0;
    std::vector<unsigned short> payload;
};
typedef std::unique_ptr<HostChunk> HostChunkP;

static HostChunkP load_chunk(const FileVersion& f, int od, int na) {
    HostChunkP h(new HostChunk);
    h->file = f;
    h->n = read_flyd(f.path, od, na, &h->payload);
    if (h->n <= 0) return nullptr;                 // (being rewritten right now: a later look finds it whole)
    return h;
}

// Reads chunks in the background, never more than one ahead of the trainer: a chunk is read only once the trainer
// has taken the one before.  Looks for fresh files every two seconds.
class Prefetch {
public:
    Prefetch(const std::string& dir, size_t newest, int od, int na) : watch_(dir, newest), od_(od), na_(na) {}
    ~Prefetch() { stop(); }
    // every fresh chunk at once (before the thread starts); how many were read
    int read_now() {
        int got = 0;
        for (const FileVersion& f : watch_.fresh()) {
            HostChunkP h = load_chunk(f, od_, na_);
            if (!h) continue;
            watch_.taken(f);
            std::lock_guard<std::mutex> g(mu_);
            ready_.push_back(std::move(h));
            ++got;
        }
        return got;
    }
    void start() { thread_ = std::thread([this] { loop(); }); }
    void stop() {
        {
            std::lock_guard<std::mutex> g(mu_);
            quit_ = true;
        }
        wake_.notify_all();
        if (thread_.joinable()) thread_.join();
    }
    HostChunkP take() {
        HostChunkP h;
        {
            std::lock_guard<std::mutex> g(mu_);
            if (ready_.empty()) return h;
            h = std::move(ready_.front());
            ready_.pop_front();
        }
        wake_.notify_all();
        return h;
    }

private:
    void loop() {
        std::unique_lock<std::mutex> lk(mu_);
        while (!quit_) {
            lk.unlock();
            std::vector<FileVersion> files = watch_.fresh();
            lk.lock();
            for (const FileVersion& f : files) {
                wake_.wait(lk, [this] { return quit_ || ready_.empty(); });
                if (quit_) break;
                lk.unlock();
                HostChunkP h = load_chunk(f, od_, na_);
                lk.lock();
                if (!h) continue;
                watch_.taken(f);
                ready_.push_back(std::move(h));
            }
            wake_.wait_for(lk, std::chrono::seconds(2), [this] { return quit_; });
        }
    }
    ChunkWatch watch_;
    int od_, na_;
    std::mutex mu_;
    std::condition_variable wake_;
    std::deque<HostChunkP> ready_;
    bool quit_ = false;
    std::thread thread_;
};

// The chunks in device memory: one allocation per chunk (its observations, then its teacher logits, binary16) in a
// slot of a device table {observations, logits, samples} that k_gather16 reads.  A batch names its samples by
// (slot, sample).
class DeviceChunks {
public:
    bool init(Core& c, int slots) {
        base_.assign((size_t)slots, nullptr);
        obs_.assign((size_t)slots, nullptr);
        lg_.assign((size_t)slots, nullptr);
        n_.assign((size_t)slots, 0);
        d_obs_ = dalloc<const unsigned short*>(c, (size_t)slots);
        d_lg_ = dalloc<const unsigned short*>(c, (size_t)slots);
        d_n_ = dalloc<long long>(c, (size_t)slots);
        return d_obs_ && d_lg_ && d_n_;
    }
    // a chunk's samples into a free slot (the host copy is then dropped); the slot, or -1
    int upload(Core& c, HostChunk& h, int od) {
        const auto free_at = std::find(base_.begin(), base_.end(), nullptr);
        if (free_at == base_.end()) { set_error("chunk table full"); return -1; }
        const size_t s = (size_t)(free_at - base_.begin()), bytes = h.payload.size() * 2;
        void* p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) {
            set_error("out of device memory for a chunk of " + std::to_string(h.n) + " samples");
            return -1;
        }
        if (!copy_in(c, p, h.payload.data(), bytes)) {
            (void)hipFree(p);
            set_error("chunk upload");
            return -1;
        }
        base_[s] = p;
        obs_[s] = static_cast<const unsigned short*>(p);
        lg_[s] = obs_[s] + (size_t)h.n * od;
        n_[s] = h.n;
        std::vector<unsigned short>().swap(h.payload);
        return publish(c) ? (int)s : -1;
    }
    void release(Core& c, int slot) {
        if (slot < 0 || !base_[(size_t)slot]) return;
        (void)hipStreamSynchronize(c.st);                  // (kernels in flight may still read it)
        (void)hipFree(base_[(size_t)slot]);
        base_[(size_t)slot] = nullptr;
        obs_[(size_t)slot] = lg_[(size_t)slot] = nullptr;
        n_[(size_t)slot] = 0;
        (void)publish(c);
    }
    int slots() const { return (int)base_.size(); }
    const unsigned short* const* obs_table() const { return d_obs_; }
    const unsigned short* const* logits_table() const { return d_lg_; }
    const long long* sizes_table() const { return d_n_; }

private:
    bool publish(Core& c) {
        if (!copy_in(c, d_obs_, obs_.data(), obs_.size() * sizeof(void*)) ||
            !copy_in(c, d_lg_, lg_.data(), lg_.size() * sizeof(void*)) ||
            !copy_in(c, d_n_, n_.data(), n_.size() * sizeof(long long))) {
            set_error("chunk table upload");
            return false;
        }
        return true;
    }
    std::vector<void*> base_;
    std::vector<const unsigned short*> obs_, lg_;
    std::vector<long long> n_;
    const unsigned short** d_obs_ = nullptr;
    const unsigned short** d_lg_ = nullptr;
    long long* d_n_ = nullptr;
};

// A chunk the trainer draws from (or holds out): its file version, samples and device slot.
struct Chunk {
    FileVersion file;
    long long n = 0;
    int slot = -1;
};

// Drawn batches on their way to the device: the (slot, sample) pairs of up to `rows` samples in one of two pinned
// buffers (the host fills one while the copy of the other may still run), then gathered on the device into staged
// float32 observations and teacher logits.
class Staging {
public:
    ~Staging() {
        for (int k = 0; k < 2; ++k) {
            if (done_[k]) {
                if (used_[k]) (void)hipEventSynchronize(done_[k]);
                (void)hipEventDestroy(done_[k]);
            }
            if (pin_[k]) (void)hipHostFree(pin_[k]);
        }
    }
    bool init(Core& c, int rows) {
        rows_ = rows;
        for (int k = 0; k < 2; ++k) {
            FG_CHECK(hipHostMalloc((void**)&pin_[k], (size_t)rows * sizeof(int2), hipHostMallocDefault), false);
            FG_CHECK(hipEventCreateWithFlags(&done_[k], hipEventDisableTiming), false);
        }
        sel_ = dalloc<int2>(c, (size_t)rows);
        obs = dalloc<float>(c, (size_t)rows * c.obs_dim);
        tl = dalloc<float>(c, (size_t)rows * c.n_act);
        return sel_ && obs && tl;
    }
    // `batches` batches of B drawn with g from the chunks of `from` (the ring's order) into obs / tl
    bool fill(Core& c, const DeviceChunks& dev, const std::vector<const Chunk*>& from, std::mt19937_64& g, int B,
              int batches) {
        const int n = B * batches;
        if (n > rows_) { set_error("staging too small"); return false; }
        std::vector<long long> sizes;
        for (const Chunk* ch : from) sizes.push_back(ch->n);
        const int k = next_;
        next_ ^= 1;
        if (used_[k]) FG_CHECK(hipEventSynchronize(done_[k]), false);    // the copy that last read it is done
        for (int i = 0; i < batches; ++i) draw_samples(g, sizes, B, pin_[k] + (size_t)i * B);
        for (int i = 0; i < n; ++i) pin_[k][i].x = from[(size_t)pin_[k][i].x]->slot;
        FG_CHECK(hipMemcpyAsync(sel_, pin_[k], (size_t)n * sizeof(int2), hipMemcpyHostToDevice, c.st), false);
        FG_CHECK(hipEventRecord(done_[k], c.st), false);
        used_[k] = true;
        k_gather16<<<(unsigned)n, 256, 0, c.st>>>(dev.obs_table(), dev.logits_table(), dev.sizes_table(), dev.slots(),
                                                  sel_, c.obs_dim, c.n_act, obs, tl);
        FG_CHECK(hipGetLastError(), false);
        return true;
    }
    float *obs = nullptr, *tl = nullptr;

private:
    int rows_ = 0, next_ = 0;
    int2* pin_[2] = {nullptr, nullptr};
    hipEvent_t done_[2] = {nullptr, nullptr};
    bool used_[2] = {false, false};
    int2* sel_ = nullptr;
};

// ================================================================================================ the trainer
static double seconds_now() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// the learning rates of one step: per group max(lr_min * base / lr, base * 0.5^(step / half_life))
static void rates_at(long long step, float lr, float lr_neuron, float lr_plug, float lr_min, double half_life,
                     float out[3]) {
    const float decay = (float)std::pow(0.5, (double)step / half_life);
    const float base[3] = {lr, lr_neuron, lr_plug};
    for (int g = 0; g < 3; ++g) out[g] = std::max(lr_min * base[g] / lr, base[g] * decay);
}

// one forward + loss + backward of a staged batch; the loss sums ADDED to stats
static bool learn_from(Core& c, const float* obs, const float* tl, int B, float it, float* stats) {
    FG_CHECK(launch_fill(c.arr(SET_G, 0), 0.f, c.PT, c.st), false);
    if (!forward(c, obs, B, c.lg, SET_P)) return false;
    FG_CHECK(launch_loss(c.lg, tl, c.dl, c.stats_part, stats, c.n_act, B, it, c.st, true), false);
    return backward(c, c.dl, B, true);                      // (the gradient was cleared above)
}

typedef std::unique_ptr<Core, void (*)(Core*)> CoreP;

static CoreP open_network(const std::string& path, int B, int flags = 0) {
    const std::vector<unsigned char> bytes = slurp(path);
    if (bytes.empty()) {
        fprintf(stderr, "cannot open %s\n", path.c_str());
        return CoreP(nullptr, release);
    }
    CoreP c(build(bytes.data(), (long long)bytes.size(), B, flags), release);
    if (!c) fprintf(stderr, "%s: %s\n", path.c_str(), last_error());
    return c;
}

// ---- --check NET PARAMS BATCH: one forward + backward of a FLYB batch, printed as export.py batch prints PyTorch's
static int check_batch_file(const char* net_path, const char* params_path, const char* batch_path) {
    BinFile f(batch_path, "rb");
    char tag[4];
    int B = 0;
    if (!f.is_open()) { fprintf(stderr, "cannot open %s\n", batch_path); return 1; }
    if (!f.get(tag, 4) || !f.get(&B) || B <= 0) { fprintf(stderr, "%s: not a batch file\n", batch_path); return 1; }
    if (B % TW) { fprintf(stderr, "%s: %d samples; the batch must be a multiple of 32\n", batch_path, B); return 2; }
    CoreP cp = open_network(net_path, B);
    if (!cp) return 1;
    Core& c = *cp;
    long long step = 0;
    if (!load_weights(c, params_path, "", step)) return 1;
    std::vector<float> x((size_t)B * c.obs_dim), t((size_t)B * c.n_act);
    if (!f.get(x.data(), x.size()) || !f.get(t.data(), t.size())) { fprintf(stderr, "%s: short batch file\n", batch_path); return 1; }
    float* dx = dalloc<float>(c, x.size());
    float* dt = dalloc<float>(c, t.size());
    if (!dx || !dt || !copy_in(c, dx, x.data(), x.size() * 4) || !copy_in(c, dt, t.data(), t.size() * 4) ||
        launch_fill(c.stats, 0.f, 4, c.st) != hipSuccess || !learn_from(c, dx, dt, B, 1.f, c.stats)) {
        fprintf(stderr, "%s\n", *last_error() ? last_error() : "device error");
        return 1;
    }
    float sums[2];
    std::vector<float> first((size_t)c.n_act);
    if (!copy_out(c, sums, c.stats, sizeof sums) || !copy_out(c, first.data(), c.lg, first.size() * 4)) {
        fprintf(stderr, "copy\n");
        return 1;
    }
    printf("native: loss %.6f agree %.4f\n   logits[0][:5]", sums[0] / B, sums[1] / B);
    for (int a = 0; a < std::min(5, c.n_act); ++a) printf(" %.6f", first[(size_t)a]);
    printf("\n");
    for (int i = 0; i < 7; ++i) {
        HostArray g(c, SET_G, i);
        if (!g.load()) { fprintf(stderr, "copy\n"); return 1; }
        double sq = 0, sum = 0;
        for (float v : g.v) { sq += (double)v * v; sum += v; }
        printf("   grad %-6s norm %.6e sum %+.6e\n", kArrays[i], std::sqrt(sq), sum);
    }
    fflush(stdout);
    return 0;
}

// The trainer's settings (the command line of flyguy_train.cu:654-677, plus --bf16).
struct Settings {
    int batch = 512, log_every = 100, eval_batches = 16, revive_batches = 4, ring = 3;
    bool revive_first = false, holdout = false;
    int flags = 0;                                  // FC_STATES_BF16 with --bf16 1
    long long steps = 0, revive_every = 0, eval_every = 0;
    double save_sec = 120, half_life = 20000, max_reuse = -1;
    float lr = 3e-4f, lr_neuron = 1e-4f, lr_plug = 3e-4f, lr_min = 3e-5f, ema = 0.999f, clip = 0.f, temp = 1.f,
          revive_target = 0.4f;

    // "--name value" pairs from argv[first]; false (with a message) for an unknown name
    bool parse(int argc, const char* const* argv, int first) {
        const std::map<std::string, std::function<void(double)>> options = {
            {"--batch", [this](double v) { batch = (int)v; }},
            {"--lr", [this](double v) { lr = (float)v; }},
            {"--lr-neuron", [this](double v) { lr_neuron = (float)v; }},
            {"--lr-plug", [this](double v) { lr_plug = (float)v; }},
            {"--lr-min", [this](double v) { lr_min = (float)v; }},
            {"--half-life", [this](double v) { half_life = v; }},
            {"--ema", [this](double v) { ema = (float)v; }},
            {"--log", [this](double v) { log_every = (int)v; }},
            {"--save-sec", [this](double v) { save_sec = v; }},
            {"--steps", [this](double v) { steps = (long long)v; }},
            {"--clip", [this](double v) { clip = (float)v; }},
            {"--temp", [this](double v) { temp = (float)v; }},
            {"--eval-batches", [this](double v) { eval_batches = (int)v; }},
            {"--eval-every", [this](double v) { eval_every = (long long)v; }},
            {"--revive-every", [this](double v) { revive_every = (long long)v; }},
            {"--revive-batches", [this](double v) { revive_batches = (int)v; }},
            {"--revive-target", [this](double v) { revive_target = (float)v; }},
            {"--revive-first", [this](double v) { revive_first = (int)v != 0; }},
            {"--max-reuse", [this](double v) { max_reuse = v; }},
            {"--ring", [this](double v) { ring = std::max(1, (int)v); }},
            {"--holdout", [this](double v) { holdout = (int)v != 0; }},
            {"--passes", [](double) {}},            // (an option of the one-chunk-at-a-time trainer: no effect)
            {"--bf16", [this](double v) { flags = v != 0 ? FC_STATES_BF16 : 0; }},
        };
        for (int i = first; i + 1 < argc; i += 2) {
            const auto opt = options.find(argv[i]);
            if (opt == options.end()) { fprintf(stderr, "unknown option %s\n", argv[i]); return false; }
            opt->second(std::atof(argv[i + 1]));
        }
        return true;
    }
};

class Trainer {
public:
    Trainer(Core& c, const Settings& o, std::string data_dir, std::string out)
        : c_(c), o_(o), data_dir_(std::move(data_dir)), out_(std::move(out)),
          prefetch_(data_dir_, (size_t)o.ring + (o.holdout ? 1 : 0), c.obs_dim, c.n_act) {}
    ~Trainer() {
        prefetch_.stop();
        (void)hipStreamSynchronize(c_.st);
        for (Chunk& ch : ring_) chunks_.release(c_, ch.slot);
        if (held_) chunks_.release(c_, held_->slot);
    }
    int run(const std::string& params_in);

private:
    bool fail(const char* what) {
        fprintf(stderr, "%s: %s\n", what, last_error());
        fflush(stderr);
        failed_ = true;
        return false;
    }
    std::vector<const Chunk*> ring_view() const {
        std::vector<const Chunk*> v;
        for (const Chunk& ch : ring_) v.push_back(&ch);
        return v;
    }
    double ring_samples() const {
        double s = 0;
        for (const Chunk& ch : ring_) s += (double)ch.n;
        return s;
    }
    bool upload(HostChunk& h, Chunk& ch) {
        ch.file = h.file;
        ch.n = h.n;
        ch.slot = chunks_.upload(c_, h, c_.obs_dim);
        return ch.slot >= 0 || fail("chunk upload");
    }
    // a chunk into the ring in modification-time order, in place of an earlier version of the same file; the oldest
    // chunks leave beyond the ring's size
    void enter_ring(const Chunk& ch) {
        for (auto it = ring_.begin(); it != ring_.end();) {
            if (it->file.name() == ch.file.name()) {
                chunks_.release(c_, it->slot);
                it = ring_.erase(it);
            } else {
                ++it;
            }
        }
        ring_.insert(std::upper_bound(ring_.begin(), ring_.end(), ch,
                                      [](const Chunk& a, const Chunk& b) { return a.file.mtime < b.file.mtime; }), ch);
        while ((int)ring_.size() > o_.ring) {
            chunks_.release(c_, ring_.front().slot);
            ring_.erase(ring_.begin());
        }
    }
    bool evaluate(const Chunk& ch, unsigned long long seed, const char* label);
    bool admit_new_chunks();
    bool revive_now();
    bool learn_one_step();
    void log_progress();
    bool save_all();
    bool stop_requested() const { return fs::exists(out_ + ".STOP"); }
    void stop_acknowledged() {
        std::error_code ec;
        fs::rename(out_ + ".STOP", out_ + ".STOP.done", ec);
        printf("stopped on request at step %lld\n", step_);
        fflush(stdout);
    }

    Core& c_;
    Settings o_;
    std::string data_dir_, out_;
    Prefetch prefetch_;
    DeviceChunks chunks_;
    Staging stage_;
    std::vector<Chunk> ring_;                       // oldest first
    std::unique_ptr<Chunk> held_;                   // --holdout 1: the newest chunk at the start, never learned from
    std::mt19937_64 draws_;
    long long step_ = 0, ran_ = 0, since_log_ = 0, last_revive_ = 0;
    double budget_ = 0;                             // draws left before the ring's samples are used up (--max-reuse)
    double t_log_ = 0, t_save_ = 0, t_new_ = 0;
    bool failed_ = false;
    bool save_failed_ = false;                      // some save failed (the exit status says so)
};

// The loss and agreement of the running average (the network that would be installed) and of the raw weights on
// eval_batches batches of one chunk, both drawn with the same seed, with the firing report of the average.
bool Trainer::evaluate(const Chunk& ch, unsigned long long seed, const char* label) {
    if (o_.eval_batches <= 0 || failed_) return !failed_;
    const std::vector<const Chunk*> one{&ch};
    Survey of[2];
    const int sets[2] = {SET_EMA, SET_P};
    for (int k = 0; k < 2; ++k) {
        std::mt19937_64 g(seed);
        if (!survey_reset(c_)) return fail("eval");
        for (int i = 0; i < o_.eval_batches; ++i)
            if (!stage_.fill(c_, chunks_, one, g, o_.batch, 1) ||
                !survey_batch(c_, stage_.obs, stage_.tl, o_.batch, sets[k], 1.f))
                return fail("eval");
        if (!survey_read(c_, of[k])) return fail("eval");
    }
    const Census census(c_);
    const std::vector<long long> fired = census.fired(of[0]);
    int silent = 0, in_play = 0;
    for (long long f : fired) {
        in_play += f >= 0;
        silent += f == 0;
    }
    printf("eval step %lld | kl %.4f agree %.4f | raw kl %.4f agree %.4f | firing%s | silent %d of %d | %s %s\n", step_,
           of[0].kl, of[0].agree, of[1].kl, of[1].agree, census.layer_shares(of[0]).c_str(), silent, in_play,
           ch.file.name().c_str(), label);
    fflush(stdout);
    return true;
}

// chunks the prefetcher has read since: each scored before anything is learned from it, then into the ring
bool Trainer::admit_new_chunks() {
    while (HostChunkP h = prefetch_.take()) {
        Chunk ch;
        if (!upload(*h, ch)) return false;
        if (!evaluate(ch, 1000003ULL * (unsigned long long)step_ + 7, "unseen")) {
            chunks_.release(c_, ch.slot);
            return false;
        }
        enter_ring(ch);
        t_new_ = seconds_now();
        budget_ = std::min(budget_ + o_.max_reuse * (double)ch.n, o_.max_reuse * ring_samples());
    }
    return true;
}

bool Trainer::revive_now() {
    const unsigned long long seed = 99991ULL * (unsigned long long)step_ + 3;
    std::mt19937_64 g(seed);
    std::string report;
    if (!stage_.fill(c_, chunks_, ring_view(), g, o_.batch, o_.revive_batches) ||
        revive(c_, stage_.obs, stage_.tl, o_.batch, o_.revive_batches, o_.revive_target, seed, step_, report) < 0)
        return fail("revive");
    printf("%s\n", report.c_str());
    fflush(stdout);
    last_revive_ = step_;
    return true;
}

bool Trainer::learn_one_step() {
    if (!stage_.fill(c_, chunks_, ring_view(), draws_, o_.batch, 1) ||
        !learn_from(c_, stage_.obs, stage_.tl, o_.batch, 1.f / o_.temp, c_.stats))
        return fail("step");
    ++step_;
    ++ran_;
    ++since_log_;
    float rates[3];
    rates_at(step_, o_.lr, o_.lr_neuron, o_.lr_plug, o_.lr_min, o_.half_life, rates);
    if (fg::step(c_, rates[0], rates[1], rates[2], o_.clip, o_.ema) < 0.f) return fail("step");
    return true;
}

// the loss and agreement since the last line (the sums are cleared after each), samples/s, the strengths' rate
void Trainer::log_progress() {
    float sums[2];
    if (!copy_out(c_, sums, c_.stats, sizeof sums) || launch_fill(c_.stats, 0.f, 4, c_.st) != hipSuccess) {
        fail("stats");
        return;
    }
    const double t = seconds_now(), n = (double)o_.batch * since_log_;
    char late[64] = "";
    if (!o_.steps && t - t_new_ > 900) snprintf(late, sizeof late, " | NO NEW DATA for %.0f min", (t - t_new_) / 60);
    const float shown = std::max(o_.lr_min, o_.lr * (float)std::pow(0.5, (double)step_ / o_.half_life));
    printf("step %lld | %.0f samples/s | kl %.4f agree %.4f | lr %.2e | ring %d, newest %s%s\n", step_,
           n / (t - t_log_), sums[0] / n, sums[1] / n, shown, (int)ring_.size(), ring_.back().file.name().c_str(), late);
    fflush(stdout);
    t_log_ = t;
    since_log_ = 0;
}

bool Trainer::save_all() {
    if (hipStreamSynchronize(c_.st) != hipSuccess || !save_weights(c_, out_ + ".bin", step_, SET_P) ||
        !save_weights(c_, out_ + ".ema.bin", step_, SET_EMA) || !save_moments(c_, out_ + ".opt.bin", step_)) {
        fprintf(stderr, "cannot save %s.bin / .ema.bin / .opt.bin\n", out_.c_str());
        return false;
    }
    printf("saved %s.bin, .ema.bin and .opt.bin at step %lld\n", out_.c_str(), step_);
    fflush(stdout);
    t_save_ = seconds_now();
    return true;
}

int Trainer::run(const std::string& params_in) {
    // a restart from this run's own save keeps the running average and the optimiser state
    const bool resuming = fs::path(params_in).lexically_normal() == fs::path(out_ + ".bin").lexically_normal();
    const std::string avg_file = out_ + ".ema.bin";
    if (!load_weights(c_, params_in, resuming && fs::exists(avg_file) ? avg_file : "", step_)) return 1;
    c_.adam_t = 0;
    const bool moments = resuming && load_moments(c_, out_ + ".opt.bin", step_);
    const int stage_rows = o_.batch * std::max(1, o_.revive_every > 0 ? o_.revive_batches : 1);
    if (!stage_.init(c_, stage_rows) || !chunks_.init(c_, o_.ring + 2)) {
        fprintf(stderr, "%s\n", last_error());
        return 1;
    }
    draws_.seed(12345 + step_);
    printf("flyguy native trainer: %d neurons, %d strengths in play, %d hops, batch %d, lr %g (neurons %g, plugs %g), "
           "teacher temperature %g, ring of %d chunks, start step %lld%s%s\n",
           c_.n_neurons, c_.n_w, c_.hops, o_.batch, o_.lr, o_.lr_neuron, o_.lr_plug, o_.temp, o_.ring, step_,
           moments ? ", optimiser state restored" : "", c_.prec ? ", bfloat16 states" : "");
    fflush(stdout);
    while (prefetch_.read_now() == 0) {
        printf("waiting for data in %s\n", data_dir_.c_str());
        fflush(stdout);
        std::this_thread::sleep_for(std::chrono::seconds(20));
    }
    std::vector<HostChunkP> first;
    while (HostChunkP h = prefetch_.take()) first.push_back(std::move(h));
    if (o_.holdout && first.size() > 1) {
        held_.reset(new Chunk);
        if (!upload(*first.back(), *held_)) return 1;
        first.pop_back();
    }
    for (HostChunkP& h : first) {
        Chunk ch;
        if (!upload(*h, ch)) return 1;
        enter_ring(ch);
    }
    if (!evaluate(held_ ? *held_ : ring_.back(), 4242, held_ ? "held out" : "at the start")) return 1;
    prefetch_.start();
    last_revive_ = o_.revive_first ? step_ - o_.revive_every : step_;
    // at most max_reuse draws per recorded sample (default 4 for an open-ended run, off for --steps): when the
    // recording stops, the trainer waits rather than learn the same chunks by heart
    if (o_.max_reuse < 0) o_.max_reuse = o_.steps ? 0 : 4;
    budget_ = o_.max_reuse * ring_samples();
    t_log_ = t_save_ = t_new_ = seconds_now();
    if (launch_fill(c_.stats, 0.f, 4, c_.st) != hipSuccess) return fail("stats"), 1;
    bool waiting = false;
    while (!o_.steps || ran_ < o_.steps) {
        if (!admit_new_chunks()) return 1;
        if (o_.max_reuse > 0 && budget_ < o_.batch) {
            if (!waiting) {
                printf("step %lld | waiting for new data: every sample of the ring has been drawn %.0f times on average\n",
                       step_, o_.max_reuse);
                fflush(stdout);
                waiting = true;
                since_log_ = 0;
                if (launch_fill(c_.stats, 0.f, 4, c_.st) != hipSuccess) return fail("stats"), 1;
            }
            if (stop_requested()) {
                save_failed_ |= !save_all();
                stop_acknowledged();
                return save_failed_ ? 1 : 0;
            }
            std::this_thread::sleep_for(std::chrono::seconds(1));
            t_log_ = seconds_now();
            continue;
        }
        waiting = false;
        budget_ -= o_.batch;
        if (o_.revive_every > 0 && step_ - last_revive_ >= o_.revive_every && !revive_now()) return 1;
        if (!learn_one_step()) return 1;
        if (since_log_ >= o_.log_every) {
            log_progress();
            if (failed_) return 1;
        }
        if (o_.eval_every > 0 && step_ % o_.eval_every == 0 &&
            !evaluate(held_ ? *held_ : ring_.back(), 4242, held_ ? "held out" : "in the ring"))
            return 1;
        const bool stop = stop_requested();
        if (stop || seconds_now() - t_save_ > o_.save_sec) {
            const bool saved = save_all();             // (a failed save is reported; the run goes on)
            save_failed_ |= !saved;
            if (stop) {
                stop_acknowledged();
                return save_failed_ ? 1 : 0;
            }
        }
    }
    save_failed_ |= !save_all();
    printf("done at step %lld\n", step_);
    fflush(stdout);
    return save_failed_ ? 1 : 0;
}

static int train_main(int argc, const char* const* argv) {
    Settings o;
    if (!o.parse(argc, argv, 5)) return 2;
    const int granule = o.flags & FC_STATES_BF16 ? TW16 : TW;
    if (o.batch <= 0 || o.batch % granule) { fprintf(stderr, "--batch must be a multiple of %d\n", granule); return 2; }
    CoreP cp = open_network(argv[1], o.batch, o.flags);
    if (!cp) return 1;
    Trainer t(*cp, o, argv[3], argv[4]);
    return t.run(argv[2]);
}

}  // namespace fg

using namespace fg;

// ================================================================================================ C-ABI
extern "C" {

int ft_main(int argc, const char* const* argv) {
    clear_error();
    if (argc >= 5 && argv[1] && !std::strcmp(argv[1], "--check")) return check_batch_file(argv[2], argv[3], argv[4]);
    if (argc < 5) {
        fprintf(stderr, "usage: flyguy_train NET PARAMS DATA_DIR OUT_PREFIX [options] | --check NET PARAMS BATCH\n");
        return 2;
    }
    return train_main(argc, argv);
}

int ft_draw(unsigned long long seed, const long long* sizes, int n_chunks, int B, int n_batches, int* out) {
    if (!sizes || !out || n_chunks <= 0 || B < 0 || n_batches < 0) return -1;
    std::vector<long long> s(sizes, sizes + n_chunks);
    long long total = 0;
    for (long long n : s) {
        if (n < 0 || n > 0x7fffffffLL) return -1;
        total += n;
    }
    if (total <= 0) return -1;
    std::mt19937_64 g(seed);
    for (int i = 0; i < n_batches; ++i) draw_samples(g, s, B, reinterpret_cast<int2*>(out) + (size_t)i * B);
    return 0;
}

void ft_lr(long long step, float lr, float lr_neuron, float lr_plug, float lr_min, double half_life, float* out) {
    if (out) rates_at(step, lr, lr_neuron, lr_plug, lr_min, half_life, out);
}

long long ft_chunk_samples(const char* path, int obs_dim, int n_act) {
    return path ? read_flyd(path, obs_dim, n_act, nullptr) : -1;
}

int ft_scan_order(const char* dir, int keep, char* out, int cap) {
    if (!dir || keep < 0 || (!out && cap > 0)) return -1;
    ChunkWatch w(dir, (size_t)keep);
    std::string names;
    int n = 0;
    for (const FileVersion& f : w.fresh()) {
        names += (n++ ? "\n" : "") + f.name();
    }
    if ((long long)names.size() + 1 > cap) return -1;
    std::memcpy(out, names.c_str(), names.size() + 1);
    return n;
}

void fd_gather16(const void* const* obs_tab, const void* const* lg_tab, const long long* n_tab, int n_chunks,
                 const int* sel, int B, int obs_dim, int n_act, float* obs, float* teacher, void* stream) {
    clear_error();
    if (B <= 0) return;
    if (!obs_tab || !lg_tab || !n_tab || !sel || !obs || !teacher || n_chunks <= 0 || obs_dim <= 0 || n_act <= 0) {
        set_error("fd_gather16: bad argument");
        return;
    }
    k_gather16<<<(unsigned)B, 256, 0, (hipStream_t)stream>>>((const unsigned short* const*)obs_tab,
                                                             (const unsigned short* const*)lg_tab, n_tab, n_chunks,
                                                             (const int2*)sel, obs_dim, n_act, obs, teacher);
    FG_CHECK(hipGetLastError(), );
}

void fd_unpack16(const void* st, int B, int obs_dim, int n_act, float* obs, float* teacher, void* stream) {
    clear_error();
    if (B <= 0) return;
    if (!st || !obs || !teacher || obs_dim <= 0 || n_act <= 0) { set_error("fd_unpack16: bad argument"); return; }
    k_unpack16<<<(unsigned)B, 256, 0, (hipStream_t)stream>>>((const unsigned short*)st, obs_dim, n_act, obs, teacher);
    FG_CHECK(hipGetLastError(), );
}

int fc_layers(void* h, int* sizes, int cap) {
    Core* c = (Core*)h;
    if (!c) { set_error("null handle"); return -1; }
    if (!sizes || cap < c->hops + 1) { set_error("fc_layers: capacity"); return -1; }
    for (int k = 0; k <= c->hops; ++k) sizes[k] = k ? c->hop[k - 1].rows : c->n_s;
    return c->hops + 1;
}

int fc_survey(void* h, const float* obs, const float* teacher, int B, int ema, float it, int reset) {
    Core* c = (Core*)h;
    if (!check_batch(c, B)) return -1;
    if (!obs || !teacher) { set_error("fc_survey: null pointer"); return -1; }
    if (reset && !survey_reset(*c)) return -1;
    return survey_batch(*c, obs, teacher, B, ema ? SET_EMA : SET_P, it) ? 0 : -1;
}

long long fc_survey_read(void* h, int* cnt, float* sq, double* stats) {
    Core* c = (Core*)h;
    if (!c) { set_error("null handle"); return -1; }
    Survey s;
    if (!survey_read(*c, s)) return -1;
    if (cnt) std::memcpy(cnt, s.cnt.data(), s.cnt.size() * 4);
    if (sq) std::memcpy(sq, s.sq.data(), s.sq.size() * 4);
    if (stats) { stats[0] = s.kl_sum; stats[1] = s.agree_sum; stats[2] = s.samples; }
    return c->rows_total;
}

int fc_revive(void* h, const float* obs, const float* teacher, int B, int batches, float target, unsigned long long seed,
              long long step, char* report, int cap) {
    Core* c = (Core*)h;
    if (!check_batch(c, B)) return -1;
    if (!obs || !teacher || batches <= 0) { set_error("fc_revive: bad argument"); return -1; }
    std::string rep;
    const int n = revive(*c, obs, teacher, B, batches, target, seed, step, rep);
    if (n >= 0 && report && cap > 0) {
        const size_t k = std::min(rep.size(), (size_t)cap - 1);
        std::memcpy(report, rep.data(), k);
        report[k] = 0;
    }
    return n;
}

}  // extern "C"
