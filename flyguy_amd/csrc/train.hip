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
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <filesystem>
#include <map>
#include <memory>
#include <mutex>
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

// ================================================================================================ host helpers
static bool get_dev(Core& c, const float* d, std::vector<float>& v, size_t n) {
    v.resize(n);
    if (n && hipMemcpyAsync(v.data(), d, n * 4, hipMemcpyDeviceToHost, c.st) != hipSuccess) return false;
    return hipStreamSynchronize(c.st) == hipSuccess;
}
static bool put_dev(Core& c, float* d, const std::vector<float>& v) {
    c.weights_written(SET_P);                  // (it may write the weights or the running average)
    c.weights_written(SET_EMA);
    if (!v.empty() && hipMemcpyAsync(d, v.data(), v.size() * 4, hipMemcpyHostToDevice, c.st) != hipSuccess) return false;
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

struct Survey {
    std::vector<int> cnt;
    std::vector<float> sq;
    float kl_sum = 0, agree_sum = 0;
    double kl = 0, agree = 0, samples = 0;        // per sample
};

static bool survey_read(Core& c, Survey& s) {
    if (!ensure_survey(c)) return false;
    s.cnt.resize((size_t)c.rows_total);
    s.sq.resize((size_t)c.rows_total);
    float st[4] = {0, 0, 0, 0};
    FG_CHECK(hipMemcpyAsync(s.cnt.data(), c.scnt, s.cnt.size() * 4, hipMemcpyDeviceToHost, c.st), false);
    FG_CHECK(hipMemcpyAsync(s.sq.data(), c.ssq, s.sq.size() * 4, hipMemcpyDeviceToHost, c.st), false);
    FG_CHECK(hipMemcpyAsync(st, c.sstats, 16, hipMemcpyDeviceToHost, c.st), false);
    FG_CHECK(hipStreamSynchronize(c.st), false);
    s.samples = c.s_samples;
    s.kl_sum = st[0];
    s.agree_sum = st[1];
    s.kl = s.samples > 0 ? st[0] / s.samples : 0;
    s.agree = s.samples > 0 ? st[1] / s.samples : 0;
    return true;
}

// a survey over `batches` staged batches of B samples (obs [batches * B][obs_dim]) at temperature 1
static bool survey_staged(Core& c, const float* obs, const float* tl, int B, int batches, int set, Survey& s) {
    if (!survey_reset(c)) return false;
    for (int i = 0; i < batches; ++i)
        if (!survey_batch(c, obs + (size_t)i * B * c.obs_dim, tl + (size_t)i * B * c.n_act, B, set, 1.f)) return false;
    return survey_read(c, s);
}

// per neuron: times it fired in any hop past the sensory layer; play = in such a hop; sens = a sensory neuron
// (flyguy_train.cu:456-461)
static void per_neuron(const Core& c, const Survey& s, std::vector<long long>& fired, std::vector<char>& play,
                       std::vector<char>& sens) {
    fired.assign((size_t)c.n_neurons, 0);
    play.assign((size_t)c.n_neurons, 0);
    sens.assign((size_t)c.n_neurons, 0);
    for (int g : c.h_n0) sens[g] = 1;
    size_t off = (size_t)c.n_s;
    for (auto& d : c.hop) {
        for (int t = 0; t < d.rows; ++t) {
            const int g = d.h_nid[t];
            play[g] = 1;
            fired[g] += s.cnt[off + t];
        }
        off += d.rows;
    }
}

// " f0 f1 ..." firing share per layer, and the silent / in-play neuron counts (flyguy_train.cu:462-471)
static std::string firing_line(const Core& c, const Survey& s, int& silent, int& in_play) {
    std::vector<long long> fired;
    std::vector<char> play, sens;
    per_neuron(c, s, fired, play, sens);
    silent = in_play = 0;
    for (int g = 0; g < c.n_neurons; ++g)
        if (play[g] && !sens[g]) {
            ++in_play;
            if (!fired[g]) ++silent;
        }
    std::string out;
    size_t off = 0;
    char b[32];
    for (int k = 0; k <= c.hops; ++k) {
        const int rows = k ? c.hop[k - 1].rows : c.n_s;
        double n = 0;
        for (int t = 0; t < rows; ++t) n += s.cnt[off + t];
        snprintf(b, sizeof b, " %.3f", n / (rows * s.samples));
        out += b;
        off += rows;
    }
    return out;
}

static float median_positive(const std::vector<float>& v) {      // flyguy_train.cu:472-478
    std::vector<float> p;
    p.reserve(v.size());
    for (float x : v)
        if (x > 0.f) p.push_back(x);
    if (p.empty()) return 0.f;
    std::nth_element(p.begin(), p.begin() + p.size() / 2, p.end());
    return p[p.size() / 2];
}

// ================================================================================================ revive
// flyguy_train.cu:486-551, over staged batches (every survey of one revive sees the same samples, as the reference's
// surveys do by drawing with the same seed)
static int revive(Core& c, const float* obs, const float* tl, int B, int batches, float target, unsigned long long seed,
                  long long step, std::string& report) {
    const int N = c.n_neurons, K = c.hops;
    char buf[512];
    Survey s0;
    if (!survey_staged(c, obs, tl, B, batches, SET_P, s0)) return -1;
    std::vector<long long> fired;
    std::vector<char> play, sens, dead((size_t)N, 0);
    per_neuron(c, s0, fired, play, sens);
    int n_dead = 0, n_play = 0;
    for (int g = 0; g < N; ++g)
        if (play[g] && !sens[g]) {
            ++n_play;
            if (!fired[g]) { dead[g] = 1; ++n_dead; }
        }
    if (!n_dead) {
        snprintf(buf, sizeof buf, "revive step %lld | no silent neuron among %d over %.0f samples", step, n_play, s0.samples);
        report = buf;
        return 0;
    }
    std::vector<float> W, gain, theta, ow;
    if (!get_dev(c, c.arr(SET_P, 0), W, c.psize[0]) || !get_dev(c, c.arr(SET_P, 1), gain, N) ||
        !get_dev(c, c.arr(SET_P, 2), theta, N) || !get_dev(c, c.arr(SET_P, 5), ow, c.psize[5])) {
        set_error("revive: copy from the device");
        return -1;
    }
    std::vector<char> mark((size_t)c.n_w, 0);     // 1: into a silent neuron (new sign), 2: from a silent one into a live one
    std::mt19937_64 r(seed * 7919ULL + 17);
    long long n_in = 0, n_out = 0;
    for (int k = 0; k < K; ++k) {
        const HopD& h = c.hop[k];
        const std::vector<int>& below = k ? c.hop[k - 1].h_nid : c.h_n0;
        for (int t = 0; t < h.rows; ++t) {
            const bool dpost = dead[h.h_nid[t]];
            for (int e = h.h_crow[t]; e < h.h_crow[t + 1]; ++e) {
                const int wi = h.h_widx[e];
                if (mark[wi]) continue;
                if (dpost) {
                    W[wi] = std::max(std::fabs(W[wi]), 1e-4f) * ((r() & 1) ? 1.f : -1.f);
                    mark[wi] = 1;
                    ++n_in;
                } else if (dead[below[h.h_col[e]]]) {
                    W[wi] = 0.f;
                    mark[wi] = 2;
                    ++n_out;
                }
            }
        }
    }
    for (int g = 0; g < N; ++g)
        if (dead[g]) { gain[g] = 1.f; theta[g] = -4.f; }
    const HopD& top = c.hop[K - 1];
    std::vector<char> dcol((size_t)c.n_dn, 0);
    int n_dn_dead = 0;
    for (int j = 0; j < c.n_dn; ++j)
        if (dead[top.h_nid[c.h_dn[j]]]) {
            dcol[j] = 1;
            ++n_dn_dead;
            for (int a = 0; a < c.n_act; ++a) ow[(size_t)a * c.n_dn + j] = 0.f;
        }
    if (!put_dev(c, c.arr(SET_P, 0), W) || !put_dev(c, c.arr(SET_P, 1), gain) || !put_dev(c, c.arr(SET_P, 2), theta) ||
        !put_dev(c, c.arr(SET_P, 5), ow)) {
        set_error("revive: copy to the device");
        return -1;
    }
    for (int pass = 0; pass < 3; ++pass) {         // hop after hop the revived neurons' inputs come to the target size
        Survey s;
        if (!survey_staged(c, obs, tl, B, batches, SET_P, s)) return -1;
        std::vector<float> rms((size_t)N, 0.f);
        size_t off = (size_t)c.n_s;
        for (auto& h : c.hop) {
            for (int t = 0; t < h.rows; ++t) {
                const int g = h.h_nid[t];
                rms[g] = std::max(rms[g], (float)std::sqrt(s.sq[off + t] / s.samples));
            }
            off += h.rows;
        }
        std::vector<char> done((size_t)c.n_w, 0);
        for (auto& h : c.hop)
            for (int t = 0; t < h.rows; ++t) {
                const int g = h.h_nid[t];
                if (!dead[g] || rms[g] <= 0.f) continue;
                const float sc = std::min(200.f, std::max(0.02f, target / rms[g]));
                for (int e = h.h_crow[t]; e < h.h_crow[t + 1]; ++e) {
                    const int wi = h.h_widx[e];
                    if (!done[wi]) { W[wi] *= sc; done[wi] = 1; }
                }
            }
        if (!put_dev(c, c.arr(SET_P, 0), W)) { set_error("revive: copy to the device"); return -1; }
    }
    Survey s1;
    if (!survey_staged(c, obs, tl, B, batches, SET_P, s1)) return -1;
    per_neuron(c, s1, fired, play, sens);
    int still = 0;
    for (int g = 0; g < N; ++g)
        if (dead[g] && !fired[g]) ++still;
    {   // the running average and Adam follow
        std::vector<float> e, m, v;
        if (!get_dev(c, c.arr(SET_EMA, 0), e, c.psize[0]) || !get_dev(c, c.arr(SET_M, 0), m, c.psize[0]) ||
            !get_dev(c, c.arr(SET_V, 0), v, c.psize[0])) { set_error("revive: copy from the device"); return -1; }
        const float fill = median_positive(v);
        for (int i = 0; i < c.n_w; ++i)
            if (mark[i]) { e[i] = W[i]; m[i] = 0.f; v[i] = fill; }
        if (!put_dev(c, c.arr(SET_EMA, 0), e) || !put_dev(c, c.arr(SET_M, 0), m) || !put_dev(c, c.arr(SET_V, 0), v)) {
            set_error("revive: copy to the device");
            return -1;
        }
        for (int p = 1; p <= 2; ++p) {
            std::vector<float> ee, mm, vv;
            if (!get_dev(c, c.arr(SET_EMA, p), ee, N) || !get_dev(c, c.arr(SET_M, p), mm, N) ||
                !get_dev(c, c.arr(SET_V, p), vv, N)) { set_error("revive: copy from the device"); return -1; }
            const float f2 = median_positive(vv);
            for (int g = 0; g < N; ++g)
                if (dead[g]) { ee[g] = p == 1 ? 1.f : -4.f; mm[g] = 0.f; vv[g] = f2; }
            if (!put_dev(c, c.arr(SET_EMA, p), ee) || !put_dev(c, c.arr(SET_M, p), mm) || !put_dev(c, c.arr(SET_V, p), vv)) {
                set_error("revive: copy to the device");
                return -1;
            }
        }
        std::vector<float> eo, mo;
        if (!get_dev(c, c.arr(SET_EMA, 5), eo, c.psize[5]) || !get_dev(c, c.arr(SET_M, 5), mo, c.psize[5])) {
            set_error("revive: copy from the device");
            return -1;
        }
        for (int j = 0; j < c.n_dn; ++j)
            if (dcol[j])
                for (int a = 0; a < c.n_act; ++a) { eo[(size_t)a * c.n_dn + j] = 0.f; mo[(size_t)a * c.n_dn + j] = 0.f; }
        if (!put_dev(c, c.arr(SET_EMA, 5), eo) || !put_dev(c, c.arr(SET_M, 5), mo)) {
            set_error("revive: copy to the device");
            return -1;
        }
    }
    snprintf(buf, sizeof buf,
             "revive step %lld | %d of %d neurons past the sensory layer silent over %.0f samples | new sign for %lld "
             "incoming strengths, zero for %lld outgoing and for %d descending neurons' action weights | %d still silent "
             "| kl %.5f -> %.5f (must be equal)",
             step, n_dead, n_play, s0.samples, n_in, n_out, n_dn_dead, still, s0.kl, s1.kl);
    report = buf;
    return n_dead;
}

// ================================================================================================ data
// flyguy_train.cu:412-424: B samples, each uniform over the concatenated chunks -> {chunk, sample}
static void draw(std::mt19937_64& r, const std::vector<long long>& sizes, int B, int2* out) {
    long long total = 0;
    for (long long n : sizes) total += n;
    std::uniform_int_distribution<long long> u(0, total - 1);
    for (int i = 0; i < B; ++i) {
        long long s = u(r);
        size_t ch = 0;
        while (s >= sizes[ch]) { s -= sizes[ch]; ++ch; }
        out[i] = make_int2((int)ch, (int)s);
    }
}

struct Chunk {
    long long n = 0;
    std::string name;
    fs::file_time_type mtime{};
    std::vector<unsigned short> obs, lg;           // host copies, dropped once on the device
    int slot = -1;                                 // place in the device table (-1: not on the device)
};
typedef std::shared_ptr<Chunk> ChunkP;

// flyguy_train.cu:372-384
static ChunkP read_chunk(const std::string& path, int od, int na) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return nullptr;
    char magic[4];
    long long n = 0;
    int fod = 0, fna = 0;
    if (fread(magic, 1, 4, f) != 4 || std::memcmp(magic, "FLYD", 4) || fread(&n, 8, 1, f) != 1 || fread(&fod, 4, 1, f) != 1 ||
        fread(&fna, 4, 1, f) != 1 || fod != od || fna != na || n <= 0 || n > 0x7fffffffLL) {
        fclose(f);
        return nullptr;
    }
    auto b = std::make_shared<Chunk>();
    b->obs.resize((size_t)n * od);
    b->lg.resize((size_t)n * na);
    const bool ok = fread(b->obs.data(), 2, b->obs.size(), f) == b->obs.size() && fread(b->lg.data(), 2, b->lg.size(), f) == b->lg.size();
    fclose(f);
    if (!ok) return nullptr;
    b->n = n;
    b->name = fs::path(path).filename().string();
    return b;
}

// flyguy_train.cu:385-411: a thread reads every chunk file that is new or rewritten since it was read (of several
// only the newest `keep`), not more than one chunk ahead of the trainer
struct Loader {
    std::mutex mu;
    std::deque<ChunkP> pending;
    std::atomic<bool> quit{false};
    std::map<std::string, fs::file_time_type> known;
    std::string dir;
    int od = 0, na = 0;
    size_t keep = 3;

    std::vector<std::pair<fs::file_time_type, std::string>> select() {
        std::vector<std::pair<fs::file_time_type, std::string>> files;
        std::error_code ec;
        for (auto& e : fs::directory_iterator(dir, ec)) {
            const auto p = e.path().filename().string();
            std::error_code e2;
            const auto mt = fs::last_write_time(e.path(), e2);
            if (e2 || p.rfind("chunk_", 0) != 0 || e.path().extension() != ".bin") continue;
            auto k = known.find(p);
            if (k == known.end() || k->second != mt) files.push_back({mt, e.path().string()});
        }
        std::sort(files.begin(), files.end());
        while (files.size() > keep) {
            known[fs::path(files.front().second).filename().string()] = files.front().first;
            files.erase(files.begin());
        }
        return files;
    }
    int scan(bool wait) {
        int got = 0;
        for (auto& fm : select()) {
            while (wait && !quit) {
                {
                    std::lock_guard<std::mutex> g(mu);
                    if (pending.empty()) break;
                }
                std::this_thread::sleep_for(std::chrono::milliseconds(200));
            }
            if (quit) break;
            ChunkP b = read_chunk(fm.second, od, na);
            if (!b) continue;                      // (being replaced right now: the next scan has it)
            b->mtime = fm.first;
            known[b->name] = fm.first;
            {
                std::lock_guard<std::mutex> g(mu);
                pending.push_back(b);
            }
            ++got;
        }
        return got;
    }
};

// The chunks in device memory: a table of slots (binary16 obs / logits and sample count per slot) that the gather
// kernel reads; a batch names its samples by (slot, sample).
struct DevRing {
    int cap = 0;
    std::vector<unsigned short*> h_obs, h_lg;
    std::vector<long long> h_n;
    unsigned short **d_obs = nullptr, **d_lg = nullptr;
    long long* d_n = nullptr;
};

static bool ring_init(Core& c, DevRing& r, int cap) {
    r.cap = cap;
    r.h_obs.assign(cap, nullptr);
    r.h_lg.assign(cap, nullptr);
    r.h_n.assign(cap, 0);
    r.d_obs = reinterpret_cast<unsigned short**>(dalloc<void*>(c, cap));
    r.d_lg = reinterpret_cast<unsigned short**>(dalloc<void*>(c, cap));
    r.d_n = dalloc<long long>(c, cap);
    return r.d_obs && r.d_lg && r.d_n;
}
static bool ring_table(Core& c, DevRing& r) {
    FG_CHECK(hipStreamSynchronize(c.st), false);
    FG_CHECK(hipMemcpy(r.d_obs, r.h_obs.data(), r.cap * sizeof(void*), hipMemcpyHostToDevice), false);
    FG_CHECK(hipMemcpy(r.d_lg, r.h_lg.data(), r.cap * sizeof(void*), hipMemcpyHostToDevice), false);
    FG_CHECK(hipMemcpy(r.d_n, r.h_n.data(), r.cap * sizeof(long long), hipMemcpyHostToDevice), false);
    return true;
}
static bool ring_put(Core& c, DevRing& r, Chunk& b) {
    if (b.slot >= 0) return true;
    int s = 0;
    while (s < r.cap && r.h_obs[s]) ++s;
    if (s == r.cap) { set_error("chunk table full"); return false; }
    void *o = nullptr, *l = nullptr;
    if (hipMalloc(&o, b.obs.size() * 2) != hipSuccess || hipMalloc(&l, b.lg.size() * 2) != hipSuccess) {
        if (o) (void)hipFree(o);
        set_error("out of device memory for a chunk of " + std::to_string(b.n) + " samples");
        return false;
    }
    FG_CHECK(hipMemcpy(o, b.obs.data(), b.obs.size() * 2, hipMemcpyHostToDevice), false);
    FG_CHECK(hipMemcpy(l, b.lg.data(), b.lg.size() * 2, hipMemcpyHostToDevice), false);
    r.h_obs[s] = (unsigned short*)o;
    r.h_lg[s] = (unsigned short*)l;
    r.h_n[s] = b.n;
    b.slot = s;
    std::vector<unsigned short>().swap(b.obs);
    std::vector<unsigned short>().swap(b.lg);
    return ring_table(c, r);
}
static void ring_drop(Core& c, DevRing& r, Chunk& b) {
    if (b.slot < 0) return;
    (void)hipStreamSynchronize(c.st);              // (kernels in flight may still read it)
    (void)hipFree(r.h_obs[b.slot]);
    (void)hipFree(r.h_lg[b.slot]);
    r.h_obs[b.slot] = r.h_lg[b.slot] = nullptr;
    r.h_n[b.slot] = 0;
    b.slot = -1;
    ring_table(c, r);
}

// Drawn batches on their way to the device: pinned (chunk slot, sample) pairs, two buffers so the host draws the
// next batch while the last copy runs; staged float32 obs / teacher rows for up to `rows` samples.
struct Feed {
    int rows = 0;
    int2* pin[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool used[2] = {false, false};
    int flip = 0;
    int2* d_sel = nullptr;
    float *obs = nullptr, *tl = nullptr;
};

static bool feed_init(Core& c, Feed& f, int rows) {
    f.rows = rows;
    for (int k = 0; k < 2; ++k) {
        FG_CHECK(hipHostMalloc((void**)&f.pin[k], (size_t)rows * sizeof(int2), hipHostMallocDefault), false);
        FG_CHECK(hipEventCreateWithFlags(&f.done[k], hipEventDisableTiming), false);
    }
    f.d_sel = dalloc<int2>(c, rows);
    f.obs = dalloc<float>(c, (size_t)rows * c.obs_dim);
    f.tl = dalloc<float>(c, (size_t)rows * c.n_act);
    return f.d_sel && f.obs && f.tl;
}
static void feed_free(Feed& f) {
    for (int k = 0; k < 2; ++k) {
        if (f.done[k]) {
            if (f.used[k]) (void)hipEventSynchronize(f.done[k]);
            (void)hipEventDestroy(f.done[k]);
        }
        if (f.pin[k]) (void)hipHostFree(f.pin[k]);
    }
}

// `batches` batches of B drawn from src with r, gathered into the staged rows
static bool draw_batches(Core& c, DevRing& ring, Feed& f, const std::vector<ChunkP>& src, std::mt19937_64& r, int B,
                         int batches) {
    const int n = B * batches;
    if (n > f.rows) { set_error("staging too small"); return false; }
    std::vector<long long> sizes;
    for (auto& b : src) sizes.push_back(b->n);
    const int k = f.flip;
    f.flip ^= 1;
    if (f.used[k]) FG_CHECK(hipEventSynchronize(f.done[k]), false);   // the copy that last read this buffer is done
    for (int i = 0; i < batches; ++i) draw(r, sizes, B, f.pin[k] + (size_t)i * B);
    for (int i = 0; i < n; ++i) f.pin[k][i].x = src[f.pin[k][i].x]->slot;
    FG_CHECK(hipMemcpyAsync(f.d_sel, f.pin[k], (size_t)n * sizeof(int2), hipMemcpyHostToDevice, c.st), false);
    FG_CHECK(hipEventRecord(f.done[k], c.st), false);
    f.used[k] = true;
    k_gather16<<<(unsigned)n, 256, 0, c.st>>>(ring.d_obs, ring.d_lg, ring.d_n, ring.cap, f.d_sel, c.obs_dim, c.n_act,
                                              f.obs, f.tl);
    FG_CHECK(hipGetLastError(), false);
    return true;
}

// ================================================================================================ parameter files
static const char* kArrName[7] = {"W", "gain", "theta", "in_w", "in_b", "out_w", "out_b"};

// flyguy_train.cu:258-274: weights from path, the running average from ema_path (else a copy); returns the step
static bool load_params(Core& c, const std::string& path, const std::string& ema_path, long long& step) {
    for (int which = 0; which < 2; ++which) {
        FILE* f = fopen(which && !ema_path.empty() ? ema_path.c_str() : path.c_str(), "rb");
        if (!f && which) f = fopen(path.c_str(), "rb");
        if (!f) { fprintf(stderr, "cannot open %s\n", path.c_str()); return false; }
        char magic[4];
        long long st = 0;
        if (fread(magic, 1, 4, f) != 4 || std::memcmp(magic, "FLYP", 4) || fread(&st, 8, 1, f) != 1) {
            fclose(f);
            fprintf(stderr, "%s: not a FLYP parameter file\n", path.c_str());
            return false;
        }
        if (!which) step = st;
        for (int i = 0; i < 7; ++i) {
            std::vector<float> v((size_t)c.psize[i]);
            if (fread(v.data(), 4, v.size(), f) != v.size()) {
                fclose(f);
                fprintf(stderr, "short params file\n");
                return false;
            }
            if (!put_dev(c, c.arr(which ? SET_EMA : SET_P, i), v)) { fclose(f); return false; }
        }
        fclose(f);
    }
    return true;
}
static bool finish_file(FILE* f, const std::string& tmp, const std::string& path) {
    const bool ok = fflush(f) == 0;
    fclose(f);
    std::error_code ec;
    fs::rename(tmp, path, ec);
    if (ec) {
        fs::remove(path, ec);
        fs::rename(tmp, path, ec);
    }
    return ok && !ec;
}
static bool save_params(Core& c, const std::string& path, long long step, bool ema) {
    const std::string tmp = path + ".tmp";
    FILE* f = fopen(tmp.c_str(), "wb");
    if (!f) return false;
    fwrite("FLYP", 1, 4, f);
    fwrite(&step, 8, 1, f);
    for (int i = 0; i < 7; ++i) {
        std::vector<float> v;
        if (!get_dev(c, c.arr(ema ? SET_EMA : SET_P, i), v, c.psize[i])) { fclose(f); return false; }
        fwrite(v.data(), 4, v.size(), f);
    }
    return finish_file(f, tmp, path);
}
static bool save_opt(Core& c, const std::string& path, long long step, long long adam_t) {     // :288-294
    const std::string tmp = path + ".tmp";
    FILE* f = fopen(tmp.c_str(), "wb");
    if (!f) return false;
    fwrite("FLYO", 1, 4, f);
    fwrite(&step, 8, 1, f);
    fwrite(&adam_t, 8, 1, f);
    for (int i = 0; i < 7; ++i) {
        std::vector<float> m, v;
        if (!get_dev(c, c.arr(SET_M, i), m, c.psize[i]) || !get_dev(c, c.arr(SET_V, i), v, c.psize[i])) { fclose(f); return false; }
        fwrite(m.data(), 4, m.size(), f);
        fwrite(v.data(), 4, v.size(), f);
    }
    return finish_file(f, tmp, path);
}
// :295-307: only a file of this very step restores Adam's state
static bool load_opt(Core& c, const std::string& path, long long step, long long& adam_t) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return false;
    char magic[4];
    long long st = -1, at = 0;
    bool ok = fread(magic, 1, 4, f) == 4 && !std::memcmp(magic, "FLYO", 4) && fread(&st, 8, 1, f) == 1 &&
              fread(&at, 8, 1, f) == 1 && st == step;
    std::vector<std::vector<float>> m(7), v(7);
    for (int i = 0; ok && i < 7; ++i) {
        m[i].resize((size_t)c.psize[i]);
        v[i].resize((size_t)c.psize[i]);
        ok = fread(m[i].data(), 4, m[i].size(), f) == m[i].size() && fread(v[i].data(), 4, v[i].size(), f) == v[i].size();
    }
    fclose(f);
    if (!ok) return false;
    for (int i = 0; i < 7; ++i)
        if (!put_dev(c, c.arr(SET_M, i), m[i]) || !put_dev(c, c.arr(SET_V, i), v[i])) return false;
    adam_t = at;
    return true;
}

static std::vector<unsigned char> read_file(const std::string& path) {
    std::vector<unsigned char> buf;
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return buf;
    unsigned char tmp[1 << 16];
    size_t k;
    while ((k = fread(tmp, 1, sizeof tmp, f)) > 0) buf.insert(buf.end(), tmp, tmp + k);
    fclose(f);
    return buf;
}

static double now() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// the learning rates of one step (flyguy_train.cu:764-769)
static void lr_of(long long step, float lr, float lr_neuron, float lr_plug, float lr_min, double half_life, float out[3]) {
    const float sched = (float)std::pow(0.5, (double)step / half_life);
    const float base[3] = {lr, lr_neuron, lr_plug};
    for (int g = 0; g < 3; ++g) out[g] = std::max(lr_min * base[g] / lr, base[g] * sched);
}

// one forward + loss + backward on the staged batch; loss sums ADDED to stats
static bool fwd_bwd(Core& c, const float* obs, const float* tl, int B, float it, float* stats) {
    FG_CHECK(launch_fill(c.arr(SET_G, 0), 0.f, c.PT, c.st), false);
    if (!forward(c, obs, B, c.lg, SET_P)) return false;
    FG_CHECK(launch_loss(c.lg, tl, c.dl, c.stats_part, stats, c.n_act, B, it, c.st, true), false);
    return backward(c, c.dl, B, true);                      // (the gradient was cleared above)
}

typedef std::unique_ptr<Core, void (*)(Core*)> CoreP;

static CoreP open_net(const std::string& path, int B, int flags = 0) {
    auto bytes = read_file(path);
    if (bytes.empty()) {
        fprintf(stderr, "cannot open %s\n", path.c_str());
        return CoreP(nullptr, release);
    }
    CoreP c(build(bytes.data(), (long long)bytes.size(), B, flags), release);
    if (!c) fprintf(stderr, "%s: %s\n", path.c_str(), last_error());
    return c;
}

// ---- --check NET PARAMS BATCH (flyguy_train.cu:632-653)
static int check_main(const char* net_path, const char* params_path, const char* batch_path) {
    FILE* f = fopen(batch_path, "rb");
    if (!f) { fprintf(stderr, "cannot open %s\n", batch_path); return 1; }
    char magic[4];
    int B = 0;
    if (fread(magic, 1, 4, f) != 4 || fread(&B, 4, 1, f) != 1 || B <= 0) {
        fclose(f);
        fprintf(stderr, "%s: not a batch file\n", batch_path);
        return 1;
    }
    if (B % TW) {
        fclose(f);
        fprintf(stderr, "%s: %d samples; the batch must be a multiple of 32\n", batch_path, B);
        return 2;
    }
    CoreP c = open_net(net_path, B);
    if (!c) { fclose(f); return 1; }
    long long step = 0;
    if (!load_params(*c, params_path, "", step)) { fclose(f); return 1; }
    std::vector<float> x((size_t)B * c->obs_dim), t((size_t)B * c->n_act);
    const bool ok = fread(x.data(), 4, x.size(), f) == x.size() && fread(t.data(), 4, t.size(), f) == t.size();
    fclose(f);
    if (!ok) { fprintf(stderr, "%s: short batch file\n", batch_path); return 1; }
    float* dx = dalloc<float>(*c, x.size());
    float* dt = dalloc<float>(*c, t.size());
    if (!dx || !dt || !put_dev(*c, dx, x) || !put_dev(*c, dt, t)) { fprintf(stderr, "%s\n", last_error()); return 1; }
    FG_CHECK(launch_fill(c->stats, 0.f, 4, c->st), 1);
    if (!fwd_bwd(*c, dx, dt, B, 1.f, c->stats)) { fprintf(stderr, "%s\n", last_error()); return 1; }
    std::vector<float> st, lg;
    if (!get_dev(*c, c->stats, st, 2) || !get_dev(*c, c->lg, lg, (size_t)c->n_act)) { fprintf(stderr, "copy\n"); return 1; }
    printf("native: loss %.6f agree %.4f\n   logits[0][:5]", st[0] / B, st[1] / B);
    for (int a = 0; a < 5 && a < c->n_act; ++a) printf(" %.6f", lg[a]);
    printf("\n");
    for (int i = 0; i < 7; ++i) {
        std::vector<float> g;
        if (!get_dev(*c, c->arr(SET_G, i), g, c->psize[i])) { fprintf(stderr, "copy\n"); return 1; }
        double ss = 0, s = 0;
        for (float v : g) { ss += (double)v * v; s += v; }
        printf("   grad %-6s norm %.6e sum %+.6e\n", kArrName[i], std::sqrt(ss), s);
    }
    fflush(stdout);
    return 0;
}

// ---- the trainer (flyguy_train.cu:654-787)
static int train_main(int argc, const char* const* argv) {
    int B = 512, log_every = 100, eval_batches = 16, revive_batches = 4, revive_first = 0, ring_k = 3, holdout = 0;
    long long max_steps = 0, revive_every = 0, eval_every = 0;
    double save_sec = 120, half_life = 20000;
    float lr = 3e-4f, lr_neuron = 1e-4f, lr_plug = 3e-4f, lr_min = 3e-5f, ema = 0.999f, clip = 0.f, temp = 1.f,
          revive_target = 0.4f;
    double max_reuse = -1;
    int flags = 0;                                      // --bf16 1: the bfloat16-state core (FC_STATES_BF16)
    for (int i = 5; i + 1 < argc; i += 2) {
        const std::string a = argv[i];
        const double v = atof(argv[i + 1]);
        if (a == "--batch") B = (int)v;
        else if (a == "--lr") lr = (float)v;
        else if (a == "--lr-neuron") lr_neuron = (float)v;
        else if (a == "--lr-plug") lr_plug = (float)v;
        else if (a == "--lr-min") lr_min = (float)v;
        else if (a == "--half-life") half_life = v;
        else if (a == "--ema") ema = (float)v;
        else if (a == "--log") log_every = (int)v;
        else if (a == "--save-sec") save_sec = v;
        else if (a == "--steps") max_steps = (long long)v;
        else if (a == "--clip") clip = (float)v;
        else if (a == "--temp") temp = (float)v;
        else if (a == "--eval-batches") eval_batches = (int)v;
        else if (a == "--eval-every") eval_every = (long long)v;
        else if (a == "--revive-every") revive_every = (long long)v;
        else if (a == "--revive-batches") revive_batches = (int)v;
        else if (a == "--revive-target") revive_target = (float)v;
        else if (a == "--revive-first") revive_first = (int)v;
        else if (a == "--max-reuse") max_reuse = v;
        else if (a == "--ring") ring_k = std::max(1, (int)v);
        else if (a == "--holdout") holdout = (int)v;
        else if (a == "--passes") { }                  // (of the one-chunk-at-a-time trainer: ignored)
        else if (a == "--bf16") flags = v != 0 ? FC_STATES_BF16 : 0;
        else { fprintf(stderr, "unknown option %s\n", a.c_str()); return 2; }
    }
    const int bq = flags & FC_STATES_BF16 ? TW16 : TW;
    if (B <= 0 || B % bq) { fprintf(stderr, "--batch must be a multiple of %d\n", bq); return 2; }
    const std::string data = argv[3], out = argv[4];
    CoreP cp = open_net(argv[1], B, flags);
    if (!cp) return 1;
    Core& c = *cp;
    // a restart from this run's own save keeps the running average and the optimiser state
    const bool own = fs::path(argv[2]).lexically_normal() == fs::path(out + ".bin").lexically_normal();
    const std::string ema_file = out + ".ema.bin";
    long long step = 0, ran = 0;
    if (!load_params(c, argv[2], own && fs::exists(ema_file) ? ema_file : "", step)) return 1;
    long long adam_t = 0;
    const bool opt = own && load_opt(c, out + ".opt.bin", step, adam_t);
    c.adam_t = adam_t;
    const int stage_batches = std::max(1, revive_every > 0 ? revive_batches : 1);
    Feed feed;
    DevRing dring;
    if (!feed_init(c, feed, B * stage_batches) || !ring_init(c, dring, ring_k + 2)) {
        fprintf(stderr, "%s\n", last_error());
        feed_free(feed);
        return 1;
    }
    std::mt19937_64 rng(12345 + step);
    const float it = 1.f / temp;
    printf("flyguy native trainer: %d neurons, %d strengths in play, %d hops, batch %d, lr %g (neurons %g, plugs %g), "
           "teacher temperature %g, ring of %d chunks, start step %lld%s%s\n",
           c.n_neurons, c.n_w, c.hops, B, lr, lr_neuron, lr_plug, temp, ring_k, step, opt ? ", optimiser state restored" : "",
           c.prec ? ", bfloat16 states" : "");
    fflush(stdout);

    Loader ld;
    ld.dir = data;
    ld.od = c.obs_dim;
    ld.na = c.n_act;
    ld.keep = (size_t)ring_k + (holdout ? 1 : 0);
    while (!ld.scan(false)) {
        printf("waiting for data in %s\n", data.c_str());
        fflush(stdout);
        std::this_thread::sleep_for(std::chrono::seconds(20));
    }
    int rc = 0;
    std::vector<ChunkP> ring;
    ChunkP held;
    bool failed = false;
    auto fail = [&](const char* what) {
        fprintf(stderr, "%s: %s\n", what, last_error());
        fflush(stderr);
        failed = true;
    };
    auto eval_on = [&](const ChunkP& b, unsigned long long seed, const char* what) {
        if (eval_batches <= 0 || failed) return;
        std::vector<ChunkP> one{b};
        Survey sv[2];
        for (int pass = 0; pass < 2; ++pass) {      // the running average (what would be installed), then the raw weights
            std::mt19937_64 r(seed);
            if (!survey_reset(c)) return fail("eval");
            for (int i = 0; i < eval_batches; ++i) {
                if (!draw_batches(c, dring, feed, one, r, B, 1) || !survey_batch(c, feed.obs, feed.tl, B, pass ? SET_P : SET_EMA, 1.f))
                    return fail("eval");
            }
            if (!survey_read(c, sv[pass])) return fail("eval");
        }
        int silent = 0, in_play = 0;
        const std::string fb = firing_line(c, sv[0], silent, in_play);
        printf("eval step %lld | kl %.4f agree %.4f | raw kl %.4f agree %.4f | firing%s | silent %d of %d | %s %s\n", step,
               sv[0].kl, sv[0].agree, sv[1].kl, sv[1].agree, fb.c_str(), silent, in_play, b->name.c_str(), what);
        fflush(stdout);
    };
    auto into_ring = [&](const ChunkP& b) {
        for (auto& o : ring)
            if (o->name == b->name && o != b) ring_drop(c, dring, *o);
        ring.erase(std::remove_if(ring.begin(), ring.end(), [&](const ChunkP& o) { return o->name == b->name; }), ring.end());
        ring.push_back(b);
        std::sort(ring.begin(), ring.end(), [](const ChunkP& x, const ChunkP& y) { return x->mtime < y->mtime; });
        while (ring.size() > (size_t)ring_k) {
            ring_drop(c, dring, *ring.front());
            ring.erase(ring.begin());
        }
    };
    {
        std::lock_guard<std::mutex> g(ld.mu);
        if (holdout && ld.pending.size() > 1) { held = ld.pending.back(); ld.pending.pop_back(); }
        for (auto& b : ld.pending) {
            if (!ring_put(c, dring, *b)) { fail("chunk upload"); break; }
            into_ring(b);
        }
        ld.pending.clear();
    }
    if (held && !ring_put(c, dring, *held)) fail("chunk upload");
    if (!failed) {
        if (held) eval_on(held, 4242, "held out");
        else eval_on(ring.back(), 4242, "at the start");
    }
    std::thread loader([&]() {
        while (!ld.quit) {
            ld.scan(true);
            for (int i = 0; i < 20 && !ld.quit; ++i) std::this_thread::sleep_for(std::chrono::milliseconds(100));
        }
    });
    long long last_revive = revive_first ? step - revive_every : step;
    // no more than max_reuse draws per recorded sample (default 4 for an open-ended run, off for --steps)
    if (max_reuse < 0) max_reuse = max_steps ? 0 : 4;
    auto ring_total = [&]() {
        double s = 0;
        for (auto& b : ring) s += (double)b->n;
        return s;
    };
    double allow = max_reuse * ring_total();
    bool waiting = false;
    double t_log = now(), t_save = now(), t_new = now();
    long long since = 0;
    auto save_all = [&]() {
        if (hipStreamSynchronize(c.st) != hipSuccess || !save_params(c, out + ".bin", step, false) ||
            !save_params(c, out + ".ema.bin", step, true) || !save_opt(c, out + ".opt.bin", step, c.adam_t)) {
            fprintf(stderr, "cannot save %s.bin / .ema.bin / .opt.bin\n", out.c_str());
            rc = 1;
            return;
        }
        printf("saved %s.bin, .ema.bin and .opt.bin at step %lld\n", out.c_str(), step);
        fflush(stdout);
        t_save = now();
    };
    auto stop_requested = [&]() { return fs::exists(out + ".STOP"); };
    auto stop_done = [&]() {
        std::error_code ec;
        fs::rename(out + ".STOP", out + ".STOP.done", ec);
        printf("stopped on request at step %lld\n", step);
        fflush(stdout);
    };
    bool stopped = false;
    if (!failed && launch_fill(c.stats, 0.f, 4, c.st) != hipSuccess) fail("stats");
    while (!failed && (!max_steps || ran < max_steps)) {
        for (;;) {                                 // a new chunk: scored before anything is learned from it
            ChunkP nb;
            {
                std::lock_guard<std::mutex> g(ld.mu);
                if (!ld.pending.empty()) { nb = ld.pending.front(); ld.pending.pop_front(); }
            }
            if (!nb) break;
            if (!ring_put(c, dring, *nb)) { fail("chunk upload"); break; }
            eval_on(nb, 1000003ULL * (unsigned long long)step + 7, "unseen");
            into_ring(nb);
            t_new = now();
            allow = std::min(allow + max_reuse * (double)nb->n, max_reuse * ring_total());
        }
        if (failed) break;
        if (max_reuse > 0 && allow < B) {
            if (!waiting) {
                printf("step %lld | waiting for new data: every sample of the ring has been drawn %.0f times on average\n",
                       step, max_reuse);
                fflush(stdout);
                waiting = true;
                t_log = now();
                since = 0;
                if (launch_fill(c.stats, 0.f, 4, c.st) != hipSuccess) { fail("stats"); break; }
            }
            if (stop_requested()) {
                save_all();
                stop_done();
                stopped = true;
                break;
            }
            std::this_thread::sleep_for(std::chrono::seconds(1));
            t_log = now();
            continue;
        }
        waiting = false;
        allow -= B;
        if (revive_every > 0 && step - last_revive >= revive_every) {
            const unsigned long long seed = 99991ULL * (unsigned long long)step + 3;
            std::mt19937_64 r(seed);
            std::string rep;
            if (!draw_batches(c, dring, feed, ring, r, B, revive_batches) ||
                revive(c, feed.obs, feed.tl, B, revive_batches, revive_target, seed, step, rep) < 0) {
                fail("revive");
                break;
            }
            printf("%s\n", rep.c_str());
            fflush(stdout);
            last_revive = step;
        }
        if (!draw_batches(c, dring, feed, ring, rng, B, 1) || !fwd_bwd(c, feed.obs, feed.tl, B, it, c.stats)) {
            fail("step");
            break;
        }
        ++step; ++ran; ++since;
        float l[3];
        lr_of(step, lr, lr_neuron, lr_plug, lr_min, half_life, l);
        if (fg::step(c, l[0], l[1], l[2], clip, ema) < 0.f) { fail("step"); break; }
        if (since >= log_every) {
            std::vector<float> stt;
            if (!get_dev(c, c.stats, stt, 2) || launch_fill(c.stats, 0.f, 4, c.st) != hipSuccess) { fail("stats"); break; }
            const double t = now();
            char late[64] = "";
            if (!max_steps && t - t_new > 900) snprintf(late, sizeof late, " | NO NEW DATA for %.0f min", (t - t_new) / 60);
            const float sched = (float)std::pow(0.5, (double)step / half_life);
            printf("step %lld | %.0f samples/s | kl %.4f agree %.4f | lr %.2e | ring %d, newest %s%s\n", step,
                   since * (double)B / (t - t_log), stt[0] / ((double)B * since), stt[1] / ((double)B * since),
                   std::max(lr_min, lr * sched), (int)ring.size(), ring.back()->name.c_str(), late);
            fflush(stdout);
            t_log = t;
            since = 0;
        }
        if (eval_every > 0 && step % eval_every == 0) {
            if (held) eval_on(held, 4242, "held out");
            else eval_on(ring.back(), 4242, "in the ring");
        }
        const bool stop = stop_requested();
        if (stop || now() - t_save > save_sec) {
            save_all();
            if (stop) {
                stop_done();
                stopped = true;
                break;
            }
        }
    }
    if (!failed && !stopped) {
        save_all();
        printf("done at step %lld\n", step);
        fflush(stdout);
    }
    ld.quit = true;
    loader.join();
    (void)hipStreamSynchronize(c.st);
    for (auto& b : ring) ring_drop(c, dring, *b);
    if (held) ring_drop(c, dring, *held);
    feed_free(feed);
    return failed ? 1 : rc;
}

}  // namespace fg

using namespace fg;

// ================================================================================================ C-ABI
extern "C" {

int ft_main(int argc, const char* const* argv) {
    clear_error();
    if (argc >= 5 && argv[1] && !std::strcmp(argv[1], "--check")) return check_main(argv[2], argv[3], argv[4]);
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
    std::mt19937_64 r(seed);
    for (int i = 0; i < n_batches; ++i) draw(r, s, B, reinterpret_cast<int2*>(out) + (size_t)i * B);
    return 0;
}

void ft_lr(long long step, float lr, float lr_neuron, float lr_plug, float lr_min, double half_life, float* out) {
    if (out) lr_of(step, lr, lr_neuron, lr_plug, lr_min, half_life, out);
}

long long ft_chunk_samples(const char* path, int obs_dim, int n_act) {
    if (!path) return -1;
    ChunkP b = read_chunk(path, obs_dim, n_act);
    return b ? b->n : -1;
}

int ft_scan_order(const char* dir, int keep, char* out, int cap) {
    if (!dir || keep < 0 || (!out && cap > 0)) return -1;
    Loader ld;
    ld.dir = dir;
    ld.keep = (size_t)keep;
    std::string s;
    int n = 0;
    for (auto& fm : ld.select()) {
        if (n) s += '\n';
        s += fs::path(fm.second).filename().string();
        ++n;
    }
    if ((long long)s.size() + 1 > cap) return -1;
    std::memcpy(out, s.c_str(), s.size() + 1);
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
