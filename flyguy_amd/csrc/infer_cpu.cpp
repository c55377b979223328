// Decisions on the host CPU: the playing network's forward pass for a caller without a GPU (one car at a time, as
// the RLBot bot asks for them), behind the C-ABI of include/fly_infer.h.
//
// A hop pushes the state of every source neuron that fires (state > 0) along its outgoing connections, which are
// stored by source (CSC order); a silent source is skipped, so a decision walks only the connections of the neurons
// that fire (about a third of them).  Re-drive rows then add the sensory drive, and each row fires
// relu(gain * z - softplus(theta)) with softplus(theta) given precomputed.  All sums are float32.  The firing of every
// neuron of the first car can be reported as one byte a neuron, 255 * tanh(1.5 * firing), layer after layer.
//
// One decision can run on several threads (fly_set_threads).  Each thread owns a range of every layer's rows and
// keeps, per hop, the connections into its rows by source in their original order.  A target row then receives its
// inputs in the same order as on one thread, so the answers are bit-identical whatever the thread count; the threads
// meet at a barrier after each layer.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

#include "../../include/fly_infer.h"

namespace {

struct Share {                     // one thread's part of a hop: the connections into its target rows [r0, r1)
    int r0 = 0, r1 = 0;
    std::vector<int> first;        // [src + 1], by source
    std::vector<int> target;
    std::vector<float> w;
};

struct PushHop {
    int rows = 0, src = 0;
    std::vector<int> first;        // [src + 1]: the outgoing connections of source j are first[j] .. first[j + 1]
    std::vector<int> target;       // the target row of each connection
    std::vector<float> w;          // its strength
    std::vector<float> gain, thr;  // per target row: gain and softplus(theta)
    std::vector<int> redrive;      // per target row: the sensory row that keeps driving it (-1: none)
    std::vector<Share> share;      // per thread (more than one thread only)
    std::vector<int> rowr;         // [threads + 1]: the target rows of each thread
};

struct CpuNet;

// The threads of a handle beyond the caller's: they wait for a decision (spinning for a while, then asleep), each
// runs its share of it, and all meet at the barrier after every layer.
struct Pool {
    std::vector<std::thread> th;
    std::mutex mu;
    std::condition_variable cv;
    std::atomic<unsigned> job{0};          // incremented for every car
    std::atomic<bool> stop{false};
    std::atomic<int> arrived{0};
    std::atomic<unsigned> sense{0};
    const float* x = nullptr;              // the car being decided
    float* out = nullptr;
    unsigned char* tap = nullptr;
};

struct CpuNet {
    int obs_dim = 0, n_act = 0, n_s = 0, n_dn = 0;
    std::vector<int> plug_first, plug_col;        // the plug by sensory row (CSR)
    std::vector<float> plug_w, plug_b, gain0, thr0;
    std::vector<PushHop> hops;
    std::vector<int> readout_rows;                 // rows of the last layer the read-out reads, in its column order
    std::vector<float> ro_w, ro_b;                 // [n_act][n_dn], [n_act]
    std::vector<float> drive, a, b;                // work space (no allocation per decision)
    std::vector<int> on;                           // (several threads) the rows of a layer that fire: thread t's
    std::vector<int> on_n;                         // in on[r0(t) ..], on_n[t] of them
    int threads = 1;
    bool shares_ok = false;                        // the per-thread shares match the network and thread count
    std::vector<int> plug_r;                       // [threads + 1]: sensory rows of each thread
    std::vector<int> act_r;                        // [threads + 1]: read-out actions of each thread
    Pool* pool = nullptr;
    bool ready() const { return n_s > 0 && n_dn > 0 && !hops.empty(); }
};

inline float fire(float gain, float z, float thr) {
    const float v = gain * z - thr;
    return v > 0.f ? v : 0.f;
}
inline unsigned char shade(float v) { return v > 0.f ? (unsigned char)(255.f * std::tanh(1.5f * v)) : 0; }

inline void pause_once() {
#if defined(__x86_64__) || defined(__i386__)
    __builtin_ia32_pause();
#else
    std::this_thread::yield();
#endif
}

// sense-reversing barrier of the handle's threads
void barrier(CpuNet& n, unsigned& local) {
    Pool& p = *n.pool;
    local ^= 1u;
    if (p.arrived.fetch_add(1, std::memory_order_acq_rel) + 1 == n.threads) {
        p.arrived.store(0, std::memory_order_relaxed);
        p.sense.store(local, std::memory_order_release);
    } else {
        for (int k = 0; p.sense.load(std::memory_order_acquire) != local; ++k)
            if (k > 4096) std::this_thread::yield(); else pause_once();
    }
}

// Thread t's part of one car.  Rows [r0, r1) of every layer are its own: it computes and fires them (and writes
// their tap bytes); the sources it reads are every thread's rows of the layer below, final after the barrier.
void decide_part(CpuNet& n, int t, const float* x, float* out, unsigned char* tap, unsigned& local) {
    const bool multi = n.threads > 1;
    float* cur = n.a.data();
    float* nxt = n.b.data();
    const int p0 = multi ? n.plug_r[t] : 0, p1 = multi ? n.plug_r[t + 1] : n.n_s;
    for (int r = p0; r < p1; ++r) {
        float z = n.plug_b[r];
        for (int e = n.plug_first[r]; e < n.plug_first[r + 1]; ++e) z += n.plug_w[e] * x[n.plug_col[e]];
        n.drive[r] = z;
        cur[r] = fire(n.gain0[r], z, n.thr0[r]);
    }
    if (tap)
        for (int r = p0; r < p1; ++r) tap[r] = shade(cur[r]);
    // with several threads, each lists its own rows that fire (ascending), so that every thread then walks the
    // firing sources in ascending order without testing every source
    int* on = n.on.data();
    auto list_firing = [&](const float* h, int r0, int r1) {
        int k = r0;
        for (int r = r0; r < r1; ++r) {
            on[k] = r;
            k += h[r] > 0.f;
        }
        n.on_n[(size_t)t] = k - r0;
    };
    if (multi) {
        list_firing(cur, p0, p1);
        barrier(n, local);
    }
    size_t tap_off = (size_t)n.n_s;
    const std::vector<int>* below = &n.plug_r;             // (several threads) each thread's rows of the layer below
    for (const PushHop& h : n.hops) {
        const int r0 = multi ? h.share[t].r0 : 0, r1 = multi ? h.share[t].r1 : h.rows;
        const int* first = multi ? h.share[t].first.data() : h.first.data();
        const int* target = multi ? h.share[t].target.data() : h.target.data();
        const float* w = multi ? h.share[t].w.data() : h.w.data();
        std::fill(nxt + r0, nxt + r1, 0.f);
        if (multi) {
            for (int u = 0; u < n.threads; ++u) {
                const int* list = on + (*below)[(size_t)u];
                for (int i = 0, m = n.on_n[(size_t)u]; i < m; ++i) {
                    const int j = list[i];
                    const float v = cur[j];
                    for (int e = first[j], e1 = first[j + 1]; e < e1; ++e) nxt[target[e]] += w[e] * v;
                }
            }
        } else {
            for (int j = 0; j < h.src; ++j) {
                const float v = cur[j];
                if (!(v > 0.f)) continue;                     // a silent neuron sends nothing
                for (int e = first[j], e1 = first[j + 1]; e < e1; ++e) nxt[target[e]] += w[e] * v;
            }
        }
        for (int r = r0; r < r1; ++r) {
            const int d = h.redrive[r];
            nxt[r] = fire(h.gain[r], d >= 0 ? nxt[r] + n.drive[d] : nxt[r], h.thr[r]);
        }
        if (tap)
            for (int r = r0; r < r1; ++r) tap[tap_off + r] = shade(nxt[r]);
        tap_off += (size_t)h.rows;
        std::swap(cur, nxt);
        if (multi) {
            barrier(n, local);                             // every thread has read the firing lists of the layer below
            list_firing(cur, r0, r1);
            below = &h.rowr;
            barrier(n, local);
        }
    }
    const int a0 = multi ? n.act_r[t] : 0, a1 = multi ? n.act_r[t + 1] : n.n_act;
    for (int a = a0; a < a1; ++a) {
        const float* wa = n.ro_w.data() + (size_t)a * n.n_dn;
        float z = n.ro_b[a];
        for (int j = 0; j < n.n_dn; ++j) z += wa[j] * cur[n.readout_rows[j]];
        out[a] = z;
    }
    if (multi) barrier(n, local);
}

void worker(CpuNet* n, int t) {
    Pool& p = *n->pool;
    unsigned seen = 0, local = 0;
    for (;;) {
        unsigned j = p.job.load(std::memory_order_acquire);
        for (int k = 0; j == seen && !p.stop.load(std::memory_order_acquire); ++k) {
            if (k < (1 << 16)) {
                pause_once();
            } else {                                       // idle for a while: sleep until the next car
                std::unique_lock<std::mutex> lk(p.mu);
                p.cv.wait(lk, [&] { return p.job.load(std::memory_order_acquire) != seen ||
                                           p.stop.load(std::memory_order_acquire); });
            }
            j = p.job.load(std::memory_order_acquire);
        }
        if (p.stop.load(std::memory_order_acquire)) return;
        seen = j;
        decide_part(*n, t, p.x, p.out, p.tap, local);
    }
}

void stop_pool(CpuNet& n) {
    if (!n.pool) return;
    {
        std::lock_guard<std::mutex> lk(n.pool->mu);
        n.pool->stop.store(true, std::memory_order_release);
    }
    n.pool->cv.notify_all();
    for (auto& t : n.pool->th) t.join();
    delete n.pool;
    n.pool = nullptr;
}

// contiguous ranges of [0, count) for n threads, cut so that each holds about the same total weight
std::vector<int> cut(int count, int n, const std::vector<long long>& weight) {
    std::vector<int> r((size_t)n + 1, count);
    r[0] = 0;
    long long total = 0;
    for (int i = 0; i < count; ++i) total += weight[(size_t)i] + 1;
    long long acc = 0;
    int k = 1;
    for (int i = 0; i < count && k < n; ++i) {
        acc += weight[(size_t)i] + 1;
        while (k < n && acc * n >= total * k) r[(size_t)k++] = i + 1;
    }
    return r;
}

// the per-thread shares and ranges for the current network and thread count
void make_shares(CpuNet& n) {
    const int T = n.threads;
    std::vector<long long> wt((size_t)n.n_s);
    for (int r = 0; r < n.n_s; ++r) wt[(size_t)r] = n.plug_first[r + 1] - n.plug_first[r];
    n.plug_r = cut(n.n_s, T, wt);
    n.on_n.assign((size_t)T, 0);
    n.act_r = cut(n.n_act, T, std::vector<long long>((size_t)n.n_act, 0));
    for (PushHop& h : n.hops) {
        std::vector<long long> indeg((size_t)h.rows, 0);
        for (int t : h.target) ++indeg[(size_t)t];
        const std::vector<int> rr = cut(h.rows, T, indeg);
        h.rowr = rr;
        std::vector<int> owner((size_t)h.rows);
        for (int t = 0; t < T; ++t)
            for (int r = rr[(size_t)t]; r < rr[(size_t)t + 1]; ++r) owner[(size_t)r] = t;
        h.share.assign((size_t)T, Share{});
        for (int t = 0; t < T; ++t) {
            Share& s = h.share[(size_t)t];
            s.r0 = rr[(size_t)t];
            s.r1 = rr[(size_t)t + 1];
            s.first.assign((size_t)h.src + 1, 0);
        }
        for (int j = 0; j < h.src; ++j) {                 // keep each source's connections in their order
            for (int t = 0; t < T; ++t) h.share[(size_t)t].first[(size_t)j] = (int)h.share[(size_t)t].target.size();
            for (int e = h.first[j]; e < h.first[j + 1]; ++e) {
                Share& s = h.share[(size_t)owner[(size_t)h.target[e]]];
                s.target.push_back(h.target[e]);
                s.w.push_back(h.w[e]);
            }
        }
        for (int t = 0; t < T; ++t) h.share[(size_t)t].first[(size_t)h.src] = (int)h.share[(size_t)t].target.size();
    }
    n.shares_ok = true;
}

void size_work(CpuNet& n) {
    size_t m = (size_t)n.n_s;
    for (const PushHop& h : n.hops) m = std::max(m, (size_t)h.rows);
    n.a.assign(m, 0.f);
    n.b.assign(m, 0.f);
    n.drive.assign((size_t)n.n_s, 0.f);
    n.on.assign(m, 0);
    n.shares_ok = false;
}

}  // namespace

extern "C" {

void* fly_create(int obs_dim, int n_act, int hops) {
    if (obs_dim <= 0 || n_act <= 0 || hops <= 0) return nullptr;
    CpuNet* n = new CpuNet;
    n->obs_dim = obs_dim;
    n->n_act = n_act;
    n->hops.resize((size_t)hops);
    return n;
}

void fly_set_plug(void* p, int n_s, int E, const int* crow, const int* col, const float* w, const float* b,
                  const float* g0, const float* t0) {
    CpuNet* n = (CpuNet*)p;
    if (!n || n_s <= 0 || E < 0) return;
    n->n_s = n_s;
    n->plug_first.assign(crow, crow + n_s + 1);
    n->plug_col.assign(col, col + E);
    n->plug_w.assign(w, w + E);
    n->plug_b.assign(b, b + n_s);
    n->gain0.assign(g0, g0 + n_s);
    n->thr0.assign(t0, t0 + n_s);
    size_work(*n);
}

void fly_set_hop(void* p, int k, int rows, int src, int E, const int* tcrow, const int* tcol, const float* w,
                 const float* g, const float* t, const int* drow) {
    CpuNet* n = (CpuNet*)p;
    if (!n || k < 0 || k >= (int)n->hops.size() || rows <= 0 || src <= 0 || E < 0) return;
    PushHop& h = n->hops[(size_t)k];
    h.rows = rows;
    h.src = src;
    h.first.assign(tcrow, tcrow + src + 1);
    h.target.assign(tcol, tcol + E);
    h.w.assign(w, w + E);
    h.gain.assign(g, g + rows);
    h.thr.assign(t, t + rows);
    h.redrive.assign(drow, drow + rows);
    size_work(*n);
}

void fly_set_out(void* p, int n_dn, const int* dn, const float* w, const float* b) {
    CpuNet* n = (CpuNet*)p;
    if (!n || n_dn <= 0) return;
    n->n_dn = n_dn;
    n->readout_rows.assign(dn, dn + n_dn);
    n->ro_w.assign(w, w + (size_t)n->n_act * n_dn);
    n->ro_b.assign(b, b + n->n_act);
    n->shares_ok = false;
}

void fly_set_threads(void* p, int threads) {
    CpuNet* n = (CpuNet*)p;
    if (!n) return;
    if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
    threads = std::min(threads, 256);
    if (threads == n->threads) return;
    stop_pool(*n);
    n->threads = threads;
    n->shares_ok = false;
    for (PushHop& h : n->hops) h.share.clear();
}

void fly_forward(void* p, const float* obs, int batch, float* logits, unsigned char* tap) {
    CpuNet* n = (CpuNet*)p;
    if (!n || !n->ready() || !obs || !logits) return;
    if (n->threads > 1) {
        try {
            if (!n->shares_ok) make_shares(*n);
            if (!n->pool) {
                n->pool = new Pool;
                for (int t = 1; t < n->threads; ++t) n->pool->th.emplace_back(worker, n, t);
            }
        } catch (...) {                                    // no memory or no threads: decide on this thread alone
            stop_pool(*n);
            n->threads = 1;
            n->shares_ok = false;
            for (PushHop& h : n->hops) h.share.clear();
        }
    }
    unsigned local = n->pool ? n->pool->sense.load(std::memory_order_acquire) : 0;
    for (int c = 0; c < batch; ++c) {
        const float* x = obs + (size_t)c * n->obs_dim;
        float* out = logits + (size_t)c * n->n_act;
        unsigned char* tp = c == 0 ? tap : nullptr;
        if (n->threads > 1) {
            Pool& pl = *n->pool;
            pl.x = x;
            pl.out = out;
            pl.tap = tp;
            {
                std::lock_guard<std::mutex> lk(pl.mu);
                pl.job.fetch_add(1, std::memory_order_acq_rel);
            }
            pl.cv.notify_all();
        }
        decide_part(*n, 0, x, out, tp, local);
    }
}

void fly_free(void* p) {
    CpuNet* n = (CpuNet*)p;
    if (!n) return;
    stop_pool(*n);
    delete n;
}

}  // extern "C"
