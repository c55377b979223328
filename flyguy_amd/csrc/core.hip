// Host side of the flyguy MI355X library: NET.bin reading and checking, row plans, device buffers, and the
// fc_* / fh_* entry points of include/flyguy_core.h.
//
// Device memory of a handle (max_batch = Bm, Tm = Bm / 32 tiles, states tiled [T][rows][32] fp32):
//   parameters: one block of 5 sets x PT floats (sets in fc_copy order: weights, running average, m, v,
//               gradient), each set holding the seven arrays at 64-float aligned offsets, so Adam is one launch;
//   structure: NET.bin's index arrays, the packed (index, weight) pairs of every product (made again from the
//              weights after every write to them), and the row plans (forward: CSR rows; backward: CSC rows);
//   states: x, drive, h0, gdrive, h_k per hop, two gz buffers, logits / dlogits (a hop layer's pre-activation z is
//           not kept: the backward needs it only where h > 0, and there it is (h + softplus(theta)) / gain);
//   partial sums: split rows, per-edge weight gradients [T or T/2][E_k], per-row gain / threshold gradients [T][rows],
//                 plug gradients [T][n_s] / [T][E_in], read-out gradients [chunks][n_act * n_dn].
#include <algorithm>
#include <cmath>
#include <cstring>
#include <cstdlib>
#include <functional>
#include <memory>
#include <numeric>
#include <string>
#include <vector>

#include "../../include/flyguy_core.h"
#include "core.h"

namespace fg {

static thread_local std::string g_err;
void set_error(const std::string& m) { g_err = m; }
const char* last_error() { return g_err.c_str(); }
void clear_error() { g_err.clear(); }

// ------------------------------------------------------------------------------------------------ row plans
// The row plan of one product (the Plan of kernels.h), built on the host.
struct HostPlan {
    std::vector<int2> wave;      // {first position, longest segment}
    std::vector<int4> seg;       // {row, slot, re-drive row, 0}
    std::vector<int4> split;     // {row, first slot, segments, re-drive row}
    std::vector<int> pos;        // plan position -> CSR edge it holds (-1: none)
    int nslot = 0;
};

// Cut rows into segments of at most seg_max edges (a longer row gets ceil(d / seg_max) segments of nearly equal
// length), order all segments longest first (equal lengths keep (row, segment) order), deal them 8 to a wave and lay
// the edges out in plan order: edge k of the segment of group g of wave w at position woff[w] + 64 (k / 8) + 8 g +
// k % 8, each wave taking 64 positions per step of its longest segment.  drow (nullable): every row's re-drive field.
// Among segments of equal length, whole rows with a re-drive line to load (drow >= 0) come first: that line comes
// from HBM, and a wave waits for it once whether one or all eight of its rows load one, so they are gathered into as
// few waves as the lengths allow (hop 1 forward 1.167 -> 1.116 ms at B=4096 on the synthetic 3-hop network).
static bool make_plan(const int* rowptr, int rows, int seg_max, const int* drow, HostPlan& p) {
    p = HostPlan{};
    if (rows < 0 || seg_max <= 0 || (rows > 0 && rowptr[0] != 0)) return false;
    struct S { int row, b, e, slot; };
    std::vector<S> segs;
    for (int r = 0; r < rows; ++r) {
        const long long d = (long long)rowptr[r + 1] - rowptr[r];
        if (d < 0) return false;
        const int dr = drow ? drow[r] : -1;
        if (d <= seg_max) {
            segs.push_back(S{r, rowptr[r], rowptr[r + 1], -1});
            continue;
        }
        const int ns = (int)((d + seg_max - 1) / seg_max);
        p.split.push_back(make_int4(r, p.nslot, ns, dr));
        for (int s = 0; s < ns; ++s) {
            const int b = rowptr[r] + (int)(d * s / ns), e = rowptr[r] + (int)(d * (s + 1) / ns);
            segs.push_back(S{r, b, e, p.nslot + s});
        }
        p.nslot += ns;
    }
    auto loads_drive = [&](const S& s) { return drow && s.slot < 0 && drow[s.row] >= 0; };
    std::stable_sort(segs.begin(), segs.end(), [&](const S& a, const S& b) {
        const int la = a.e - a.b, lb = b.e - b.b;
        return la != lb ? la > lb : loads_drive(a) > loads_drive(b);
    });
    const size_t n = segs.size(), nw = (n + 7) / 8;
    long long npos = 0;
    p.wave.resize(nw);
    for (size_t w = 0; w < nw; ++w) {
        int longest = 0;
        for (size_t i = 8 * w; i < std::min(n, 8 * w + 8); ++i) longest = std::max(longest, segs[i].e - segs[i].b);
        p.wave[w] = make_int2((int)npos, longest);
        npos += 64LL * ((longest + 7) / 8);
        if (npos > 0x7fffff00LL) return false;              // positions are 32-bit
    }
    p.pos.assign((size_t)npos, -1);
    p.seg.resize(n);
    for (size_t i = 0; i < n; ++i) {
        const S& g = segs[i];
        p.seg[i] = make_int4(g.row, g.slot, drow ? drow[g.row] : -1, 0);
        const long long base = p.wave[i / 8].x + 8LL * (long long)(i % 8);
        for (int k = 0; k < g.e - g.b; ++k) p.pos[(size_t)(base + 64LL * (k / 8) + k % 8)] = g.b + k;
    }
    return true;
}

// a plan into caller-owned arrays (fc_plan_rows, fc_net_plan): counts[0..4] = waves, segments, split rows, slots,
// positions; 0, or -1 when a capacity is too small
static int plan_out(const HostPlan& p, const char* who, int* wave_out, long long wave_cap, int* seg_out,
                    long long seg_cap, int* split_out, long long split_cap, int* pos_out, long long pos_cap,
                    long long* counts) {
    if (counts) {
        counts[0] = (long long)p.wave.size(); counts[1] = (long long)p.seg.size(); counts[2] = (long long)p.split.size();
        counts[3] = p.nslot; counts[4] = (long long)p.pos.size();
    }
    if ((long long)p.wave.size() > wave_cap || (long long)p.seg.size() > seg_cap || (long long)p.split.size() > split_cap ||
        (long long)p.pos.size() > pos_cap) {
        set_error(std::string(who) + ": capacity");
        return -1;
    }
    if (wave_out && !p.wave.empty()) std::memcpy(wave_out, p.wave.data(), p.wave.size() * sizeof(int2));
    if (seg_out && !p.seg.empty()) std::memcpy(seg_out, p.seg.data(), p.seg.size() * sizeof(int4));
    if (split_out && !p.split.empty()) std::memcpy(split_out, p.split.data(), p.split.size() * sizeof(int4));
    if (pos_out && !p.pos.empty()) std::memcpy(pos_out, p.pos.data(), p.pos.size() * sizeof(int));
    return 0;
}

template <class T>
static T* upload(Core& c, const std::vector<T>& v) {
    T* p = dalloc<T>(c, v.size());
    if (p && !v.empty() && hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) {
        set_error("hipMemcpy to device failed");
        return nullptr;
    }
    return p;
}
// How a plan's pairs are stored (Plan::pb): in 6 bytes when the state its product gathers has at most PAIR6_MAX_ROWS
// rows and its waves walk 3 steps or more on average, else in 8.  Every tile reads the pairs again, and 6-byte
// pairs cut that stream by a quarter: float32 forward 3.062 -> 3.013 ms, teaching step 6.975 -> 6.914 ms at B=4096.
// A wave of one or two steps waits for its first pairs before any gather, and the 6-byte form's unpacking lies on
// that path: the plug (2 steps a wave) took 0.160 -> 0.163 ms and hop 3's backward (1.4) 0.513 -> 0.519 ms with them,
// so those keep 8 bytes.  FLYGUY_PAIR_BYTES=8 keeps every plan at 8 bytes, =6 stores every plan whose gathered state
// allows it in 6 (the results are the same bit for bit).
static int pair_storage(int gathered_rows, const HostPlan& h) {
    if (const char* f = std::getenv("FLYGUY_PAIR_BYTES")) {
        if (std::atoi(f) == 8) return 8;
        if (std::atoi(f) == 6 && gathered_rows <= PAIR6_MAX_ROWS) return 6;
    }
    const long long steps = (long long)h.pos.size() / 64, waves = (long long)h.wave.size();
    return gathered_rows <= PAIR6_MAX_ROWS && steps >= 3 * waves ? 6 : 8;
}

// the plan on the device, with its positions resolved through col (source rows) and idx (weight index of a CSR edge;
// nullptr: the edge itself); gathered: the rows of the state its product gathers
static bool upload_plan(Core& c, const HostPlan& h, int rows, const std::vector<int>& col, const std::vector<int>* idx,
                        int gathered, DevPlan& d) {
    d.rows = rows;
    d.pb = pair_storage(gathered, h);
    d.nwave = (int)h.wave.size();
    d.nseg = (int)h.seg.size();
    d.nsplit = (int)h.split.size();
    d.nslot = h.nslot;
    d.npos = (long long)h.pos.size();
    std::vector<int> pcol(h.pos.size()), pidx(h.pos.size());
    for (size_t i = 0; i < h.pos.size(); ++i) {
        const int e = h.pos[i];
        pcol[i] = e >= 0 ? col[(size_t)e] : NO_ROW;
        pidx[i] = e >= 0 ? (idx ? (*idx)[(size_t)e] : e) : -1;
    }
    d.wave = upload(c, h.wave);
    d.seg = upload(c, h.seg);
    d.split = upload(c, h.split);
    d.pcol = upload(c, pcol);
    d.pidx = upload(c, pidx);
    return d.wave && d.seg && d.split && d.pcol && d.pidx;
}

void release(Core* c) {
    if (!c) return;
    for (auto& r : c->prof.rec) (void)hipEventDestroy(r.first);
    for (auto e : c->prof.pool) (void)hipEventDestroy(e);
    for (void* p : c->allocs) (void)hipFree(p);
    delete c;
}

// fold the recorded events into per-stage totals (waits for them)
bool prof_collect(Core& c) {
    std::vector<hipEvent_t> open(ST_COUNT, nullptr);
    bool ok = true;
    for (auto& r : c.prof.rec) {
        const int stg = r.second / 2;
        if (r.second % 2 == 0) { open[stg] = r.first; continue; }
        if (open[stg]) {
            float ms = 0.f;
            if (hipEventSynchronize(r.first) != hipSuccess || hipEventElapsedTime(&ms, open[stg], r.first) != hipSuccess) ok = false;
            c.prof.ms[stg] += ms;
            c.prof.n[stg] += 1;
            c.prof.pool.push_back(open[stg]);
            open[stg] = nullptr;
        }
        c.prof.pool.push_back(r.first);
    }
    c.prof.rec.clear();
    return ok;
}

// ------------------------------------------------------------------------------------------------ NET.bin
struct Reader {
    const unsigned char* p;
    long long n, at = 0;
    bool ok = true;
    std::vector<int> ints(long long k) {
        std::vector<int> v;
        if (k < 0 || at + 4 * k > n) {
            ok = false;
            return v;
        }
        v.resize((size_t)k);
        if (k) std::memcpy(v.data(), p + at, (size_t)(4 * k));
        at += 4 * k;
        return v;
    }
};

static bool in_range(const std::vector<int>& v, long long lo, long long hi) {   // lo <= v < hi
    for (int x : v)
        if (x < lo || x >= hi) return false;
    return true;
}
static bool rowptr_ok(const std::vector<int>& rp, long long E) {
    if (rp.empty() || rp[0] != 0 || rp.back() != E) return false;
    for (size_t i = 1; i < rp.size(); ++i)
        if (rp[i] < rp[i - 1]) return false;
    return true;
}
// Whether a layer's backward takes two tiles per workgroup: it stores half the weight-gradient partials, but holds
// two tiles' lines of the gathered gradient rows in the L2 at once.  That pays where the 16384 most gathered rows
// (two tiles of their 128-byte lines fill an XCD's 4 MiB L2) take at least 3/4 of the gathers: 0.87-0.91 on the
// lognormal fan-in of the benchmark networks (4% faster), 0.43-0.50 on an Erdos-Renyi control (5% slower).
// FLYGUY_BWD_TILES=1 or 2 overrides the choice (for tests of both kernels).
static bool pair_tiles(const std::vector<int>& crow, int rows) {
    if (const char* f = std::getenv("FLYGUY_BWD_TILES")) {
        if (f[0] == '1') return false;
        if (f[0] == '2') return true;
    }
    const long long E = crow[rows];
    if (E <= 0) return false;
    std::vector<int> deg(rows);
    for (int i = 0; i < rows; ++i) deg[i] = crow[i + 1] - crow[i];
    const int top = std::min(rows, 16384);
    std::nth_element(deg.begin(), deg.begin() + (top - 1), deg.end(), std::greater<int>());
    long long s = 0;
    for (int i = 0; i < top; ++i) s += deg[i];
    return 4 * s >= 3 * E;
}

// Whether a layer's backward skips the gathers of source rows that are silent on a tile (the test needs the row's own
// h line first, so its gathers wait for that load): only where its waves walk more than two steps on average.  A
// shorter wave is a chain of dependent loads, and the wait costs more than the skip saves.  FLYGUY_BWD_SKIP=0 or 1
// overrides the choice (FLYGUY_SKIP_SILENT=0 turns off every skip).
static bool bwd_skip_rows(const HostPlan& b) {
    if (const char* f = std::getenv("FLYGUY_BWD_SKIP")) {
        if (f[0] == '0') return false;
        if (f[0] == '1') return true;
    }
    return (long long)b.pos.size() > 2LL * 64 * (long long)b.wave.size();
}

// Which rows a hop's backward stages in LDS (k_bwd_lds): its backward gathers the hop's own rows, each as often as its
// in-degree; the `cap` most gathered (ties by row) go into `hot`, most gathered first.  The hop takes the kernel when
// the rows left out take at most 1/64 of the gathers, so that few steps gather anything through the vector-memory
// path: the hop into the descending layer (1,332 rows) of the benchmark networks and of the shipped graph (1,216 rows
// staged, the other 116 about 0.2% of the gathers).  Returns the number staged, 0 when the hop does not take it.
static int bwd_lds_choice(const std::vector<int>& crow, int rows, int cap, std::vector<int>& hot) {
    hot.clear();
    const long long E = crow[rows];
    if (cap <= 0 || rows <= 0 || E <= 0 || (long long)std::min(rows, cap) + rows > PAIR6_MAX_ROWS) return 0;
    std::vector<int> order(rows);
    for (int i = 0; i < rows; ++i) order[i] = i;
    std::stable_sort(order.begin(), order.end(),
                     [&](int a, int b) { return crow[a + 1] - crow[a] > crow[b + 1] - crow[b]; });
    const int n = std::min(rows, cap);
    long long out = 0;
    for (int r = n; r < rows; ++r) out += crow[order[r] + 1] - crow[order[r]];
    if (64 * out > E) return 0;
    hot.assign(order.begin(), order.begin() + n);
    return n;
}

// k_bwd_lds from this many tiles up (one workgroup per CU: at fewer tiles each workgroup stages its 152 kB for fewer
// rows).  FLYGUY_BWD_LDS=0 turns it off, =1 takes it at every batch.
constexpr int BWD_LDS_MIN_TILES = 16;

static bool distinct(const std::vector<int>& v, long long n, bool skip_negative) {
    std::vector<unsigned char> seen((size_t)std::max<long long>(n, 1), 0);
    for (int x : v) {
        if (x < 0 && skip_negative) continue;
        if (x < 0 || x >= n || seen[x]) return false;
        seen[x] = 1;
    }
    return true;
}

// Whether the by-source form of a hop (tcrow, tcol, twidx: per source row its connections' target rows and weight
// indices) holds exactly the connections of its by-target form (crow, col, widx), as (target, source, weight index)
// triples.  Both forms' weight indices are already known to be distinct and below n_w, and both hold E connections,
// so it is enough that each by-source connection meets a by-target one of its weight index with the same target and
// source.  The forward gathers through one form and the backward through the other: were they different graphs, the
// gradients would belong to another network than the logits.  edge_of: scratch, n_w entries of -1 on return.
static bool transposes(const std::vector<int>& crow, const std::vector<int>& col, const std::vector<int>& widx,
                       const std::vector<int>& tcrow, const std::vector<int>& tcol, const std::vector<int>& twidx,
                       int n_w, std::vector<int>& edge_of) {
    if (edge_of.size() != (size_t)std::max(n_w, 0)) edge_of.assign((size_t)std::max(n_w, 0), -1);
    const int srcs = (int)tcrow.size() - 1;
    const long long E = (long long)col.size();
    for (long long e = 0; e < E; ++e) edge_of[(size_t)widx[e]] = (int)e;      // weight index -> by-target connection
    bool ok = tcol.size() == col.size();
    for (int j = 0; j < srcs && ok; ++j)
        for (int e = tcrow[j]; e < tcrow[j + 1] && ok; ++e) {
            const int f = edge_of[(size_t)twidx[e]], r = tcol[e];           // (tcol is range-checked: a row)
            ok = f >= 0 && col[f] == j && crow[r] <= f && f < crow[r + 1];
        }
    for (long long e = 0; e < E; ++e) edge_of[(size_t)widx[e]] = -1;
    return ok;
}

// ------------------------------------------------------------------------------------------------ the host half
// NET.bin's arrays after every check, and the plans made from them: everything a handle holds that needs no device.
// build() uploads it; fc_net_plan / fc_net_marks hand it to the host (the plans the kernels run, for tests).
struct HopHost { std::vector<int> nid, crow, col, widx, tcrow, tcol, twidx, drow; };
struct NetHost {
    int obs_dim = 0, n_act = 0, hops = 0, n_neurons = 0, n_w = 0, n_s = 0, fan = 0, n_dn = 0, E_in = 0;
    std::vector<int> sizes, E, in_crow, in_col, n0, dn;
    std::vector<HopHost> hop;
};

static bool read_net(const unsigned char* bytes, long long len, NetHost& n) {
    if (!bytes || len < 36 || std::memcmp(bytes, "FLY1", 4) != 0) {
        set_error("not a FLY1 network file");
        return false;
    }
    Reader r{bytes, len, 4};
    auto hd = r.ints(8);
    if (!r.ok) { set_error("short network file (header)"); return false; }
    n.obs_dim = hd[0]; n.n_act = hd[1]; n.hops = hd[2]; n.n_neurons = hd[3];
    n.n_w = hd[4]; n.n_s = hd[5]; n.fan = hd[6]; n.n_dn = hd[7];
    if (n.obs_dim <= 0 || n.n_act <= 0 || n.hops <= 0 || n.hops > 64 || n.n_neurons <= 0 || n.n_w < 0 ||
        n.n_s <= 0 || n.fan <= 0 || n.n_dn <= 0) {
        set_error("bad network header");
        return false;
    }
    const int K = n.hops;
    n.sizes = r.ints(K + 1);
    n.E = r.ints(K);
    if (!r.ok) { set_error("short network file (sizes)"); return false; }
    if (n.sizes[0] != n.n_s) { set_error("sizes[0] != n_s"); return false; }
    for (int k = 0; k <= K; ++k)
        if (n.sizes[k] <= 0) { set_error("empty layer"); return false; }
    for (int k = 0; k < K; ++k)
        if (n.E[k] < 0) { set_error("negative edge count"); return false; }
    n.E_in = n.n_s * n.fan;
    n.in_crow = r.ints(n.n_s + 1);
    n.in_col = r.ints(n.E_in);
    r.ints(n.obs_dim + 1); r.ints(n.E_in); r.ints(n.E_in);      // the plug's transposed form: not used here
    n.n0 = r.ints(n.n_s);
    if (!r.ok) { set_error("short network file (plug)"); return false; }
    if (!rowptr_ok(n.in_crow, n.E_in) || !in_range(n.in_col, 0, n.obs_dim) || !distinct(n.n0, n.n_neurons, false)) {
        set_error("bad plug index arrays");
        return false;
    }
    n.hop.resize(K);
    std::vector<int> edge_of;                                       // (scratch of transposes())
    for (int k = 0; k < K; ++k) {
        HopHost& h = n.hop[k];
        const int rows = n.sizes[k + 1], src = n.sizes[k], E = n.E[k];
        h.nid = r.ints(rows); h.crow = r.ints(rows + 1); h.col = r.ints(E); h.widx = r.ints(E);
        h.tcrow = r.ints(src + 1); h.tcol = r.ints(E); h.twidx = r.ints(E); h.drow = r.ints(rows);
        if (!r.ok) { set_error("short network file (hop " + std::to_string(k + 1) + ")"); return false; }
        bool ok = distinct(h.nid, n.n_neurons, false) && rowptr_ok(h.crow, E) && in_range(h.col, 0, src) &&
                  distinct(h.widx, n.n_w, false) && rowptr_ok(h.tcrow, E) && in_range(h.tcol, 0, rows) &&
                  distinct(h.twidx, n.n_w, false) && in_range(h.drow, -1, n.n_s) && distinct(h.drow, n.n_s, true);
        if (!ok) { set_error("bad index arrays in hop " + std::to_string(k + 1)); return false; }
        if (!transposes(h.crow, h.col, h.widx, h.tcrow, h.tcol, h.twidx, n.n_w, edge_of)) {
            set_error("hop " + std::to_string(k + 1) + ": the by-source form (tcrow, tcol, twidx) is not the transpose "
                      "of the by-target form (crow, col, widx)");
            return false;
        }
    }
    {   // a strength is one connection: in every hop that uses it, the same source and target neuron (the revive
        // surgery and the first-write marks take a strength's neurons from any of its hops)
        std::vector<int> src_of((size_t)std::max(n.n_w, 1), -1), dst_of((size_t)std::max(n.n_w, 1), -1);
        for (int k = 0; k < K; ++k) {
            const HopHost& h = n.hop[k];
            const std::vector<int>& below = k ? n.hop[k - 1].nid : n.n0;
            for (int t = 0; t + 1 < (int)h.crow.size(); ++t)
                for (int e = h.crow[t]; e < h.crow[t + 1]; ++e) {
                    const size_t wi = (size_t)h.widx[(size_t)e];
                    const int pre = below[(size_t)h.col[(size_t)e]], post = h.nid[(size_t)t];
                    if (dst_of[wi] < 0) {
                        src_of[wi] = pre;
                        dst_of[wi] = post;
                    } else if (src_of[wi] != pre || dst_of[wi] != post) {
                        set_error("strength " + std::to_string(wi) + " joins different neurons in different hops");
                        return false;
                    }
                }
        }
    }
    n.dn = r.ints(n.n_dn);
    r.ints(n.n_w);                                                  // wmap: the caller's business
    if (!r.ok) { set_error("short network file (read-out)"); return false; }
    if (!distinct(n.dn, n.sizes[K], false)) { set_error("bad read-out rows"); return false; }
    return true;
}

// The plans of every product and the backward's per-column and first-write tables.
struct NetPlans {
    HostPlan plug;                          // the plug's rows (its forward and its gradients' pass)
    std::vector<HostPlan> fwd, bwd;         // per hop: CSR rows (forward), CSC rows = the layer below (backward)
    std::vector<std::vector<int>> gidx;     // per hop: neuron of each gain / threshold partial column of the backward
    std::vector<std::vector<int>> ridx;     // per hop: strength of each backward plan position, first writes marked
    std::vector<std::vector<int>> gridx;    // per hop: gidx with first writes marked
    std::vector<int> top_ridx;              // the top layer's neurons, first writes marked
};

static bool plan_net(const NetHost& n, NetPlans& p) {
    const int K = n.hops;
    if (!make_plan(n.in_crow.data(), n.n_s, seg_cap(n.E_in), nullptr, p.plug)) return false;
    // The re-drive field of the transposed plans' segments, which is read by the backward only.  The backward writes
    // the drive's gradient layer by layer from the top, so the top layer writes each of its re-drive rows first and
    // a lower layer's row writes its re-drive row first when no layer above re-drives that row (a sensory row
    // appears at most once per layer).  A first write starts from zero and reads nothing: its row is encoded as
    // -(d + 3).  A sensory row that no layer re-drives reads zero: it is encoded -2 (others -1).  The gradient
    // buffer then needs no clearing before a backward.
    std::vector<std::vector<int>> bwd_drow(K);
    std::vector<char> touched(n.n_s, 0);
    for (int L = K; L >= 1; --L) {
        const std::vector<int>& dr = n.hop[L - 1].drow;
        if (L < K) {
            bwd_drow[L - 1].resize(dr.size());
            for (size_t r = 0; r < dr.size(); ++r)
                bwd_drow[L - 1][r] = dr[r] >= 0 && !touched[dr[r]] ? -(dr[r] + 3) : dr[r];
        }
        for (int v : dr)
            if (v >= 0) touched[v] = 1;
    }
    std::vector<int> sensory_drow(n.n_s);
    for (int j = 0; j < n.n_s; ++j) sensory_drow[j] = touched[j] ? -1 : -2;
    p.fwd.resize(K); p.bwd.resize(K); p.gidx.resize(K); p.ridx.resize(K); p.gridx.resize(K);
    std::vector<std::vector<int>> bwd_w(K);            // per hop: strength per backward position
    for (int k = 0; k < K; ++k) {
        const HopHost& h = n.hop[k];
        const int rows = n.sizes[k + 1], src = n.sizes[k], E = n.E[k];
        // the transposed plan's rows are the layer below, with their re-drive fields as above
        const int* below_drow = k >= 1 ? bwd_drow[k - 1].data() : sensory_drow.data();
        HostPlan& f = p.fwd[k];
        HostPlan& b = p.bwd[k];
        if (!make_plan(h.crow.data(), rows, seg_cap(E), h.drow.data(), f) ||
            !make_plan(h.tcrow.data(), src, seg_cap(E), below_drow, b))
            return false;
        // the backward stores the layer below's gain and threshold partials in plan columns: a whole row at its
        // segment, split row i after the segments (coalesced stores); each column's neuron, for the reduction
        const std::vector<int>& nid_below = k >= 1 ? n.hop[k - 1].nid : n.n0;
        std::vector<int>& gidx = p.gidx[k];
        gidx.assign(b.seg.size() + b.split.size(), -1);
        for (size_t si = 0; si < b.seg.size(); ++si)
            if (b.seg[si].y < 0) gidx[si] = nid_below[(size_t)b.seg[si].x];
        for (size_t i = 0; i < b.split.size(); ++i) gidx[b.seg.size() + i] = nid_below[(size_t)b.split[i].x];
        bwd_w[k].resize(b.pos.size());
        for (size_t i = 0; i < b.pos.size(); ++i) bwd_w[k][i] = b.pos[i] >= 0 ? h.twidx[(size_t)b.pos[i]] : -1;
    }
    // the first sum into each gradient entry in a backward's order of reductions: the top layer's neurons, then
    // hop K's strengths and the layer below's neurons, ..., hop 1's (a teaching step stores those sums)
    auto mark = [](const std::vector<int>& idx, std::vector<unsigned char>& seen) {
        std::vector<int> m(idx.size());
        for (size_t i = 0; i < idx.size(); ++i) {
            const int v = idx[i];
            m[i] = v < 0 ? -1 : (seen[(size_t)v] ? v : -(v + 2));
            if (v >= 0) seen[(size_t)v] = 1;
        }
        return m;
    };
    std::vector<unsigned char> wseen((size_t)std::max(n.n_w, 1), 0), nseen((size_t)std::max(n.n_neurons, 1), 0);
    p.top_ridx = mark(n.hop[K - 1].nid, nseen);
    for (int k = K - 1; k >= 0; --k) {
        p.ridx[k] = mark(bwd_w[k], wseen);
        p.gridx[k] = mark(p.gidx[k], nseen);
    }
    return true;
}

Core* build(const unsigned char* bytes, long long len, int max_batch, int prec) {
    clear_error();
    if (!bytes || len < 36 || std::memcmp(bytes, "FLY1", 4) != 0) {
        set_error("not a FLY1 network file");
        return nullptr;
    }
    if (max_batch <= 0) {
        set_error("max_batch must be positive");
        return nullptr;
    }
    if (prec != 0 && prec != 1) {
        set_error("unknown state precision");
        return nullptr;
    }
    NetHost n;
    if (!read_net(bytes, len, n)) return nullptr;
    NetPlans P;
    if (!plan_net(n, P)) {
        set_error("row plan");
        return nullptr;
    }
    std::unique_ptr<Core, void (*)(Core*)> c(new Core, release);
    c->prec = prec;
    c->obs_dim = n.obs_dim; c->n_act = n.n_act; c->hops = n.hops; c->n_neurons = n.n_neurons;
    c->n_w = n.n_w; c->n_s = n.n_s; c->fan = n.fan; c->n_dn = n.n_dn; c->E_in = n.E_in;
    c->sizes = n.sizes;
    c->E = n.E;
    const int K = n.hops;

    // plans on the device
    const int tq = prec ? TW16 : TW;
    const int bm = (max_batch + tq - 1) / tq * tq;
    c->maxB = bm;
    c->Tm = bm / TW;
    if (!upload_plan(*c, P.plug, c->n_s, n.in_col, nullptr, c->obs_dim, c->pp)) {
        if (!*last_error()) set_error("plug plan");
        return nullptr;
    }
    c->in_cw = dalloc<int2>(*c, (size_t)(pair_bytes(c->pp.npos, c->pp.pb) / 8));
    long long max_slot = c->pp.nslot, max_pos = 1, max_rows = 1;
    c->hop.resize(K);
    if (const char* f = std::getenv("FLYGUY_BWD_LDS")) c->bwd_lds = f[0] == '0' ? 0 : (f[0] == '1' ? 1 : -1);
    const int lds_cap = c->bwd_lds == 0 ? 0 : (prec ? bwd_lds_rows16() : bwd_lds_rows());
    {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&c->cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            c->cus = 0;
    }
    for (int k = 0; k < K; ++k) {
        HopD& d = c->hop[k];
        HopHost& h = n.hop[k];
        d.rows = c->sizes[k + 1]; d.src = c->sizes[k]; d.E = c->E[k];
        if (!upload_plan(*c, P.fwd[k], d.rows, h.col, &h.widx, d.src, d.fp) ||
            !upload_plan(*c, P.bwd[k], d.src, h.tcol, &h.twidx, d.rows, d.bp))
            return nullptr;
        d.gcols = (int)P.gidx[k].size();
        d.gidx = upload(*c, P.gidx[k]);
        d.ridx = upload(*c, P.ridx[k]);
        d.gridx = upload(*c, P.gridx[k]);
        d.has_drive = std::any_of(h.drow.begin(), h.drow.end(), [](int v) { return v >= 0; });
        d.pair_bwd = pair_tiles(h.crow, d.rows);
        d.bwd_skip = bwd_skip_rows(P.bwd[k]);
        d.nid = upload(*c, h.nid);
        d.drow = upload(*c, h.drow);
        d.cw = dalloc<int2>(*c, (size_t)(pair_bytes(d.fp.npos, d.fp.pb) / 8));
        d.tcw = dalloc<int2>(*c, (size_t)(pair_bytes(d.bp.npos, d.bp.pb) / 8));
        if (!d.gidx || !d.ridx || !d.gridx || !d.nid || !d.drow || !d.cw || !d.tcw) return nullptr;
        // the last hop's backward (a hop layer below it) through k_bwd_lds / k_cbwd16_lds
        std::vector<int> hot;
        if (k == K - 1 && K >= 2 && lds_cap > 0 && bwd_lds_choice(h.crow, d.rows, lds_cap, hot) > 0) {
            std::vector<int> rank(d.rows, -1);
            for (size_t r = 0; r < hot.size(); ++r) rank[hot[r]] = (int)r;
            const int nh = (int)hot.size();
            const HostPlan& b = P.bwd[k];
            std::vector<int> code(b.pos.size());
            for (size_t i = 0; i < b.pos.size(); ++i) {
                const int e = b.pos[i];
                const int row = e >= 0 ? h.tcol[(size_t)e] : -1;
                code[i] = row < 0 ? NO_ROW : (rank[row] >= 0 ? rank[row] : nh + row);
            }
            std::vector<int2> wl(b.wave);           // (plan waves with a pair outside the LDS marked)
            for (auto& v : wl) {
                const long long end = v.x + 64LL * ((v.y + 7) / 8);
                for (long long i = v.x; i < end; ++i)
                    if (code[(size_t)i] >= nh && code[(size_t)i] < nh + d.rows) {
                        v.y |= WLDS_COLD;
                        break;
                    }
            }
            d.lds_hot = nh;
            d.hot_rows = upload(*c, hot);
            d.pcol_lds = upload(*c, code);
            d.wave_lds = upload(*c, wl);
            d.tcw_lds = dalloc<int2>(*c, (size_t)(pair_bytes(d.bp.npos, d.bp.pb) / 8));
            if (!d.hot_rows || !d.pcol_lds || !d.wave_lds || !d.tcw_lds) return nullptr;
        }
        d.h_nid = std::move(h.nid); d.h_crow = std::move(h.crow); d.h_col = std::move(h.col); d.h_widx = std::move(h.widx);
        max_slot = std::max<long long>({max_slot, d.fp.nslot, d.bp.nslot});
        max_pos = std::max<long long>(max_pos, d.bp.npos);
        max_rows = std::max<long long>(max_rows, d.rows);
    }
    c->top_ridx = upload(*c, P.top_ridx);
    if (!c->top_ridx) return nullptr;
    std::vector<int> dn_inv(c->sizes[K], -1);
    for (int j = 0; j < c->n_dn; ++j) dn_inv[n.dn[j]] = j;
    c->in_crow = upload(*c, n.in_crow); c->in_col = upload(*c, n.in_col); c->n0 = upload(*c, n.n0);
    c->dn = upload(*c, n.dn); c->dn_inv = upload(*c, dn_inv);
    c->rows_total = c->n_s;
    for (auto& d : c->hop) c->rows_total += d.rows;
    c->h_n0 = std::move(n.n0);
    c->h_dn = std::move(n.dn);
    if (!c->in_crow || !c->in_col || !c->n0 || !c->dn || !c->dn_inv || !c->in_cw) return nullptr;
    // parameters: 5 sets x 7 arrays
    const long long ps[7] = {c->n_w, c->n_neurons, c->n_neurons, c->E_in, c->n_s, (long long)c->n_act * c->n_dn, c->n_act};
    long long o = 0;
    for (int i = 0; i < 7; ++i) {
        c->psize[i] = ps[i];
        c->off[i] = o;
        o += (ps[i] + 63) / 64 * 64;
    }
    c->off[7] = o;
    c->PT = o;
    c->pm = dalloc<float>(*c, (size_t)(5 * o));
    if (!c->pm) return nullptr;

    // states (float32 or bfloat16, max_batch samples per row) and partial sums.  Per-tile partials take one row per
    // tile of the handle's own width (32 samples, or 64 with bfloat16 states); the weight-gradient partials one row
    // per tile, or per pair of tiles when every hop's backward takes two (the bfloat16 sensory layer takes one).
    const size_t Tm = c->Tm, S = TW, Tp = (size_t)bm / tq;
    size_t gw_rows = 0;
    for (int k = 1; k <= K; ++k) {       // (k_bwd_lds takes one tile per workgroup)
        const bool pair = c->hop[k - 1].pair_bwd && (prec == 0 || k >= 2) && !c->hop[k - 1].lds_hot;
        gw_rows = std::max(gw_rows, pair ? (Tp + 1) / 2 : Tp);
    }
    auto state = [&](long long rows) -> float* {
        return prec ? reinterpret_cast<float*>(dalloc<unsigned short>(*c, (size_t)bm * rows))
                    : dalloc<float>(*c, (size_t)bm * rows);
    };
    c->x = state(c->obs_dim);
    c->drive = state(c->n_s);
    c->h0 = state(c->n_s);
    c->gdrive = dalloc<float>(*c, Tm * c->n_s * S);
    c->gz[0] = state(max_rows);
    c->gz[1] = state(max_rows);
    for (auto& d : c->hop) {
        d.h = state(d.rows);
        // (its partials' columns: the plan of the hop above, or the rows themselves for the top layer's read-out)
        const size_t gc = &d != &c->hop.back() ? (size_t)std::max(d.rows, (&d + 1)->gcols) : (size_t)d.rows;
        d.ggp = dalloc<float>(*c, Tp * gc);
        d.gsp = dalloc<float>(*c, Tp * gc);
        d.info = dalloc<float4>(*c, d.rows);
        d.sinfo = dalloc<float4>(*c, d.fp.nseg);
        d.bsinfo = dalloc<float4>(*c, d.bp.nseg);
        if (!d.h || !d.ggp || !d.gsp || !d.info || !d.sinfo || !d.bsinfo) return nullptr;
    }
    c->info0 = dalloc<float4>(*c, c->n_s);
    c->sinfo0 = dalloc<float4>(*c, c->pp.nseg);
    if (!c->info0 || !c->sinfo0) return nullptr;
    if (const char* f = std::getenv("FLYGUY_SKIP_SILENT")) c->skip_silent = f[0] != '0';
    if (const char* f = std::getenv("FLYGUY_PLUG_LDS")) c->plug_lds = std::min(std::max(std::atoi(f), 0), 64);
    if (!(prec ? lds_plug_fits16() : lds_plug_fits())) c->plug_lds = 0;     // (a device with less LDS per workgroup)
    for (int l = 0; l < K; ++l) {                   // (the top layer's would have no reader)
        c->fire_bytes.push_back(dalloc<unsigned char>(*c, Tp * (size_t)fires_bytes_ld(c->sizes[l])));
        c->fire_bits.push_back(dalloc<unsigned>(*c, Tp * (size_t)fires_ld(c->sizes[l])));
        if (!c->fire_bytes.back() || !c->fire_bits.back()) return nullptr;
    }
    c->lg = dalloc<float>(*c, (size_t)bm * c->n_act);
    c->dl = dalloc<float>(*c, (size_t)bm * c->n_act);
    c->part = dalloc<float>(*c, Tm * std::max<long long>(max_slot, 1) * S);
    c->gwpart = dalloc<float>(*c, gw_rows * max_pos);
    c->ggp0 = dalloc<float>(*c, Tp * (size_t)std::max(c->n_s, c->hop[0].gcols));
    c->gsp0 = dalloc<float>(*c, Tp * (size_t)std::max(c->n_s, c->hop[0].gcols));
    c->ginb = dalloc<float>(*c, Tp * c->n_s);
    c->ginw = dalloc<float>(*c, Tp * c->E_in);
    c->gow_p = dalloc<float>(*c, (size_t)readout_chunks(bm) * c->n_act * c->n_dn);
    c->gob_p = dalloc<float>(*c, (size_t)readout_chunks(bm) * c->n_act);
    c->stats_part = dalloc<float>(*c, (size_t)2 * ((bm + 31) / 32));     // one pair per 32 samples (k_loss)
    c->stats = dalloc<float>(*c, 4);
    c->red = dalloc<float>(*c, 1024);
    c->nrm = dalloc<float>(*c, 1);
    c->owT = dalloc<float>(*c, (size_t)c->n_dn * readout_pad(c->n_act));
    c->lpart = dalloc<float>(*c, (size_t)RO_SPLIT * bm * c->n_act);
    if (!c->x || !c->drive || !c->h0 || !c->gdrive || !c->gz[0] || !c->gz[1] || !c->lg || !c->dl || !c->part ||
        !c->gwpart || !c->ggp0 || !c->gsp0 || !c->ginb || !c->ginw || !c->gow_p || !c->gob_p || !c->stats_part ||
        !c->stats || !c->red || !c->nrm || !c->owT || !c->lpart)
        return nullptr;
    if (hipDeviceSynchronize() != hipSuccess) { set_error("device error after set-up"); return nullptr; }
    return c.release();
}

bool check_batch(const Core* c, int B) {
    if (!c) { set_error("null handle"); return false; }
    const int q = c->prec ? TW16 : TW;
    if (B <= 0 || B % q != 0 || B > c->maxB) {
        set_error("batch " + std::to_string(B) + " must be a positive multiple of " + std::to_string(q) + " and at most " +
                  std::to_string(c->maxB));
        return false;
    }
    return true;
}

// ------------------------------------------------------------------------------------------------ passes
// the per-row neuron records of every layer from this set's gain and theta
static hipError_t rowinfo(Core& c, const float* gain, const float* theta, const float* bias) {
    std::vector<RowJob> j;
    j.push_back({c.n0, nullptr, c.info0, c.n_s, nullptr, bias});          // (the plug's rows carry their bias)
    j.push_back({c.n0, nullptr, c.sinfo0, c.pp.nseg, c.pp.seg, bias});
    for (size_t k = 0; k < c.hop.size(); ++k) {
        HopD& d = c.hop[k];
        j.push_back({d.nid, d.has_drive ? d.drow : nullptr, d.info, d.rows});
        j.push_back({d.nid, d.has_drive ? d.drow : nullptr, d.sinfo, d.fp.nseg, d.fp.seg});
        // the backward of hop k + 1 finishes the rows of the layer below (its transposed plan's rows)
        j.push_back({k ? c.hop[k - 1].nid : c.n0, nullptr, d.bsinfo, d.bp.nseg, d.bp.seg});
    }
    hipError_t e = hipSuccess;
    for (size_t k = 0; k < j.size() && e == hipSuccess; k += ROW_JOBS)
        e = launch_rowinfo_n(j.data() + k, (int)std::min<size_t>(ROW_JOBS, j.size() - k), gain, theta, c.st);
    return e;
}

// the packed (source, weight) pairs of the forward plans (plug and hops) or of the hops' transposed plans, in launches
// of up to PACK_JOBS plans
static hipError_t pack(Core& c, int set, bool transposed, bool bf16w) {
    std::vector<PackJob> j;
    const float* W = c.arr(set, 0);
    if (!transposed) j.push_back({c.pp.pcol, c.pp.pidx, c.arr(set, 3), c.in_cw, c.pp.npos, c.pp.pb});
    for (auto& d : c.hop) {
        j.push_back(transposed ? PackJob{d.bp.pcol, d.bp.pidx, W, d.tcw, d.bp.npos, d.bp.pb}
                               : PackJob{d.fp.pcol, d.fp.pidx, W, d.cw, d.fp.npos, d.fp.pb});
        if (transposed && d.lds_hot)    // (the same pairs with LDS codes, for k_bwd_lds)
            j.push_back(PackJob{d.pcol_lds, d.bp.pidx, W, d.tcw_lds, d.bp.npos, d.bp.pb});
    }
    hipError_t e = hipSuccess;
    for (size_t k = 0; k < j.size() && e == hipSuccess; k += PACK_JOBS)
        e = launch_pack_n(j.data() + k, (int)std::min<size_t>(PACK_JOBS, j.size() - k), c.st, bf16w);
    return e;
}

// The forward's packed pairs and per-row records from `set`, unless they were made from its current version
static hipError_t derive_forward(Core& c, int set, bool bf16w, const float* gain, const float* theta) {
    if (!c.made_fpairs.same(set, c.wver[set])) {
        const hipError_t e = pack(c, set, false, bf16w);
        if (e != hipSuccess) return e;
        c.made_fpairs = {set, c.wver[set]};
    }
    if (!c.made_info.same(set, c.wver[set])) {
        const hipError_t e = rowinfo(c, gain, theta, c.arr(set, 4));
        if (e != hipSuccess) return e;
        c.made_info = {set, c.wver[set]};
    }
    return hipSuccess;
}
// The backward's transposed pairs and per-row records from the weights (SET_P), unless current
static hipError_t derive_backward(Core& c, bool bf16w, const float* gain, const float* theta) {
    if (!c.made_tpairs.same(SET_P, c.wver[SET_P])) {
        const hipError_t e = pack(c, SET_P, true, bf16w);
        if (e != hipSuccess) return e;
        c.made_tpairs = {SET_P, c.wver[SET_P]};
    }
    if (!c.made_info.same(SET_P, c.wver[SET_P])) {
        const hipError_t e = rowinfo(c, gain, theta, c.arr(SET_P, 4));
        if (e != hipSuccess) return e;
        c.made_info = {SET_P, c.wver[SET_P]};
    }
    return hipSuccess;
}

static bool forward16(Core& c, const float* obs, int B, float* logits, int set);
static bool backward16(Core& c, const float* dlogits, int B, bool fresh);

// Workgroups per tile of the plug staged in LDS (launch_fwd_lds; launch_plug_bwd_lds for its gradients), or 0 for
// the plug through launch_fwd (its gradients in the sensory finish).  The staging pays when the workgroups have rows
// enough to walk after copying the slab: at 64 tiles or more (B >= 2048), about `total` workgroups in all.  Measured
// at B=4096 on the benchmark network: the forward's plug, 0.191 ms through launch_fwd, took 0.202 / 0.153 / 0.153 /
// 0.154 / 0.164 / 0.179 ms at 4 / 8 / 12 / 16 / 32 / 64 workgroups per tile (total 2048); hop 1's backward with the
// gradient kernel 1.409 / 1.418 / 1.429 / 1.442 ms at 8 / 16 / 24 / 32 (total 1024).  FLYGUY_PLUG_LDS=0 turns both
// off, =S forces S workgroups per tile.
static int plug_split(const Core& c, int T, int total = 2048) {
    if ((size_t)c.obs_dim * TW * 4 > FWD_LDS_BYTES || c.plug_lds == 0) return 0;
    if (c.plug_lds > 0) return c.plug_lds;
    return T >= 64 ? std::max(1, total / T) : 0;
}

bool forward(Core& c, const float* obs, int B, float* logits, int set) {
    if (c.prec) return forward16(c, obs, B, logits, set);
    const int T = B / TW;
    hipStream_t st = c.st;
    { Timed t(c, ST_OBS); FG_CHECK(launch_obs_in(obs, c.x, c.obs_dim, B, st), false); }
    const float *gain = c.arr(set, 1), *theta = c.arr(set, 2);
    // tables made in an earlier pass: the caches have moved on since (see the plug below)
    const bool old_tables = c.made_fpairs.same(set, c.wver[set]) && c.made_info.same(set, c.wver[set]);
    {
        Timed t(c, ST_PACK);
        FG_CHECK(derive_forward(c, set, false, gain, theta), false);
    }
    // each layer below the top records which rows fire on each tile; its bitmaps are packed before the next hop
    auto bytes = [&](int layer) { return c.skip_silent ? c.fire_bytes[(size_t)layer] : nullptr; };
    auto bits = [&](int layer) { return c.skip_silent ? c.fire_bits[(size_t)layer] : nullptr; };
    FwdEpi e0;
    e0.bias = c.arr(set, 4);
    e0.info = c.info0;
    e0.sinfo = c.sinfo0;
    e0.z = c.drive; e0.lz = tiled(c.n_s);
    e0.h = c.h0; e0.lh = tiled(c.n_s);
    e0.fires = bytes(0);
    {
        Timed t(c, ST_PLUG);
        const int S = plug_split(c, T);
        if (S && old_tables) {
            // Every workgroup of the LDS plug starts on the plug's plan at once; tables made in an earlier pass come
            // from HBM then, tables just made (a teaching step's) from the infinity cache.  Reading them into every
            // XCD's L2 first took repeated forwards at B=4096 from 3.085 to 3.071 ms (the plug with the read from
            // 0.183 to 0.167 ms); in a teaching step it would only cost its launch.
            TouchJob tj;
            tj.p[0] = reinterpret_cast<const uint4*>(c.in_cw); tj.n[0] = pair_bytes(c.pp.npos, c.pp.pb) / 16;
            tj.p[1] = reinterpret_cast<const uint4*>(c.sinfo0); tj.n[1] = c.pp.nseg;
            tj.p[2] = reinterpret_cast<const uint4*>(c.pp.seg); tj.n[2] = c.pp.nseg;
            tj.p[3] = reinterpret_cast<const uint4*>(c.pp.wave); tj.n[3] = c.pp.nwave / 2;
            FG_CHECK(launch_touch(tj, st), false);
        }
        if (S)
            FG_CHECK(launch_fwd_lds(c.pp.view(), c.in_cw, c.x, c.obs_dim, e0, c.part, tiled(c.pp.nslot), T, S, st), false);
        else
            FG_CHECK(launch_fwd(c.pp.view(), c.in_cw, c.x, tiled(c.obs_dim), c.obs_dim, e0, c.part, tiled(c.pp.nslot), T, st),
                     false);
        if (c.skip_silent) FG_CHECK(launch_fires_pack(bytes(0), c.n_s, bits(0), T, st), false);
    }
    const float* hp = c.h0;
    int hk = 0;
    for (auto& d : c.hop) {
        FwdEpi e;
        e.info = d.info;
        e.sinfo = d.sinfo;
        if (d.has_drive) { e.drive = c.drive; e.ldrive = tiled(c.n_s); }
        e.h = d.h; e.lh = tiled(d.rows);
        if (c.keep_z) { e.z = d.zk; e.lz = tiled(d.rows); }
        const bool record = hk + 1 < c.hops;
        if (record) e.fires = bytes(hk + 1);
        {
            Timed t(c, ST_HOP + std::min(hk, 7));
            FG_CHECK(launch_fwd(d.fp.view(), d.cw, hp, tiled(d.src), d.src, e, c.part, tiled(d.fp.nslot), T, st, bits(hk)), false);
            if (record && c.skip_silent) FG_CHECK(launch_fires_pack(bytes(hk + 1), d.rows, bits(hk + 1), T, st), false);
        }
        hp = d.h;
        ++hk;
    }
    {
        Timed t(c, ST_LOGITS);
        FG_CHECK(launch_logits_mfma(hp, false, c.sizes[c.hops], c.dn, c.n_dn, c.arr(set, 5), c.arr(set, 6), c.n_act, c.owT,
                                    c.lpart, logits, B, st, c.made_owT.same(set, c.wver[set])), false);
        c.made_owT = {set, c.wver[set]};
    }
    c.B = B;
    return true;
}

bool backward(Core& c, const float* dlogits, int B, bool fresh) {
    if (c.prec) return backward16(c, dlogits, B, fresh);
    const int T = B / TW, K = c.hops;
    hipStream_t st = c.st;
    const float *gain = c.arr(SET_P, 1), *theta = c.arr(SET_P, 2);
    float* G[7];
    for (int i = 0; i < 7; ++i) G[i] = c.arr(SET_G, i);
    {
        Timed t(c, ST_PACK);
        FG_CHECK(derive_backward(c, false, gain, theta), false);
    }

    HopD& top = c.hop[K - 1];
    BwdEpi et;
    et.mode = 1;
    et.h = top.h; et.lh = tiled(top.rows);
    et.info = top.info;
    et.drow = top.has_drive ? top.drow : nullptr;
    et.gz_out = c.gz[0]; et.lgz = tiled(top.rows);
    et.gdrive = c.gdrive; et.lgd = tiled(c.n_s);
    et.first = true;                                 // (the top layer writes each of its re-drive rows first)
    et.ggain_part = top.ggp; et.gsum_part = top.gsp; et.gp_ld = top.rows;
    {
        Timed t(c, ST_RBWD);
        if (!c.made_owT.same(SET_P, c.wver[SET_P])) {
            FG_CHECK(launch_owT(c.arr(SET_P, 5), c.n_act, c.n_dn, c.owT, st), false);
            c.made_owT = {SET_P, c.wver[SET_P]};
        }
        FG_CHECK(launch_readout_bwd_h_mfma(dlogits, c.owT, c.dn_inv, c.n_act, top.rows, et, B, st), false);
        FG_CHECK(launch_readout_bwd_w_mfma(dlogits, top.h, false, top.rows, c.dn, c.n_dn, c.n_act, c.gow_p, c.gob_p, B, st),
                 false);
    }
    const int nch = readout_chunks(B);
    {
        Timed t(c, ST_REDUCE);
        const long long now = (long long)c.n_act * c.n_dn;
        const RedJob jobs[4] = {{c.gow_p, now, now, nch, nullptr, nullptr, G[5], fresh},
                                {c.gob_p, c.n_act, c.n_act, nch, nullptr, nullptr, G[6], fresh},
                                {top.ggp, top.rows, top.rows, T, c.top_ridx, nullptr, G[1], fresh},
                                {top.gsp, top.rows, top.rows, T, c.top_ridx, theta, G[2], fresh}};
        FG_CHECK(launch_reduce_n(jobs, 4, st), false);
    }

    int cur = 0;
    for (int k = K; k >= 1; --k) {
        HopD& d = c.hop[k - 1];
        BwdEpi e;
        e.gdrive = c.gdrive; e.lgd = tiled(c.n_s);
        e.skip_silent = c.skip_silent && d.bwd_skip;
        const float* hbelow;
        int rows_below;
        float *ggp, *gsp;
        if (k >= 2) {
            HopD& b = c.hop[k - 2];
            e.mode = 1;
            e.h = b.h; e.lh = tiled(b.rows);
            e.info = b.info;
            e.gz_out = c.gz[cur ^ 1]; e.lgz = tiled(b.rows);
            hbelow = b.h; rows_below = b.rows; ggp = b.ggp; gsp = b.gsp;
        } else {
            e.mode = 2;
            e.h = c.h0; e.lh = tiled(c.n_s);
            e.z = c.drive; e.lz = tiled(c.n_s);
            e.info = c.info0;
            e.in_crow = c.in_crow; e.in_col = c.in_col; e.x = c.x; e.lx = tiled(c.obs_dim); e.x_rows = c.obs_dim;
            e.ginb_part = c.ginb; e.gb_ld = c.n_s;
            e.ginw_part = c.ginw; e.gw_ld = c.E_in;
            hbelow = c.h0; rows_below = c.n_s; ggp = c.ggp0; gsp = c.gsp0;
        }
        e.ggain_part = ggp; e.gsum_part = gsp; e.gp_ld = d.gcols;
        e.sinfo = d.bsinfo;
        // the plug's gradients in a kernel of their own with the observations in LDS, where the forward's plug is
        // (plug_split): the sensory finish then leaves the drive's complete gradient in gdrive for it
        const int ps = k == 1 ? plug_split(c, T, 1024) : 0;
        if (ps) e.in_crow = nullptr;
        // the gathered rows staged in LDS (bwd_lds_choice), one workgroup per CU
        const bool lds = d.lds_hot > 0 && e.mode == 1 && (c.bwd_lds == 1 || (c.bwd_lds < 0 && T >= BWD_LDS_MIN_TILES));
        {
            Timed t(c, ST_BHOP + std::min(k - 1, 7));
            if (lds)
                FG_CHECK(launch_bwd_lds(d.bp.view(), d.wave_lds, d.tcw_lds, c.gz[cur], d.rows, d.hot_rows, d.lds_hot, hbelow,
                                        tiled(rows_below), c.gwpart, d.bp.npos, e, c.part, tiled(d.bp.nslot), T,
                                        std::max(1, (c.cus > 0 ? c.cus : 256) / T), st), false);
            else
                FG_CHECK(launch_bwd(d.bp.view(), d.tcw, c.gz[cur], tiled(d.rows), d.rows, hbelow, tiled(rows_below),
                                    c.gwpart, d.bp.npos, e, c.part, tiled(d.bp.nslot), T, st, d.pair_bwd), false);
            if (ps)
                FG_CHECK(launch_plug_bwd_lds(c.gdrive, c.x, c.obs_dim, c.in_crow, c.in_col, c.n_s, c.ginb, c.n_s, c.ginw,
                                             c.E_in, T, ps, st), false);
        }
        Timed t(c, ST_REDUCE);
        // the layer's sums in one launch: each writes its own gradient array
        const int np = d.pair_bwd && !lds ? (T + 1) / 2 : T;   // (a two-tile backward: partials per pair of tiles)
        const RedJob jobs[5] = {{c.gwpart, d.bp.npos, d.bp.npos, np, d.ridx, nullptr, G[0], fresh},
                                {ggp, d.gcols, d.gcols, np, d.gridx, nullptr, G[1], fresh},
                                {gsp, d.gcols, d.gcols, np, d.gridx, theta, G[2], fresh},
                                {c.ginb, c.n_s, c.n_s, T, nullptr, nullptr, G[4], fresh},
                                {c.ginw, c.E_in, c.E_in, T, nullptr, nullptr, G[3], fresh}};
        FG_CHECK(launch_reduce_n(jobs, k == 1 ? 5 : 3, st), false);
        cur ^= 1;
    }
    return true;
}

// ---- the same passes over bfloat16 states (core16.hip): tiles of 64 samples
typedef unsigned short u16;
static u16* s16(float* p) { return reinterpret_cast<u16*>(p); }

static bool forward16(Core& c, const float* obs, int B, float* logits, int set) {
    const int T = B / TW16;
    hipStream_t st = c.st;
    { Timed t(c, ST_OBS); FG_CHECK(launch_obs_in16(obs, s16(c.x), c.obs_dim, B, st), false); }
    const float *gain = c.arr(set, 1), *theta = c.arr(set, 2);
    {
        Timed t(c, ST_PACK);
        FG_CHECK(derive_forward(c, set, true, gain, theta), false);
    }
    auto bytes = [&](int layer) { return c.skip_silent ? c.fire_bytes[(size_t)layer] : nullptr; };   // (as forward)
    auto bits = [&](int layer) { return c.skip_silent ? c.fire_bits[(size_t)layer] : nullptr; };
    FwdEpi16 e0;
    e0.bias = c.arr(set, 4);
    e0.info = c.info0;
    e0.sinfo = c.sinfo0;
    e0.z = s16(c.drive);
    e0.h = s16(c.h0);
    e0.rows = c.n_s;
    e0.fires = bytes(0);
    {
        Timed t(c, ST_PLUG);
        if (const int S = plug_split(c, T))
            FG_CHECK(launch_fwd16c_lds(c.pp.view(), c.in_cw, s16(c.x), c.obs_dim, e0, c.part, T, S, st), false);
        else
            FG_CHECK(launch_fwd16c(c.pp.view(), c.in_cw, s16(c.x), c.obs_dim, e0, c.part, T, st), false);
        if (c.skip_silent) FG_CHECK(launch_fires_pack(bytes(0), c.n_s, bits(0), T, st), false);
    }
    const u16* hp = s16(c.h0);
    int hk = 0;
    for (auto& d : c.hop) {
        FwdEpi16 e;
        e.info = d.info;
        e.sinfo = d.sinfo;
        if (d.has_drive) { e.drive = s16(c.drive); e.n_s = c.n_s; }
        e.h = s16(d.h);
        if (c.keep_z) e.z = s16(d.zk);
        e.rows = d.rows;
        const bool record = hk + 1 < c.hops;
        if (record) e.fires = bytes(hk + 1);
        {
            Timed t(c, ST_HOP + std::min(hk, 7));
            FG_CHECK(launch_fwd16c(d.fp.view(), d.cw, hp, d.src, e, c.part, T, st, bits(hk)), false);
            if (record && c.skip_silent) FG_CHECK(launch_fires_pack(bytes(hk + 1), d.rows, bits(hk + 1), T, st), false);
        }
        hp = s16(d.h);
        ++hk;
    }
    {
        Timed t(c, ST_LOGITS);
        FG_CHECK(launch_logits_mfma(hp, true, c.sizes[c.hops], c.dn, c.n_dn, c.arr(set, 5), c.arr(set, 6), c.n_act, c.owT,
                                    c.lpart, logits, B, st, c.made_owT.same(set, c.wver[set])), false);
        c.made_owT = {set, c.wver[set]};
    }
    c.B = B;
    return true;
}

static bool backward16(Core& c, const float* dlogits, int B, bool fresh) {
    const int T = B / TW16, K = c.hops;
    hipStream_t st = c.st;
    const float *gain = c.arr(SET_P, 1), *theta = c.arr(SET_P, 2);
    float* G[7];
    for (int i = 0; i < 7; ++i) G[i] = c.arr(SET_G, i);
    {
        Timed t(c, ST_PACK);
        FG_CHECK(derive_backward(c, true, gain, theta), false);
    }
    HopD& top = c.hop[K - 1];
    BwdEpi16 et;
    et.mode = 1;
    et.h = s16(top.h);
    et.rows = top.rows;
    et.info = top.info;
    et.drow = top.has_drive ? top.drow : nullptr;
    et.gz_out = s16(c.gz[0]);
    et.gdrive = c.gdrive;
    et.first = true;
    et.n_s = c.n_s;
    et.ggain_part = top.ggp; et.gsum_part = top.gsp; et.gp_ld = top.rows;
    {
        Timed t(c, ST_RBWD);
        if (!c.made_owT.same(SET_P, c.wver[SET_P])) {
            FG_CHECK(launch_owT(c.arr(SET_P, 5), c.n_act, c.n_dn, c.owT, st), false);
            c.made_owT = {SET_P, c.wver[SET_P]};
        }
        FG_CHECK(launch_readout_bwd_h16_mfma(dlogits, c.owT, c.dn_inv, c.n_act, top.rows, et, B, st), false);
        FG_CHECK(launch_readout_bwd_w_mfma(dlogits, top.h, true, top.rows, c.dn, c.n_dn, c.n_act, c.gow_p, c.gob_p, B, st),
                 false);
    }
    const int nch = readout_chunks(B);
    {
        Timed t(c, ST_REDUCE);
        const long long now = (long long)c.n_act * c.n_dn;
        const RedJob jobs[4] = {{c.gow_p, now, now, nch, nullptr, nullptr, G[5], fresh},
                                {c.gob_p, c.n_act, c.n_act, nch, nullptr, nullptr, G[6], fresh},
                                {top.ggp, top.rows, top.rows, T, c.top_ridx, nullptr, G[1], fresh},
                                {top.gsp, top.rows, top.rows, T, c.top_ridx, theta, G[2], fresh}};
        FG_CHECK(launch_reduce_n(jobs, 4, st), false);
    }
    int cur = 0;
    for (int k = K; k >= 1; --k) {
        HopD& d = c.hop[k - 1];
        // (the sensory layer's backward always takes one tile; the gathered rows staged in LDS as in backward())
        const bool lds = d.lds_hot > 0 && k >= 2 && (c.bwd_lds == 1 || (c.bwd_lds < 0 && T >= BWD_LDS_MIN_TILES));
        const bool pair = k >= 2 && d.pair_bwd && !lds;
        BwdEpi16 e;
        e.gdrive = c.gdrive;
        e.n_s = c.n_s;
        e.skip_silent = c.skip_silent && d.bwd_skip;
        float *ggp, *gsp;
        if (k >= 2) {
            HopD& b = c.hop[k - 2];
            e.mode = 1;
            e.h = s16(b.h);
            e.rows = b.rows;
            e.info = b.info;
            e.gz_out = s16(c.gz[cur ^ 1]);
            ggp = b.ggp; gsp = b.gsp;
        } else {
            e.mode = 2;
            e.h = s16(c.h0);
            e.z = s16(c.drive);
            e.rows = c.n_s;
            e.info = c.info0;
            e.in_crow = c.in_crow; e.in_col = c.in_col; e.x = s16(c.x); e.x_rows = c.obs_dim;
            e.ginb_part = c.ginb; e.gb_ld = c.n_s;
            e.ginw_part = c.ginw; e.gw_ld = c.E_in;
            ggp = c.ggp0; gsp = c.gsp0;
        }
        e.ggain_part = ggp; e.gsum_part = gsp; e.gp_ld = d.gcols;
        e.sinfo = d.bsinfo;
        {
            Timed t(c, ST_BHOP + std::min(k - 1, 7));
            if (lds)
                FG_CHECK(launch_bwd16c_lds(d.bp.view(), d.wave_lds, d.tcw_lds, s16(c.gz[cur]), d.rows, d.hot_rows,
                                           d.lds_hot, c.gwpart, d.bp.npos, e, c.part, T,
                                           std::max(1, (c.cus > 0 ? c.cus : 256) / T), st), false);
            else
                FG_CHECK(launch_bwd16c(d.bp.view(), d.tcw, s16(c.gz[cur]), d.rows, c.gwpart, d.bp.npos, e, c.part, T, st,
                                       pair), false);
        }
        Timed t(c, ST_REDUCE);
        // the layer's sums in one launch: each writes its own gradient array
        const int np = pair ? (T + 1) / 2 : T;        // (a two-tile backward stores its partials per pair of tiles)
        const RedJob jobs[5] = {{c.gwpart, d.bp.npos, d.bp.npos, np, d.ridx, nullptr, G[0], fresh},
                                {ggp, d.gcols, d.gcols, np, d.gridx, nullptr, G[1], fresh},
                                {gsp, d.gcols, d.gcols, np, d.gridx, theta, G[2], fresh},
                                {c.ginb, c.n_s, c.n_s, T, nullptr, nullptr, G[4], fresh},
                                {c.ginw, c.E_in, c.E_in, T, nullptr, nullptr, G[3], fresh}};
        FG_CHECK(launch_reduce_n(jobs, k == 1 ? 5 : 3, st), false);
        cur ^= 1;
    }
    return true;
}

float grad_norm(Core& c) {
    if (launch_sumsq(c.arr(SET_G, 0), c.PT, c.red, c.nrm, c.st) != hipSuccess) { set_error("grad norm launch"); return -1.f; }
    float ss = 0.f;
    FG_CHECK(hipMemcpyAsync(&ss, c.nrm, 4, hipMemcpyDeviceToHost, c.st), -1.f);
    FG_CHECK(hipStreamSynchronize(c.st), -1.f);
    return sqrtf(ss);
}

float step(Core& c, float lr, float lr_neuron, float lr_plug, float max_norm, float ema) {
    float g = 0.f;
    if (max_norm > 0.f) {
        g = grad_norm(c);
        if (g < 0.f) return -1.f;
    }
    const float gs = (max_norm > 0.f && g > max_norm) ? max_norm / g : 1.f;
    ++c.adam_t;
    const long long t = std::min<long long>(c.adam_t, 100000);
    const float c1 = 1.f - (float)std::pow(0.9, (double)t), c2 = 1.f - (float)std::pow(0.999, (double)t);
    AdamSeg s;
    for (int i = 0; i < 8; ++i) s.off[i] = c.off[i];
    for (int i = 0; i < 7; ++i) s.lr[i] = i == 0 ? lr : (i <= 2 ? lr_neuron : lr_plug);
    Timed tm(c, ST_ADAM);
    hipError_t e = launch_adam(c.arr(SET_P, 0), c.arr(SET_G, 0), c.arr(SET_M, 0), c.arr(SET_V, 0), c.arr(SET_EMA, 0), s,
                               c1, c2, nullptr, gs, ema, c.st);
    c.weights_written(SET_P);
    c.weights_written(SET_EMA);
    if (e != hipSuccess) { set_error(std::string("adam: ") + hipGetErrorString(e)); return -1.f; }
    return g;
}

}  // namespace fg

using namespace fg;

// ================================================================================================ C-ABI
extern "C" {

const char* fc_last_error(void) { return fg::last_error(); }
void fc_clear_error(void) { fg::clear_error(); }

void* fc_create_from_memory(const void* net_bytes, long long len, int max_batch) {
    return build((const unsigned char*)net_bytes, len, max_batch);
}

void* fc_create_ex(const void* net_bytes, long long len, int max_batch, int flags) {
    if (flags & ~FC_STATES_BF16) {
        set_error("fc_create_ex: unknown flags");
        return nullptr;
    }
    return build((const unsigned char*)net_bytes, len, max_batch, (flags & FC_STATES_BF16) ? 1 : 0);
}

void* fc_create(const char* net_path, int max_batch) {
    clear_error();
    FILE* f = net_path ? fopen(net_path, "rb") : nullptr;
    if (!f) { set_error(std::string("cannot open ") + (net_path ? net_path : "(null)")); return nullptr; }
    std::vector<unsigned char> buf;
    unsigned char tmp[1 << 16];
    size_t k;
    while ((k = fread(tmp, 1, sizeof tmp, f)) > 0) buf.insert(buf.end(), tmp, tmp + k);
    fclose(f);
    return build(buf.data(), (long long)buf.size(), max_batch);
}

void fc_free(void* h) { release((Core*)h); }

void fc_set_stream(void* h, void* stream) {
    Core* c = (Core*)h;
    if (!c) return;
    if (c->st != (hipStream_t)stream)           // (tables made on another stream are made again on this one)
        c->made_fpairs = c->made_info = c->made_owT = c->made_tpairs = Core::Stamp{};
    c->st = (hipStream_t)stream;
}

void fc_sizes(void* h, long long* out) {
    Core* c = (Core*)h;
    if (!c || !out) { set_error("null argument"); return; }
    for (int i = 0; i < 7; ++i) out[i] = c->psize[i];
    out[7] = c->obs_dim; out[8] = c->n_act; out[9] = c->maxB;
}

void fc_copy(void* h, int which, int to_core, float** ptrs) {
    Core* c = (Core*)h;
    if (!c || !ptrs || which < 0 || which > 4) { set_error("fc_copy: bad argument"); return; }
    for (int i = 0; i < 7; ++i) {
        if (!ptrs[i]) continue;
        float* lib = c->arr(which, i);
        FG_CHECK(hipMemcpyAsync(to_core ? lib : ptrs[i], to_core ? ptrs[i] : lib, c->psize[i] * 4, hipMemcpyDeviceToDevice,
                                c->st), );
        if (to_core) c->weights_written(which);
    }
    FG_CHECK(hipStreamSynchronize(c->st), );
}

void fc_forward(void* h, const float* obs, int B, float* logits, int ema) {
    Core* c = (Core*)h;
    if (!check_batch(c, B)) return;
    if (!obs || !logits) { set_error("fc_forward: null pointer"); return; }
    forward(*c, obs, B, logits, ema ? SET_EMA : SET_P);
}

void fc_zero_grad(void* h) {
    Core* c = (Core*)h;
    if (!c) { set_error("null handle"); return; }
    FG_CHECK(launch_fill(c->arr(SET_G, 0), 0.f, c->PT, c->st), );
}

void fc_backward(void* h, const float* dlogits, int B) {
    Core* c = (Core*)h;
    if (!check_batch(c, B)) return;
    if (!dlogits) { set_error("fc_backward: null pointer"); return; }
    if (B != c->B) { set_error("fc_backward: batch differs from the last forward's"); return; }
    backward(*c, dlogits, B);
}

float fc_grad_norm(void* h) {
    Core* c = (Core*)h;
    if (!c) { set_error("null handle"); return -1.f; }
    return grad_norm(*c);
}

float fc_step(void* h, float lr, float lr_neuron, float lr_plug, float max_norm, float ema) {
    Core* c = (Core*)h;
    if (!c) { set_error("null handle"); return -1.f; }
    return step(*c, lr, lr_neuron, lr_plug, max_norm, ema);
}

long long fc_adam_t(void* h, long long set) {
    Core* c = (Core*)h;
    if (!c) { set_error("null handle"); return -1; }
    if (set >= 0) c->adam_t = set;
    return c->adam_t;
}

void fc_sync(void*) { FG_CHECK(hipDeviceSynchronize(), ); }

void fc_kl_loss(void* h, const float* logits, const float* teacher, int B, float it, float* dlogits, float* stats) {
    Core* c = (Core*)h;
    if (!c || !logits || !teacher || !dlogits || !stats || B <= 0 || B > c->maxB) { set_error("fc_kl_loss: bad argument"); return; }
    FG_CHECK(launch_loss(logits, teacher, dlogits, c->stats_part, stats, c->n_act, B, it, c->st), );
}

float fc_teach_step(void* h, const float* obs, const float* teacher, int B, float it, float lr, float lr_neuron,
                    float lr_plug, float max_norm, float ema, float* stats) {
    Core* c = (Core*)h;
    if (!check_batch(c, B)) return -1.f;
    if (!obs || !teacher) { set_error("fc_teach_step: null pointer"); return -1.f; }
    { Timed t(*c, ST_ZERO); FG_CHECK(launch_fill(c->arr(SET_G, 0), 0.f, c->PT, c->st), -1.f); }
    if (!forward(*c, obs, B, c->lg, SET_P)) return -1.f;
    {
        Timed t(*c, ST_LOSS);
        FG_CHECK(launch_loss(c->lg, teacher, c->dl, c->stats_part, stats ? stats : c->stats, c->n_act, B, it, c->st), -1.f);
    }
    if (!backward(*c, c->dl, B, true)) return -1.f;          // (the gradient was cleared above)
    return step(*c, lr, lr_neuron, lr_plug, max_norm, ema);
}

void fc_export_state(void* h, int layer, int what, float* dst, int B) {
    Core* c = (Core*)h;
    if (!check_batch(c, B) || !dst || what < 0 || what > 2 || layer < 0 || layer > (c ? c->hops : 0)) {
        if (!*last_error()) set_error("fc_export_state: bad argument");
        return;
    }
    const float* src;
    int rows;
    if (c->prec) {
        if (what == 2) { src = c->x; rows = c->obs_dim; }
        else if (layer == 0) { src = what == 0 ? c->h0 : c->drive; rows = c->n_s; }
        else if (what == 1) { set_error("fc_export_state: a hop layer's pre-activation is not kept (only h)"); return; }
        else { src = c->hop[layer - 1].h; rows = c->hop[layer - 1].rows; }
        FG_CHECK(launch_export16(reinterpret_cast<const unsigned short*>(src), rows, dst, B, c->st), );
        return;
    }
    if (what == 2) { src = c->x; rows = c->obs_dim; }
    else if (layer == 0) { src = what == 0 ? c->h0 : c->drive; rows = c->n_s; }
    else {
        if (what == 1) { set_error("fc_export_state: a hop layer's pre-activation is not kept (only h)"); return; }
        const HopD& d = c->hop[layer - 1];
        src = d.h;
        rows = d.rows;
    }
    FG_CHECK(launch_export(src, tiled(rows), dst, rows, B, c->st), );
}

void fc_profile(void* h, int on) {
    Core* c = (Core*)h;
    if (!c) { set_error("null handle"); return; }
    if (on < 0 || on >= 2 + ST_COUNT) { set_error("fc_profile: on must be 0, 1 or 2 + a stage"); return; }
    if (c->prof.on) prof_collect(*c);            // (events recorded so far count under the old setting)
    c->prof.on = on != 0;
    c->prof.only = on >= 2 ? on - 2 : -1;
}

int fc_profile_read(void* h, double* ms, long long* counts, int n, int reset) {
    Core* c = (Core*)h;
    if (!c || n < 0) { set_error("fc_profile_read: bad argument"); return -1; }
    if (!prof_collect(*c)) { set_error("fc_profile_read: event error"); return -1; }
    for (int i = 0; i < n && i < ST_COUNT; ++i) {
        if (ms) ms[i] = c->prof.ms[i];
        if (counts) counts[i] = c->prof.n[i];
    }
    if (reset)
        for (int i = 0; i < ST_COUNT; ++i) { c->prof.ms[i] = 0; c->prof.n[i] = 0; }
    return ST_COUNT;
}

int fc_plan_rows(const int* rowptr, int rows, int seg_max, int* wave_out, long long wave_cap, int* seg_out,
                 long long seg_cap, int* split_out, long long split_cap, int* pos_out, long long pos_cap,
                 long long* counts) {
    HostPlan p;
    if (!rowptr || !make_plan(rowptr, rows, seg_max, nullptr, p)) {
        set_error("fc_plan_rows: malformed row pointer");
        return -1;
    }
    return plan_out(p, "fc_plan_rows", wave_out, wave_cap, seg_out, seg_cap, split_out, split_cap, pos_out, pos_cap,
                    counts);
}

int fc_net_plan(const char* net, long long len, int product, int backward, int* wave_out, long long wave_cap,
                int* seg_out, long long seg_cap, int* split_out, long long split_cap, int* pos_out, long long pos_cap,
                long long* counts) {
    clear_error();
    NetHost n;
    NetPlans P;
    if (!read_net(reinterpret_cast<const unsigned char*>(net), len, n)) return -1;
    if (product < 0 || product > n.hops || backward < 0 || backward > 1 || (product == 0 && backward)) {
        set_error("fc_net_plan: product 0 (the plug, forward only) or 1 .. hops, backward 0 or 1");
        return -1;
    }
    if (!plan_net(n, P)) {
        set_error("fc_net_plan: row plan");
        return -1;
    }
    const HostPlan& p = product == 0 ? P.plug : (backward ? P.bwd[product - 1] : P.fwd[product - 1]);
    return plan_out(p, "fc_net_plan", wave_out, wave_cap, seg_out, seg_cap, split_out, split_cap, pos_out, pos_cap,
                    counts);
}

long long fc_net_marks(const char* net, long long len, int hop, int which, int* out, long long cap) {
    clear_error();
    NetHost n;
    NetPlans P;
    if (!read_net(reinterpret_cast<const unsigned char*>(net), len, n)) return -1;
    if (which < 0 || which > 3 || (which < 3 && (hop < 1 || hop > n.hops))) {
        set_error("fc_net_marks: which 0 .. 2 with hop 1 .. hops, or which 3");
        return -1;
    }
    if (!plan_net(n, P)) {
        set_error("fc_net_marks: row plan");
        return -1;
    }
    const std::vector<int>& v = which == 0 ? P.gidx[hop - 1] : which == 1 ? P.ridx[hop - 1]
                                : which == 2 ? P.gridx[hop - 1] : P.top_ridx;
    if (out) {
        if ((long long)v.size() > cap) {
            set_error("fc_net_marks: capacity");
            return -1;
        }
        if (!v.empty()) std::memcpy(out, v.data(), v.size() * sizeof(int));
    }
    return (long long)v.size();
}

}  // extern "C"
