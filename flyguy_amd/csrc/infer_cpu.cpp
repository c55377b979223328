// Decisions on the host CPU: the playing network's forward pass for a caller without a GPU (one car at a time, as
// the RLBot bot asks for them), behind the C-ABI of include/fly_infer.h.
//
// A hop pushes the state of every source neuron that fires (state > 0) along its outgoing connections, which are
// stored by source (CSC order); a silent source is skipped, so a decision walks only the connections of the neurons
// that fire (about a third of them).  Re-drive rows then add the sensory drive, and each row fires
// relu(gain * z - softplus(theta)) with softplus(theta) given precomputed.  All sums are float32.  The firing of every
// neuron of the first car can be reported as one byte a neuron, 255 * tanh(1.5 * firing), layer after layer.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/fly_infer.h"

namespace {

struct PushHop {
    int rows = 0, src = 0;
    std::vector<int> first;        // [src + 1]: the outgoing connections of source j are first[j] .. first[j + 1]
    std::vector<int> target;       // the target row of each connection
    std::vector<float> w;          // its strength
    std::vector<float> gain, thr;  // per target row: gain and softplus(theta)
    std::vector<int> redrive;      // per target row: the sensory row that keeps driving it (-1: none)
};

struct CpuNet {
    int obs_dim = 0, n_act = 0, n_s = 0, n_dn = 0;
    std::vector<int> plug_first, plug_col;        // the plug by sensory row (CSR)
    std::vector<float> plug_w, plug_b, gain0, thr0;
    std::vector<PushHop> hops;
    std::vector<int> readout_rows;                 // rows of the last layer the read-out reads, in its column order
    std::vector<float> ro_w, ro_b;                 // [n_act][n_dn], [n_act]
    std::vector<float> drive, cur, nxt;            // work space (no allocation per decision)
    bool ready() const { return n_s > 0 && n_dn > 0 && !hops.empty(); }
};

inline float fire(float gain, float z, float thr) {
    const float v = gain * z - thr;
    return v > 0.f ? v : 0.f;
}
inline unsigned char shade(float v) { return v > 0.f ? (unsigned char)(255.f * std::tanh(1.5f * v)) : 0; }

// one car: x [obs_dim] -> out [n_act]; tap (nullable): the firing bytes of every layer
void decide(CpuNet& n, const float* x, float* out, unsigned char* tap) {
    float* cur = n.cur.data();
    float* nxt = n.nxt.data();
    for (int r = 0; r < n.n_s; ++r) {
        float z = n.plug_b[r];
        for (int e = n.plug_first[r]; e < n.plug_first[r + 1]; ++e) z += n.plug_w[e] * x[n.plug_col[e]];
        n.drive[r] = z;
        cur[r] = fire(n.gain0[r], z, n.thr0[r]);
    }
    if (tap)
        for (int r = 0; r < n.n_s; ++r) *tap++ = shade(cur[r]);
    for (const PushHop& h : n.hops) {
        std::fill(nxt, nxt + h.rows, 0.f);
        const int* first = h.first.data();
        const int* target = h.target.data();
        const float* w = h.w.data();
        for (int j = 0; j < h.src; ++j) {
            const float v = cur[j];
            if (!(v > 0.f)) continue;                     // a silent neuron sends nothing
            for (int e = first[j], e1 = first[j + 1]; e < e1; ++e) nxt[target[e]] += w[e] * v;
        }
        for (int r = 0; r < h.rows; ++r) {
            const int d = h.redrive[r];
            nxt[r] = fire(h.gain[r], d >= 0 ? nxt[r] + n.drive[d] : nxt[r], h.thr[r]);
        }
        if (tap)
            for (int r = 0; r < h.rows; ++r) *tap++ = shade(nxt[r]);
        std::swap(cur, nxt);
    }
    for (int a = 0; a < n.n_act; ++a) {
        const float* wa = n.ro_w.data() + (size_t)a * n.n_dn;
        float z = n.ro_b[a];
        for (int j = 0; j < n.n_dn; ++j) z += wa[j] * cur[n.readout_rows[j]];
        out[a] = z;
    }
}

void size_work(CpuNet& n) {
    size_t m = (size_t)n.n_s;
    for (const PushHop& h : n.hops) m = std::max(m, (size_t)h.rows);
    n.cur.assign(m, 0.f);
    n.nxt.assign(m, 0.f);
    n.drive.assign((size_t)n.n_s, 0.f);
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
}

void fly_forward(void* p, const float* obs, int batch, float* logits, unsigned char* tap) {
    CpuNet* n = (CpuNet*)p;
    if (!n || !n->ready() || !obs || !logits) return;
    for (int c = 0; c < batch; ++c)
        decide(*n, obs + (size_t)c * n->obs_dim, logits + (size_t)c * n->n_act, c == 0 ? tap : nullptr);
}

void fly_free(void* p) { delete (CpuNet*)p; }

}  // extern "C"
