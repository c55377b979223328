// Internal interface of the library's core (not part of the C-ABI): the device state of one network handle and
// the passes over it, shared by the entry points of core.hip and the teaching trainer of train.hip.
#pragma once
#include <algorithm>
#include <string>
#include <utility>
#include <vector>

#include "kernels.h"

namespace fg {

struct DevPlan {
    int2* wave = nullptr;
    int4* seg = nullptr;
    int4* split = nullptr;
    int *pcol = nullptr, *pidx = nullptr;      // per position: source row and weight index (-1: no edge)
    int nwave = 0, nseg = 0, nsplit = 0, nslot = 0, rows = 0;
    long long npos = 0;
    int pb = 8;                                 // pair storage (Plan::pb)
    Plan view() const { return Plan{wave, nwave, seg, nseg, split, nsplit, rows, nslot, npos, pb}; }
};

struct HopD {
    int rows = 0, src = 0, E = 0;
    int *nid = nullptr, *drow = nullptr;
    bool has_drive = false;
    bool pair_bwd = false;           // the layer's backward takes two tiles per workgroup (pair_tiles in core.hip)
    bool bwd_skip = true;            // the layer's backward skips silent source rows (bwd_skip_rows in core.hip)
    int gcols = 0;                   // the backward's gain / threshold partials of the layer below: plan columns
    int* gidx = nullptr;             //   (segments, then split rows) and each column's neuron (-1: none)
    // The reductions' indices, with the first writer of each gradient entry in a backward marked: -1 nothing,
    // -(i + 2) entry i written here first, i >= 0 entry i written before (by a hop above, or the top layer).
    // ridx: per backward plan position, the strength; gridx: per plan column, the neuron (gidx's marking).
    int* ridx = nullptr;
    int* gridx = nullptr;
    int2 *cw = nullptr, *tcw = nullptr;
    // The backward through k_bwd_lds (launch_bwd_lds), for a hop whose gathered rows mostly fit the LDS (bwd_lds_choice
    // in core.hip): lds_hot rows staged (0: the hop never takes it), hot_rows (most gathered first), and the transposed
    // plan's pairs with LDS codes (tcw_lds, packed from pcol_lds like tcw from bp.pcol)
    int lds_hot = 0;
    int *hot_rows = nullptr, *pcol_lds = nullptr;
    int2 *tcw_lds = nullptr, *wave_lds = nullptr;   // (wave_lds: bp's wave records with WLDS_COLD marks)
    DevPlan fp, bp;
    float *h = nullptr, *ggp = nullptr, *gsp = nullptr;
    float4* info = nullptr;          // per row {gain, softplus(theta), re-drive row}, from the current weights
    float4* sinfo = nullptr;         // the same per segment of the forward plan fp (a wave's 8 in one line)
    float4* bsinfo = nullptr;        // the layer below's records per segment of the transposed plan bp
    float* zk = nullptr;             // the pre-activation, kept only by survey passes (allocated on first use)
    std::vector<int> h_nid, h_crow, h_col, h_widx;   // host copies of the index arrays (the revive surgery)
};

// Stages timed with HIP events on the library's stream when profiling is on (fc_profile): where the time of a
// forward / backward / step goes, kernel by kernel.
enum Stage {
    ST_OBS = 0, ST_PACK = 1, ST_PLUG = 2, ST_HOP = 3,            // ST_HOP + k: forward of hop k+1 (k < 8)
    ST_LOGITS = 11, ST_LOSS = 12, ST_RBWD = 13, ST_BHOP = 14,    // ST_BHOP + k: backward of hop k+1 (k < 8)
    ST_REDUCE = 22, ST_ADAM = 23, ST_ZERO = 24, ST_COUNT = 25
};

struct Prof {
    bool on = false;
    int only = -1;                                   // >= 0: only this stage is timed
    std::vector<std::pair<hipEvent_t, int>> rec;   // (event, stage*2 + 0 start / 1 end) in recording order
    std::vector<hipEvent_t> pool;
    double ms[ST_COUNT] = {0};
    long long n[ST_COUNT] = {0};
    hipEvent_t get() {
        if (!pool.empty()) { hipEvent_t e = pool.back(); pool.pop_back(); return e; }
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        return e;
    }
};

struct Core {
    int obs_dim = 0, n_act = 0, hops = 0, n_neurons = 0, n_w = 0, n_s = 0, fan = 0, n_dn = 0, E_in = 0;
    std::vector<int> sizes, E;
    int maxB = 0, Tm = 0;
    int *in_crow = nullptr, *in_col = nullptr, *n0 = nullptr, *dn = nullptr, *dn_inv = nullptr;
    int2* in_cw = nullptr;
    float4* info0 = nullptr;
    float4* sinfo0 = nullptr;        // the sensory rows' records per segment of the plug's plan
    int* top_ridx = nullptr;         // the top layer's neurons for its gain / threshold sums, marked as HopD::ridx
    DevPlan pp;
    std::vector<HopD> hop;
    float* pm = nullptr;
    long long PT = 0, off[8] = {0}, psize[7] = {0};
    float *x = nullptr, *drive = nullptr, *h0 = nullptr, *gdrive = nullptr, *gz[2] = {nullptr, nullptr};
    float *lg = nullptr, *dl = nullptr, *part = nullptr, *gwpart = nullptr, *ggp0 = nullptr, *gsp0 = nullptr;
    float *ginb = nullptr, *ginw = nullptr, *gow_p = nullptr, *gob_p = nullptr, *stats_part = nullptr;
    float *stats = nullptr, *red = nullptr, *nrm = nullptr;
    float* owT = nullptr;            // the read-out weights transposed for the matrix cores, n_dn x readout_pad(n_act)
    float* lpart = nullptr;          // the logits' sums over the RO_SPLIT ranges of read-out rows, RO_SPLIT x maxB x n_act
    std::vector<int> h_n0, h_dn;     // host copies: the sensory rows' neurons, the read-out rows
    bool keep_z = false;             // forward passes store every hop layer's pre-activation (surveys)
    int* scnt = nullptr;             // survey sums per row of every layer (sensory rows, then each hop's rows):
    float* ssq = nullptr;            //   samples for which the row fires, sum of its squared pre-activation
    float* sstats = nullptr;         //   and the loss sums {KL, agreements}
    double s_samples = 0;
    long long rows_total = 0;
    int prec = 0;                    // 0: float32 states [B/32][rows][32]; 1: bfloat16 states [B/64][rows][64]
    // Whether rows fire, for layers 0 .. hops-1: per (tile, row) a byte written by the layer's forward
    // (fire_bytes[layer], [Tm][fires_bytes_ld(rows)]) and the bitmaps packed from them (fire_bits[layer], [Tm][fires_ld(rows)]).
    // The forward of hop k skips the gathers of layer k-1's rows that fire on no sample of a tile, and the backward
    // those of rows whose own output is zero on the tile.  skip_silent false (FLYGUY_SKIP_SILENT=0): neither (the
    // results are the same).
    bool skip_silent = true;
    int plug_lds = -1;               // the plug staged in LDS: -1 by batch size, 0 never, S > 0 with S workgroups per tile
    int bwd_lds = -1;                // k_bwd_lds for the hops that have it: -1 from BWD_LDS_MIN_TILES tiles up, 0 never,
                                     //   1 at every batch (FLYGUY_BWD_LDS)
    int cus = 0;                     // the device's CUs (k_bwd_lds takes one workgroup per CU)
    // What the derived tables were made from.  wver[set] counts the writes to the weights (set 0) and to the running
    // average (set 1): fc_copy into the handle, an Adam step, the trainer's host-side edits.  A table made from a
    // set at its current version is not made again: the forward's packed pairs and per-row records (from one set),
    // the transposed read-out weights (from one set) and the backward's packed pairs (from the weights).
    struct Stamp {
        int set = -1;
        unsigned long long ver = 0;
        bool same(int s, unsigned long long v) const { return set == s && ver == v; }
    };
    unsigned long long wver[2] = {1, 1};
    Stamp made_fpairs, made_info, made_owT, made_tpairs;
    void weights_written(int set) { if (set == 0 || set == 1) ++wver[set]; }
    std::vector<unsigned char*> fire_bytes;
    std::vector<unsigned*> fire_bits;
    long long adam_t = 0;
    int B = 0;
    hipStream_t st = nullptr;
    std::vector<void*> allocs;
    Prof prof;
    float* arr(int set, int i) const { return pm + (long long)set * PT + off[i]; }
};

// RAII: events before and after the launches of one stage (no-op unless profiling)
struct Timed {
    Core& c;
    int stage;
    Timed(Core& c_, int s) : c(c_), stage(s) { mark(0); }
    ~Timed() { mark(1); }
    void mark(int end) {
        if (!c.prof.on || (c.prof.only >= 0 && c.prof.only != stage)) return;
        hipEvent_t e = c.prof.get();
        if (e && hipEventRecord(e, c.st) == hipSuccess) c.prof.rec.push_back({e, stage * 2 + end});
    }
};

enum { SET_P = 0, SET_EMA = 1, SET_M = 2, SET_V = 3, SET_G = 4 };

template <class T>
T* dalloc(Core& c, size_t n) {
    void* p = nullptr;
    const size_t bytes = std::max<size_t>(n, 1) * sizeof(T);
    if (hipMalloc(&p, bytes) != hipSuccess) {
        set_error("out of device memory (" + std::to_string(bytes) + " bytes)");
        return nullptr;
    }
    c.allocs.push_back(p);
    if (hipMemset(p, 0, bytes) != hipSuccess) {
        set_error("hipMemset failed");
        return nullptr;
    }
    return (T*)p;
}

// prec: 0 float32 states, 1 bfloat16 states (the batch then a multiple of 64)
Core* build(const unsigned char* bytes, long long len, int max_batch, int prec = 0);
void release(Core* c);
bool check_batch(const Core* c, int B);
bool prof_collect(Core& c);
// forward of a batch through the weight set `set` (SET_P or SET_EMA); obs [B][obs_dim] row-major on the device;
// logits [B][n_act]
bool forward(Core& c, const float* obs, int B, float* logits, int set);
// backward of the last forward (through SET_P) from dlogits [B][n_act]: gradients ADDED to the SET_G arrays
// fresh: the gradient arrays are zero and this backward is the only one adding to them (a teaching step), so the
// first sum into each entry is stored instead of added (no read of the entry)
bool backward(Core& c, const float* dlogits, int B, bool fresh = false);
float grad_norm(Core& c);
// Adam + running average over all seven arrays; lr for W, lr_neuron for gain / theta, lr_plug for the rest
float step(Core& c, float lr, float lr_neuron, float lr_plug, float max_norm, float ema);

}  // namespace fg
