// Kernel argument blocks and launch wrappers of the flyguy MI355X library (kernels.hip).
#pragma once
#include "common.h"

namespace fg {

// element (tile, row, col) of a state tensor lives at tile * tile_ld + row * row_ld + col (floats)
struct Lay {
    long long tile;
    int row;
};
inline Lay tiled(int rows) { return Lay{(long long)rows * TW, TW}; }   // [T][rows][32]
inline Lay plain(int B) { return Lay{TW, B}; }                          // [rows][B]

// A segment is a run of at most SEG_MAX edges of one row: {row, e_begin, e_end, slot}; slot < 0: the whole row
// (the kernel finishes it), else the index of its partial sum in the split scratch.  A split row is
// {row, first slot, number of segments, 0}; its partial sums are added in segment order.
// rows / E / nslot bound what a segment may name: a segment outside them is skipped (the library's own plans never
// are; the bounds guard plans handed in through the fh_* entry points).
struct Plan {
    const int4* seg = nullptr;
    int nseg = 0;
    const int4* split = nullptr;
    int nsplit = 0;
    int rows = 0;
    int nslot = 0;
    long long E = 0;
};

// Per row of a layer, refreshed from the weights at every pass (k_rowinfo): {gain[nid], softplus(theta[nid]),
// re-drive row in the sensory layer as int bits (-1: none), 0}.  One 16-byte load gives a row's whole neuron.
// What follows the sum over a row's edges in the forward pass (flyguy_train.cu:84-94):
// acc (+ bias) (+ drive[drow]) -> z; h = relu(gain * z - softplus(theta)).  info == nullptr: z only (raw product).
struct FwdEpi {
    const float* bias = nullptr;
    const float4* info = nullptr;
    const float* drive = nullptr;     // the sensory layer's drive, for re-drive rows (nullptr: none in this layer)
    Lay ldrive{};
    float* z = nullptr;               // the pre-activation: stored for the sensory layer (the drive) and raw products
    Lay lz{};
    float* h = nullptr;
    Lay lh{};
};

// The backward through a layer of neurons (flyguy_train.cu:143-156 and, for the sensory layer, 174-179 and the
// plug's per-connection gradient, 158-167), applied to the gradient gh of the layer's output.
struct BwdEpi {
    int mode = 0;                 // 0: store gh raw into gh_out; 1: a hop layer; 2: the sensory layer (+ plug)
    float* gh_out = nullptr;
    Lay lgh{};
    const float* h = nullptr;
    Lay lh{};
    const float* z = nullptr;     // the sensory layer's pre-activation (the drive); hop layers do not keep theirs:
    Lay lz{};                     //   where h > 0 it is (h + softplus(theta)) / gain, and elsewhere it is not needed
    const float4* info = nullptr; // per row {gain, softplus(theta), re-drive row}
    float* gz_out = nullptr;      // mode 1
    Lay lgz{};
    float* gdrive = nullptr;
    Lay lgd{};
    float* ggain_part = nullptr;  // [T][rows]: sum over the tile of g * z
    float* gsum_part = nullptr;   // [T][rows]: sum over the tile of g
    long long gp_ld = 0;
    // mode 2: the plug
    const int* in_crow = nullptr;
    const int2* in_cw = nullptr;
    const float* x = nullptr;
    Lay lx{};
    float* ginb_part = nullptr;   // [T][n_s]
    long long gb_ld = 0;
    float* ginw_part = nullptr;   // [T][E_in]
    long long gw_ld = 0;
};

// launch wrappers (all asynchronous on `st`)
hipError_t launch_pack(const int* col, const int* idx, const float* w, int2* cw, long long E, hipStream_t st);
hipError_t launch_pack64(const int* col, const long long* idx, const float* w, int2* cw, long long E, hipStream_t st);
hipError_t launch_reduce64(const float* part, long long ld, long long n, int nt, const long long* idx, float* G,
                           hipStream_t st);
// src_rows / gz_rows: rows of the gathered state (a gather of a row outside it reads zeros)
hipError_t launch_fwd(const Plan& p, const int2* cw, const float* src, Lay ls, int src_rows, const FwdEpi& epi,
                      float* part, Lay lp, int T, hipStream_t st);
hipError_t launch_bwd(const Plan& p, const int2* cw, const float* gz, Lay lg, int gz_rows, const float* hsrc, Lay lhs,
                      float* gwpart, long long gw_ld, const BwdEpi& epi, float* part, Lay lp, int T, hipStream_t st);
hipError_t launch_obs_in(const float* obs, float* x, int obs_dim, int B, hipStream_t st);
hipError_t launch_logits(const float* hK, Lay lh, const int* dn, int n_dn, const float* ow, const float* ob, int n_act,
                         float* logits, int B, hipStream_t st);
hipError_t launch_readout_bwd_h(const float* dl, const float* ow, const int* dn_inv, int n_dn, int n_act, int rows,
                                const BwdEpi& epi, int B, hipStream_t st);
hipError_t launch_readout_bwd_w(const float* dl, const float* hK, Lay lh, const int* dn, int n_dn, int n_act,
                                float* gow_part, float* gob_part, int B, hipStream_t st);
int readout_chunks(int B);
hipError_t launch_reduce(const float* part, long long ld, long long n, int nt, const int* idx, const float* theta,
                         float* G, hipStream_t st);
hipError_t launch_loss(const float* lg, const float* tl, float* dl, float* stats_part, float* stats, int n_act, int B,
                       float it, hipStream_t st);
hipError_t launch_fill(float* p, float v, long long n, hipStream_t st);
hipError_t launch_sumsq(const float* g, long long n, float* part, float* out, hipStream_t st);
struct AdamSeg {
    long long off[8];
    float lr[7];
};
hipError_t launch_adam(float* P, const float* G, float* M, float* V, float* EMA, const AdamSeg& s, float c1, float c2,
                       const float* gs_dev, float gs, float decay, hipStream_t st);
hipError_t launch_export(const float* src, Lay ls, float* dst, int rows, int B, hipStream_t st);
hipError_t launch_rowinfo(const int* nid, const int* drow, const float* gain, const float* theta, float4* info, int rows,
                          hipStream_t st);

}  // namespace fg
