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

// The row plan of one sparse product.  Every row is cut into segments of at most seg_cap edges, the segments are
// sorted longest first and dealt out 8 to a wave (one per 8-lane group).  The (source, weight) pairs of a product
// live in plan order, interleaved per wave: the pair of edge 8j+s of the segment of group g of wave w is at position
// woff[w] + 64 j + 8 g + s, so the 64 pairs one wave uses in one step are one contiguous 512-byte block, and the
// per-(edge, tile) partials of the weight gradient are stored the same way.  Positions no edge uses hold the pair
// (NO_ROW, 0).
//   wave[w]  = {woff, longest segment of the wave}: the wave runs ceil(longest / 8) steps
//   seg[i]   = {row, slot, re-drive row, 0} of segment i (group i % 8 of wave i / 8); slot < 0: the whole row, which
//              the kernel finishes; else the index of the segment's partial sum in the split scratch.  The re-drive
//              row (-1: none) is the row's input from the sensory layer, handed in here so that its load does not
//              wait for another one.
//   split[k] = {row, first slot, number of segments, 0} of a split row; its partial sums are added in segment order
// rows / nslot / npos bound what the plan may name: a wave or segment outside them is skipped (the library's own
// plans never are; the bounds guard plans handed in through the fh_* entry points).
// pb: how the pairs are stored.  8: an int2 (source, float bits) per position, as above.  6 (a tiled product whose
// gathered state has at most 65,535 rows): per block of 64 positions (one wave's step) the 64 float weights (256 bytes)
// and then the 64 sources as 16-bit indices (128 bytes), 0xFFFF where no edge is; 384 bytes a step instead of 512.
// Every tile of a pass reads a product's pairs again, so they are a large share of what its gathers fetch past the L2.
struct Plan {
    const int2* wave = nullptr;
    int nwave = 0;
    const int4* seg = nullptr;
    int nseg = 0;
    const int4* split = nullptr;
    int nsplit = 0;
    int rows = 0;
    int nslot = 0;
    long long npos = 0;
    int pb = 8;
};
// the bytes the pairs of npos positions take
inline long long pair_bytes(long long npos, int pb) { return npos * (pb == 6 ? 6 : 8); }
// the largest gathered state (rows) whose products may store their pairs in 6 bytes (0xFFFF names no row)
constexpr int PAIR6_MAX_ROWS = 65535;

// A source index that no slab reaches: as a buffer offset (index * 128 B) it lies past every slab, so a buffer load
// of it returns zeros without touching memory; a masked global load of it is skipped.
constexpr int NO_ROW = 0x01FFFFFF;

// Per row of a layer, made from the weights after every write to them (k_rowinfo): {gain[nid], softplus(theta[nid]),
// re-drive row in the sensory layer as int bits (-1: none), 0}.  One 16-byte load gives a row's whole neuron.
// What follows the sum over a row's edges in the forward pass (flyguy_train.cu:84-94):
// acc (+ bias) (+ drive[drow]) -> z; h = relu(gain * z - softplus(theta)).  info == nullptr: z only (raw product).
struct FwdEpi {
    const float* bias = nullptr;
    const float4* info = nullptr;
    const float4* sinfo = nullptr;    // the same records per segment of the product's plan: whole rows read these
                                      // (k_fwd), split rows info (k_fwd_combine); both or neither are given.  With
                                      // a bias, whole rows take it from sinfo (the records' fourth field)
    const float* drive = nullptr;     // the sensory layer's drive, for re-drive rows (nullptr: none in this layer)
    Lay ldrive{};
    float* z = nullptr;               // the pre-activation: stored for the sensory layer (the drive) and raw products
    Lay lz{};
    float* h = nullptr;
    Lay lh{};
    // Per tile a byte per row: 1 when the row fires (h > 0) on some sample of the tile, else 0 ([T][fires_bytes_ld(rows)];
    // every row of the tile is written).  launch_fires_pack turns them into the bitmap the next hop reads.  nullptr: off.
    unsigned char* fires = nullptr;
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
    const float4* sinfo = nullptr;// the same per segment of the plan (a wave's 8 in one line): whole rows read these,
                                  //   split rows read info (k_bwd_combine); null: info throughout
    const int* drow = nullptr;    // per row: the re-drive row (-1: none), for kernels that do not follow a row plan
    float* gz_out = nullptr;      // mode 1
    Lay lgz{};
    float* gdrive = nullptr;      // the drive's gradient: a re-drive row d >= 0 adds into it; -(d + 3): writes it
    Lay lgd{};                    //   first (no load); a sensory row of re-drive field -2 reads 0 from it
    bool first = false;           // mode 1: every re-drive row of the rows writes first (the top layer)
    bool skip_silent = true;      // modes 1, 2: skip the gathers of a source row whose output is zero on the tile
    float* ggain_part = nullptr;  // [T][gp_ld]: sum over the tile of g * z, in plan columns: a whole row at its
    float* gsum_part = nullptr;   //   segment, split row i at nseg + i (the read-out kernel: the row itself);
    long long gp_ld = 0;          //   [T][gp_ld]: sum over the tile of g
    // mode 2: the plug (in_crow nullptr: the finish stores the drive's complete gradient into gdrive instead, for
    // launch_plug_bwd_lds)
    const int* in_crow = nullptr;     // the plug's CSR: connections in_crow[j] .. in_crow[j+1] of sensory row j
    const int* in_col = nullptr;      //   read observation rows in_col[f]
    const float* x = nullptr;         // the observations, tiled, x_rows of them
    Lay lx{};
    int x_rows = 0;
    float* ginb_part = nullptr;   // [T][n_s]
    long long gb_ld = 0;
    float* ginw_part = nullptr;   // [T][E_in], in the plug's CSR order
    long long gw_ld = 0;
};

// launch wrappers (all asynchronous on `st`)
// cw[p] = (pcol[p], w[pidx[p]]) for the npos positions of a plan; pidx[p] < 0: (NO_ROW, 0).  bf16w: the weight
// rounded to bfloat16 (nearest even), as the float32 of that value (the bfloat16-state core's products)
hipError_t launch_pack(const int* pcol, const int* pidx, const float* w, int2* cw, long long npos, hipStream_t st,
                       bool bf16w = false);
// the same for up to PACK_JOBS plans in one launch
struct PackJob {
    const int *pcol = nullptr, *pidx = nullptr;
    const float* w = nullptr;
    int2* cw = nullptr;
    long long n = 0;
    int pb = 8;                       // the plan's pair storage (Plan::pb); 6 takes n a multiple of 64
};
constexpr int PACK_JOBS = 4;
hipError_t launch_pack_n(const PackJob* jobs, int n, hipStream_t st, bool bf16w = false);
// src_rows / gz_rows: rows of the gathered state (a gather of a row outside it reads zeros).  src_fires: the source
// layer's firing bitmaps (launch_fires_pack; fires_ld(src_rows) words per tile; tiled states only), or nullptr
hipError_t launch_fwd(const Plan& p, const int2* cw, const float* src, Lay ls, int src_rows, const FwdEpi& epi,
                      float* part, Lay lp, int T, hipStream_t st, const unsigned* src_fires = nullptr);
// Tables to bring into every XCD's L2 ahead of a kernel (launch_touch): n[k] 16-byte words at p[k] (n 0: none)
constexpr int TOUCH_JOBS = 4;
struct TouchJob {
    const uint4* p[TOUCH_JOBS] = {};
    long long n[TOUCH_JOBS] = {};
};
hipError_t launch_touch(const TouchJob& j, hipStream_t st);
// The same over a tiled source whose tile slab (src_rows x 128 bytes) fits FWD_LDS_BYTES: each of the S workgroups
// per tile stages the slab in LDS once and gathers from there (the plug: few source rows, each gathered many times)
constexpr int FWD_LDS_NW = 8;                     // waves per workgroup
constexpr size_t FWD_LDS_BYTES = 144 * 1024;      // largest slab
hipError_t launch_fwd_lds(const Plan& p, const int2* cw, const float* src, int src_rows, const FwdEpi& epi, float* part,
                          Lay lp, int T, int S, hipStream_t st);
// The plug's bias and per-connection gradient partials (ginb [T][gb_ld], ginw [T][gw_ld]) from the drive's complete
// gradient gd ([T][n_s][32], left by a sensory-layer backward whose BwdEpi has no in_crow), with each tile's
// observation slab (x_rows x 128 bytes) staged in LDS by each of its S workgroups
// Whether the current device gives a workgroup the LDS the staged plug kernels ask for (FWD_LDS_BYTES of dynamic LDS
// plus their own static LDS): float32 (k_fwd_lds, k_plug_bwd_lds) or bfloat16 (k_cfwd16_lds) states.  Where it does
// not, the plug runs through launch_fwd and its gradients in the sensory finish.
bool lds_plug_fits();
bool lds_plug_fits16();
hipError_t launch_plug_bwd_lds(const float* gd, const float* x, int x_rows, const int* in_crow, const int* in_col,
                               int n_s, float* ginb, long long gb_ld, float* ginw, long long gw_ld, int T, int S,
                               hipStream_t st);
// A tile's firing bitmap: 4 header words (word 0: the number of rows that fire on no sample of the tile), then a
// bit per row (row r: bit r % 32 of word 4 + r / 32), padded to whole 16-byte units.
inline int fires_ld(int rows) { return 4 + ((rows + 31) / 32 + 3) / 4 * 4; }
// the bytes of a tile, rows rounded up to whole 32-row words (the pack reads each word's bytes as two 16-byte loads)
__host__ __device__ inline int fires_bytes_ld(int rows) { return (rows + 31) / 32 * 32; }
// the largest bitmap (words per tile) a hop kernel stages in LDS; a larger source layer's bits are not used
constexpr int FIRES_LDS_WORDS = 8192;
// bytes [T][fires_bytes_ld(rows)] (FwdEpi::fires) -> bitmaps [T][fires_ld(rows)]
hipError_t launch_fires_pack(const unsigned char* bytes, int rows, unsigned* bits, int T, hipStream_t st);
// gwpart: the per-position weight-gradient partials, gw_ld apart, one row per tile; with pair (a tiled layer backward,
// modes 1 and 2, whose hsrc must be epi.h: the layer's own output) one row per pair of tiles (tiles 2p and 2p + 1
// summed), ceil(T / 2) rows, and so are the rows' gain and threshold partials (epi.ggain_part, epi.gsum_part)
hipError_t launch_bwd(const Plan& p, const int2* cw, const float* gz, Lay lg, int gz_rows, const float* hsrc, Lay lhs,
                      float* gwpart, long long gw_ld, const BwdEpi& epi, float* part, Lay lp, int T, hipStream_t st,
                      bool pair = false);
// The backward of a hop layer (epi.mode 1) whose gathered gradient rows (gz_rows, the hop's own rows) mostly fit the
// LDS: each of the S workgroups per tile stages rows hot_rows[0 .. hot) of its tile's gz slab in LDS (LDS row r holds
// slab row hot_rows[r]; row `hot` holds zeros) and gathers from there.  The pairs cw carry codes instead of rows: code < hot names LDS row
// code, hot <= code < hot + gz_rows names slab row code - hot (gathered through the vector-memory path, only in steps
// that need one), anything else no row.  One tile per workgroup: gwpart and the gain / threshold partials take one
// row per tile, as launch_bwd without pair.  epi.sinfo is required (the rows' records in plan order).
constexpr int BWD_LDS_NW = 12;                    // waves per workgroup (the slab takes a CU's LDS: one workgroup)
constexpr int BWD_LDS_WREC = 4;                   // a wave walks at most 64 * BWD_LDS_WREC plan waves
constexpr int BWD_LDS_MAXROWS = 1231;             // most rows staged: 154 kB with a row of zeros, and 6 kB of pair
                                                  // staging beside them
// the rows k_bwd_lds can stage on the current device (its LDS per workgroup less the kernel's static LDS, at most
// BWD_LDS_MAXROWS), 0 if none
int bwd_lds_rows();
// wlds: the plan's wave records with WLDS_COLD set in the longest-segment field of every plan wave that has a pair
// naming a slab row outside the LDS
constexpr int WLDS_COLD = 1 << 30;
hipError_t launch_bwd_lds(const Plan& p, const int2* wlds, const int2* cw, const float* gz, int gz_rows,
                          const int* hot_rows, int hot, const float* hsrc, Lay lhs, float* gwpart, long long gw_ld,
                          const BwdEpi& epi, float* part, Lay lp, int T, int S, hipStream_t st);
hipError_t launch_obs_in(const float* obs, float* x, int obs_dim, int B, hipStream_t st);
// the read-out on the matrix cores (readout.hip): owT, n_dn x readout_pad(n_act) floats of scratch for the
// transposed weights; hK float32 tiles of 32 or (bf16_states) bfloat16 tiles of 64
int readout_pad(int n_act);
hipError_t launch_owT(const float* ow, int n_act, int n_dn, float* owT, hipStream_t st);
hipError_t launch_readout_bwd_w_mfma(const float* dl, const void* hK, bool bf16_states, int rows, const int* dn,
                                     int n_dn, int n_act, float* gow_part, float* gob_part, int B, hipStream_t st);
hipError_t launch_readout_bwd_h_mfma(const float* dl, const float* owT, const int* dn_inv, int n_act, int rows,
                                     const BwdEpi& epi, int B, hipStream_t st);
// lpart: RO_SPLIT x B x n_act floats of scratch (the sums over each split of the read-out rows)
constexpr int RO_SPLIT = 8;
// (owT_current: owT already holds ow transposed, so the transpose is not launched again)
hipError_t launch_logits_mfma(const void* hK, bool bf16_states, int rows, const int* dn, int n_dn, const float* ow,
                              const float* ob, int n_act, float* owT, float* lpart, float* logits, int B,
                              hipStream_t st, bool owT_current = false);
// the read-out weights' gradient partials come per chunk of RO_CHUNK_S samples: readout_chunks(B) of them
constexpr int RO_CHUNK_S = 128;
int readout_chunks(int B);
// G[idx[i]] += sum over nt tiles of part[t * ld + i] (times -sigmoid(theta[idx[i]]) if theta); idx[i] = -1: skipped,
// idx[i] = -(j + 2): entry j, the first sum into it in this backward; idx == nullptr: i itself (always the first).
// fresh (the gradient was cleared and only this backward adds to it): a first sum is stored, not added.  The indices
// a launch names are distinct, so no two threads write one entry.
hipError_t launch_reduce(const float* part, long long ld, long long n, int nt, const int* idx, const float* theta,
                         float* G, hipStream_t st);
// The same for up to RED_JOBS sums in one launch (a layer's weight, gain and threshold gradients, say).  The jobs of
// a launch write different arrays, or different entries of one, so their order does not matter; each entry's sum is
// the one launch_reduce forms.
struct RedJob {
    const float* part = nullptr;
    long long ld = 0, n = 0;
    int nt = 0;
    const int* idx = nullptr;
    const float* theta = nullptr;
    float* G = nullptr;
    int fresh = 0;
};
constexpr int RED_JOBS = 5;
hipError_t launch_reduce_n(const RedJob* jobs, int n, hipStream_t st);
// The core with bfloat16 states (core16.hip): the epilogues of FwdEpi / BwdEpi on [T = B/64][rows][64] tiles, with
// float32 tensors (partials, the drive's gradient) in the same tiling.
struct FwdEpi16 {
    const float* bias = nullptr;
    const float4* info = nullptr;
    const float4* sinfo = nullptr;           // per segment of the plan, as FwdEpi::sinfo
    const unsigned short* drive = nullptr;   // re-drive source: the sensory layer's drive (nullptr: none here)
    int n_s = 0;                             // rows of drive
    unsigned short* z = nullptr;             // the sensory layer's pre-activation (its drive)
    unsigned short* h = nullptr;
    int rows = 0;                            // rows of z and h
    unsigned char* fires = nullptr;          // as FwdEpi::fires, per tile of 64 samples
};
struct BwdEpi16 {
    int mode = 1;                            // 1: a hop layer; 2: the sensory layer (+ plug)
    const unsigned short* h = nullptr;       // the layer's output (also the per-edge gradient's source operand)
    const unsigned short* z = nullptr;       // the sensory layer's drive
    int rows = 0;
    const float4* info = nullptr;
    const float4* sinfo = nullptr;           // as in BwdEpi
    const int* drow = nullptr;               // per row: re-drive row (read-out kernel only)
    unsigned short* gz_out = nullptr;        // mode 1: the layer's gz, gathered by the next backward
    float* gdrive = nullptr;                 // float32 [T][n_s][64], re-drive fields as in BwdEpi
    bool first = false;                      // as in BwdEpi
    bool skip_silent = true;                 // as in BwdEpi
    int n_s = 0;
    float *ggain_part = nullptr, *gsum_part = nullptr;
    long long gp_ld = 0;
    const int *in_crow = nullptr, *in_col = nullptr;
    const unsigned short* x = nullptr;
    int x_rows = 0;
    float* ginb_part = nullptr;
    long long gb_ld = 0;
    float* ginw_part = nullptr;
    long long gw_ld = 0;
};
hipError_t launch_obs_in16(const float* obs, unsigned short* x, int obs_dim, int B, hipStream_t st);
hipError_t launch_fwd16c(const Plan& p, const int2* cw, const unsigned short* src, int src_rows, const FwdEpi16& epi,
                         float* part, int T, hipStream_t st, const unsigned* src_fires = nullptr);
// the same with each tile's source slab staged in LDS (launch_fwd_lds)
hipError_t launch_fwd16c_lds(const Plan& p, const int2* cw, const unsigned short* src, int src_rows,
                             const FwdEpi16& epi, float* part, int T, int S, hipStream_t st);
// gwpart: per-position weight-gradient partials, gw_ld apart, one row per tile; with pair (a hop layer, mode 1) one
// row per pair of tiles, ceil(T / 2) rows (the sensory layer, mode 2, always takes one tile per workgroup)
hipError_t launch_bwd16c(const Plan& p, const int2* cw, const unsigned short* gz, int gz_rows, float* gwpart,
                         long long gw_ld, const BwdEpi16& epi, float* part, int T, hipStream_t st, bool pair = false);
// the last hop's backward with the descending layer's gradient staged in LDS (launch_bwd_lds over bfloat16 states;
// one tile of 64 samples per workgroup), and the rows it can stage on the current device
hipError_t launch_bwd16c_lds(const Plan& p, const int2* wlds, const int2* cw, const unsigned short* gz, int gz_rows,
                             const int* hot_rows, int hot, float* gwpart, long long gw_ld, const BwdEpi16& epi,
                             float* part, int T, int S, hipStream_t st);
int bwd_lds_rows16();
hipError_t launch_export16(const unsigned short* src, int rows, float* dst, int B, hipStream_t st);
hipError_t launch_readout_bwd_h16_mfma(const float* dl, const float* owT, const int* dn_inv, int n_act, int rows,
                                       const BwdEpi16& epi, int B, hipStream_t st);

// KL(teacher || student) per sample (flyguy_train.cu:104-123): dl [B][n_act]; stats {KL sum, agreements} set, or
// added to when accumulate
hipError_t launch_loss(const float* lg, const float* tl, float* dl, float* stats_part, float* stats, int n_act, int B,
                       float it, hipStream_t st, bool accumulate = false);
hipError_t launch_fill(float* p, float v, long long n, hipStream_t st);
hipError_t launch_sumsq(const float* g, long long n, float* part, float* out, hipStream_t st);
struct AdamSeg {
    long long off[8];
    float lr[7];
};
hipError_t launch_adam(float* P, const float* G, float* M, float* V, float* EMA, const AdamSeg& s, float c1, float c2,
                       const float* gs_dev, float gs, float decay, hipStream_t st);
hipError_t launch_export(const float* src, Lay ls, float* dst, int rows, int B, hipStream_t st);
// per row of a layer its record {gain[nid], softplus(theta[nid]), re-drive row, 0} (see FwdEpi::info), for up to
// ROW_JOBS layers in one launch
struct RowJob {
    const int *nid = nullptr, *drow = nullptr;
    float4* info = nullptr;
    int rows = 0;
    // non-null: the records in the order of a row plan's segments instead (rows = the plan's segments, row = seg.x),
    // so that a wave's 8 rows read one 128-byte line (FwdEpi::sinfo)
    const int4* seg = nullptr;
    const float* bias = nullptr;      // non-null: the records' fourth field is bias[row] (the plug's rows), else 0
};
constexpr int ROW_JOBS = 8;
hipError_t launch_rowinfo_n(const RowJob* jobs, int n, const float* gain, const float* theta, hipStream_t st);

}  // namespace fg
