/* flyguy MI355X library: the C-ABI of the fly actor's batched forward, backward, KL loss and Adam on one GPU.
 *
 * Drop-in for the reference's FLYGUY_CORE library (flyguy/native/flyguy_train.cu:553-629, loaded by
 * flyguy/fly_native.py:34,127-159 through ctypes).  The ten fc_* functions of the reference keep their names,
 * argument meaning and ownership rules; the functions after them are additions, each marked as such.
 *
 * Conventions (as in the reference):
 *   - all float pointers passed in or out are DEVICE pointers owned by the caller (PyTorch tensors), fp32,
 *     row-major: obs [B][obs_dim], logits / dlogits / teacher logits [B][n_act];
 *   - B is a multiple of 32 and at most the max_batch given to fc_create (fly_native.py:53,200);
 *   - the seven weight arrays are, in this order: W (strengths in play, n_w), gain (n_neurons),
 *     theta (n_neurons), in_w (n_s * fan), in_b (n_s), out_w (n_act * n_dn, row = action), out_b (n_act);
 *   - work runs on one HIP stream (the null stream unless fc_set_stream names another), in call order.
 * Errors: where the reference prints and ends the process (flyguy_train.cu:47), this library records a message,
 * skips the work and returns (NULL / 0 / -1 where the function returns something); fc_last_error() reads it.
 * Arguments are checked before any kernel is launched (sizes, B, and every index array read from NET.bin).
 */
#ifndef FLYGUY_CORE_H
#define FLYGUY_CORE_H

#ifdef __cplusplus
extern "C" {
#endif

/* Reads NET.bin ("FLY1", written by export.write_net, flyguy/native/export.py:52-65) and allocates every device
 * buffer for batches up to max_batch.  Replaces fc_create, flyguy_train.cu:569-575.  NULL on error. */
void* fc_create(const char* net_path, int max_batch);

/* out[0..6]: lengths of the seven weight arrays; out[7..9]: obs_dim, n_act, max_batch.
 * Replaces fc_sizes, flyguy_train.cu:577-581. */
void fc_sizes(void* core, long long* out);

/* Copies the seven arrays of one set between the library and seven caller device arrays (NULL = skip).
 * which: 0 weights, 1 running average (EMA), 2 Adam m, 3 Adam v, 4 gradient; to_core 1: caller -> library,
 * 0: library -> caller.  Synchronous.  Replaces fc_copy, flyguy_train.cu:584-589. */
void fc_copy(void* core, int which, int to_core, float** ptrs);

/* obs [B][obs_dim] -> logits [B][n_act] with the weights (ema 0) or their running average (ema 1); the states
 * stay in the library for fc_backward.  Replaces fc_forward, flyguy_train.cu:592-598.
 * The tables a pass derives from a set (packed (source, weight) pairs, per-row records, the transposed read-out
 * weights) are made again only after that set was written (fc_copy into it, an Adam step, the trainer's edits) or
 * the stream changed; so repeated forwards with the same weights skip that work.  A forward captured in a HIP graph
 * replays the tables it made (or found) at capture: capture again after writing the weights. */
void fc_forward(void* core, const float* obs, int B, float* logits, int ema);

/* Sets the gradient of all seven arrays to zero.  Replaces fc_zero_grad, flyguy_train.cu:599-602. */
void fc_zero_grad(void* core);

/* dlogits [B][n_act]: gradient of the loss w.r.t. the logits of the last fc_forward(..., ema 0); the weights'
 * gradients are ADDED to the library's.  Replaces fc_backward, flyguy_train.cu:604-609. */
void fc_backward(void* core, const float* dlogits, int B);

/* Length of the gathered gradient (all seven arrays).  Replaces fc_grad_norm, flyguy_train.cu:610-616. */
float fc_grad_norm(void* core);

/* One Adam step (beta 0.9 / 0.999, eps 1e-8, bias corrections with t capped at 100000) with rate lr for W,
 * lr_neuron for gain and theta, lr_plug for the plugs; the gradient is first scaled down to max_norm when it is
 * longer (0: no limit); the running average follows with decay `ema`.  Returns the gradient's length before
 * scaling (0 when max_norm is 0).  Replaces fc_step, flyguy_train.cu:619-627. */
float fc_step(void* core, float lr, float lr_neuron, float lr_plug, float max_norm, float ema);

/* Adam's step count: set >= 0 sets it; returns the count.  Replaces fc_adam_t, flyguy_train.cu:628. */
long long fc_adam_t(void* core, long long set);

/* Waits for the device.  Replaces fc_sync, flyguy_train.cu:629. */
void fc_sync(void* core);

/* ---- additions (no counterpart in the reference's library) ---- */

/* The last error message of the calling thread ("" if none); fc_clear_error() forgets it. */
const char* fc_last_error(void);
void fc_clear_error(void);

/* fc_create from NET.bin bytes already in memory (len bytes). */
void* fc_create_from_memory(const void* net_bytes, long long len, int max_batch);

/* fc_create_from_memory with options.  FC_STATES_BF16: the states (observations, drive, every layer's output, the
 * gradients the backward gathers) are kept as bfloat16, rounded to nearest even, in tiles of 64 samples, and the
 * sparse products (plug and hops, forward and backward) use the connection strengths and plug weights rounded to
 * bfloat16; sums, gradients, the float32 master weights and Adam stay float32.  Batches are then a multiple of 64.
 * Every other entry point works on such a handle as on a float32 one (the surveys of include/flyguy_train.h count
 * and square its stored bfloat16 states). */
#define FC_STATES_BF16 1
void* fc_create_ex(const void* net_bytes, long long len, int max_batch, int flags);

/* Frees every buffer of the handle (the reference's handles live until the process ends). */
void fc_free(void* core);

/* Runs the library's work on this HIP stream (hipStream_t; NULL = the null stream) from now on.  A new stream
 * makes the next passes derive their tables again, on that stream. */
void fc_set_stream(void* core, void* stream);

/* KL(teacher || student) over n_act actions for a batch: logits and teacher [B][n_act] device arrays,
 * it = 1 / temperature of the teacher; writes dlogits [B][n_act] = d(mean KL)/d logits and stats[0] = sum of
 * the per-sample KL, stats[1] = number of samples whose argmax agrees (first maximum wins).  The trainer's
 * k_loss, flyguy_train.cu:104-123, as a function of its own. */
void fc_kl_loss(void* core, const float* logits, const float* teacher, int B, float it, float* dlogits, float* stats);

/* One teaching step as the standalone trainer's loop does it (flyguy_train.cu:361-365 then 758-764):
 * zero the gradient, forward on obs, KL loss against teacher (it as above), backward, Adam step.  stats (device,
 * 2 floats, or NULL) receives the loss sums as in fc_kl_loss.  Returns what fc_step returns. */
float fc_teach_step(void* core, const float* obs, const float* teacher, int B, float it, float lr, float lr_neuron,
                    float lr_plug, float max_norm, float ema, float* stats);

/* Copies an internal state of the last forward to dst [rows][B] (device): layer 0 is the sensory layer,
 * layer k the output of hop k; what 0: h (firing), 1: z (input before the neuron; layer 0: the drive),
 * 2: the observation batch x [obs_dim][B] (layer ignored).  For tests and diagnostics. */
void fc_export_state(void* core, int layer, int what, float* dst, int B);

/* Profiling: with on = 1 every stage of the library's work is bracketed by HIP events on its stream; with
 * on = 2 + s only stage s is (two events per run of it, so timing the whole call is not disturbed); 0 stops.
 * fc_profile_read waits for the recorded events and writes, per stage, the summed milliseconds and the number of
 * timed runs (reset != 0 clears the totals); returns the number of stages (25) or -1.  Stages: 0 observation
 * transpose, 1 (index, weight) packing, 2 plug + sensory layer, 3+k forward of hop k+1, 11 read-out, 12 loss,
 * 13 read-out backward, 14+k backward of hop k+1, 22 gradient reductions, 23 Adam, 24 zeroing.  The reference
 * timed its library from Python (flyguy/native/rl_profile.py:49-86). */
void fc_profile(void* core, int on);
int fc_profile_read(void* core, double* ms, long long* counts, int n, int reset);

/* The gather ceiling (measurement): the time per gathered 128-byte line, for the whole device, when every CU's 8-lane
 * groups do nothing but gather, as the hop kernels gather: per step each lane of a group draws one connection at
 * random and takes its row, row_of[e] (device, n_edges entries, each in 0 .. rows - 1; NULL: rows drawn uniformly),
 * the group shares the 8 rows and loads each row's line, 16 bytes a lane (8 lines per wave instruction), from each
 * of `tiles` slabs of rows x 128 bytes (1, or 2 for a backward that takes two tiles per workgroup).  reps timed
 * launches after an untimed one, on `stream` (a hipStream_t, or NULL); writes nanoseconds per line to ns_per_line.
 * Allocates and frees its own scratch.  Returns 0, or -1 (fc_last_error).  (No counterpart in the reference.) */
int fc_gather_ceiling(int rows, int tiles, const int* row_of, long long n_edges, int reps, void* stream,
                      double* ns_per_line);

/* The row plan of one sparse product, computed on the host (no device needed).  Every row is cut into segments of
 * at most seg_max edges; the segments are sorted longest first (ties: row, then segment order) and dealt 8 to a
 * wave; the edges are laid out in plan order, edge k of the segment of group g of wave w at position
 * woff[w] + 64 (k / 8) + 8 g + k % 8 (a wave takes 64 positions per 8 edges of its longest segment).
 *   wave_out:  2 ints per wave {woff, longest segment}
 *   seg_out:   4 ints per segment {row, slot, -1, 0} (slot -1: the whole row, else the index of its partial sum)
 *   split_out: 4 ints per split row {row, first slot, segments, -1}
 *   pos_out:   per position the CSR edge it holds (-1: none)
 * counts[0..4] = waves, segments, split rows, slots, positions.  Null outputs with zero capacities return the counts
 * only.  Returns 0, or -1 if a capacity is too small or rowptr (rows+1 entries) is malformed.  (No counterpart in
 * the reference, whose kernels take plain CSR arrays, flyguy_train.cu:75-101.) */
int fc_plan_rows(const int* rowptr, int rows, int seg_max, int* wave_out, long long wave_cap, int* seg_out,
                 long long seg_cap, int* split_out, long long split_cap, int* pos_out, long long pos_cap,
                 long long* counts);

/* The plans a handle's kernels run, computed on the host from NET.bin bytes (no device; the network is checked as
 * fc_create checks it).  product 0: the plug's rows (forward only; its gradient pass walks the same plan); product k
 * = 1 .. hops: hop k, backward 0 its CSR rows (forward), backward 1 its CSC rows, i.e. the layer below (backward).
 * Outputs as fc_plan_rows, with these differences: the segment length cap is the library's own (at least 4096
 * segments, 16 .. 512 edges per segment); among segments of equal length, whole rows that read a line of the drive
 * (forward: a re-drive row; backward: the drive gradient written so far) come first; the third int of a segment
 * and the fourth of a split row are that row's re-drive field: the sensory row it re-drives (>= 0), -1 none, and in
 * the backward -(d + 3) when its hop is the first (from the top) to write sensory row d's gradient, -2 for a sensory
 * row that no hop re-drives.  Returns 0 or -1 (fc_last_error).  (No counterpart in the reference.) */
int fc_net_plan(const char* net, long long len, int product, int backward, int* wave_out, long long wave_cap,
                int* seg_out, long long seg_cap, int* split_out, long long split_cap, int* pos_out, long long pos_cap,
                long long* counts);

/* The backward's reduction tables of a network, from NET.bin bytes on the host (no device).  which 0: for hop
 * 1 .. hops, the neuron of each gain / threshold partial column of its backward (the plan's segments, then its split
 * rows; -1 for a segment of a split row); 1: the strength of each backward plan position, 2: the column neurons,
 * 3: the top layer's neurons (hop ignored), each with the first write in a backward's order of reductions (top
 * layer, then hop K's strengths and columns, down to hop 1) marked -(i + 2) for entry i, later writes i, nothing -1.
 * Copies at most cap ints into out (null: none) and returns the length, or -1 (fc_last_error).  (No counterpart in
 * the reference.) */
long long fc_net_marks(const char* net, long long len, int hop, int which, int* out, long long cap);

/* ---- the HopCuda-style hop (flyguy/fly_cuda.py:78-115): states [rows][B] row-major, B % 32 == 0 ---- */

/* out[n_rows][B] = A h for the CSR matrix A (n_rows rows over n_src sources, E weights w in CSR order), through the
 * row plan of its row pointer (fc_plan_rows, copied to the device): wave (2 ints per wave), seg (4 ints per
 * segment), split (4 ints per split row), nslot; pcol / pidx: per plan position its source row col[pos] and weight
 * index pos (both for an unused position: pidx -1).  cw: scratch of npos (col, w) pairs; scratch: nslot * B floats.
 * All device.  Replaces the spmm_f kernel, fly_cuda.py:27-33. */
void fh_spmm(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
             const int* pcol, const int* pidx, long long npos, const float* w, const float* h, float* out, int n_rows,
             int n_src, int B, void* cw, float* scratch, void* stream);

/* fh_spmm without the two workspace arguments, for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops that forbid allocation).  No counterpart in the reference: the pairs and the split rows'
 * partial sums go to a static device workspace of FH_STATIC_BYTES per GPU (held until the process ends), so a call
 * allocates nothing.  A product needs 8 bytes per plan position (rounded up to 256) + 4 * nslot * B bytes; a larger
 * one is refused with an error (fc_last_error).  Calls on one GPU share its workspace: calls that overlap on one GPU
 * (several streams or threads) race. */
#define FH_STATIC_BYTES (32u << 20)
void fh_spmm_static(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                    const int* pcol, const int* pidx, long long npos, const float* w, const float* h, float* out,
                    int n_rows, int n_src, int B, void* stream);

/* Backward of fh_spmm: gh[n_src][B] = A^T gz and gw[e] += sum_b gz[row_e][b] h[col_e][b] (gw is added to), through the
 * row plan of the transposed (CSC) row pointer: pcol / pidx per position the CSC column tcol[pos] (a row of gz) and
 * the CSR edge tperm[pos] it is.  gwpart: scratch of npos * B/32 floats (unused when gw is null); scratch: nslot * B
 * floats.  Replaces sddmm_f + spmm_f over the CSC, fly_cuda.py:45-50,93-115. */
void fh_spmm_bwd(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                 const int* pcol, const int* pidx, long long npos, const float* w, const float* gz, const float* h,
                 float* gh, float* gw, int n_rows, int n_src, int B, void* cw, float* gwpart, float* scratch,
                 void* stream);

/* ---- the same products over states copied to the tiled layout [B/32][rows][32] (a row's 32 samples of a tile in
 * one 128-byte line, a tile's rows contiguous).  No counterpart in the reference: the gathers of a product read one
 * tile's slab of rows at a time, which the tiled layout keeps in a few MB of contiguous memory, where the row-major
 * layout scatters it at a stride of B floats; on MI355X the tiled products take about half the time. ---- */

/* out[B/32][rows][32] = x[rows][B] (B % 32 == 0): the layout fh_spmm_tiled and fh_spmm_bwd_tiled read. */
void fh_to_tiled(const float* x, int rows, int B, float* out, void* stream);

/* fh_spmm with the states ht tiled (fh_to_tiled); out stays [n_rows][B] row-major.  Arguments as fh_spmm. */
void fh_spmm_tiled(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                   const int* pcol, const int* pidx, long long npos, const float* w, const float* ht, float* out,
                   int n_rows, int n_src, int B, void* cw, float* scratch, void* stream);

/* fh_spmm_bwd with the gradient gzt tiled (fh_to_tiled, [B/32][n_rows][32]); h and gh stay [n_src][B] row-major.
 * Arguments as fh_spmm_bwd. */
void fh_spmm_bwd_tiled(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                       const int* pcol, const int* pidx, long long npos, const float* w, const float* gzt, const float* h,
                       float* gh, float* gw, int n_rows, int n_src, int B, void* cw, float* gwpart, float* scratch,
                       void* stream);

/* ---- the neuron activation of FlyActor's GPU path, h = relu(g z - t) per row, for the PyTorch elementwise steps of
 * fly.py:296-304 (fire).  No counterpart in the library of the reference: its GPU actor path (fly.py:170-185) forms
 * it from three PyTorch operations, each a pass over the states.  z, h: [rows][B] row-major float32, B % 4 == 0;
 * g, t: per row (the gain and softplus(theta) of the row's neuron).  The product and the difference are rounded
 * separately, as PyTorch rounds them, so h is PyTorch's bit for bit. ---- */
void fh_fire(const float* z, const float* g, const float* t, int rows, int B, float* h, void* stream);

/* The backward of fh_fire from gh, the gradient of h: gz = gh g where g z - t is not <= 0 (PyTorch's relu passes a
 * NaN's gradient on), else 0; per row the gradients of g and t, gg = sum of gh z and gt = -(sum of gh) over those
 * samples. */
void fh_fire_bwd(const float* gh, const float* z, const float* g, const float* t, int rows, int B, float* gz, float* gg,
                 float* gt, void* stream);

/* ---- 16-bit states (the reference's half path, fly_cuda.py:34-56, 93-115): products read states and gradients as
 * IEEE binary16 and accumulate in float32.  A 16-bit state tensor is tiled: [ceil(B/64)][rows][64] halves, samples
 * past B zero. ---- */

/* out (tiled binary16) = x / (*scale, when scale is not null) rounded to nearest even; x is row-major float32
 * [rows][B], B % 32 == 0.  The reference's h.half() and (gz / scale).half(), fly_cuda.py:93, 103-104. */
void fh_to_half(const float* x, int rows, int B, const float* scale, void* out, void* stream);

/* *out = max(max |x[i]|, 1e-30) over n floats (device scalar): the reference's gz.abs().max().clamp_min(1e-30),
 * fly_cuda.py:103 (a NaN in x is not propagated). */
void fh_absmax(const float* x, long long n, float* out, void* stream);

/* fh_spmm with the states hs in binary16 (tiled, from fh_to_half): out[n_rows][B] float32.  scratch: nslot *
 * ceil(B/64) * 64 floats.  Replaces spmm_h, fly_cuda.py:34-39. */
void fh_spmm_h(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
               const int* pcol, const int* pidx, long long npos, const float* w, const void* hs, float* out, int n_rows,
               int n_src, int B, void* cw, float* scratch, void* stream);

/* fh_spmm_bwd with binary16 gradients gzs = half(gz / scale) and states hs (both tiled): gh[n_src][B] = scale *
 * A^T gzs, and gw[e] += scale * sum_b gzs[row_e][b] hs[col_e][b].  scale: device scalar (fh_absmax).  gwpart:
 * npos * ceil(B/64) floats; scratch: nslot * ceil(B/64) * 64 floats.  Replaces sddmm_h + spmm_h over the CSC and
 * the scaling of fly_cuda.py:100-114. */
void fh_spmm_bwd_h(const int* wave, int nwave, const int* seg, int nseg, const int* split, int nsplit, int nslot,
                   const int* pcol, const int* pidx, long long npos, const float* w, const void* gzs, const void* hs,
                   const float* scale, float* gh, float* gw, int n_rows, int n_src, int B, void* cw, float* gwpart,
                   float* scratch, void* stream);

#ifdef __cplusplus
}
#endif
#endif
