/* The standalone teaching trainer of the flyguy MI355X library (libflyguy_core.so), and the pieces of its data path,
 * survey and revive surgery that callers and tests reach directly.  C-ABI: plain pointers and sizes.
 *
 * Replaces the reference's trainer executable flyguy/native/flyguy_train.cu (main, :631-787) and its host
 * helpers.  Files (little endian):
 *   FLYD chunk  "FLYD", n (int64), obs_dim (int32), n_act (int32), obs [n][obs_dim] binary16, teacher logits
 *               [n][n_act] binary16                                                (flyguy_train.cu:372-384)
 *   FLYP params "FLYP", step (int64), float32 W, gain, theta, in_w, in_b, out_w, out_b          (:258-286)
 *   FLYO Adam   "FLYO", step (int64), adam_t (int64), then per array m and v (float32)          (:288-307)
 *   FLYB batch  "FLYB", B (int32), obs [B][obs_dim] float32, teacher [B][n_act] float32         (:632-653)
 * Device pointers are marked (device); everything else is host memory.
 */
#ifndef FLYGUY_TRAIN_H
#define FLYGUY_TRAIN_H

#ifdef __cplusplus
extern "C" {
#endif

/* The trainer's command line (flyguy_train.cu:631-787):
 *   NET PARAMS_IN DATA_DIR OUT_PREFIX [--batch 512] [--lr 3e-4] [--lr-neuron 1e-4] [--lr-plug 3e-4] [--lr-min 3e-5]
 *     [--half-life 20000] [--passes 1] [--ema 0.999] [--log 100] [--save-sec 120] [--steps 0] [--clip 0] [--temp 1]
 *     [--eval-batches 16] [--revive-every 0] [--revive-batches 4] [--revive-target 0.4] [--revive-first 0]
 *     [--ring 3] [--max-reuse 4] [--holdout 0] [--eval-every 0] [--bf16 0]
 *   --bf16 1 trains on the library core with bfloat16 states and edge weights (FC_STATES_BF16; the batch a multiple
 *   of 64): an addition of this library, the reference's trainer is float32 only.
 *   --check NET PARAMS BATCH      one forward + backward of a FLYB batch; prints loss, agreement, logits, gradients
 * argv[0] is the program name.  Returns the process exit status (0 done or stopped, 1 file or device error,
 * 2 usage).  Writes OUT_PREFIX.bin, .ema.bin, .opt.bin; a file OUT_PREFIX.STOP ends the run after a save. */
int ft_main(int argc, const char* const* argv);

/* The batch draw of the trainer (flyguy_train.cu:412-424): n_batches consecutive batches of B samples from one
 * std::mt19937_64 seeded with `seed`; each sample uniform over the concatenation of the chunks (sizes[i] samples
 * in chunk i).  out [n_batches * B][2] = {chunk, sample}.  Returns 0, or -1 on bad arguments. */
int ft_draw(unsigned long long seed, const long long* sizes, int n_chunks, int B, int n_batches, int* out);

/* The learning rates of one step (flyguy_train.cu:764-769): sched = 0.5^(step / half_life); per group
 * max(lr_min * base / lr, base * sched) for base = lr, lr_neuron, lr_plug -> out[3]. */
void ft_lr(long long step, float lr, float lr_neuron, float lr_plug, float lr_min, double half_life, float* out);

/* Samples in a FLYD chunk file that the trainer accepts for a network of (obs_dim, n_act): the whole file is read
 * and checked as the trainer reads it (:372-384).  -1 if the file is missing, short, or of other sizes. */
long long ft_chunk_samples(const char* path, int obs_dim, int n_act);

/* The chunk files a first scan of `dir` loads, oldest first (:392-404): the names of chunk_*.bin, sorted by
 * modification time, of several only the newest `keep`; written '\n'-separated into out (cap bytes).  Returns
 * the number of names, or -1 if they do not fit. */
int ft_scan_order(const char* dir, int keep, char* out, int cap);

/* Rows of the drawn samples from chunks in device memory (flyguy_train.cu:56-61): sample b is sample sel[b].y of
 * chunk sel[b].x (obs_tab / lg_tab / n_tab (device): per chunk the binary16 obs [n][obs_dim], logits [n][n_act]
 * and n).  Writes obs [B][obs_dim] and teacher [B][n_act] float32 (device).  A selection outside the chunks
 * gives a row of NaN. */
void fd_gather16(const void* const* obs_tab, const void* const* lg_tab, const long long* n_tab, int n_chunks,
                 const int* sel, int B, int obs_dim, int n_act, float* obs, float* teacher, void* stream);

/* A staged batch st [B][obs_dim + n_act] binary16 (device) -> obs [B][obs_dim], teacher [B][n_act] float32
 * (flyguy_train.cu:62-66). */
void fd_unpack16(const void* st, int B, int obs_dim, int n_act, float* obs, float* teacher, void* stream);

/* Layer sizes of a network handle: sizes[0] sensory rows, sizes[k] rows of hop k; returns hops + 1 (or -1 when
 * cap is too small).  Survey arrays hold the rows of every layer in this order. */
int fc_layers(void* core, int* sizes, int cap);

/* One batch of a survey (flyguy_train.cu:181-187, 436-454): forward through the weights (ema = 1: the running
 * average) of obs [B][obs_dim] (device), the loss against teacher [B][n_act] (device) at 1/temperature `it`,
 * and per row of every layer the samples for which it fires (h > 0) and the sum of its squared pre-activation
 * (hop layers; 0 for the sensory layer).  reset = 1 clears the sums first.  Replaces the states of the last
 * forward (an fc_backward must follow a new fc_forward).  On a bfloat16-state handle (FC_STATES_BF16) the counts
 * and squares are those of the stored bfloat16 states and pre-activations.  Returns 0 or -1. */
int fc_survey(void* core, const float* obs, const float* teacher, int B, int ema, float it, int reset);

/* The survey sums so far: cnt, sq [rows of every layer]; stats = {KL sum, agreements, samples}.  Returns the
 * number of rows, or -1. */
long long fc_survey_read(void* core, int* cnt, float* sq, double* stats);

/* Silent neurons back to work with the network's output unchanged (flyguy_train.cu:479-551): every neuron past
 * the sensory layer that fires for none of the samples gets new signs on its incoming strengths (std::mt19937_64
 * seeded seed * 7919 + 17), gain 1 and threshold -4, zero outgoing strengths onto live neurons and onto the
 * actions, then its incoming strengths are scaled in three surveys until its input's rms is `target`; the running
 * average and Adam's state follow.  obs / teacher (device): `batches` batches of B samples, [batches * B][...].
 * report (cap bytes): the trainer's report line.  Returns the number of silent neurons, or -1. */
int fc_revive(void* core, const float* obs, const float* teacher, int B, int batches, float target,
              unsigned long long seed, long long step, char* report, int cap);

#ifdef __cplusplus
}
#endif
#endif
