/* Decisions on the host CPU (flyguy_amd/libfly_infer.so): the playing network's forward pass for callers without a
 * GPU.  C-ABI of the reference's flyguy/native/fly_infer.cpp (:33-98), which flyguy/fly.py:186-250 loads with
 * ctypes; same functions, arguments and meaning.  Every pointer is host memory; the library keeps copies of the
 * arrays it is given.  Not thread-safe per handle. */
#ifndef FLY_INFER_H
#define FLY_INFER_H

#ifdef __cplusplus
extern "C" {
#endif

/* A network of `hops` hops reading obs_dim observation values and scoring n_act actions (fly_infer.cpp:33). */
void* fly_create(int obs_dim, int n_act, int hops);

/* The plug and the sensory layer (fly_infer.cpp:37): n_s rows, E connections in CSR order (crow [n_s + 1], col
 * [E] observation index, w [E]), bias b [n_s], gain g0 [n_s] and softplus(theta) t0 [n_s] per sensory row. */
void fly_set_plug(void* net, int n_s, int E, const int* crow, const int* col, const float* w, const float* b,
                  const float* g0, const float* t0);

/* Hop k (0-based) (fly_infer.cpp:43): rows target rows, src source rows, E connections by SOURCE (tcrow [src + 1],
 * tcol [E] target row, w [E]), gain g [rows], softplus(theta) t [rows], drow [rows] the sensory row that keeps
 * driving a target row (-1: none). */
void fly_set_hop(void* net, int k, int rows, int src, int E, const int* tcrow, const int* tcol, const float* w,
                 const float* g, const float* t, const int* drow);

/* The read-out (fly_infer.cpp:48): dn [n_dn] rows of the last layer, w [n_act][n_dn], b [n_act]. */
void fly_set_out(void* net, int n_dn, const int* dn, const float* w, const float* b);

/* obs [batch][obs_dim] -> logits [batch][n_act] (fly_infer.cpp:57-98); tap (or NULL): one byte per neuron state of
 * the first car, layer after layer (sensory first), 255 * tanh(1.5 * firing). */
void fly_forward(void* net, const float* obs, int batch, float* logits, unsigned char* tap);

/* An addition with no counterpart in the reference: decide each car on `threads` threads (<= 0: one per hardware
 * thread; default 1), the calling thread among them.  Each thread owns a range of every layer's rows; the answers
 * and tap bytes are bit-identical to one thread's.  The other threads wait for the next car, spinning for about a
 * millisecond and then asleep; fly_free ends them. */
void fly_set_threads(void* net, int threads);

void fly_free(void* net);

#ifdef __cplusplus
}
#endif
#endif
