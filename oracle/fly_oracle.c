/* ORACLE - test infrastructure only.  A CPU restatement of the reference's arithmetic for the fly actor's
 * forward, KL loss, backward and Adam, against which tests/, __graft_entry__.smoke() and bench.py's CPU baseline
 * hold the MI355X library.  It is never part of the product path.
 *
 * Compiled twice (oracle/Makefile): REAL=float follows the reference kernels' per-element arithmetic and
 * summation order (flyguy/native/flyguy_train.cu, fused multiply-adds as nvcc contracts them); REAL=double
 * is the same algorithm in double precision, the accuracy yardstick.  Reductions over the batch (per-connection
 * and per-neuron gradients), which the reference sums in a scheduling-dependent order (warp trees + atomics,
 * flyguy_train.cu:153-166), are accumulated in double in both builds.
 *
 * It reads NET.bin ("FLY1", flyguy/native/export.py:9-15,52-65) with its own parser.  States are [rows][B].
 *
 * Functions and the reference lines they follow:
 *   or_forward   k_plug :73-78, k_act0 :79-83 (softplus :51), k_hop :84-94, k_logits :95-101,
 *                forward_logits :320-332
 *   or_loss      k_loss :104-123
 *   or_backward  backward :339-359: k_out_bwd_w :125-135, k_out_bwd_h :136-141, k_hop_bwd :143-156,
 *                k_sddmm :158-167, k_spmmT :168-173, k_rowsum :174-179
 *   or_adam      k_adam :194-203 with fc_step's bias corrections :619-627
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifndef REAL
#define REAL double
#endif

#ifdef ORACLE_F32
#define FMA fmaf
#define EXP expf
#define LOG logf
#define LOG1P log1pf
#else
#define FMA fma
#define EXP exp
#define LOG log
#define LOG1P log1p
#endif

typedef struct {
    int rows, src, E;
    int *nid, *crow, *col, *widx, *tcrow, *tcol, *twidx, *drow;
    REAL *z, *h, *gh;
} OHop;

typedef struct {
    int obs_dim, n_act, hops, n_neurons, n_w, n_s, fan, n_dn, E_in;
    int *sizes, *in_crow, *in_col, *n0, *dn;
    OHop* hop;
    long long psize[7];
    REAL* p[7];                 /* W, gain, theta, in_w, in_b, out_w, out_b */
    int B;
    REAL *x, *drive, *h0, *gh0, *gdrive;
    int cap_B;
} Oracle;

static int rd_ints(const unsigned char* b, long long n, long long* at, int* out, long long k) {
    if (k < 0 || *at + 4 * k > n) return -1;
    if (k) memcpy(out, b + *at, (size_t)(4 * k));
    *at += 4 * k;
    return 0;
}
static int* take(const unsigned char* b, long long n, long long* at, long long k, int* bad) {
    int* v = (int*)malloc((size_t)(k > 0 ? k : 1) * sizeof(int));
    if (!v || rd_ints(b, n, at, v, k)) *bad = 1;
    return v;
}

void or_free(void* h);

void* or_create(const void* net, long long len) {
    const unsigned char* b = (const unsigned char*)net;
    long long at = 4;
    int hd[8], bad = 0, k;
    if (!b || len < 36 || memcmp(b, "FLY1", 4) || rd_ints(b, len, &at, hd, 8)) return NULL;
    Oracle* o = (Oracle*)calloc(1, sizeof(Oracle));
    o->obs_dim = hd[0]; o->n_act = hd[1]; o->hops = hd[2]; o->n_neurons = hd[3];
    o->n_w = hd[4]; o->n_s = hd[5]; o->fan = hd[6]; o->n_dn = hd[7];
    if (o->hops <= 0 || o->hops > 64 || o->n_s <= 0 || o->fan <= 0) { free(o); return NULL; }
    o->E_in = o->n_s * o->fan;
    o->sizes = take(b, len, &at, o->hops + 1, &bad);
    int* E = take(b, len, &at, o->hops, &bad);
    if (bad) { free(E); or_free(o); return NULL; }
    o->in_crow = take(b, len, &at, o->n_s + 1, &bad);
    o->in_col = take(b, len, &at, o->E_in, &bad);
    at += 4LL * (o->obs_dim + 1 + 2LL * o->E_in);            /* the plug's transposed form */
    o->n0 = take(b, len, &at, o->n_s, &bad);
    o->hop = (OHop*)calloc((size_t)o->hops, sizeof(OHop));
    for (k = 0; k < o->hops && !bad; ++k) {
        OHop* h = &o->hop[k];
        h->rows = o->sizes[k + 1]; h->src = o->sizes[k]; h->E = E[k];
        h->nid = take(b, len, &at, h->rows, &bad); h->crow = take(b, len, &at, h->rows + 1, &bad);
        h->col = take(b, len, &at, h->E, &bad); h->widx = take(b, len, &at, h->E, &bad);
        h->tcrow = take(b, len, &at, h->src + 1, &bad); h->tcol = take(b, len, &at, h->E, &bad);
        h->twidx = take(b, len, &at, h->E, &bad); h->drow = take(b, len, &at, h->rows, &bad);
    }
    free(E);
    o->dn = take(b, len, &at, o->n_dn, &bad);
    if (bad) { or_free(o); return NULL; }
    long long ps[7] = {o->n_w, o->n_neurons, o->n_neurons, o->E_in, o->n_s, (long long)o->n_act * o->n_dn, o->n_act};
    for (k = 0; k < 7; ++k) { o->psize[k] = ps[k]; o->p[k] = (REAL*)calloc((size_t)(ps[k] > 0 ? ps[k] : 1), sizeof(REAL)); }
    return o;
}

void or_free(void* ptr) {
    Oracle* o = (Oracle*)ptr;
    int k;
    if (!o) return;
    if (o->hop)
        for (k = 0; k < o->hops; ++k) {
            OHop* h = &o->hop[k];
            free(h->nid); free(h->crow); free(h->col); free(h->widx); free(h->tcrow); free(h->tcol); free(h->twidx);
            free(h->drow); free(h->z); free(h->h); free(h->gh);
        }
    free(o->hop); free(o->sizes); free(o->in_crow); free(o->in_col); free(o->n0); free(o->dn);
    for (k = 0; k < 7; ++k) free(o->p[k]);
    free(o->x); free(o->drive); free(o->h0); free(o->gh0); free(o->gdrive);
    free(o);
}

void or_sizes(void* ptr, long long* out) {
    Oracle* o = (Oracle*)ptr;
    int k;
    for (k = 0; k < 7; ++k) out[k] = o->psize[k];
    out[7] = o->obs_dim; out[8] = o->n_act; out[9] = o->hops;
}

/* the seven weight arrays (float, as the reference stores them) */
void or_set_params(void* ptr, const float* const* p7) {
    Oracle* o = (Oracle*)ptr;
    long long i;
    int k;
    for (k = 0; k < 7; ++k)
        for (i = 0; i < o->psize[k]; ++i) o->p[k][i] = (REAL)p7[k][i];
}

static void ensure(Oracle* o, int B) {
    int k;
    if (B <= o->cap_B) return;
    free(o->x); free(o->drive); free(o->h0); free(o->gh0); free(o->gdrive);
    o->x = (REAL*)calloc((size_t)o->obs_dim * B, sizeof(REAL));
    o->drive = (REAL*)calloc((size_t)o->n_s * B, sizeof(REAL));
    o->h0 = (REAL*)calloc((size_t)o->n_s * B, sizeof(REAL));
    o->gh0 = (REAL*)calloc((size_t)o->n_s * B, sizeof(REAL));
    o->gdrive = (REAL*)calloc((size_t)o->n_s * B, sizeof(REAL));
    for (k = 0; k < o->hops; ++k) {
        OHop* h = &o->hop[k];
        free(h->z); free(h->h); free(h->gh);
        h->z = (REAL*)calloc((size_t)h->rows * B, sizeof(REAL));
        h->h = (REAL*)calloc((size_t)h->rows * B, sizeof(REAL));
        h->gh = (REAL*)calloc((size_t)h->rows * B, sizeof(REAL));
    }
    o->cap_B = B;
}

static REAL softplus(REAL v) { return v > (REAL)20 ? v : LOG1P(EXP(v)); }
static REAL relu(REAL v) { return v > (REAL)0 ? v : (REAL)0; }

/* obs [B][obs_dim] -> logits [B][n_act]; the states are kept for or_backward */
int or_forward(void* ptr, const float* obs, int B, float* logits) {
    Oracle* o = (Oracle*)ptr;
    const REAL *W = o->p[0], *gain = o->p[1], *theta = o->p[2], *in_w = o->p[3], *in_b = o->p[4], *ow = o->p[5], *ob = o->p[6];
    int t, b, k, a, j, e;
    if (B <= 0) return -1;
    ensure(o, B);
    o->B = B;
    for (b = 0; b < B; ++b)
        for (t = 0; t < o->obs_dim; ++t) o->x[(size_t)t * B + b] = (REAL)obs[(size_t)b * o->obs_dim + t];
#pragma omp parallel for private(b, e)
    for (t = 0; t < o->n_s; ++t) {                               /* plug + sensory layer */
        REAL* d = o->drive + (size_t)t * B;
        const REAL sp = softplus(theta[o->n0[t]]), g = gain[o->n0[t]];
        for (b = 0; b < B; ++b) d[b] = in_b[t];
        for (e = o->in_crow[t]; e < o->in_crow[t + 1]; ++e) {
            const REAL w = in_w[e], *xs = o->x + (size_t)o->in_col[e] * B;
            for (b = 0; b < B; ++b) d[b] = FMA(w, xs[b], d[b]);
        }
        for (b = 0; b < B; ++b) o->h0[(size_t)t * B + b] = relu(FMA(g, d[b], -sp));
    }
    const REAL* hp = o->h0;
    for (k = 0; k < o->hops; ++k) {
        OHop* h = &o->hop[k];
#pragma omp parallel for private(b, e)
        for (t = 0; t < h->rows; ++t) {
            REAL* z = h->z + (size_t)t * B;
            const int n = h->nid[t];
            const REAL sp = softplus(theta[n]), g = gain[n];
            for (b = 0; b < B; ++b) z[b] = 0;
            for (e = h->crow[t]; e < h->crow[t + 1]; ++e) {
                const REAL w = W[h->widx[e]], *s = hp + (size_t)h->col[e] * B;
                for (b = 0; b < B; ++b) z[b] = FMA(w, s[b], z[b]);
            }
            if (h->drow[t] >= 0) {
                const REAL* d = o->drive + (size_t)h->drow[t] * B;
                for (b = 0; b < B; ++b) z[b] += d[b];
            }
            for (b = 0; b < B; ++b) h->h[(size_t)t * B + b] = relu(FMA(g, z[b], -sp));
        }
        hp = h->h;
    }
#pragma omp parallel for private(a, j)
    for (b = 0; b < B; ++b)
        for (a = 0; a < o->n_act; ++a) {
            REAL acc = ob[a];
            for (j = 0; j < o->n_dn; ++j) acc = FMA(ow[(size_t)a * o->n_dn + j], hp[(size_t)o->dn[j] * B + b], acc);
            logits[(size_t)b * o->n_act + a] = (float)acc;
        }
    return 0;
}

/* a state of the last forward -> out [rows][B]: layer 0 sensory, k the output of hop k; what 0 h, 1 z (drive) */
int or_state(void* ptr, int layer, int what, float* out) {
    Oracle* o = (Oracle*)ptr;
    const REAL* s;
    long long n, i;
    if (layer < 0 || layer > o->hops) return -1;
    if (layer == 0) { s = what ? o->drive : o->h0; n = (long long)o->n_s * o->B; }
    else { s = what ? o->hop[layer - 1].z : o->hop[layer - 1].h; n = (long long)o->hop[layer - 1].rows * o->B; }
    for (i = 0; i < n; ++i) out[i] = (float)s[i];
    return 0;
}

/* KL(teacher || student) per sample; dl [B][n_act]; stats[0] = sum of KL, stats[1] = argmax agreements */
int or_loss(const float* lg, const float* tl, int B, int n_act, float it, float* dl, double* stats) {
    int b, a;
    stats[0] = stats[1] = 0.0;
    for (b = 0; b < B; ++b) {
        const float* s = lg + (size_t)b * n_act;
        const float* t = tl + (size_t)b * n_act;
        REAL ms = (REAL)-1e30, mt = (REAL)-1e30, zs = 0, zt = 0, kl = 0;
        int as = 0, at = 0;
        for (a = 0; a < n_act; ++a) {
            const REAL sv = (REAL)s[a], tv = (REAL)t[a] * (REAL)it;
            if (sv > ms) { ms = sv; as = a; }
            if (tv > mt) { mt = tv; at = a; }
        }
        for (a = 0; a < n_act; ++a) { zs += EXP((REAL)s[a] - ms); zt += EXP((REAL)t[a] * (REAL)it - mt); }
        const REAL ls = ms + LOG(zs), lt = mt + LOG(zt);
        for (a = 0; a < n_act; ++a) {
            const REAL lps = (REAL)s[a] - ls, lpt = (REAL)t[a] * (REAL)it - lt, pt = EXP(lpt);
            kl += pt * (lpt - lps);
            dl[(size_t)b * n_act + a] = (float)((EXP(lps) - pt) / (REAL)B);
        }
        stats[0] += (double)kl;
        stats[1] += as == at ? 1.0 : 0.0;
    }
    return 0;
}

/* the neuron backward of one layer (k_hop_bwd): g = gh where h > 0; gz = g * gain; re-drive; gain / threshold */
static void neuron_bwd(Oracle* o, int rows, int B, const REAL* gh, const REAL* h, const REAL* z, const int* nid,
                       const int* drow, int sensory, REAL* gz, double* ggain, double* gtheta) {
    const REAL *gain = o->p[1], *theta = o->p[2];
    int t, b;
#pragma omp parallel for private(b)
    for (t = 0; t < rows; ++t) {
        const int n = nid[t];
        const int d = sensory ? t : drow[t];
        const REAL sig = (REAL)1 / ((REAL)1 + EXP(-theta[n]));
        double sa = 0, sc = 0;
        for (b = 0; b < B; ++b) {
            const size_t i = (size_t)t * B + b;
            const REAL g = h[i] > (REAL)0 ? gh[i] : (REAL)0;
            const REAL gzv = g * gain[n];
            if (gz) gz[i] = gzv;
            if (d >= 0) o->gdrive[(size_t)d * B + b] += gzv;
            sa += (double)(g * z[i]);
            sc += (double)(-g * sig);
        }
        ggain[n] += sa;
        gtheta[n] += sc;
    }
}

/* dlogits [B][n_act] of the last forward -> gradients ADDED to g7 (float arrays of the seven sizes) */
int or_backward(void* ptr, const float* dlogits, int B, float* const* g7) {
    Oracle* o = (Oracle*)ptr;
    const REAL *W = o->p[0], *ow = o->p[5];
    int t, b, k, a, j, e;
    if (B != o->B) return -1;
    double* G[7];
    for (k = 0; k < 7; ++k) G[k] = (double*)calloc((size_t)(o->psize[k] > 0 ? o->psize[k] : 1), sizeof(double));
    REAL* gz = NULL;
    size_t mx = (size_t)o->n_s;
    for (k = 0; k < o->hops; ++k) if ((size_t)o->hop[k].rows > mx) mx = (size_t)o->hop[k].rows;
    gz = (REAL*)calloc(mx * B, sizeof(REAL));
    memset(o->gdrive, 0, (size_t)o->n_s * B * sizeof(REAL));
    OHop* top = &o->hop[o->hops - 1];
    /* read-out weights: sum over the batch in order (k_out_bwd_w) */
#pragma omp parallel for private(j, b)
    for (a = 0; a < o->n_act; ++a) {
        REAL sb = 0;
        for (b = 0; b < B; ++b) sb += (REAL)dlogits[(size_t)b * o->n_act + a];
        G[6][a] += (double)sb;
        for (j = 0; j < o->n_dn; ++j) {
            REAL acc = 0;
            const REAL* hr = top->h + (size_t)o->dn[j] * B;
            for (b = 0; b < B; ++b) acc = FMA((REAL)dlogits[(size_t)b * o->n_act + a], hr[b], acc);
            G[5][(size_t)a * o->n_dn + j] += (double)acc;
        }
    }
    /* gh of the read-out rows (k_out_bwd_h); other top rows get 0 */
    memset(top->gh, 0, (size_t)top->rows * B * sizeof(REAL));
#pragma omp parallel for private(b, a)
    for (j = 0; j < o->n_dn; ++j)
        for (b = 0; b < B; ++b) {
            REAL acc = 0;
            for (a = 0; a < o->n_act; ++a) acc = FMA(ow[(size_t)a * o->n_dn + j], (REAL)dlogits[(size_t)b * o->n_act + a], acc);
            top->gh[(size_t)o->dn[j] * B + b] = acc;
        }
    for (k = o->hops - 1; k >= 0; --k) {
        OHop* h = &o->hop[k];
        const REAL* below = k ? o->hop[k - 1].h : o->h0;
        REAL* ghb = k ? o->hop[k - 1].gh : o->gh0;
        const int rows_below = k ? o->hop[k - 1].rows : o->n_s;
        neuron_bwd(o, h->rows, B, h->gh, h->h, h->z, h->nid, h->drow, 0, gz, G[1], G[2]);
        /* per-connection gradient (k_sddmm): sum over the batch */
#pragma omp parallel for private(e, b)
        for (t = 0; t < h->rows; ++t)
            for (e = h->crow[t]; e < h->crow[t + 1]; ++e) {
                double s = 0;
                const REAL *gr = gz + (size_t)t * B, *hr = below + (size_t)h->col[e] * B;
                for (b = 0; b < B; ++b) s += (double)gr[b] * (double)hr[b];
                G[0][h->widx[e]] += s;
            }
        /* transposed product (k_spmmT), CSC order */
#pragma omp parallel for private(e, b)
        for (j = 0; j < rows_below; ++j) {
            REAL* out = ghb + (size_t)j * B;
            for (b = 0; b < B; ++b) out[b] = 0;
            for (e = h->tcrow[j]; e < h->tcrow[j + 1]; ++e) {
                const REAL w = W[h->twidx[e]], *gr = gz + (size_t)h->tcol[e] * B;
                for (b = 0; b < B; ++b) out[b] = FMA(w, gr[b], out[b]);
            }
        }
    }
    /* the sensory layer (drive as its input), then the plug (k_rowsum, k_sddmm without widx) */
    neuron_bwd(o, o->n_s, B, o->gh0, o->h0, o->drive, o->n0, NULL, 1, NULL, G[1], G[2]);
#pragma omp parallel for private(e, b)
    for (t = 0; t < o->n_s; ++t) {
        const REAL* gd = o->gdrive + (size_t)t * B;
        double s = 0;
        for (b = 0; b < B; ++b) s += (double)gd[b];
        G[4][t] += s;
        for (e = o->in_crow[t]; e < o->in_crow[t + 1]; ++e) {
            const REAL* xr = o->x + (size_t)o->in_col[e] * B;
            double sw = 0;
            for (b = 0; b < B; ++b) sw += (double)gd[b] * (double)xr[b];
            G[3][e] += sw;
        }
    }
    for (k = 0; k < 7; ++k) {
        long long i;
        for (i = 0; i < o->psize[k]; ++i) g7[k][i] += (float)G[k][i];
        free(G[k]);
    }
    free(gz);
    return 0;
}

/* one Adam step with the running average, as k_adam; c1 / c2 from adam_t as fc_step computes them */
void or_adam(float* p, const float* g, float* m, float* v, float* ema, long long n, float lr, long long adam_t,
             float gs, float decay) {
    const long long t = adam_t < 100000 ? adam_t : 100000;
    const float c1 = 1.f - (float)pow(0.9, (double)t), c2 = 1.f - (float)pow(0.999, (double)t);
    long long i;
    for (i = 0; i < n; ++i) {
        const float gr = g[i] * gs;
        const float mi = fmaf(0.9f, m[i], 0.1f * gr), vi = fmaf(0.999f, v[i], 0.001f * gr * gr);
        m[i] = mi;
        v[i] = vi;
        const float pi = p[i] - lr * (mi / c1) / (sqrtf(vi / c2) + 1e-8f);
        p[i] = pi;
        ema[i] = fmaf(decay, ema[i], (1.f - decay) * pi);
    }
}
