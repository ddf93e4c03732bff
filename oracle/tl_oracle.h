/* tl_oracle.h -- CPU oracle for the fp32 GEMM hot path of tinylm.c.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links this: only tests/,
 * __graft_entry__.smoke() (as the checker) and bench.py's cpu_baseline leg
 * load it.  It restates, from scratch, the arithmetic of the reference's
 * portable kernels so that a GPU result can be compared with what tinylm.c
 * computes on identical inputs.
 *
 * Pinning (how each function is checked, so a dropped term / wrong index /
 * transposed operand fails somewhere):
 *   orc_mm, orc_mm_bt, orc_mm_atb   golden fixtures written by the reference's
 *                                   own compiled kernels (tests/golden), the
 *                                   fp64 textbook loops below, and invariants
 *                                   (set vs accumulate, identity W, linearity).
 *   orc_*_f64                       closed-form textbook GEMM in double; checked
 *                                   against exact small-integer cases and brute
 *                                   force in tests/test_oracle.py.
 *   orc_rng_*                       the reference's xorshift/Box-Muller draw,
 *                                   pinned by the fixtures' stored inputs.
 *   orc_moe_*                       brute-force per-token expert evaluation in
 *                                   fp64 (tests/test_oracle.py) and the reference
 *                                   MoE compiled from its own source (fixtures).
 *   orc_rmsnorm_*, orc_rope*,       (tl_oracle_step.c) fixtures written by the
 *   orc_attn_*, orc_adamw,          reference's own compiled functions
 *   orc_gradnorm, orc_train_step    (tests/golden/step_*.npz), fp64 forms and
 *                                   closed forms (rotation norms, softmax rows
 *                                   summing to one, finite-difference
 *                                   gradients) in tests/test_oracle.py.
 *   orc_xent, orc_embed_*           the whole-step fixtures (loss and the
 *                                   embedding gradient) and closed forms.
 */
#ifndef TL_ORACLE_H
#define TL_ORACLE_H
#include <stdint.h>
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- the three primitives, same argument meaning as tinylm.c ---------- */
/* Y[M*N]  = X[M*K] @ W[K*N]          (set)         tinylm.c:438-478 */
void orc_mm(float *Y, const float *X, const float *W, int M, int K, int N);
/* dX[M*K] += dY[M*N] @ W[K*N]^T      (accumulate)  tinylm.c:480-508 */
void orc_mm_bt(float *dX, const float *dY, const float *W, int M, int K, int N);
/* dW[K*N] += X[M*K]^T @ dY[M*N]      (accumulate)  tinylm.c:510-537 */
void orc_mm_atb(float *dW, const float *X, const float *dY, int M, int K, int N);

/* Decode-pool dispatch emulation (tinylm.c:237-245, :446, :486).  nt<=1 is
 * the training setting (OpenMP), nt>1 emulates a live tl_for pool of nt
 * workers: ranges of fewer than nt items run serially on the caller. */
void orc_set_pool(int nt);
int  orc_threads(void);            /* OpenMP threads the oracle will use */
/* on != 0: M <= 8 mm / mm_bt calls split their outputs over the OpenMP
 * threads (column / W-row ranges, each element's chain unchanged): the
 * threaded variant of the CPU decode baseline.  0 (default): the
 * reference's dispatch. */
void orc_set_gemv_split(int on);
void orc_set_threads(int nt);      /* omp_set_num_threads */

/* ---- fp64 textbook references (the selftest pattern, tinylm.c:4764-4766),
 * extended with the accumulator prefill that mm_bt / mm_atb add into. ---- */
void orc_mm_f64(float *Y, const float *X, const float *W, int M, int K, int N);
void orc_mm_bt_f64(float *dX, const float *dY, const float *W, int M, int K, int N);
void orc_mm_atb_f64(float *dW, const float *X, const float *dY, int M, int K, int N);

/* ---- RNG: xorshift64 (13,7,17) + Box-Muller, tinylm.c:127-134 ---------- */
void     orc_rng_seed(uint64_t s);
uint64_t orc_rng_state(void);
uint64_t orc_xorshift(void);
float    orc_rnd_normal(void);
void     orc_fill_normal(float *p, size_t n, float scale);

/* ---- top-1 MoE (tinylm.c:814-827, :857-947), K=1 routing, no router bias.
 * fnorm[N*D], fin[N*D] -> out[N*D]; assign[N], gate[N], rprobs[N*E] written.
 * w1,w3: E x [D*F], w2: E x [F*D], wr: [D*E]; scratch handled internally. */
void orc_moe_forward(int N, int D, int F, int E,
                     const float *fnorm, const float *fin, float *out,
                     const float *wr, const float *w1, const float *w3, const float *w2,
                     int *assign, float *gate, float *rprobs);
/* dout[N*D] -> d_fnorm[N*D] (set); gw1/gw3/gw2/gwr accumulate. */
void orc_moe_backward(int N, int D, int F, int E,
                      const float *fnorm, const float *dout, float *d_fnorm,
                      const float *wr, const float *w1, const float *w3, const float *w2,
                      float *gwr, float *gw1, float *gw3, float *gw2,
                      const int *assign, const float *gate, const float *rprobs);

/* ---- training-step glue (tl_oracle_step.c), tinylm.c:539-1176 ---------- */
void   orc_embed_fwd(float *out, const float *emb, const int *tok, int N, int D);           /* :972-976   */
void   orc_embed_bwd(float *demb, const float *dout, const int *tok, int N, int D);        /* :1149-1153 */
void   orc_rmsnorm_fwd(const float *x, const float *g, float *out, float *rinv, int rows, int D); /* :540 */
void   orc_rmsnorm_bwd(const float *x, const float *g, const float *rinv, const float *dy, float *dx,
                       float *dg, int rows, int D);                                         /* :565-588 */
void   orc_rope_table(float *cs, float *sn, int maxpos, int hd, float base);               /* :605-619 */
void   orc_rope(float *buf, const int *pos, int T, int rows, int nh, int hd, const float *cs,
                const float *sn, int back);                                                 /* :630-651 */
void   orc_attn_fwd(const float *q, const float *k, const float *v, float *out, int B, int T, int H,
                    int KV, int hd, int win);                                               /* :699-732 */
void   orc_attn_bwd(const float *q, const float *k, const float *v, const float *datt, float *dq,
                    float *dk, float *dv, int B, int T, int H, int KV, int hd, int win);    /* :734-783 */
double orc_xent(const float *logits, const int *tgt, float *dl, float scale, int N, int V);
float  orc_gradnorm(const float *G, size_t n);                                               /* :1171 */
void   orc_adamw(float *P, const float *G, float *M, float *V, size_t n, float lr, float b1, float b2,
                 float wd, int t, float gscale);                                             /* :1159 */

/* A model (tinylm.c Cfg :35-59 without shared experts) and its flat
 * parameter layout (map_weights :361-393: the QK-norm gains qn, kn (hd each)
 * between wo and an2 when qknorm, wr and the E expert slots when n_exp > 0).
 * The training step runs qknorm = 0 only (the reference refuses to train
 * QK-norm models, :2707-2713); the decoder runs both. */
typedef struct { int V, D, L, H, KV, F, T, n_mtp, n_exp, win, full_every; float rope_base; int qknorm; } OrcModel;
typedef struct { size_t emb, an1, wq, wk, wv, wo, qn, kn, an2, wr, w1, w3, w2, nf, mtp0, total; } OrcLayerMap;
void  orc_param_map(const OrcModel *m, int layer, OrcLayerMap *o);
/* init_params (:395-419) from the reference generator seeded with `seed` */
void  orc_init_params(const OrcModel *m, float *P, uint64_t seed);
/* forward + memset(G) + backward of one batch of B sequences; returns the
 * loss.  tgt_mtp: n_mtp x (B*T) targets of the MTP heads. */
float orc_train_step(const OrcModel *m, int B, const float *P, float *G, const int *tok, const int *tgt,
                     const int *tgt_mtp);

/* qknorm_apply (:597-605): each of rows x nheads head vectors of hd values
 * becomes v * s * gain with s = 1 / sqrt(sum(v^2) / hd + 1e-5). */
void orc_qknorm(float *buf, const float *gain, int rows, int nheads, int hd);
/* The decode MoE layer (moe_forward_q8's fp32 branch, :3433-3458): router
 * logits fnorm . wr, softmax (expf) and the first maximum per row; out = fin,
 * then per expert in order its rows (in row order): a = silu(x W1) * (x W3),
 * out[n] += gate[n] * (a W2).  K = 1 routing, no router bias. */
void orc_dec_moe(int N, int D, int F, int E, const float *fnorm, const float *fin, float *out, const float *wr,
                 const float *w1, const float *w3, const float *w2, int *assign, float *gate, float *rprobs);

/* ---- decode: forward_chunk (:3721-3830), fp32 weights ---------------------
 * A ring KV cache of W positions per layer stored as f32 (kvdt 0) or f16
 * (kvdt 1, the reference default), the unsplit attention path, and the
 * softmax exponential fast_expf (exact_exp 0, the default) or expf.  maxpos
 * sizes the RoPE table (positions 0..maxpos-1). */
typedef struct OrcDec OrcDec;
OrcDec *orc_dec_new(const OrcModel *m, int W, int kvdt, int exact_exp, int maxpos);
void    orc_dec_free(OrcDec *d);
void    orc_dec_chunk(OrcDec *d, const float *P, const int *tok, int m, int start_pos, float *logits);
/* orc_dec_chunk that also returns the final-normed rows fn [m][D] (the rows
 * the MTP heads read, gn->fn of forward_chunk :3828). */
void    orc_dec_chunk_fn(OrcDec *d, const float *P, const int *tok, int m, int start_pos, float *logits,
                         float *fn);
/* mtp_argmax (:3930-3936): head k's draft from a final-normed row fn1 [D]:
 * argmax_v((fn1 + silu(fn1 Wk)) emb^T); its logits [V] into logits. */
int     orc_mtp_argmax(const OrcModel *m, const float *P, const float *fn1, int k, float *logits);
/* One layer's attention step of orc_dec_chunk: ring stores of the m new K / V
 * rows, then attention of the m query rows (q [m][D], k / v [m][KD], ctx
 * [m][D]). */
void    orc_dec_attn(OrcDec *d, int l, const float *q, const float *k, const float *v, int m, int start_pos,
                     float *ctx);
/* Test hooks for checking a decoder whose f16 ring rounds K / V rows computed
 * in another fp32 order: overwrite layer l's ring with given contents ([W][KD]
 * in the ring's storage type), and switch the chunk's ring stores off (store
 * 0) so attention reads the ring as given -- the state a chunk attends over
 * after its hoisted stores, when the given ring was taken after that chunk. */
void    orc_dec_set_ring(OrcDec *d, int l, const void *K, const void *V);
const void *orc_dec_ring(const OrcDec *d, int l, int v);       /* layer l's K (v 0) or V ring */
void    orc_dec_set_store(OrcDec *d, int store);
float          orc_fast_expf(float x);         /* :3181-3191 */
unsigned short orc_f2h(float f);               /* :3158-3168 (F16C path) */
float          orc_h2f(unsigned short h);      /* :3147-3157 */

/* A plan's call list run in C (CPU baseline of short calls): op 0 mm,
 * 1 mm_bt, 2 mm_atb, 3 memset of n floats; `reps` passes over the list. */
typedef struct { int op; float *out; const float *a, *b; int M, K, N; size_t n; } OrcCall;
void orc_run_calls(const OrcCall *c, int n, int reps);

#ifdef __cplusplus
}
#endif
#endif
