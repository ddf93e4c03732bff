/* tltrain.h -- the non-GEMM kernels of tinylm.c's training step, on device
 * pointers (libtlgemm.so, gfx950).  With the GEMM entry points of tlgemm.h
 * they keep a whole forward + backward + AdamW step resident in HBM; the C
 * step driver tinylm-c_amd/host/tl_train.c strings them together in the
 * reference's order.
 *
 * Conventions (as tlgemm.h): every entry is asynchronous on `stream` (a
 * hipStream_t), returns TLG_OK or an error code with tlg_last_error() set,
 * and takes row-major buffers whose row widths are multiples of 4 floats and
 * whose base pointers are 16-byte aligned.  Calls on one stream run in order;
 * calls that need scratch share one library arena, so two streams must not
 * run them concurrently, and the first call at a new size synchronizes the
 * device (so it cannot be captured into a graph -- run one step eagerly
 * before capturing).  Every result is deterministic: no floating-point
 * atomics, fixed reduction orders.
 */
#ifndef TLTRAIN_H
#define TLTRAIN_H
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

/* forward's embedding gather, tinylm.c:972-976: out[n][:] = emb[tok[n]][:]
 * (N x D); a token outside [0, V) makes its row NaN. */
int tlg_dev_embed_fwd(float *out, const float *emb, const int *tok, int N, int D, int V, void *stream);

/* backward's embedding scatter, tinylm.c:1149-1153: demb[tok[n]] += dout[n],
 * the rows of one token added in increasing n as the reference's loop does
 * (bit-identical sums).  Tokens outside [0, V) are skipped. */
int tlg_dev_embed_bwd(float *demb, const float *dout, const int *tok, int N, int D, int V, void *stream);

/* rmsnorm_fwd, tinylm.c:540-563: per row, s = 1/sqrt(mean(x^2) + 1e-5),
 * rinv[r] = s (if rinv), out = x * s * g. */
int tlg_dev_rmsnorm_fwd(const float *x, const float *g, float *out, float *rinv, int rows, int D, void *stream);

/* tlg_dev_embed_fwd into x, then tlg_dev_rmsnorm_fwd of x, in one pass: the
 * forward's embedding gather (:972-976) and its first layer's norm
 * (:540-563), the same x, out and rinv bit for bit (no counterpart as one
 * call).  emb [V][D]; x, out [N][D]. */
int tlg_dev_embed_rmsnorm_fwd(const float *emb, const int *tok, int V, float *x, const float *g, float *out,
                              float *rinv, int N, int D, void *stream);

/* rmsnorm_bwd, tinylm.c:565-588: dx = base + s g dy - (s^3/D)(x . g dy) x with
 * base = dx_in, which may be dx itself (the reference's dx +=), or zero when
 * dx_in is NULL (the memset + rmsnorm_bwd of :1089-1090); dg += sum_r x s dy
 * (fixed order).  D <= 2048. */
int tlg_dev_rmsnorm_bwd(const float *x, const float *g, const float *rinv, const float *dy, const float *dx_in,
                        float *dx, float *dg, int rows, int D, void *stream);

/* rmsnorm_bwd as above (tinylm.c:565-588) with the dg sum deferred: the
 * per-row-block partials of dg go to `part` (at least ceil(rows/16) * D
 * floats, 16-byte aligned, owned by the caller), and their fixed-order
 * column sum into dg rides along in the next grouped GEMM or expert launch
 * on the stream (or tlg_dev_gemm_flush), as a split GEMM's reduction does;
 * a launch on another stream first runs it on this stream.
 * dg is complete only after that launch; `part` must not be written before
 * it (a later call on the same `part` flushes the earlier sum first).  No
 * counterpart in the reference, whose rmsnorm_bwd adds into dg directly: it
 * saves the gain-sum launch of every RMSNorm backward in a training step.
 * The result equals tlg_dev_rmsnorm_bwd's bit for bit. */
int tlg_dev_rmsnorm_bwd_defer(const float *x, const float *g, const float *rinv, const float *dy,
                              const float *dx_in, float *dx, float *dg, int rows, int D, float *part,
                              size_t part_floats, void *stream);

/* rope_apply, tinylm.c:630-651, in place on [rows][nheads*hd]: row r is at
 * position pos[r] (device ints), or r % T when pos is NULL (forward's
 * pos[n] = n % T, :975).  cos_t / sin_t are rope_init's tables
 * ([maxpos][hd/2], :611-618) in device memory; back = 1 is the transpose. */
int tlg_dev_rope(float *buf, const int *pos, int T, int rows, int nheads, int hd, const float *cos_t,
                 const float *sin_t, int maxpos, int back, void *stream);

/* attn_fwd, tinylm.c:699-732: causal GQA attention of B sequences of T rows,
 * q [B*T][H*hd], k / v [B*T][KV*hd], out [B*T][H*hd]; head h reads KV head
 * h / (H/KV); win > 0 is the sliding window (cfg_lwin, :64-68).  Also writes
 * lse [B*T][H], the base-2 log-sum-exp of each row's scaled scores (log2 of
 * sum_s 2^(q.k_s * scale * log2 e)), for attn_bwd.  hd must be 32. */
int tlg_dev_attn_fwd(const float *q, const float *k, const float *v, float *out, float *lse, int B, int T, int H,
                     int KV, int hd, int win, void *stream);

/* attn_bwd, tinylm.c:734-783: dq, dk, dv (written, not accumulated: the
 * reference clears them first, :1129-1131) from datt, given the forward's
 * out and lse. */
int tlg_dev_attn_bwd(const float *q, const float *k, const float *v, const float *out, const float *lse,
                     const float *datt, float *dq, float *dk, float *dv, int B, int T, int H, int KV, int hd,
                     int win, void *stream);

/* rope_apply fused into attention (no reference counterpart as one call: it
 * replaces the sequence rope_apply(q), rope_apply(k), attn_fwd of
 * tinylm.c:988-990 and attn_bwd, rope_apply^T(dq), rope_apply^T(dk) of
 * :1130-1133).  q and k are the projections before rope_apply; cos_t / sin_t
 * are rope_init's tables for positions 0..T-1 (row r of a sequence is at
 * position r, :975), 16-byte aligned; dq and dk are the gradients of the
 * pre-rope q and k.  H / KV must be a multiple of 4 (the GQA-group kernels). */
int tlg_dev_attn_fwd_rope(const float *q, const float *k, const float *v, float *out, float *lse, int B, int T,
                          int H, int KV, int hd, int win, const float *cos_t, const float *sin_t, void *stream);
int tlg_dev_attn_bwd_rope(const float *q, const float *k, const float *v, const float *out, const float *lse,
                          const float *datt, float *dq, float *dk, float *dv, int B, int T, int H, int KV, int hd,
                          int win, const float *cos_t, const float *sin_t, void *stream);
/* tlg_dev_attn_bwd_rope with the per-row term D[r][h] = datt[r][h] . out[r][h]
 * (tinylm.c:750-768; [B*T][H]) given, as the O-projection backward's grouped
 * launch forms it (TlgGemmCall.dotB / dotOut, include/tlgemm.h), so the
 * backward starts with its dQ / dK / dV launch (no counterpart as one call). */
int tlg_dev_attn_bwd_rope_d(const float *q, const float *k, const float *v, const float *out, const float *lse,
                            const float *datt, const float *D, float *dq, float *dk, float *dv, int B, int T, int H,
                            int KV, int hd, int win, const float *cos_t, const float *sin_t, void *stream);

/* residual adds, tinylm.c:994-995, :1009-1010, :1062: y[i] += x[i]. */
int tlg_dev_add(float *y, const float *x, size_t n, void *stream);

/* SwiGLU forward, tinylm.c:1005-1006 (and the recompute :1097-1098):
 * act = silu(g) * u with silu(z) = z / (1 + e^-z) (:786). */
int tlg_dev_swiglu_fwd(float *act, const float *g, const float *u, size_t n, void *stream);

/* SwiGLU backward, tinylm.c:1103-1109: dg = dact u silu'(g), du = dact silu(g). */
int tlg_dev_swiglu_bwd(const float *dact, const float *g, const float *u, float *dg, float *du, size_t n,
                       void *stream);

/* mtp_grad's head input, tinylm.c:1046: hk = fn + silu(t1). */
int tlg_dev_silu_res(float *hk, const float *fn, const float *t1, size_t n, void *stream);

/* mtp_grad's dt1, tinylm.c:1063-1064: dt1 = dhk silu'(t1). */
int tlg_dev_silu_bwd(float *dt1, const float *dhk, const float *t1, size_t n, void *stream);

/* softmax + cross-entropy over logits [N][V] with the gradient in the same
 * pass: forward's loss, tinylm.c:1019-1028, and backward's dlogits,
 * :1076-1082 (scale = 1/N), or mtp_grad's weighted head gradient, :1051-1055
 * (scale = wk/N): dlogits = softmax * scale, minus scale at the target.  When
 * loss is given, loss[0] = mean over rows of -log(p[target] + 1e-12) (summed
 * in double, :1026-1028). */
int tlg_dev_xent(const float *logits, const int *tgt, float *dlogits, float *loss, float scale, int N, int V,
                 void *stream);

/* tlg_dev_xent without the loss sum: each row's -log(p[target] + 1e-12) goes
 * to rows[N] (doubles, caller-owned), for tlg_dev_gradnorm_loss to average
 * later in the step (no counterpart as one call). */
int tlg_dev_xent_rows(const float *logits, const int *tgt, float *dlogits, double *rows, float scale, int N, int V,
                      void *stream);

/* global_gradnorm, tinylm.c:1171-1176: norm[0] = sqrt(sum G^2) (double sum). */
int tlg_dev_gradnorm(const float *G, size_t n, float *norm, void *stream);
/* tlg_dev_gradnorm that also sets loss[0] = the mean of rows[0, N) from
 * tlg_dev_xent_rows, the same sum in the same order as tlg_dev_xent's loss
 * (:1026-1028), in the norm's last kernel: a training step's loss costs no
 * launch of its own (no counterpart as one call). */
int tlg_dev_gradnorm_loss(const float *G, size_t n, float *norm, const double *rows, int N, float *loss,
                          void *stream);

/* adamw, tinylm.c:1159-1170, with the clip of train_loop folded in
 * (:2630-2633): hyper = device floats {lr, b1, b2, wd, 1 - b1^t, 1 - b2^t};
 * gscale = 1/norm[0] when norm[0] > 1 (norm from tlg_dev_gradnorm, or NULL
 * for gscale = 1).  Keeping the step-dependent values in device memory lets
 * a captured step be replayed at any t. */
int tlg_dev_adamw(float *P, const float *G, float *M, float *V, size_t n, const float *hyper, const float *norm,
                  void *stream);

#ifdef __cplusplus
}
#endif
#endif
