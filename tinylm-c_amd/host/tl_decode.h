/* tl_decode.h -- device-resident decoding of tinylm.c (libtlhost.so, plain C
 * over include/tlgemm.h, tltrain.h and tldecode.h).
 *
 * One TlDecode holds a model's fp32 weights (map_weights' layout) and a KV
 * ring cache of W positions per layer in HBM and runs forward_chunk
 * (tinylm.c:3721-3830) for chunks of m <= mmax rows: the embedding at the
 * chunk's positions, per layer RMSNorm -> [Q, K, V] -> RoPE -> ring store ->
 * attention over the ring window -> [O] + residual -> RMSNorm -> [W1, W3] ->
 * SwiGLU -> [W2] + residual, the final norm and [logits].  By default the
 * glue rides in the neighbouring launches (tldecode.h's fused entries: the
 * norms and SwiGLU as GEMV prologues, the residual adds as GEMV epilogues,
 * RoPE and the ring store inside the attention launch): 5 launches per layer
 * plus the embedding, the head and the argmax.  The cache holds f16 (the
 * reference's default, kv_dtype_env :3138-3146) or f32 elements; the softmax
 * uses the reference's fast_expf (default) or expf.
 *
 * Greedy decoding stays on the device: the argmax of the last logits row
 * becomes the next step's token and position in a device-side state, so one
 * captured step per weight copy replays token after token with no host
 * round trip.  Scope: head_dim 32, W <= 4096; dense or top-1 MoE layers
 * (moe_forward_q8's fp32 branch, :3433-3458), with or without QK-norm; the
 * MTP heads draft for self-speculative generation.  The persistent kernels
 * (tl_decode_persist, tl_decode_chunks) run the dense model without QK-norm
 * and return TLG_EINVAL for the others.
 */
#ifndef TL_DECODE_H
#define TL_DECODE_H
#include <stddef.h>
#include "tl_train.h"
#ifdef __cplusplus
extern "C" {
#endif

typedef struct TlDecode TlDecode;

/* W: ring positions (the reference uses the training context T); kv_f16: 1
 * f16 cache (default), 0 f32; exact_exp: 0 fast_expf (default), 1 expf;
 * maxpos: RoPE table length (positions 0..maxpos-1); mmax: largest chunk
 * (1..8, the GEMV kernels' row limit);
 * pool: copies of the weights, the greedy graph steps rotate through them so
 * the weights stream from HBM rather than the last-level cache.  NULL on
 * bad shapes or allocation failure. */
TlDecode *tl_decode_new(const TlModel *m, int W, int kv_f16, int exact_exp, int maxpos, int mmax, int pool);
void      tl_decode_free(TlDecode *d);
size_t    tl_decode_nparams(const TlDecode *d);
float    *tl_decode_params(TlDecode *d, int copy);      /* device P (copy < pool) */
float    *tl_decode_logits(TlDecode *d);                /* device [mmax][V]        */
/* Device addresses of layer l's K and V rings ([W][KD], f16 bits or f32 as
 * created; slot = position mod W); NULL for l out of range. */
void     *tl_decode_ring(TlDecode *d, int l, int v);

/* Copy host weights into every copy (and their decode layout, as
 * tl_decode_pack); clear the caches and the state. */
int tl_decode_upload(TlDecode *d, const float *P, void *stream);
/* Rebuild the decode layout of every copy from its P (after writing P
 * through tl_decode_params): the fused step's GEMVs read each linear weight
 * transposed (tldecode.h tlg_dev_transpose); the unfused step and the
 * persistent kernels read P. */
int tl_decode_pack(TlDecode *d, void *stream);
int tl_decode_reset(TlDecode *d, void *stream);
/* forward_chunk of m host tokens at positions start..start+m-1 (weights
 * copy 0); logits -> tl_decode_logits. */
int tl_decode_chunk(TlDecode *d, const int *tok, int m, int start, void *stream);
/* Prefill a prompt in chunks of <= mmax (positions 0..n-1), then take the
 * greedy token: the state now holds position n and that token. */
int tl_decode_prime(TlDecode *d, const int *prompt, int n, void *stream);
/* One greedy token step from the device state (weights copy `copy`). */
int tl_decode_greedy_step(TlDecode *d, int copy, void *stream);
/* MTP head k's greedy draft (mtp_argmax, tinylm.c:3930-3936) from row `row`
 * of the last chunk: fn = RMSNorm(x_row, nf), hh = fn + silu(fn Wk), the
 * argmax_v of hh emb^T -> dtok_out[0] (device).  Weights copy 0. */
int tl_decode_mtp_draft(TlDecode *d, int row, int k, int *dtok_out, void *stream);
/* Greedy self-speculative generation with the MTP heads (run_generation's
 * greedy path, tinylm.c:3985-4001): prefill the prompt (positions
 * 0..np-1); then per round the current row's greedy token x1 and the n_mtp
 * heads' drafts go through ONE chunk of n_mtp + 1 rows, and the drafts are
 * kept while each equals the greedy token of the row before it.  Writes n
 * tokens to toks (host) -- the same tokens greedy decoding gives -- and the
 * number of verification chunks to *chunks.  Needs n_mtp >= 1 and n_mtp + 1
 * <= mmax; weights copy 0. */
int tl_decode_generate_spec(TlDecode *d, const int *prompt, int np, int n, int *toks, int *chunks, void *stream);
/* Capture the greedy step once per weight copy; tl_decode_graph_step
 * replays the next copy's graph. */
int tl_decode_graph_build(TlDecode *d, void *stream);
int tl_decode_graph_step(TlDecode *d, void *stream);
/* 1 (default): the fused launches; 0: every glue op as its own launch, as
 * the reference orders them (for comparison).  Drops captured graphs. */
int tl_decode_set_fused(TlDecode *d, int fused);
/* n greedy token steps from the device state in ONE persistent launch
 * (tldecode.h tlg_dev_dec_persist), weight copies rotating per token;
 * toks_out: device [n] for the chosen tokens, or NULL.  Same state, logits
 * and cache as n tl_decode_greedy_step calls.  Needs D = 32 H <= 384,
 * F <= 1024 (F % 32 == 0), V % 8 == 0, W <= 256.  tl_decode_persist_status
 * synchronizes and reports an aborted launch (TLG_EHIP; then reset). */
int tl_decode_persist(TlDecode *d, int n, int *toks_out, void *stream);
/* n chunks of m rows (m = 1, 2, 4, 8; m <= mmax) of the device tokens dtoks[n
 * m] in ONE persistent launch (tldecode.h tlg_dev_dec_chunks): forward_chunk
 * over given tokens (prefill, speculative verification); toks_out[n m] (device,
 * or NULL) gets every row's argmax, logits the last chunk's m rows.  Same
 * shape limits as tl_decode_persist. */
int tl_decode_chunks(TlDecode *d, int m, const int *dtoks, int n, int *toks_out, void *stream);
int tl_decode_persist_status(TlDecode *d, void *stream);
/* Synchronize and read the state: {next position, rows, last token}. */
int tl_decode_state(TlDecode *d, int *state, void *stream);

#ifdef __cplusplus
}
#endif
#endif
