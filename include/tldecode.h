/* tldecode.h -- the non-GEMM kernels of tinylm.c's decode step, on device
 * pointers (libtlgemm.so, gfx950).  With the GEMV path of tlgemm.h
 * (tlg_dev_gemm_group at M <= 8) and the norms / RoPE / SwiGLU of
 * tltrain.h they run forward_chunk (tinylm.c:3721-3830) on the device; the C
 * driver tinylm-c_amd/host/tl_decode.c strings them together.
 *
 * Conventions as tlgemm.h / tltrain.h: asynchronous on `stream`, TLG_OK or
 * an error code with tlg_last_error() set, 16-byte aligned rows whose widths
 * are multiples of 4 floats.  The KV cache of one layer is two [W][KV*hd]
 * arrays of f32 or f16 (IEEE binary16, round to nearest even), position p in
 * slot p % W.  A device `state` of 3 ints lets a captured step run at the
 * position it finds there: state[0] = first position of the next chunk,
 * state[1] = its rows, state[2] = the last greedy token.
 */
#ifndef TLDECODE_H
#define TLDECODE_H
#ifdef __cplusplus
extern "C" {
#endif

/* forward_chunk's embedding, tinylm.c:3727-3728: x[j] = emb[tok[j]] and
 * pos[j] = p0 + j for j < m, with p0 = state[0] (or `start` when state is
 * NULL).  A token outside [0, V) makes its row NaN. */
int tlg_dev_dec_embed(float *x, int *pos, const float *emb, const int *tok, const int *state, int start, int m,
                      int D, int V, void *stream);

/* kv_store, tinylm.c:3236-3250 (f32 and f16 elements), for the m new rows:
 * K / V cache slot pos[j] % W <- k[j] / v[j] (RoPE already applied to k). */
int tlg_dev_kv_store(const float *k, const float *v, const int *pos, int m, int KD, int W, int f16, void *Kc,
                     void *Vc, void *stream);

/* attn_body's unsplit path, tinylm.c:3639-3715 (with forward_chunk's window
 * clamp :3768): for row j at position pos[j] and head h, attend over
 * positions max(0, pos - wlim + 1) .. pos of the ring (wlim = win when
 * 0 < win < W, else W): scores q.k * hd^-1/2, softmax with fast_expf
 * (:3181-3191, exact_exp 0, the reference default) or expf, normalised, then
 * ctx = sum p_t v_t.  hd must be 32, W <= 4096. */
int tlg_dev_dec_attn(const float *q, const void *Kc, const void *Vc, const int *pos, float *ctx, int m, int H,
                     int KV, int hd, int W, int win, int f16, int exact_exp, void *stream);

/* Greedy decoding, argmax_v (tinylm.c:3844: the first maximum) of the last
 * of m rows of logits [m][V]; then state[0] += m, state[1] = 1,
 * state[2] = tok[0] = the token, so the next step decodes it. */
int tlg_dev_dec_argmax(const float *logits, int V, int m, int *state, int *tok, void *stream);

#ifdef __cplusplus
}
#endif
#endif
