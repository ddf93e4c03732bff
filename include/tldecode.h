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

/* ---- fused decode launches (no reference counterpart: the reference runs
 * the glue between its GEMVs as separate loops; these fold it into the
 * GEMV and attention launches so a token step needs 5 launches per layer).
 *
 * One GEMV of a decode run: mm (op 0) or mm_bt (op 1) with the reference's
 * argument labels (M <= 8), whose activation rows A [M][R] (R = K for mm, N
 * for mm_bt) pass through a prologue as they are read:
 *   pro 0  A as it is
 *   pro 1  rmsnorm_fwd (tinylm.c:540-548): A[m][r] * s_m * gain[r] with
 *          s_m = 1 / sqrt(sum_r A[m][r]^2 / R + 1e-5)
 *   pro 2  SwiGLU (:786, :3821-3823): silu(A[m][r]) * A2[m][r], silu(z) =
 *          z / (1 + e^-z)
 * and beta = 1 adds the result into C (the residual adds x += tmp of
 * forward_chunk, :3818, :3824), beta = 0 sets it. */
typedef struct {
    int op;                  /* 0 mm, 1 mm_bt */
    int beta;                /* 1 C += result, 0 C = result */
    float *C;
    int M, K, N;
    const float *A, *B;      /* X and W (mm), dY and W (mm_bt) */
    int pro;                 /* 0 none, 1 rmsnorm with gain, 2 SwiGLU with A2 */
    const float *gain;       /* pro 1: [R] */
    const float *A2;         /* pro 2: [M][R] */
    /* optional (zero = none), for a MoE layer's expert rows: the weight is
     * B + bsel[0] * bstride with bsel in device memory (the row's expert,
     * chosen on the device), and the result is multiplied by cgate[0] (the
     * row's gate) before it is stored or added: out[n] += gate[n] * y
     * (moe_scatter_body, tinylm.c:3347-3353) */
    const int *bsel;
    long long bstride;
    const float *cgate;
} TlgDecGemv;

/* Up to 8 independent GEMVs (none reads what another writes) in one launch. */
int tlg_dev_dec_gemv(const TlgDecGemv *calls, int n, void *stream);

/* qknorm_apply (tinylm.c:597-605, applied to q and k before RoPE,
 * :3752-3754): each of the m rows' H query heads of q [m][H*hd] and KV key
 * heads of k [m][KV*hd] becomes v * s * gain with s = 1 / sqrt(sum(v^2) / hd +
 * 1e-5), gain qn (queries) or kn (keys) of hd floats.  hd must be 32. */
int tlg_dev_dec_qknorm(float *q, float *k, const float *qn, const float *kn, int m, int H, int KV, int hd,
                       void *stream);
/* The decode MoE router's top-1 (moe_rt_body, tinylm.c:3332-3341) for m <= 64
 * rows of router logits rt [m][E] (E <= 64): softmax with expf, the first
 * maximum of the normalised probabilities -> assign[j], its probability ->
 * gate[j]. */
int tlg_dev_dec_moe_route(const float *rt, int m, int E, int *assign, float *gate, void *stream);
/* mtp_argmax's middle (tinylm.c:3933): hh[i] = fn[i] + silu(ht[i]), fn =
 * rmsnorm_fwd(x, nf) (:540-548) of one row x [D]. */
int tlg_dev_dec_mtp_mix(float *hh, const float *x, const float *nf, const float *ht, int D, void *stream);
/* argmax_v (tinylm.c:3844, the first maximum) of each of m rows of logits
 * [m][V] into out[m] (device), leaving the decode state alone. */
int tlg_dev_argmax_rows(const float *logits, int V, int m, int *out, void *stream);

/* The decode weight layout (no reference counterpart in fp32; the reference
 * repacks its weights for the int8 decode path, qmat_KN3 / qmat_KN_ilv,
 * tinylm.c:2945-2972): dst[c][r] = src[r][c] for a rows x cols matrix.  A
 * linear weight W [K][N] (map_weights' [in][out]) stored as W^T [N][K] turns
 * the decode GEMV mm(M, K, N) into an mm_bt form (op 1 with K and N swapped),
 * whose rows run along the reduction: every workgroup streams whole
 * contiguous rows.  dst and src must not overlap. */
int tlg_dev_transpose(float *dst, const float *src, int rows, int cols, void *stream);

/* RoPE, the ring store and the attention of forward_chunk (:3766-3815) in one
 * launch, for the m new rows at positions pos[j]: q [m][H*hd] and k [m][KD]
 * arrive before RoPE (rope_apply :645-651 with the tables cs / sn [maxpos][hd/2]
 * of rope_init :605-618, a position outside them gives NaN), v [m][KD];
 * every row's K and V go to slot pos % W (rounded to f16 for an f16 cache),
 * and row j attends as tlg_dev_dec_attn does, over the ring as the
 * reference's hoisted stores leave it (a slot written by this chunk holds
 * the new row).  q, k and v are left as they are.  The m positions must be
 * consecutive (pos[j] = pos[0] + j), as forward_chunk's are. */
int tlg_dev_dec_rope_attn(const float *q, const float *k, const float *v, const int *pos, const float *cs,
                          const float *sn, int maxpos, void *Kc, void *Vc, float *ctx, int m, int H, int KV, int hd,
                          int W, int win, int f16, int exact_exp, void *stream);

/* Greedy decoding, argmax_v (tinylm.c:3844: the first maximum) of the last
 * of m rows of logits [m][V]; then state[0] += m, state[1] = 1,
 * state[2] = tok[0] = the token, so the next step decodes it. */
int tlg_dev_dec_argmax(const float *logits, int V, int m, int *state, int *tok, void *stream);

/* ---- persistent greedy decoding (no reference counterpart: the reference
 * calls forward_chunk once per generated token, :3721-3830 and :3844; this
 * runs n such single-token steps, each followed by the greedy argmax, in ONE
 * cooperative launch of one workgroup per CU).
 *
 * The step is forward_chunk at m = 1 on a dense model with head_dim 32
 * (D = 32 H <= 384), F <= 1024 and F % 32 == 0, V % 8 == 0 and V <= 4096,
 * W <= 256, L <= 32, with or without QK-norm (qknorm): per layer RMSNorm ->
 * Q, K, V -> [QK-norm ->] RoPE -> ring store ->
 * attention over the window -> O + residual -> RMSNorm -> W1, W3 -> SwiGLU ->
 * W2 + residual; the final norm and the tied head; argmax_v (the first
 * maximum).  Token i of the launch decodes at position state[0] + i with
 * weights P[(copy0 + i) % pool] (map_weights' layout, every copy equal), the
 * first token being state[2].  At the end state = {state[0] + n, 1, last
 * greedy token, exchange sequence}, tok[0] = the last greedy token, logits =
 * the last step's logits row and toks_out[i] (if not NULL) = the token that
 * step i chose.  Arithmetic: the reference's formulas (RMSNorm, RoPE,
 * fast_expf or expf, SwiGLU, f16 or f32 ring elements), with fp32 sums in a
 * fixed order that differs from the reference's sequential one.  `exact`
 * selects expf for the attention exponentials only: SwiGLU's silu, the
 * softmax normalisation and RMSNorm's 1/sqrt use the hardware exp2,
 * reciprocal and rsqrt either way (within the fp32 bar, not bit for bit).
 *
 * xbuf is an exchange area of tlg_dec_persist_xbytes() bytes that must be
 * zero before the first launch and after every reset of state[3] (the
 * workgroups pass each phase's outputs through it, tagged with a sequence
 * number kept in state[3]).  Launches on one decoder must not overlap.  A
 * workgroup that waits 0.5 s for its inputs aborts the launch; then
 * tlg_dec_persist_status() returns TLG_EHIP and the decoder's state and
 * cache are undefined until it is reset. */
#define TLG_PD_MAXL 32
typedef struct {
    const float *P[16];      /* weight copies                                */
    int pool, copy0;
    int V, D, L, H, KV, F;
    int win, full_every;     /* sliding window per layer (cfg_lwin :64-68)   */
    int W, f16, exact, maxpos;
    const float *cs, *sn;    /* RoPE tables [maxpos][16]                     */
    void *Kc[TLG_PD_MAXL], *Vc[TLG_PD_MAXL];
    float *logits;           /* [V]                                          */
    int *state;              /* 4 ints                                       */
    int *tok;                /* 1 int                                        */
    int *toks_out;           /* [n] or NULL                                  */
    void *xbuf;
    int qknorm;              /* 1: QK-norm model (qknorm_apply, tinylm.c:597-605,
                                on q and k before RoPE, :3752-3754; the gains qn,
                                kn of 32 floats each lie after wo, as map_weights
                                places them); tlg_dev_dec_persist only       */
} TlgDecPersist;

size_t tlg_dec_persist_xbytes(int V, int D, int L, int F);
int tlg_dev_dec_persist(const TlgDecPersist *a, int n, void *stream);
/* forward_chunk (tinylm.c:3721-3830) at m rows (m = 1, 2, 4 or 8; m <= W)
 * for n chunks of given tokens, in ONE cooperative launch of one workgroup
 * per CU -- the prefill loop (:3977) and speculative decoding's verification
 * chunk (:3989) at the decoder's shapes (those of tlg_dev_dec_persist).
 * Chunk i feeds toks[i m .. i m + m) (device memory) at positions state[0] +
 * i m .. + m - 1 with weights P[(copy0 + i) % pool].  At the end state =
 * {state[0] + n m, 1, argmax of the last row, exchange sequence}, tok[0] =
 * that argmax, logits[m][V] = the last chunk's rows and toks_out[i m + j]
 * (if not NULL) = argmax_v of chunk i's row j.  Ring rows are stored as the
 * reference's hoisted kv_store leaves them (:3775-3780): a window key whose
 * slot a later row of the chunk overwrote reads that row's key.  xbuf, the
 * state and the abort behaviour are shared with tlg_dev_dec_persist.  QK-norm
 * models are refused (qknorm must be 0). */
int tlg_dev_dec_chunks(const TlgDecPersist *a, int m, const int *toks, int n, void *stream);
/* Synchronize `stream`; TLG_OK, or TLG_EHIP if a launch on xbuf aborted. */
int tlg_dec_persist_status(void *xbuf, void *stream);

#ifdef __cplusplus
}
#endif
#endif
