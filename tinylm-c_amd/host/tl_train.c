/* tl_train.c -- a device-resident training step of tinylm.c over the
 * libtlgemm C ABI (see tl_train.h).
 *
 * The step issues, on one stream and in the reference's order, the GEMMs of
 * forward / mtp_grad / backward (tinylm.c:968-1154) as grouped launches (the
 * calls the reference makes back to back with nothing between them share a
 * launch, tlg_dev_gemm_group), the non-GEMM work through include/tltrain.h,
 * then global_gradnorm and AdamW (:2630-2633).  memset + mm_bt pairs become
 * setting mm_bt calls (beta = 0), and the reference's memcpy(dfin, dout) /
 * memcpy(dain, dfin) / memcpy(dout, dain) become rmsnorm_bwd bases and a
 * pointer swap.
 */
#include "tl_train.h"
#include "../../include/tlgemm.h"
#include "../../include/tltrain.h"
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <limits.h>
#include <string.h>

typedef struct { size_t emb, an1, wq, wk, wv, wo, an2, wr, w1, w3, w2, nf, mtp0, total; } Map;

struct TlTrain {
    TlModel m;
    int B, N, hd, KD, E;
    size_t np;
    void *arena;
    float *P, *G, *Mo, *Vo;
    int *tok, *tgt, *tgt_mtp, *assign;
    float *hyper, *loss, *gnorm, *rcos, *rsin;
    /* per layer, L slices each (the Acts fields the backward pass reads) */
    float *a_in, *a_norm, *q, *k, *v, *ctx, *f_in, *f_norm, *g, *u, *act, *a_rinv, *f_rinv, *lse, *gate, *rprobs;
    /* one each */
    float *x_final, *fn, *fn_rinv, *logits, *dl, *dout, *dfnorm, *dfin, *datt, *dq, *dk, *dv, *dnorm, *dain, *dfn;
    float *attn_d;             /* the attention backward's D = datt . ctx [N][H] */
    double *lrows;             /* per-row losses of a step's forward [N] */
    /* RMSNorm backward's per-row-block gain partials; their column sum rides
     * along in the next grouped GEMM launch */
    float *rms_part;
    size_t rms_part_n;
    /* MoE layers: each layer's kept forward state (expert index and rows),
     * read by its backward instead of a recompute */
    char *moe_keep;
    size_t moe_keep_b;
    float hyper_host[8];
    void *graph;
    /* per grouped GEMM launch of a step, in call order: tile configuration + 1
     * (0 = the library's automatic policy) and split target (0 = automatic);
     * tl_train_autotune(_split) fills them */
    int gi, lcfg[TL_TRAIN_MAXG], lrt[TL_TRAIN_MAXG];
    void **tev;                         /* timing events (autotune only): 2 per launch */
    int tcap;
};

/* map_weights (tinylm.c:361-393) without QK-norm: emb | per layer an1 wq wk
 * wv wo an2 [wr] w1 w3 w2 (E expert slots) | nf | mtp heads. */
static void wmap(const TlTrain *t, int l, Map *o)
{
    const TlModel *m = &t->m;
    const size_t D = m->D, KD = t->KD, F = m->F, E = t->E > 0 ? t->E : 1, R = t->E > 0 ? D * t->E : 0;
    const size_t per = D + D * D + 2 * D * KD + D * D + D + R + E * 3 * D * F;
    o->emb = 0;
    o->an1 = (size_t)m->V * D + (size_t)l * per;
    o->wq = o->an1 + D;
    o->wk = o->wq + D * D;
    o->wv = o->wk + D * KD;
    o->wo = o->wv + D * KD;
    o->an2 = o->wo + D * D;
    o->wr = o->an2 + D;
    o->w1 = o->wr + R;
    o->w3 = o->w1 + E * D * F;
    o->w2 = o->w3 + E * D * F;
    o->nf = (size_t)m->V * D + (size_t)m->L * per;
    o->mtp0 = o->nf + D;
    o->total = o->mtp0 + (size_t)m->n_mtp * D * D;
}

static int lwin(const TlModel *m, int l)        /* cfg_lwin, tinylm.c:64-68 */
{
    if (m->win <= 0) return 0;
    if (m->full_every > 0 && ((l + 1) % m->full_every) == 0) return 0;
    return m->win;
}

/* ---- allocation ---------------------------------------------------------- */
typedef struct { void **dst; size_t bytes; } Slot;

TlTrain *tl_train_new(const TlModel *m, int B)
{
    if (!m || B <= 0 || m->V <= 0 || m->D <= 0 || m->L <= 0 || m->H <= 0 || m->KV <= 0 || m->F <= 0 ||
        m->T <= 0 || m->n_mtp < 0 || m->n_exp < 0 || m->n_exp == 1 || m->qknorm || m->D % m->H || m->H % m->KV ||
        m->D / m->H != 32 || m->D % 4 || m->F % 4 || m->V % 4)
        return NULL;
    TlTrain *t = calloc(1, sizeof *t);
    if (!t) return NULL;
    t->m = *m;
    t->B = B;
    t->N = B * m->T;
    t->hd = m->D / m->H;
    t->KD = m->KV * t->hd;
    t->E = m->n_exp;
    Map mp;
    wmap(t, 0, &mp);
    t->np = mp.total;
    const size_t N = t->N, L = m->L, D = m->D, KD = t->KD, F = m->F, V = m->V, H = m->H, E = t->E;
    const size_t ND = N * D, NK = N * KD, NF = N * F, half = t->hd / 2;
    const int dense = E == 0;
    t->rms_part_n = (N + 15) / 16 * D;       /* RMSNorm backward: 16 rows per workgroup */
    t->moe_keep_b = dense ? 0 : (tlg_moe_keep_bytes((int)N, (int)D, (int)F, (int)E) + 255) & ~(size_t)255;
    Slot s[] = {
        {(void **)&t->P, 4 * t->np}, {(void **)&t->G, 4 * t->np}, {(void **)&t->Mo, 4 * t->np},
        {(void **)&t->Vo, 4 * t->np}, {(void **)&t->tok, 4 * N}, {(void **)&t->tgt, 4 * N},
        {(void **)&t->tgt_mtp, 4 * N * (m->n_mtp ? m->n_mtp : 1)}, {(void **)&t->hyper, 32},
        {(void **)&t->loss, 4}, {(void **)&t->gnorm, 4}, {(void **)&t->rcos, 4 * m->T * half},
        {(void **)&t->rsin, 4 * m->T * half},
        {(void **)&t->a_in, 4 * L * ND}, {(void **)&t->a_norm, 4 * L * ND}, {(void **)&t->q, 4 * L * ND},
        {(void **)&t->k, 4 * L * NK}, {(void **)&t->v, 4 * L * NK}, {(void **)&t->ctx, 4 * L * ND},
        {(void **)&t->f_in, 4 * L * ND}, {(void **)&t->f_norm, 4 * L * ND},
        {(void **)&t->g, dense ? 4 * L * NF : 0}, {(void **)&t->u, dense ? 4 * L * NF : 0},
        {(void **)&t->a_rinv, 4 * L * N}, {(void **)&t->f_rinv, 4 * L * N}, {(void **)&t->lse, 4 * L * N * H},
        {(void **)&t->assign, 4 * L * N * !dense}, {(void **)&t->gate, 4 * L * N * !dense},
        {(void **)&t->rprobs, 4 * L * N * E},
        {(void **)&t->x_final, 4 * ND}, {(void **)&t->fn, 4 * ND}, {(void **)&t->fn_rinv, 4 * N},
        {(void **)&t->logits, 4 * N * V}, {(void **)&t->dl, 4 * N * V}, {(void **)&t->dout, 4 * ND},
        {(void **)&t->act, dense ? 4 * L * NF : 0}, {(void **)&t->dfnorm, 4 * ND}, {(void **)&t->dfin, 4 * ND},
        {(void **)&t->datt, 4 * ND}, {(void **)&t->dq, 4 * ND}, {(void **)&t->dk, 4 * NK},
        {(void **)&t->dv, 4 * NK}, {(void **)&t->dnorm, 4 * ND}, {(void **)&t->dain, 4 * ND},
        {(void **)&t->dfn, 4 * ND}, {(void **)&t->attn_d, 4 * (size_t)N * H}, {(void **)&t->lrows, 8 * (size_t)N},
        {(void **)&t->rms_part, 4 * t->rms_part_n},
        {(void **)&t->moe_keep, L * t->moe_keep_b},
    };
    const int ns = (int)(sizeof s / sizeof s[0]);
    size_t total = 0;
    for (int i = 0; i < ns; i++) total += (s[i].bytes + 255) & ~(size_t)255;
    t->arena = tlg_dev_malloc(total);
    if (!t->arena) { free(t); return NULL; }
    char *p = t->arena;
    for (int i = 0; i < ns; i++) {
        *s[i].dst = s[i].bytes ? p : NULL;
        p += (s[i].bytes + 255) & ~(size_t)255;
    }
    /* rope_init's tables (tinylm.c:611-618) for positions 0..T-1 */
    float *cs = malloc(4 * m->T * half), *sn = malloc(4 * m->T * half);
    int rc = !cs || !sn;
    for (int tt = 0; !rc && tt < m->T; tt++)
        for (size_t i = 0; i < half; i++) {
            const float inv = powf(m->rope_base, -(2.0f * i) / t->hd);
            const float a = tt * inv;
            cs[tt * half + i] = cosf(a);
            sn[tt * half + i] = sinf(a);
        }
    void *st = tlg_stream_create();
    if (!rc) rc = tlg_memcpy_h2d(t->rcos, cs, 4 * m->T * half, st) || tlg_memcpy_h2d(t->rsin, sn, 4 * m->T * half, st);
    for (int i = 0; !rc && i < 4; i++) rc = tlg_dev_zero(tl_train_buf(t, i), t->np, st);
    if (!rc) rc = tlg_stream_sync(st);
    if (!rc) rc = tl_train_set_hyper(t, 3e-4f, 0.9f, 0.95f, 0.1f, 1, st);
    if (st) tlg_stream_destroy(st);
    free(cs);
    free(sn);
    if (rc) { tl_train_free(t); return NULL; }
    return t;
}

void tl_train_free(TlTrain *t)
{
    if (!t) return;
    if (t->graph) tlg_graph_destroy(t->graph);
    if (t->arena) tlg_dev_free(t->arena);
    free(t);
}

size_t tl_train_nparams(const TlTrain *t) { return t ? t->np : 0; }

float *tl_train_buf(TlTrain *t, int which)
{
    switch (which) {
    case 0: return t->P;
    case 1: return t->G;
    case 2: return t->Mo;
    case 3: return t->Vo;
    default: return NULL;
    }
}

float *tl_train_act(TlTrain *t, const char *name, int layer)
{
    const size_t N = t->N, ND = N * t->m.D, NK = N * t->KD, NF = N * t->m.F;
    const size_t l = layer < 0 || layer >= t->m.L ? 0 : (size_t)layer;
    struct { const char *n; float *p; size_t per; } tab[] = {
        {"a_in", t->a_in, ND}, {"a_norm", t->a_norm, ND}, {"q", t->q, ND}, {"k", t->k, NK}, {"v", t->v, NK},
        {"att_ctx", t->ctx, ND}, {"f_in", t->f_in, ND}, {"f_norm", t->f_norm, ND}, {"g", t->g, NF},
        {"u", t->u, NF}, {"act", t->act, NF}, {"a_rinv", t->a_rinv, N}, {"f_rinv", t->f_rinv, N}, {"lse", t->lse, N * t->m.H},
        {"x_final", t->x_final, 0}, {"fn_norm", t->fn, 0}, {"fn_rinv", t->fn_rinv, 0},
        {"logits", t->logits, 0}, {"dlogits", t->dl, 0}, {"dfn", t->dfn, 0},
    };
    for (size_t i = 0; i < sizeof tab / sizeof tab[0]; i++)
        if (!strcmp(name, tab[i].n)) return tab[i].p ? tab[i].p + l * tab[i].per : NULL;
    return NULL;
}

/* ---- host <-> device at step boundaries ------------------------------------ */
int tl_train_upload(TlTrain *t, const float *P, void *st)
{
    int rc = tlg_memcpy_h2d(t->P, P, 4 * t->np, st);
    if (!rc) rc = tlg_dev_zero(t->Mo, t->np, st);
    if (!rc) rc = tlg_dev_zero(t->Vo, t->np, st);
    if (!rc) rc = tlg_stream_sync(st);
    return rc;
}

int tl_train_set_batch(TlTrain *t, const int *tok, const int *tgt, const int *tgt_mtp, void *st)
{
    const int N = t->N, V = t->m.V, nm = t->m.n_mtp;
    for (int i = 0; i < N; i++)
        if (tok[i] < 0 || tok[i] >= V || tgt[i] < 0 || tgt[i] >= V) return TLG_EINVAL;
    for (int i = 0; i < N * nm; i++)
        if (!tgt_mtp || tgt_mtp[i] < 0 || tgt_mtp[i] >= V) return TLG_EINVAL;
    int rc = tlg_memcpy_h2d(t->tok, tok, 4 * (size_t)N, st);
    if (!rc) rc = tlg_memcpy_h2d(t->tgt, tgt, 4 * (size_t)N, st);
    if (!rc && nm) rc = tlg_memcpy_h2d(t->tgt_mtp, tgt_mtp, 4 * (size_t)N * nm, st);
    if (!rc) rc = tlg_stream_sync(st);
    return rc;
}

int tl_train_set_hyper(TlTrain *t, float lr, float b1, float b2, float wd, int step, void *st)
{
    float *h = t->hyper_host;
    h[0] = lr; h[1] = b1; h[2] = b2; h[3] = wd;
    h[4] = 1.0f - powf(b1, step);                 /* adamw's bc1, bc2 (:1161) */
    h[5] = 1.0f - powf(b2, step);
    int rc = tlg_memcpy_h2d(t->hyper, h, 8 * sizeof(float), st);
    if (!rc) rc = tlg_stream_sync(st);
    return rc;
}

static float read1(const float *dev, void *st)
{
    float x = NAN;
    if (tlg_memcpy_d2h(&x, dev, 4, st) || tlg_stream_sync(st)) return NAN;
    return x;
}
float tl_train_loss(TlTrain *t, void *st) { return read1(t->loss, st); }
float tl_train_gnorm(TlTrain *t, void *st) { return read1(t->gnorm, st); }

/* ---- GEMM calls ------------------------------------------------------------ */
static TlgGemmCall MM(float *Y, const float *X, const float *W, int M, int K, int N)
{
    TlgGemmCall c;
    memset(&c, 0, sizeof c);
    c.op = 0; c.C = Y; c.M = M; c.K = K; c.N = N; c.nseg = 1; c.A[0] = X; c.B[0] = W;
    return c;
}
/* Y = R + X W: mm and the residual add after it in one call */
static TlgGemmCall MMR(float *Y, const float *X, const float *W, int M, int K, int N, const float *R)
{
    TlgGemmCall c = MM(Y, X, W, M, K, N);
    c.R = R;
    return c;
}
static TlgGemmCall BT(float *dX, int beta, const float *dY, const float *W, int M, int K, int N)
{
    TlgGemmCall c = MM(dX, dY, W, M, K, N);
    c.op = 1; c.beta = beta;
    return c;
}
static TlgGemmCall ATB(float *dW, const float *X, const float *dY, int M, int K, int N)
{
    TlgGemmCall c = MM(dW, X, dY, M, K, N);
    c.op = 2; c.beta = 1;
    return c;
}
/* dX (beta ? += : =) sum_s dY_s W_s^T, s < n (an mm_bt chain into one dX) */
static TlgGemmCall BTN(float *dX, int beta, int M, int K, int n, const float *const *dY, const float *const *W,
                       const int *Ns)
{
    TlgGemmCall c = BT(dX, beta, dY[0], W[0], M, K, Ns[0]);
    c.nseg = n;
    for (int s = 1; s < n; s++) { c.A[s] = dY[s]; c.B[s] = W[s]; c.Nseg[s] = Ns[s]; }
    return c;
}

#define CK(x) do { int rc_ = (x); if (rc_) return rc_; } while (0)

/* One grouped GEMM launch, the step's k-th: pinned to its tile configuration
 * when the step has a table, bracketed by events while autotuning. */
static int group(TlTrain *t, const TlgGemmCall *cs, int n, void *st)
{
    const int k = t->gi++;
    const int cfg = k < TL_TRAIN_MAXG ? t->lcfg[k] : 0;
    const int rt = k < TL_TRAIN_MAXG ? t->lrt[k] : 0;
    const int timed = t->tev && k < t->tcap;
    int rc = cfg > 0 ? tlg_tune_group(cfg - 1) : 0;
    if (!rc && rt) rc = tlg_tune_group_split(rt);
    if (!rc && timed) rc = tlg_event_record(t->tev[2 * k], st);
    if (!rc) rc = tlg_dev_gemm_group(cs, n, st);
    if (!rc && timed) rc = tlg_event_record(t->tev[2 * k + 1], st);
    if (cfg > 0) {
        const int r2 = tlg_tune_group(-1);
        if (!rc) rc = r2;
    }
    if (rt) {
        const int r2 = tlg_tune_group_split(0);
        if (!rc) rc = r2;
    }
    return rc;
}
#define GROUP(st, ...) do { TlgGemmCall cs_[] = {__VA_ARGS__}; \
        CK(group(t, cs_, (int)(sizeof cs_ / sizeof cs_[0]), st)); } while (0)

/* rope_apply runs inside the attention kernels when the GQA-group kernels
 * take the model (H / KV a multiple of 4); else as its own pass. */
static int rope_fused(const TlModel *m) { return (m->H / m->KV) % 4 == 0; }

/* ---- forward, tinylm.c:968-1029 ------------------------------------------- */
/* clear_g (inside a step): memset(G) (:2628) rides in the logits launch (a
 * clear item of the grouped launch, nothing there reads or writes G), so the
 * backward need not launch it; and the per-row losses go to lrows, averaged
 * by the gradnorm's last kernel (tl_train_optimize's), not by a kernel here */
static int forward_impl(TlTrain *t, int clear_g, void *st)
{
    const TlModel *m = &t->m;
    const int N = t->N, D = m->D, KD = t->KD, F = m->F, V = m->V, H = m->H, KV = m->KV, T = m->T, E = t->E;
    const size_t ND = (size_t)N * D, NK = (size_t)N * KD, NF = (size_t)N * F;
    const float *P = t->P;
    Map w;
    wmap(t, 0, &w);
    t->gi = 0;                                   /* the step's first grouped launch */
    const float *emb = P + w.emb;
    for (int l = 0; l < m->L; l++) {
        wmap(t, l, &w);
        float *xin = t->a_in + l * ND, *an = t->a_norm + l * ND, *q = t->q + l * ND, *k = t->k + l * NK,
              *v = t->v + l * NK, *cx = t->ctx + l * ND, *fi = t->f_in + l * ND, *fnl = t->f_norm + l * ND;
        if (l == 0)     /* the embedding gather and the first norm in one pass */
            CK(tlg_dev_embed_rmsnorm_fwd(emb, t->tok, V, xin, P + w.an1, an, t->a_rinv, N, D, st));
        else
            CK(tlg_dev_rmsnorm_fwd(xin, P + w.an1, an, t->a_rinv + (size_t)l * N, N, D, st));
        GROUP(st, MM(q, an, P + w.wq, N, D, D), MM(k, an, P + w.wk, N, D, KD), MM(v, an, P + w.wv, N, D, KD));
        if (rope_fused(m)) {
            /* q, k stay pre-rope; the attention kernels rotate as they load */
            CK(tlg_dev_attn_fwd_rope(q, k, v, cx, t->lse + (size_t)l * N * H, t->B, T, H, KV, t->hd, lwin(m, l),
                                     t->rcos, t->rsin, st));
        } else {
            CK(tlg_dev_rope(q, NULL, T, N, H, t->hd, t->rcos, t->rsin, T, 0, st));
            CK(tlg_dev_rope(k, NULL, T, N, KV, t->hd, t->rcos, t->rsin, T, 0, st));
            CK(tlg_dev_attn_fwd(q, k, v, cx, t->lse + (size_t)l * N * H, t->B, T, H, KV, t->hd, lwin(m, l), st));
        }
        GROUP(st, MMR(fi, cx, P + w.wo, N, D, D, xin));                 /* + residual, :994-995 */
        CK(tlg_dev_rmsnorm_fwd(fi, P + w.an2, fnl, t->f_rinv + (size_t)l * N, N, D, st));
        float *out = l + 1 < m->L ? t->a_in + (l + 1) * ND : t->x_final;
        if (E > 0) {
            CK(tlg_dev_moe_grouped_fwd_keep(fnl, fi, out, N, D, F, E, P + w.wr, P + w.w1, P + w.w3, P + w.w2,
                                            t->assign + (size_t)l * N, t->gate + (size_t)l * N,
                                            t->rprobs + (size_t)l * N * E, t->moe_keep + l * t->moe_keep_b,
                                            t->moe_keep_b, st));
        } else {
            /* g, u and act = silu(g) u (:1002-1006) from one launch; act is
             * kept per layer, so the backward's recompute (:1098-1100) is a read */
            float *g = t->g + l * NF, *u = t->u + l * NF, *act = t->act + l * NF;
            CK(tlg_dev_swiglu_mm(fnl, P + w.w1, P + w.w3, act, g, u, N, D, F, st));
            GROUP(st, MMR(out, act, P + w.w2, N, F, D, fi));               /* + residual, :1009-1010 */
        }
    }
    CK(tlg_dev_rmsnorm_fwd(t->x_final, P + w.nf, t->fn, t->fn_rinv, N, D, st));
    if (clear_g) {
        TlgGemmCall z;
        memset(&z, 0, sizeof z);
        z.op = 3; z.C = t->G; z.M = 1; z.N = (int)t->np;
        GROUP(st, BT(t->logits, 0, t->fn, P + w.emb, N, V, D), z);
    } else {
        GROUP(st, BT(t->logits, 0, t->fn, P + w.emb, N, V, D));
    }
    /* softmax-CE, with backward's dlogits (:1076-1082) from the same pass */
    if (clear_g)
        CK(tlg_dev_xent_rows(t->logits, t->tgt, t->dl, t->lrows, 1.0f / N, N, V, st));
    else
        CK(tlg_dev_xent(t->logits, t->tgt, t->dl, t->loss, 1.0f / N, N, V, st));
    return 0;
}

int tl_train_forward(TlTrain *t, void *st) { return forward_impl(t, 0, st); }

/* ---- backward, tinylm.c:1072-1154 with mtp_grad :1036-1069 ---------------- */
/* g_clear: G was cleared by the forward before it (forward_impl) */
static int backward_impl(TlTrain *t, int g_clear, void *st)
{
    const TlModel *m = &t->m;
    const int N = t->N, D = m->D, KD = t->KD, F = m->F, V = m->V, H = m->H, KV = m->KV, T = m->T, E = t->E;
    const size_t ND = (size_t)N * D, NK = (size_t)N * KD, NF = (size_t)N * F;
    const float *P = t->P;
    float *G = t->G;
    Map w;
    wmap(t, 0, &w);
    if (!g_clear) CK(tlg_dev_zero(G, t->np, st));                     /* memset(G), :2628 */
    GROUP(st, MM(t->dfn, t->dl, P + w.emb, N, V, D), ATB(G + w.emb, t->dl, t->fn, N, V, D));
    for (int h = 0; h < m->n_mtp; h++) {
        const float wk = 0.2f * powf(0.8f, (float)h);
        const float *Wk = P + w.mtp0 + (size_t)h * D * D;
        float *t1 = t->datt, *hk = t->dnorm, *dhk = t->dq, *dt1 = t->dain;   /* the reference's scratch */
        GROUP(st, MM(t1, t->fn, Wk, N, D, D));
        CK(tlg_dev_silu_res(hk, t->fn, t1, ND, st));
        GROUP(st, BT(t->logits, 0, hk, P + w.emb, N, V, D));
        CK(tlg_dev_xent(t->logits, t->tgt_mtp + (size_t)h * N, t->dl, NULL, wk / N, N, V, st));
        GROUP(st, ATB(G + w.emb, t->dl, hk, N, V, D), MM(dhk, t->dl, P + w.emb, N, V, D));
        CK(tlg_dev_add(t->dfn, dhk, ND, st));
        CK(tlg_dev_silu_bwd(dt1, dhk, t1, ND, st));
        GROUP(st, ATB(G + w.mtp0 + (size_t)h * D * D, t->fn, dt1, N, D, D), BT(t->dfn, 1, dt1, Wk, N, D, D));
    }
    float *dout = t->dout, *dain = t->dain;
    CK(tlg_dev_rmsnorm_bwd_defer(t->x_final, P + w.nf, t->fn_rinv, t->dfn, NULL, dout, G + w.nf, N, D,
                                 t->rms_part, t->rms_part_n, st));
    for (int l = m->L - 1; l >= 0; l--) {
        wmap(t, l, &w);
        float *xin = t->a_in + l * ND, *an = t->a_norm + l * ND, *q = t->q + l * ND, *k = t->k + l * NK,
              *v = t->v + l * NK, *cx = t->ctx + l * ND, *fi = t->f_in + l * ND, *fnl = t->f_norm + l * ND;
        if (E > 0) {
            CK(tlg_dev_moe_grouped_bwd_kept(fnl, dout, t->dfnorm, t->assign + (size_t)l * N,
                                            t->gate + (size_t)l * N, t->rprobs + (size_t)l * N * E, N, D, F, E,
                                            P + w.wr, P + w.w1, P + w.w3, P + w.w2, G + w.wr, G + w.w1, G + w.w3,
                                            G + w.w2, t->moe_keep + l * t->moe_keep_b, t->moe_keep_b, st));
        } else {
            /* d_act = dout W2^T with the SwiGLU backward in its epilogue
             * (:1103-1109): g, u of this layer become dg, du in place */
            float *g = t->g + l * NF, *u = t->u + l * NF, *act = t->act + l * NF;
            CK(tlg_dev_mm_bt_swiglu_bwd(dout, P + w.w2, g, u, N, F, D, st));
            const float *dy[2] = {g, u}, *wt[2] = {P + w.w1, P + w.w3};
            const int ns[2] = {F, F};
            GROUP(st, BTN(t->dfnorm, 0, N, D, 2, dy, wt, ns), ATB(G + w.w1, fnl, g, N, D, F),
                  ATB(G + w.w3, fnl, u, N, D, F), ATB(G + w.w2, act, dout, N, F, D));   /* dW2, :1101 */
        }
        CK(tlg_dev_rmsnorm_bwd_defer(fi, P + w.an2, t->f_rinv + (size_t)l * N, t->dfnorm, dout, t->dfin,
                                     G + w.an2, N, D, t->rms_part, t->rms_part_n, st));
        if (rope_fused(m)) {
            /* datt = dfin Wo^T with the attention backward's D = datt . ctx per
             * row and head formed in the same launch (:750-768) */
            TlgGemmCall ob = BT(t->datt, 0, t->dfin, P + w.wo, N, D, D);
            ob.dotB = cx;
            ob.dotOut = t->attn_d;
            GROUP(st, ob, ATB(G + w.wo, cx, t->dfin, N, D, D));
            CK(tlg_dev_attn_bwd_rope_d(q, k, v, cx, t->lse + (size_t)l * N * H, t->datt, t->attn_d, t->dq, t->dk,
                                       t->dv, t->B, T, H, KV, t->hd, lwin(m, l), t->rcos, t->rsin, st));
        } else {
            GROUP(st, BT(t->datt, 0, t->dfin, P + w.wo, N, D, D), ATB(G + w.wo, cx, t->dfin, N, D, D));
            CK(tlg_dev_attn_bwd(q, k, v, cx, t->lse + (size_t)l * N * H, t->datt, t->dq, t->dk, t->dv, t->B, T, H,
                                KV, t->hd, lwin(m, l), st));
            CK(tlg_dev_rope(t->dq, NULL, T, N, H, t->hd, t->rcos, t->rsin, T, 1, st));
            CK(tlg_dev_rope(t->dk, NULL, T, N, KV, t->hd, t->rcos, t->rsin, T, 1, st));
        }
        const float *dy[3] = {t->dq, t->dk, t->dv}, *wt[3] = {P + w.wq, P + w.wk, P + w.wv};
        const int ns[3] = {D, KD, KD};
        GROUP(st, BTN(t->dnorm, 0, N, D, 3, dy, wt, ns), ATB(G + w.wq, an, t->dq, N, D, D),
              ATB(G + w.wk, an, t->dk, N, D, KD), ATB(G + w.wv, an, t->dv, N, D, KD));
        CK(tlg_dev_rmsnorm_bwd_defer(xin, P + w.an1, t->a_rinv + (size_t)l * N, t->dnorm, t->dfin, dain,
                                     G + w.an1, N, D, t->rms_part, t->rms_part_n, st));
        float *tmp = dout; dout = dain; dain = tmp;                    /* memcpy(dout, dain), :1146 */
    }
    wmap(t, 0, &w);
    CK(tlg_dev_embed_bwd(G + w.emb, dout, t->tok, N, D, V, st));
    CK(tlg_dev_gemm_flush(st));
    return 0;
}

int tl_train_backward(TlTrain *t, void *st) { return backward_impl(t, 0, st); }

/* ---- global_gradnorm + AdamW, tinylm.c:2630-2633 -------------------------- */
/* loss_rows: also average the forward's lrows into loss (forward_impl's
 * clear_g form) */
static int optimize_impl(TlTrain *t, int loss_rows, void *st)
{
    if (loss_rows)
        CK(tlg_dev_gradnorm_loss(t->G, t->np, t->gnorm, t->lrows, t->N, t->loss, st));
    else
        CK(tlg_dev_gradnorm(t->G, t->np, t->gnorm, st));
    CK(tlg_dev_adamw(t->P, t->G, t->Mo, t->Vo, t->np, t->hyper, t->gnorm, st));
    return 0;
}

int tl_train_optimize(TlTrain *t, void *st) { return optimize_impl(t, 0, st); }

int tl_train_step(TlTrain *t, void *st)
{
    const int fold = t->np <= (size_t)INT_MAX;         /* the clear item's extent is an int */
    CK(forward_impl(t, fold, st));
    CK(backward_impl(t, fold, st));
    return optimize_impl(t, fold, st);
}

int tl_train_graph_build(TlTrain *t, void *st)
{
    if (t->graph) { tlg_graph_destroy(t->graph); t->graph = NULL; }
    CK(tlg_graph_begin(st));
    const int rc = tl_train_step(t, st);
    void *g = tlg_graph_end(st);
    if (rc) { if (g) tlg_graph_destroy(g); return rc; }
    if (!g) return TLG_EHIP;
    t->graph = g;
    return 0;
}

int tl_train_graph_step(TlTrain *t, void *st)
{
    if (!t->graph) return TLG_EINVAL;
    return tlg_graph_launch(t->graph, st);
}

/* Per grouped launch, the fastest of `cands` (with each split target of rts)
 * over `reps` timed forward + backward passes (P, M and V are not touched; G
 * and the activations are). */
int tl_train_autotune(TlTrain *t, const int *cands, int ncands, int reps, void *st)
{
    const int policy = 0;
    return tl_train_autotune_split(t, cands, ncands, &policy, 1, reps, st);
}

int tl_train_autotune_split(TlTrain *t, const int *cands, int ncands, const int *rts, int nrts, int reps,
                            void *st)
{
    if (!t || !cands || ncands <= 0 || !rts || nrts <= 0 || reps <= 0) return TLG_EINVAL;
    for (int c = 0; c < ncands; c++)
        if (cands[c] < 0) return TLG_EINVAL;
    for (int s = 0; s < nrts; s++)
        if (rts[s] != 0 && rts[s] < 64) return TLG_EINVAL;
    memset(t->lcfg, 0, sizeof t->lcfg);
    memset(t->lrt, 0, sizeof t->lrt);
    CK(tl_train_forward(t, st));                  /* counts the launches, sizes the scratch */
    CK(tl_train_backward(t, st));
    const int ng = t->gi;
    if (ng <= 0 || ng > TL_TRAIN_MAXG) return TLG_EINVAL;
    void **ev = calloc((size_t)2 * ng, sizeof(void *));
    double *best = malloc(sizeof(double) * (size_t)ng), *acc = malloc(sizeof(double) * (size_t)ng);
    int *pick = calloc((size_t)ng, sizeof(int)), *prt = calloc((size_t)ng, sizeof(int));
    int rc = (!ev || !best || !acc || !pick || !prt) ? TLG_ENOMEM : 0;
    for (int i = 0; !rc && i < 2 * ng; i++)
        if (!(ev[i] = tlg_event_create())) rc = TLG_EHIP;
    for (int k = 0; k < ng && best; k++) best[k] = 1e30;
    for (int cs = 0; !rc && cs < ncands * nrts; cs++) {
        const int c = cs / nrts, rt = rts[cs % nrts];
        for (int k = 0; k < ng; k++) { t->lcfg[k] = cands[c] + 1; t->lrt[k] = rt; }
        t->tev = NULL;
        rc = tl_train_forward(t, st);            /* warm this shape up */
        if (!rc) rc = tl_train_backward(t, st);
        for (int k = 0; k < ng; k++) acc[k] = 0.0;
        t->tev = ev;
        t->tcap = ng;
        for (int r = 0; !rc && r < reps; r++) {
            rc = tl_train_forward(t, st);
            if (!rc) rc = tl_train_backward(t, st);
            if (!rc) rc = tlg_stream_sync(st);
            for (int k = 0; !rc && k < ng; k++) {
                const float ms = tlg_event_elapsed_ms(ev[2 * k], ev[2 * k + 1]);
                if (ms < 0) rc = TLG_EHIP;
                acc[k] += ms;
            }
        }
        for (int k = 0; !rc && k < ng; k++)
            if (acc[k] < best[k]) { best[k] = acc[k]; pick[k] = cands[c] + 1; prt[k] = rt; }
    }
    t->tev = NULL;
    t->tcap = 0;
    if (!rc) {
        memcpy(t->lcfg, pick, sizeof(int) * (size_t)ng);
        memcpy(t->lrt, prt, sizeof(int) * (size_t)ng);
    } else {
        memset(t->lcfg, 0, sizeof t->lcfg);
        memset(t->lrt, 0, sizeof t->lrt);
    }
    for (int i = 0; ev && i < 2 * ng; i++)
        if (ev[i]) tlg_event_destroy(ev[i]);
    free(ev); free(best); free(acc); free(pick); free(prt);
    return rc;
}

int tl_train_splits(const TlTrain *t, int *rt, int cap)
{
    int n = 0;
    for (int k = 0; k < TL_TRAIN_MAXG && k < cap; k++) {
        rt[k] = t->lrt[k];
        if (t->lcfg[k]) n = k + 1;
    }
    return n;
}

int tl_train_tiles(const TlTrain *t, int *cfg, int cap)
{
    int n = 0;
    for (int k = 0; k < TL_TRAIN_MAXG && k < cap; k++) {
        cfg[k] = t->lcfg[k] - 1;
        if (t->lcfg[k]) n = k + 1;
    }
    return n;
}

int tl_train_time_phases(TlTrain *t, float *ms, void *st)
{
    void *ev[4];
    for (int i = 0; i < 4; i++) if (!(ev[i] = tlg_event_create())) return TLG_EHIP;
    int rc = tlg_event_record(ev[0], st);
    if (!rc) rc = tl_train_forward(t, st);
    if (!rc) rc = tlg_event_record(ev[1], st);
    if (!rc) rc = tl_train_backward(t, st);
    if (!rc) rc = tlg_event_record(ev[2], st);
    if (!rc) rc = tl_train_optimize(t, st);
    if (!rc) rc = tlg_event_record(ev[3], st);
    if (!rc) rc = tlg_stream_sync(st);
    for (int i = 0; !rc && i < 3; i++) ms[i] = tlg_event_elapsed_ms(ev[i], ev[i + 1]);
    for (int i = 0; i < 4; i++) tlg_event_destroy(ev[i]);
    return rc;
}
