/* tl_decode.c -- device-resident decoding of tinylm.c (see tl_decode.h). */
#include "tl_decode.h"
#include "../../include/tldecode.h"
#include "../../include/tlgemm.h"
#include "../../include/tltrain.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define TLD_MAXPOOL 16
#define TLD_MAXM 8

typedef struct { size_t emb, an1, wq, wk, wv, wo, qn, kn, an2, wr, w1, w3, w2, nf, mtp0, total; } DMap;

struct TlDecode {
    TlModel m;
    int W, f16, exact, maxpos, mmax, pool, hd, KD;
    size_t np;
    void *arena;
    float *P[TLD_MAXPOOL];
    float *Pt[TLD_MAXPOOL];      /* the decode layout: every linear weight transposed, same offsets */
    void **Kc, **Vc;
    float *rcos, *rsin, *x, *xn, *q, *k, *v, *ctx, *tmp, *g, *u, *act, *fn, *logits;
    float *rt, *gt, *gu;         /* MoE: router logits [mmax][E], gates [mmax], expert rows [mmax][2F] */
    float *ht, *hh, *hlog;       /* MTP draft of one row: fn Wk [D], fn + silu [D], logits [V] */
    int *pos, *tok, *state;
    int *as;                     /* MoE: each row's expert [mmax] */
    int *dtok;                   /* drafts and verified tokens [16] */
    void *xbuf;                  /* the persistent decode's exchange area */
    size_t xbytes;
    void *graph[TLD_MAXPOOL];
    int next_graph;
    int next_copy;               /* weight copy of the next persistent step */
    int unfused;                 /* 1: the glue as separate launches (tl_decode_set_fused) */
};

/* map_weights (tinylm.c:361-393): the QK-norm gains qn, kn (hd each) between
 * wo and an2 when qknorm; the router wr [D][E] and E expert slots of w1, w3,
 * w2 when n_exp > 0; the n_mtp heads after nf */
static void dmap(const TlDecode *d, int l, DMap *o)
{
    const size_t D = d->m.D, KD = d->KD, F = d->m.F, hd = d->hd, E = d->m.n_exp > 0 ? d->m.n_exp : 1;
    const size_t QK = d->m.qknorm ? 2 * hd : 0, R = d->m.n_exp > 0 ? D * d->m.n_exp : 0;
    const size_t per = D + D * D + 2 * D * KD + D * D + QK + D + R + 3 * E * D * F;
    o->emb = 0;
    o->an1 = (size_t)d->m.V * D + (size_t)l * per;
    o->wq = o->an1 + D;
    o->wk = o->wq + D * D;
    o->wv = o->wk + D * KD;
    o->wo = o->wv + D * KD;
    o->qn = o->wo + D * D;
    o->kn = o->qn + (d->m.qknorm ? hd : 0);
    o->an2 = o->wo + D * D + QK;
    o->wr = o->an2 + D;
    o->w1 = o->wr + R;
    o->w3 = o->w1 + E * D * F;
    o->w2 = o->w3 + E * D * F;
    o->nf = (size_t)d->m.V * D + (size_t)d->m.L * per;
    o->mtp0 = o->nf + D;
    o->total = o->mtp0 + (size_t)d->m.n_mtp * D * D;
}

static int dwin(const TlModel *m, int l)         /* cfg_lwin, tinylm.c:64-68 */
{
    if (m->win <= 0) return 0;
    if (m->full_every > 0 && ((l + 1) % m->full_every) == 0) return 0;
    return m->win;
}

typedef struct { void **dst; size_t bytes; } DSlot;

TlDecode *tl_decode_new(const TlModel *m, int W, int kv_f16, int exact_exp, int maxpos, int mmax, int pool)
{
    if (!m || m->n_exp < 0 || m->n_exp == 1 || m->n_exp > 64 || m->n_mtp < 0 || m->D <= 0 || m->H <= 0 ||
        m->KV <= 0 || m->D % m->H || m->H % m->KV ||
        m->D / m->H != 32 || m->D % 4 || m->F % 4 || m->V % 4 || m->L <= 0 || W <= 0 || W > 4096 ||
        maxpos <= 0 || mmax <= 0 || mmax > 8 || mmax > W || pool <= 0 || pool > TLD_MAXPOOL)
        return NULL;
    TlDecode *d = calloc(1, sizeof *d);
    if (!d) return NULL;
    d->m = *m;
    d->W = W; d->f16 = kv_f16 ? 1 : 0; d->exact = exact_exp ? 1 : 0; d->maxpos = maxpos; d->mmax = mmax;
    d->pool = pool;
    d->hd = m->D / m->H;
    d->KD = m->KV * d->hd;
    DMap mp;
    dmap(d, 0, &mp);
    d->np = mp.total;
    d->Kc = calloc(m->L, sizeof(void *));
    d->Vc = calloc(m->L, sizeof(void *));
    if (!d->Kc || !d->Vc) { tl_decode_free(d); return NULL; }
    const size_t M = mmax, D = m->D, KD = d->KD, F = m->F, V = m->V, half = d->hd / 2;
    const size_t kvb = (size_t)W * KD * (d->f16 ? 2 : 4);
    DSlot fixed[] = {
        {(void **)&d->rcos, 4 * maxpos * half}, {(void **)&d->rsin, 4 * maxpos * half},
        {(void **)&d->x, 4 * M * D}, {(void **)&d->xn, 4 * M * D}, {(void **)&d->q, 4 * M * D},
        {(void **)&d->k, 4 * M * KD}, {(void **)&d->v, 4 * M * KD}, {(void **)&d->ctx, 4 * M * D},
        {(void **)&d->tmp, 4 * M * D}, {(void **)&d->g, 4 * M * F}, {(void **)&d->u, 4 * M * F},
        {(void **)&d->act, 4 * M * F}, {(void **)&d->fn, 4 * M * D}, {(void **)&d->logits, 4 * M * V},
        {(void **)&d->pos, 4 * M}, {(void **)&d->tok, 4 * M}, {(void **)&d->state, 16},
        {(void **)&d->rt, 4 * M * (size_t)(m->n_exp > 0 ? m->n_exp : 1)}, {(void **)&d->gt, 4 * M},
        {(void **)&d->gu, 8 * M * F}, {(void **)&d->as, 4 * M},
        {(void **)&d->ht, 4 * D}, {(void **)&d->hh, 4 * D}, {(void **)&d->hlog, 4 * V}, {(void **)&d->dtok, 64},
    };
    const int nf = (int)(sizeof fixed / sizeof fixed[0]);
    size_t total = 0;
    for (int i = 0; i < nf; i++) total += (fixed[i].bytes + 255) & ~(size_t)255;
    d->xbytes = tlg_dec_persist_xbytes(m->V, m->D, m->L, m->F);
    total += (d->xbytes + 255) & ~(size_t)255;
    total += (size_t)2 * pool * ((4 * d->np + 255) & ~(size_t)255);
    total += (size_t)m->L * 2 * ((kvb + 255) & ~(size_t)255);
    d->arena = tlg_dev_malloc(total);
    if (!d->arena) { tl_decode_free(d); return NULL; }
    char *p = d->arena;
    for (int i = 0; i < nf; i++) { *fixed[i].dst = p; p += (fixed[i].bytes + 255) & ~(size_t)255; }
    d->xbuf = p;
    p += (d->xbytes + 255) & ~(size_t)255;
    for (int c = 0; c < pool; c++) { d->P[c] = (float *)p; p += (4 * d->np + 255) & ~(size_t)255; }
    for (int c = 0; c < pool; c++) { d->Pt[c] = (float *)p; p += (4 * d->np + 255) & ~(size_t)255; }
    for (int l = 0; l < m->L; l++) {
        d->Kc[l] = p; p += (kvb + 255) & ~(size_t)255;
        d->Vc[l] = p; p += (kvb + 255) & ~(size_t)255;
    }
    /* rope_init's tables (tinylm.c:611-618) for positions 0..maxpos-1 */
    float *cs = malloc(4 * maxpos * half), *sn = malloc(4 * maxpos * half);
    int rc = !cs || !sn;
    for (int t = 0; !rc && t < maxpos; t++)
        for (size_t i = 0; i < half; i++) {
            const float inv = powf(m->rope_base, -(2.0f * i) / d->hd);
            const float a = t * inv;
            cs[t * half + i] = cosf(a);
            sn[t * half + i] = sinf(a);
        }
    void *st = tlg_stream_create();
    if (!rc) rc = tlg_memcpy_h2d(d->rcos, cs, 4 * maxpos * half, st) || tlg_memcpy_h2d(d->rsin, sn, 4 * maxpos * half, st);
    if (!rc) rc = tlg_stream_sync(st);
    if (!rc) rc = tl_decode_reset(d, st);
    if (st) tlg_stream_destroy(st);
    free(cs);
    free(sn);
    if (rc) { tl_decode_free(d); return NULL; }
    return d;
}

void tl_decode_free(TlDecode *d)
{
    if (!d) return;
    for (int c = 0; c < TLD_MAXPOOL; c++) if (d->graph[c]) tlg_graph_destroy(d->graph[c]);
    if (d->arena) tlg_dev_free(d->arena);
    free(d->Kc);
    free(d->Vc);
    free(d);
}

size_t tl_decode_nparams(const TlDecode *d) { return d ? d->np : 0; }
float *tl_decode_params(TlDecode *d, int copy) { return copy >= 0 && copy < d->pool ? d->P[copy] : NULL; }
float *tl_decode_logits(TlDecode *d) { return d->logits; }
void *tl_decode_ring(TlDecode *d, int l, int v)
{
    return d && l >= 0 && l < d->m.L ? (v ? d->Vc[l] : d->Kc[l]) : NULL;
}

int tl_decode_reset(TlDecode *d, void *st)
{
    const size_t kvf = (size_t)d->W * d->KD * (d->f16 ? 2 : 4) / 4;
    for (int l = 0; l < d->m.L; l++) {
        int rc = tlg_dev_zero((float *)d->Kc[l], kvf, st);
        if (!rc) rc = tlg_dev_zero((float *)d->Vc[l], kvf, st);
        if (rc) return rc;
    }
    int rc = tlg_dev_zero((float *)d->xbuf, d->xbytes / 4, st);   /* sequence 0: every tag stale */
    if (rc) return rc;
    const int zero[4] = {0, 0, 0, 0};
    rc = tlg_memcpy_h2d(d->state, zero, sizeof zero, st);
    if (!rc) rc = tlg_stream_sync(st);
    return rc;
}

int tl_decode_upload(TlDecode *d, const float *P, void *st)
{
    for (int c = 0; c < d->pool; c++) {
        int rc = tlg_memcpy_h2d(d->P[c], P, 4 * d->np, st);
        if (rc) return rc;
    }
    int rc = tl_decode_pack(d, st);
    return rc ? rc : tl_decode_reset(d, st);
}

/* The decode layout of every copy (tldecode.h tlg_dev_transpose): each
 * linear weight W [in][out] of P[c] as W^T [out][in] at the same offset of
 * Pt[c]; the embedding and the norm gains are read from P[c]. */
int tl_decode_pack(TlDecode *d, void *st)
{
    const int D = d->m.D, KD = d->KD, F = d->m.F, E = d->m.n_exp;
    const size_t DF = (size_t)D * F;
    for (int c = 0; c < d->pool; c++) {
        float *Pt = d->Pt[c];
        const float *P = d->P[c];
        for (int l = 0; l < d->m.L; l++) {
            DMap w;
            dmap(d, l, &w);
            const struct { size_t off; int rows, cols; } mats[] = {
                {w.wq, D, D}, {w.wk, D, KD}, {w.wv, D, KD}, {w.wo, D, D},
            };
            for (size_t i = 0; i < sizeof mats / sizeof mats[0]; i++) {
                int rc = tlg_dev_transpose(Pt + mats[i].off, P + mats[i].off, mats[i].rows, mats[i].cols, st);
                if (rc) return rc;
            }
            int rc = TLG_OK;
            if (E == 0) {
                rc = tlg_dev_transpose(Pt + w.w1, P + w.w1, D, F, st);
                if (!rc) rc = tlg_dev_transpose(Pt + w.w3, P + w.w3, D, F, st);
                if (!rc) rc = tlg_dev_transpose(Pt + w.w2, P + w.w2, F, D, st);
                if (rc) return rc;
                continue;
            }
            /* experts: W1_e^T and W3_e^T back to back at w1 + 2 e D F (one
             * [2F][D] matrix per expert), W2_e^T [D][F] at w2 + e D F; the
             * router as wr^T [E][D] */
            rc = tlg_dev_transpose(Pt + w.wr, P + w.wr, D, E, st);
            for (int e = 0; e < E && !rc; e++) {
                rc = tlg_dev_transpose(Pt + w.w1 + 2 * e * DF, P + w.w1 + e * DF, D, F, st);
                if (!rc) rc = tlg_dev_transpose(Pt + w.w1 + (2 * e + 1) * DF, P + w.w3 + e * DF, D, F, st);
                if (!rc) rc = tlg_dev_transpose(Pt + w.w2 + e * DF, P + w.w2 + e * DF, F, D, st);
            }
            if (rc) return rc;
        }
        DMap w0;
        dmap(d, 0, &w0);
        for (int k = 0; k < d->m.n_mtp; k++) {
            int rc = tlg_dev_transpose(Pt + w0.mtp0 + (size_t)k * D * D, P + w0.mtp0 + (size_t)k * D * D, D, D, st);
            if (rc) return rc;
        }
    }
    return TLG_OK;
}

/* ---- forward_chunk ---------------------------------------------------------- */
static TlgGemmCall MMc(float *Y, const float *X, const float *Wt, int M, int K, int N)
{
    TlgGemmCall c;
    memset(&c, 0, sizeof c);
    c.op = 0; c.C = Y; c.M = M; c.K = K; c.N = N; c.nseg = 1; c.A[0] = X; c.B[0] = Wt;
    return c;
}

#define CK(x) do { int rc_ = (x); if (rc_) return rc_; } while (0)
#define GROUP(st, ...) do { TlgGemmCall cs_[] = {__VA_ARGS__}; \
        CK(tlg_dev_gemm_group(cs_, (int)(sizeof cs_ / sizeof cs_[0]), st)); } while (0)

static TlgDecGemv DG(int op, int beta, float *C, int M, int K, int N, const float *A, const float *Bw, int pro,
                     const float *gain, const float *A2)
{
    TlgDecGemv c;
    memset(&c, 0, sizeof c);
    c.op = op; c.beta = beta; c.C = C; c.M = M; c.K = K; c.N = N; c.A = A; c.B = Bw;
    c.pro = pro; c.gain = gain; c.A2 = A2;
    return c;
}

#define DGEMV(st, ...) do { TlgDecGemv cs_[] = {__VA_ARGS__}; \
        CK(tlg_dev_dec_gemv(cs_, (int)(sizeof cs_ / sizeof cs_[0]), st)); } while (0)

/* A MoE layer of forward_chunk (tinylm.c:3815-3818 with moe_forward_q8's fp32
 * branch :3433-3458) on the decode layout: router logits of RMSNorm(x) (gain
 * an2), each row's top-1 expert and gate on the device, then per row the
 * chosen expert's [W1 | W3] (RMSNorm prologue) and W2 (SwiGLU prologue) with
 * x += gate * y in the W2 store -- the residual copy out = fin and the
 * scatter-add of moe_scatter_body in one step.  4 launches. */
static int run_moe_fused(TlDecode *d, const DMap *w, int m, const float *P, const float *Pt, void *st)
{
    const int D = d->m.D, F = d->m.F, E = d->m.n_exp;
    DGEMV(st, DG(1, 0, d->rt, m, E, D, d->x, Pt + w->wr, 1, P + w->an2, NULL));
    CK(tlg_dev_dec_moe_route(d->rt, m, E, d->as, d->gt, st));
    TlgDecGemv c13[TLD_MAXM], c2[TLD_MAXM];
    for (int j = 0; j < m; j++) {
        c13[j] = DG(1, 0, d->gu + (size_t)j * 2 * F, 1, 2 * F, D, d->x + (size_t)j * D, Pt + w->w1, 1, P + w->an2,
                    NULL);
        c13[j].bsel = d->as + j;
        c13[j].bstride = 2LL * D * F;
        c2[j] = DG(1, 1, d->x + (size_t)j * D, 1, D, F, d->gu + (size_t)j * 2 * F, Pt + w->w2, 2, NULL,
                   d->gu + (size_t)j * 2 * F + F);
        c2[j].bsel = d->as + j;
        c2[j].bstride = (long long)D * F;
        c2[j].cgate = d->gt + j;
    }
    CK(tlg_dev_dec_gemv(c13, m, st));
    CK(tlg_dev_dec_gemv(c2, m, st));
    return 0;
}

/* The same layer on the reference layout with the glue as separate launches,
 * in the reference's order: RMSNorm, router mm, top-1, per row W1 and W3 of
 * its expert, SwiGLU, per row W2 with out[n] = x[n] + gate[n] y. */
static int run_moe_unfused(TlDecode *d, const DMap *w, int m, const float *P, void *st)
{
    const int D = d->m.D, F = d->m.F, E = d->m.n_exp;
    CK(tlg_dev_rmsnorm_fwd(d->x, P + w->an2, d->xn, NULL, m, D, st));
    DGEMV(st, DG(0, 0, d->rt, m, D, E, d->xn, P + w->wr, 0, NULL, NULL));
    CK(tlg_dev_dec_moe_route(d->rt, m, E, d->as, d->gt, st));
    TlgDecGemv c1[TLD_MAXM], c3[TLD_MAXM], c2[TLD_MAXM];
    for (int j = 0; j < m; j++) {
        c1[j] = DG(0, 0, d->g + (size_t)j * F, 1, D, F, d->xn + (size_t)j * D, P + w->w1, 0, NULL, NULL);
        c3[j] = DG(0, 0, d->u + (size_t)j * F, 1, D, F, d->xn + (size_t)j * D, P + w->w3, 0, NULL, NULL);
        c2[j] = DG(0, 1, d->x + (size_t)j * D, 1, F, D, d->act + (size_t)j * F, P + w->w2, 0, NULL, NULL);
        c1[j].bsel = c3[j].bsel = c2[j].bsel = d->as + j;
        c1[j].bstride = c3[j].bstride = c2[j].bstride = (long long)D * F;
        c2[j].cgate = d->gt + j;
    }
    CK(tlg_dev_dec_gemv(c1, m, st));
    CK(tlg_dev_dec_gemv(c3, m, st));
    CK(tlg_dev_swiglu_fwd(d->act, d->g, d->u, (size_t)m * F, st));
    CK(tlg_dev_dec_gemv(c2, m, st));
    return 0;
}

/* The fused form: per layer 5 launches --
 *   [RMSNorm -> Q, K, V]  [RoPE, ring store, attention]  [O, x += ]
 *   [RMSNorm -> W1, W3]   [SwiGLU -> W2, x += ]
 * then [final RMSNorm -> logits]. */
static int run_chunk_fused(TlDecode *d, int m, int use_state, int start, int copy, void *st)
{
    const TlModel *md = &d->m;
    const int D = md->D, H = md->H, KV = md->KV, KD = d->KD, F = md->F, V = md->V, hd = d->hd;
    const float *P = d->P[copy], *Pt = d->Pt[copy];
    DMap w;
    dmap(d, 0, &w);
    CK(tlg_dev_dec_embed(d->x, d->pos, P + w.emb, d->tok, use_state ? d->state : NULL, start, m, D, V, st));
    /* every projection mm(m, in, out) on the decode layout: the mm_bt form
     * (op 1) of W^T [out][in], labels (m, out, in) */
    for (int l = 0; l < md->L; l++) {
        dmap(d, l, &w);
        DGEMV(st, DG(1, 0, d->q, m, D, D, d->x, Pt + w.wq, 1, P + w.an1, NULL),
              DG(1, 0, d->k, m, KD, D, d->x, Pt + w.wk, 1, P + w.an1, NULL),
              DG(1, 0, d->v, m, KD, D, d->x, Pt + w.wv, 1, P + w.an1, NULL));
        if (md->qknorm) CK(tlg_dev_dec_qknorm(d->q, d->k, P + w.qn, P + w.kn, m, H, KV, hd, st));   /* :3752-3754 */
        CK(tlg_dev_dec_rope_attn(d->q, d->k, d->v, d->pos, d->rcos, d->rsin, d->maxpos, d->Kc[l], d->Vc[l], d->ctx, m,
                                 H, KV, hd, d->W, dwin(md, l), d->f16, d->exact, st));
        DGEMV(st, DG(1, 1, d->x, m, D, D, d->ctx, Pt + w.wo, 0, NULL, NULL));
        if (md->n_exp > 0) {
            CK(run_moe_fused(d, &w, m, P, Pt, st));
            continue;
        }
        DGEMV(st, DG(1, 0, d->g, m, F, D, d->x, Pt + w.w1, 1, P + w.an2, NULL),
              DG(1, 0, d->u, m, F, D, d->x, Pt + w.w3, 1, P + w.an2, NULL));
        DGEMV(st, DG(1, 1, d->x, m, D, F, d->g, Pt + w.w2, 2, NULL, d->u));
    }
    dmap(d, 0, &w);
    DGEMV(st, DG(1, 0, d->logits, m, V, D, d->x, P + w.emb, 1, P + w.nf, NULL));   /* memset + mm_bt */
    return 0;
}

/* m rows of d->tok at positions state[0] + j (use_state) or start + j */
static int run_chunk(TlDecode *d, int m, int use_state, int start, int copy, void *st)
{
    if (!d->unfused) return run_chunk_fused(d, m, use_state, start, copy, st);
    const TlModel *md = &d->m;
    const int D = md->D, H = md->H, KV = md->KV, KD = d->KD, F = md->F, V = md->V, hd = d->hd;
    const float *P = d->P[copy];
    DMap w;
    dmap(d, 0, &w);
    CK(tlg_dev_dec_embed(d->x, d->pos, P + w.emb, d->tok, use_state ? d->state : NULL, start, m, D, V, st));
    for (int l = 0; l < md->L; l++) {
        dmap(d, l, &w);
        CK(tlg_dev_rmsnorm_fwd(d->x, P + w.an1, d->xn, NULL, m, D, st));
        GROUP(st, MMc(d->q, d->xn, P + w.wq, m, D, D), MMc(d->k, d->xn, P + w.wk, m, D, KD),
              MMc(d->v, d->xn, P + w.wv, m, D, KD));
        if (md->qknorm) CK(tlg_dev_dec_qknorm(d->q, d->k, P + w.qn, P + w.kn, m, H, KV, hd, st));
        CK(tlg_dev_rope(d->q, d->pos, 1, m, H, hd, d->rcos, d->rsin, d->maxpos, 0, st));
        CK(tlg_dev_rope(d->k, d->pos, 1, m, KV, hd, d->rcos, d->rsin, d->maxpos, 0, st));
        CK(tlg_dev_kv_store(d->k, d->v, d->pos, m, KD, d->W, d->f16, d->Kc[l], d->Vc[l], st));
        CK(tlg_dev_dec_attn(d->q, d->Kc[l], d->Vc[l], d->pos, d->ctx, m, H, KV, hd, d->W, dwin(md, l), d->f16,
                            d->exact, st));
        GROUP(st, MMc(d->tmp, d->ctx, P + w.wo, m, D, D));
        CK(tlg_dev_add(d->x, d->tmp, (size_t)m * D, st));
        if (md->n_exp > 0) {
            CK(run_moe_unfused(d, &w, m, P, st));
            continue;
        }
        CK(tlg_dev_rmsnorm_fwd(d->x, P + w.an2, d->xn, NULL, m, D, st));
        GROUP(st, MMc(d->g, d->xn, P + w.w1, m, D, F), MMc(d->u, d->xn, P + w.w3, m, D, F));
        CK(tlg_dev_swiglu_fwd(d->act, d->g, d->u, (size_t)m * F, st));
        GROUP(st, MMc(d->tmp, d->act, P + w.w2, m, F, D));
        CK(tlg_dev_add(d->x, d->tmp, (size_t)m * D, st));
    }
    dmap(d, 0, &w);
    CK(tlg_dev_rmsnorm_fwd(d->x, P + w.nf, d->fn, NULL, m, D, st));
    TlgGemmCall head = MMc(d->logits, d->fn, P + w.emb, m, V, D);
    head.op = 1;                                     /* memset + mm_bt (mmbt_dec :3033-3036) */
    head.beta = 0;
    CK(tlg_dev_gemm_group(&head, 1, st));
    return tlg_dev_gemm_flush(st);
}

int tl_decode_chunk(TlDecode *d, const int *tok, int m, int start, void *st)
{
    if (m <= 0 || m > d->mmax || start < 0 || start + m > d->maxpos) return TLG_EINVAL;
    for (int j = 0; j < m; j++) if (tok[j] < 0 || tok[j] >= d->m.V) return TLG_EINVAL;
    CK(tlg_memcpy_h2d(d->tok, tok, 4 * (size_t)m, st));
    CK(tlg_stream_sync(st));
    return run_chunk(d, m, 0, start, 0, st);
}

int tl_decode_prime(TlDecode *d, const int *prompt, int n, void *st)
{
    if (n <= 0) return TLG_EINVAL;
    int i = 0, m = 0;
    while (i < n) {
        m = n - i < d->mmax ? n - i : d->mmax;
        CK(tl_decode_chunk(d, prompt + i, m, i, st));
        i += m;
    }
    const int s[3] = {n - m, m, 0};                   /* the last chunk; argmax advances it */
    CK(tlg_memcpy_h2d(d->state, s, sizeof s, st));    /* state[3] (exchange sequence) is kept */
    CK(tlg_dev_dec_argmax(d->logits, d->m.V, m, d->state, d->tok, st));
    return tlg_stream_sync(st);
}

int tl_decode_mtp_draft(TlDecode *d, int row, int k, int *dtok_out, void *st)
{
    if (!d || !dtok_out || k < 0 || k >= d->m.n_mtp || row < 0 || row >= d->mmax) return TLG_EINVAL;
    const int D = d->m.D, V = d->m.V;
    const float *P = d->P[0], *Pt = d->Pt[0];
    DMap w;
    dmap(d, 0, &w);
    const float *xr = d->x + (size_t)row * D;
    /* ht = fn Wk (mm_dec(1, D, D), the head's W^T on the decode layout, with
     * fn = RMSNorm(x, nf) as the prologue), hh = fn + silu(ht), logits_k =
     * hh emb^T (mmbt_dec), argmax_v */
    DGEMV(st, DG(1, 0, d->ht, 1, D, D, xr, Pt + w.mtp0 + (size_t)k * D * D, 1, P + w.nf, NULL));
    CK(tlg_dev_dec_mtp_mix(d->hh, xr, P + w.nf, d->ht, D, st));
    DGEMV(st, DG(1, 0, d->hlog, 1, V, D, d->hh, P + w.emb, 0, NULL, NULL));
    return tlg_dev_argmax_rows(d->hlog, V, 1, dtok_out, st);
}

int tl_decode_generate_spec(TlDecode *d, const int *prompt, int np, int n, int *toks, int *chunks, void *st)
{
    const int K = d ? d->m.n_mtp : 0;
    if (!d || !prompt || np <= 0 || n <= 0 || !toks || K < 1 || K + 1 > d->mmax || K + 1 > 16) return TLG_EINVAL;
    /* prefill in chunks of mmax (positions 0..np-1), as tl_decode_prime */
    int i = 0, m = 0;
    while (i < np) {
        m = np - i < d->mmax ? np - i : d->mmax;
        CK(tl_decode_chunk(d, prompt + i, m, i, st));
        i += m;
    }
    int pos = np, cur = m - 1, got = 0, nch = 0;
    int draft[16], best[16];
    while (got < n) {
        /* x1 = argmax of the current row, the heads' drafts from its fn */
        CK(tlg_dev_argmax_rows(d->logits + (size_t)cur * d->m.V, d->m.V, 1, d->dtok, st));
        for (int k = 0; k < K; k++) CK(tl_decode_mtp_draft(d, cur, k, d->dtok + 1 + k, st));
        CK(tlg_memcpy_d2h(draft, d->dtok, sizeof(int) * (size_t)(K + 1), st));
        CK(tlg_stream_sync(st));
        if (pos + K + 1 > d->maxpos) return TLG_EINVAL;
        /* one chunk verifies the drafts: row r's argmax must equal draft r + 1 */
        CK(tl_decode_chunk(d, draft, K + 1, pos, st));
        nch++;
        toks[got++] = draft[0];
        CK(tlg_dev_argmax_rows(d->logits, d->m.V, K + 1, d->dtok, st));
        CK(tlg_memcpy_d2h(best, d->dtok, sizeof(int) * (size_t)(K + 1), st));
        CK(tlg_stream_sync(st));
        int acc = 0;
        for (int r = 0; r < K && got < n; r++) {
            if (draft[r + 1] != best[r]) break;
            toks[got++] = best[r];
            acc++;
        }
        pos += acc + 1;
        cur = acc;
    }
    if (chunks) *chunks = nch;
    return 0;
}

int tl_decode_greedy_step(TlDecode *d, int copy, void *st)
{
    if (copy < 0 || copy >= d->pool) return TLG_EINVAL;
    CK(run_chunk(d, 1, 1, 0, copy, st));
    return tlg_dev_dec_argmax(d->logits, d->m.V, 1, d->state, d->tok, st);
}

int tl_decode_graph_build(TlDecode *d, void *st)
{
    for (int c = 0; c < d->pool; c++) {
        if (d->graph[c]) { tlg_graph_destroy(d->graph[c]); d->graph[c] = NULL; }
        CK(tlg_graph_begin(st));
        const int rc = tl_decode_greedy_step(d, c, st);
        void *g = tlg_graph_end(st);
        if (rc) { if (g) tlg_graph_destroy(g); return rc; }
        if (!g) return TLG_EHIP;
        d->graph[c] = g;
    }
    d->next_graph = 0;
    return 0;
}

int tl_decode_graph_step(TlDecode *d, void *st)
{
    void *g = d->graph[d->next_graph];
    if (!g) return TLG_EINVAL;
    d->next_graph = (d->next_graph + 1) % d->pool;
    return tlg_graph_launch(g, st);
}

int tl_decode_state(TlDecode *d, int *state, void *st)
{
    int s[4];
    CK(tlg_memcpy_d2h(s, d->state, sizeof s, st));
    CK(tlg_stream_sync(st));
    memcpy(state, s, 3 * sizeof(int));
    return 0;
}

int tl_decode_set_fused(TlDecode *d, int fused)
{
    if (!d) return TLG_EINVAL;
    d->unfused = fused ? 0 : 1;
    for (int c = 0; c < TLD_MAXPOOL; c++)          /* captured steps are stale */
        if (d->graph[c]) { tlg_graph_destroy(d->graph[c]); d->graph[c] = NULL; }
    return 0;
}

/* ---- persistent greedy decoding (tldecode.h tlg_dev_dec_persist) ------------- */
static int persist_args(TlDecode *d, TlgDecPersist *pa, int *toks_out);

int tl_decode_persist(TlDecode *d, int n, int *toks_out, void *st)
{
    if (!d || n <= 0) return TLG_EINVAL;
    TlgDecPersist a;
    CK(persist_args(d, &a, toks_out));
    CK(tlg_dev_dec_persist(&a, n, st));
    d->next_copy = (d->next_copy + n) % d->pool;
    return 0;
}

int tl_decode_chunks(TlDecode *d, int m, const int *dtoks, int n, int *toks_out, void *st)
{
    if (!d || n <= 0 || m <= 0 || m > d->mmax || !dtoks) return TLG_EINVAL;
    TlgDecPersist a;
    CK(persist_args(d, &a, toks_out));
    CK(tlg_dev_dec_chunks(&a, m, dtoks, n, st));
    d->next_copy = (d->next_copy + n) % d->pool;
    return 0;
}

static int persist_args(TlDecode *d, TlgDecPersist *pa, int *toks_out)
{
    const TlModel *md = &d->m;
    TlgDecPersist a;
    memset(&a, 0, sizeof a);
    /* the persistent kernels run the dense model (the single-token one also
     * with QK-norm; tlg_dev_dec_chunks refuses it) */
    if (md->L > TLG_PD_MAXL || md->n_exp > 0) return TLG_EINVAL;
    for (int c = 0; c < d->pool; c++) a.P[c] = d->P[c];
    a.pool = d->pool;
    a.copy0 = d->next_copy;
    a.V = md->V; a.D = md->D; a.L = md->L; a.H = md->H; a.KV = md->KV; a.F = md->F;
    a.win = md->win; a.full_every = md->full_every;
    a.W = d->W; a.f16 = d->f16; a.exact = d->exact; a.maxpos = d->maxpos;
    a.cs = d->rcos; a.sn = d->rsin;
    for (int l = 0; l < md->L; l++) { a.Kc[l] = d->Kc[l]; a.Vc[l] = d->Vc[l]; }
    a.logits = d->logits; a.state = d->state; a.tok = d->tok; a.toks_out = toks_out; a.xbuf = d->xbuf;
    a.qknorm = md->qknorm ? 1 : 0;
    *pa = a;
    return 0;
}

int tl_decode_persist_status(TlDecode *d, void *st)
{
    return d ? tlg_dec_persist_status(d->xbuf, st) : TLG_EINVAL;
}
