/* tl_decode.c -- device-resident decoding of tinylm.c (see tl_decode.h). */
#include "tl_decode.h"
#include "../../include/tldecode.h"
#include "../../include/tlgemm.h"
#include "../../include/tltrain.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define TLD_MAXPOOL 16

typedef struct { size_t emb, an1, wq, wk, wv, wo, an2, w1, w3, w2, nf, total; } DMap;

struct TlDecode {
    TlModel m;
    int W, f16, exact, maxpos, mmax, pool, hd, KD;
    size_t np;
    void *arena;
    float *P[TLD_MAXPOOL];
    float *Pt[TLD_MAXPOOL];      /* the decode layout: every linear weight transposed, same offsets */
    void **Kc, **Vc;
    float *rcos, *rsin, *x, *xn, *q, *k, *v, *ctx, *tmp, *g, *u, *act, *fn, *logits;
    int *pos, *tok, *state;
    void *xbuf;                  /* the persistent decode's exchange area */
    size_t xbytes;
    void *graph[TLD_MAXPOOL];
    int next_graph;
    int next_copy;               /* weight copy of the next persistent step */
    int unfused;                 /* 1: the glue as separate launches (tl_decode_set_fused) */
};

/* map_weights (tinylm.c:361-393), dense FFN, no QK-norm */
static void dmap(const TlDecode *d, int l, DMap *o)
{
    const size_t D = d->m.D, KD = d->KD, F = d->m.F;
    const size_t per = D + D * D + 2 * D * KD + D * D + D + 3 * D * F;
    o->emb = 0;
    o->an1 = (size_t)d->m.V * D + (size_t)l * per;
    o->wq = o->an1 + D;
    o->wk = o->wq + D * D;
    o->wv = o->wk + D * KD;
    o->wo = o->wv + D * KD;
    o->an2 = o->wo + D * D;
    o->w1 = o->an2 + D;
    o->w3 = o->w1 + D * F;
    o->w2 = o->w3 + D * F;
    o->nf = (size_t)d->m.V * D + (size_t)d->m.L * per;
    o->total = o->nf + D + (size_t)d->m.n_mtp * D * D;
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
    if (!m || m->n_exp != 0 || m->D <= 0 || m->H <= 0 || m->KV <= 0 || m->D % m->H || m->H % m->KV ||
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
    const int D = d->m.D, KD = d->KD, F = d->m.F;
    for (int c = 0; c < d->pool; c++)
        for (int l = 0; l < d->m.L; l++) {
            DMap w;
            dmap(d, l, &w);
            const struct { size_t off; int rows, cols; } mats[] = {
                {w.wq, D, D}, {w.wk, D, KD}, {w.wv, D, KD}, {w.wo, D, D}, {w.w1, D, F}, {w.w3, D, F}, {w.w2, F, D},
            };
            for (size_t i = 0; i < sizeof mats / sizeof mats[0]; i++) {
                int rc = tlg_dev_transpose(d->Pt[c] + mats[i].off, d->P[c] + mats[i].off, mats[i].rows, mats[i].cols,
                                           st);
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
    c.op = op; c.beta = beta; c.C = C; c.M = M; c.K = K; c.N = N; c.A = A; c.B = Bw;
    c.pro = pro; c.gain = gain; c.A2 = A2;
    return c;
}

#define DGEMV(st, ...) do { TlgDecGemv cs_[] = {__VA_ARGS__}; \
        CK(tlg_dev_dec_gemv(cs_, (int)(sizeof cs_ / sizeof cs_[0]), st)); } while (0)

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
        CK(tlg_dev_dec_rope_attn(d->q, d->k, d->v, d->pos, d->rcos, d->rsin, d->maxpos, d->Kc[l], d->Vc[l], d->ctx, m,
                                 H, KV, hd, d->W, dwin(md, l), d->f16, d->exact, st));
        DGEMV(st, DG(1, 1, d->x, m, D, D, d->ctx, Pt + w.wo, 0, NULL, NULL));
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
        CK(tlg_dev_rope(d->q, d->pos, 1, m, H, hd, d->rcos, d->rsin, d->maxpos, 0, st));
        CK(tlg_dev_rope(d->k, d->pos, 1, m, KV, hd, d->rcos, d->rsin, d->maxpos, 0, st));
        CK(tlg_dev_kv_store(d->k, d->v, d->pos, m, KD, d->W, d->f16, d->Kc[l], d->Vc[l], st));
        CK(tlg_dev_dec_attn(d->q, d->Kc[l], d->Vc[l], d->pos, d->ctx, m, H, KV, hd, d->W, dwin(md, l), d->f16,
                            d->exact, st));
        GROUP(st, MMc(d->tmp, d->ctx, P + w.wo, m, D, D));
        CK(tlg_dev_add(d->x, d->tmp, (size_t)m * D, st));
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
    if (md->L > TLG_PD_MAXL) return TLG_EINVAL;
    for (int c = 0; c < d->pool; c++) a.P[c] = d->P[c];
    a.pool = d->pool;
    a.copy0 = d->next_copy;
    a.V = md->V; a.D = md->D; a.L = md->L; a.H = md->H; a.KV = md->KV; a.F = md->F;
    a.win = md->win; a.full_every = md->full_every;
    a.W = d->W; a.f16 = d->f16; a.exact = d->exact; a.maxpos = d->maxpos;
    a.cs = d->rcos; a.sn = d->rsin;
    for (int l = 0; l < md->L; l++) { a.Kc[l] = d->Kc[l]; a.Vc[l] = d->Vc[l]; }
    a.logits = d->logits; a.state = d->state; a.tok = d->tok; a.toks_out = toks_out; a.xbuf = d->xbuf;
    *pa = a;
    return 0;
}

int tl_decode_persist_status(TlDecode *d, void *st)
{
    return d ? tlg_dec_persist_status(d->xbuf, st) : TLG_EINVAL;
}
