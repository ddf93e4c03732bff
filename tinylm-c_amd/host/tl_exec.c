/* tl_exec.c -- runs a TlPlan on the GPU through the libtlgemm C ABI.
 *
 * Every plan buffer lives in one HBM arena (256-byte aligned slices), so a
 * step moves no data over the host link.  The parameter buffer P can be
 * replicated `pool` times and rotated per step: the decode weights of a token
 * (52.7 MB at m8 width) would otherwise stay in the 256 MB Infinity Cache
 * and the measured bandwidth would not be HBM's.
 */
#include "tl_plan.h"
#include "../../include/tlgemm.h"
#include <stdlib.h>
#include <string.h>

#define TL_MAXPOOL 16

struct TlRun {
    const TlPlan *plan;
    float *arena;
    size_t off[TL_MAXBUF];      /* float offset of each buffer in the arena */
    size_t p_stride;            /* floats between pool copies of P */
    int p_id;                   /* buffer id of P (-1 if none) */
    int pool, cur;
    void *graph[TL_MAXPOOL];
};

static size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

TlRun *tl_run_new(const TlPlan *p, int pool)
{
    if (!p || p->nbuf <= 0) return NULL;
    if (pool < 1) pool = 1;
    if (pool > TL_MAXPOOL) pool = TL_MAXPOOL;
    TlRun *r = calloc(1, sizeof *r);
    if (!r) return NULL;
    r->plan = p;
    r->pool = pool;
    r->p_id = tl_plan_find(p, "P");
    size_t total = 0;
    for (int i = 0; i < p->nbuf; i++) {
        r->off[i] = total;
        size_t n = round_up(p->buf[i].floats, 64);
        if (i == r->p_id) {
            r->p_stride = n;
            n *= (size_t)pool;
        }
        total += n;
    }
    r->arena = (float *)tlg_dev_malloc(total * sizeof(float));
    if (!r->arena) { free(r); return NULL; }
    return r;
}

void tl_run_free(TlRun *r)
{
    if (!r) return;
    for (int i = 0; i < TL_MAXPOOL; i++)
        if (r->graph[i]) tlg_graph_destroy(r->graph[i]);
    tlg_dev_free(r->arena);
    free(r);
}

float *tl_run_buf(TlRun *r, int id)
{
    if (!r || id < 0 || id >= r->plan->nbuf) return NULL;
    return r->arena + r->off[id];
}

static float *ptr(TlRun *r, int id, size_t off)
{
    float *b = r->arena + r->off[id];
    if (id == r->p_id) b += (size_t)r->cur * r->p_stride;
    return b + off;
}

int tl_run_fill(TlRun *r, unsigned long long seed, void *stream)
{
    static const float scale[] = {1.0f, 0.02f, 0.01f, 0.0f};
    for (int i = 0; i < r->plan->nbuf; i++) {
        const TlBuf *b = &r->plan->buf[i];
        const int copies = (i == r->p_id) ? r->pool : 1;
        for (int c = 0; c < copies; c++) {
            float *d = r->arena + r->off[i] + (size_t)c * r->p_stride;
            int rc = (b->init == TL_INIT_ZERO)
                   ? tlg_dev_zero(d, b->floats, stream)
                   : tlg_dev_fill_normal(d, b->floats, seed * 1000003ull + (unsigned long long)i,
                                         scale[b->init], stream);
            if (rc) return rc;
        }
    }
    return 0;
}

int tl_run_call(TlRun *r, int i, void *stream)
{
    const TlCall *c = &r->plan->call[i];
    float *o = ptr(r, c->out, c->out_off);
    switch (c->op) {
    case TL_ZERO:
        return tlg_dev_zero(o, c->n, stream);
    case TL_MM:
        return tlg_dev_sgemm_nn(o, ptr(r, c->a, c->a_off), ptr(r, c->b, c->b_off), c->M, c->K, c->N, stream);
    case TL_MM_BT:
        return tlg_dev_sgemm_nt_acc(o, ptr(r, c->a, c->a_off), ptr(r, c->b, c->b_off), c->M, c->K, c->N, stream);
    case TL_MM_ATB:
        return tlg_dev_sgemm_tn_acc(o, ptr(r, c->a, c->a_off), ptr(r, c->b, c->b_off), c->M, c->K, c->N, stream);
    default:
        return TLG_EINVAL;
    }
}

int tl_run_step(TlRun *r, void *stream)
{
    for (int i = 0; i < r->plan->ncall; i++) {
        int rc = tl_run_call(r, i, stream);
        if (rc) return rc;
    }
    r->cur = (r->cur + 1) % r->pool;
    return 0;
}

int tl_run_graph_build(TlRun *r, void *stream)
{
    for (int c = 0; c < r->pool; c++) {
        if (r->graph[c]) { tlg_graph_destroy(r->graph[c]); r->graph[c] = NULL; }
        r->cur = c;
        int rc = tlg_graph_begin(stream);
        if (rc) return rc;
        for (int i = 0; i < r->plan->ncall && rc == 0; i++) rc = tl_run_call(r, i, stream);
        void *g = tlg_graph_end(stream);
        if (rc) return rc;
        if (!g) return TLG_EHIP;
        r->graph[c] = g;
    }
    r->cur = 0;
    return 0;
}

int tl_run_graph_step(TlRun *r, void *stream)
{
    if (!r->graph[r->cur]) return TLG_ESTATE;
    int rc = tlg_graph_launch(r->graph[r->cur], stream);
    r->cur = (r->cur + 1) % r->pool;
    return rc;
}
