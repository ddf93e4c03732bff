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
#include <limits.h>
#include <stdlib.h>
#include <string.h>

#define TL_MAXPOOL 16
#define TL_MAXLAUNCH 1024

struct TlRun {
    const TlPlan *plan;
    float *arena;
    size_t off[TL_MAXBUF];      /* float offset of each buffer in the arena */
    size_t p_stride;            /* floats between pool copies of P */
    int p_id;                   /* buffer id of P (-1 if none) */
    int pool, cur;
    void *graph[TL_MAXPOOL];
    /* optional per-launch timing of grouped steps (tl_run_time_launches) */
    void **ev;
    int nev;
    double lflops[TL_MAXLAUNCH], lbytes[TL_MAXLAUNCH];
    int lkind[TL_MAXLAUNCH];             /* 0 grouped GEMM, 1 clear, 2 flush */
    const char *lname[TL_MAXLAUNCH];     /* kernel of each launch (NULL: none) */
    /* tile configuration of each grouped launch: 0 = the library's automatic
     * policy, else config + 1 (set by tl_run_autotune) */
    int lcfg[TL_MAXLAUNCH];
    /* split target of each grouped launch (tlg_tune_group_split; 0 = the
     * library's automatic target) */
    int lrt[TL_MAXLAUNCH];
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

/* ---- grouped step ------------------------------------------------------- */
/* Float range [lo, hi) of buffer `id` touched by an operand. */
typedef struct { int id; size_t lo, hi; } Span;

static int spans_overlap(Span a, Span b) { return a.id == b.id && a.lo < b.hi && b.lo < a.hi; }

/* Output and input ranges of a GEMM call (reference argument meaning). */
static void call_spans(const TlCall *c, Span *out, Span *a, Span *b)
{
    const size_t M = c->M, K = c->K, N = c->N;
    size_t no, na, nb;
    switch (c->op) {
    case TL_MM:    no = M * N; na = M * K; nb = K * N; break;
    case TL_MM_BT: no = M * K; na = M * N; nb = K * N; break;
    default:       no = K * N; na = M * K; nb = M * N; break;
    }
    if (c->op == TL_ZERO) no = c->n;
    out->id = c->out; out->lo = c->out_off; out->hi = c->out_off + no;
    a->id = c->a; a->lo = c->a_off; a->hi = c->a_off + na;
    b->id = c->b; b->lo = c->b_off; b->hi = c->b_off + nb;
}

#define TL_GROUP_MAX 8

typedef struct {
    TlgGemmCall call[TL_GROUP_MAX];
    Span wr[TL_GROUP_MAX], rd[2 * TL_GROUP_MAX * 3];
    int n, nrd;
} Group;

/* Record the event that opens launch k (timing runs only). */
static int mark(TlRun *r, int k, void *stream)
{
    if (!r->ev || k >= r->nev) return 0;
    return tlg_event_record(r->ev[k], stream);
}

static void note(TlRun *r, int k, int kind, double flops, double bytes)
{
    if (k >= TL_MAXLAUNCH) return;
    r->lkind[k] = kind;
    r->lflops[k] = flops;
    r->lbytes[k] = bytes;
}

static double gemm_flops(const TlgGemmCall *c)
{
    if (c->op == 3) return 0.0;
    double f = 0.0;
    for (int s = 0; s < c->nseg; s++)
        f += 2.0 * c->M * c->K * (double)(s ? c->Nseg[s] : c->N);
    return f;
}

static double gemm_bytes(const TlgGemmCall *c)
{
    if (c->op == 3) return 4.0 * (double)c->M * (double)c->N;
    const double M = c->M, K = c->K;
    double b = 0.0;
    for (int s = 0; s < c->nseg; s++) {
        const double N = s ? c->Nseg[s] : c->N;
        if (c->op == 0) b += M * K + K * N;
        else if (c->op == 1) b += M * N + K * N;
        else b += M * K + M * N;
    }
    const double out = c->op == 0 ? M * c->N : (c->op == 1 ? M * K : K * c->N);
    return 4.0 * (b + out * (c->beta ? 2.0 : 1.0));
}

static int group_launch(TlRun *r, Group *g, void *stream, int dry, int *launches)
{
    if (g->n == 0) return 0;
    double fl = 0.0, by = 0.0;
    for (int k = 0; k < g->n; k++) { fl += gemm_flops(&g->call[k]); by += gemm_bytes(&g->call[k]); }
    note(r, *launches, 0, fl, by);
    int rc = dry ? 0 : mark(r, *launches, stream);
    if (!rc && !dry) {
        const int cfg = *launches < TL_MAXLAUNCH ? r->lcfg[*launches] - 1 : -1;
        const int rt = *launches < TL_MAXLAUNCH ? r->lrt[*launches] : 0;
        if (cfg >= 0) rc = tlg_tune_group(cfg);
        if (!rc && rt) rc = tlg_tune_group_split(rt);
        if (!rc) rc = tlg_dev_gemm_group(g->call, g->n, stream);
        if (cfg >= 0) { const int rc2 = tlg_tune_group(-1); if (!rc) rc = rc2; }
        if (rt) { const int rc2 = tlg_tune_group_split(0); if (!rc) rc = rc2; }
    }
    if (!rc && !dry && *launches < TL_MAXLAUNCH) r->lname[*launches] = tlg_group_kernel();
    (*launches)++;
    g->n = g->nrd = 0;
    return rc;
}

/* Does call c conflict with what group g already reads or writes? */
static int group_conflict(const Group *g, const TlCall *c)
{
    Span o, a, b;
    call_spans(c, &o, &a, &b);
    for (int k = 0; k < g->n; k++)
        if (spans_overlap(o, g->wr[k]) || spans_overlap(a, g->wr[k]) || spans_overlap(b, g->wr[k]))
            return 1;
    for (int k = 0; k < g->nrd; k++)
        if (spans_overlap(o, g->rd[k])) return 1;
    return 0;
}

/* Index of the first GEMM after call z (same run) that writes exactly the
 * range z clears, accumulating, with nothing in between touching it; -1 if
 * the clear must stay a clear. */
static int clear_target(const TlPlan *p, int z, int end)
{
    Span zo, za, zb;
    call_spans(&p->call[z], &zo, &za, &zb);
    for (int j = z + 1; j < end; j++) {
        const TlCall *c = &p->call[j];
        Span o, a, b;
        call_spans(c, &o, &a, &b);
        if (c->op == TL_ZERO) { if (spans_overlap(o, zo)) return -1; continue; }
        if (spans_overlap(a, zo) || spans_overlap(b, zo)) return -1;
        if (spans_overlap(o, zo))
            return (c->op != TL_MM && o.lo == zo.lo && o.hi == zo.hi) ? j : -1;
    }
    return -1;
}

static int grouped(TlRun *r, void *stream, int dry)
{
    const TlPlan *p = r->plan;
    int launches = 0, rc = 0;
    char *set = calloc((size_t)p->ncall, 1);       /* GEMM turned into a setting one */
    char *gone = calloc((size_t)p->ncall, 1);      /* clear folded into a GEMM */
    if (!set || !gone) { free(set); free(gone); return TLG_ENOMEM; }
    Group g;
    g.n = g.nrd = 0;
    for (int i = 0; i < p->ncall && rc == 0;) {
        int end = i;
        while (end < p->ncall && p->call[end].run == p->call[i].run) end++;
        for (int z = i; z < end; z++)
            if (p->call[z].op == TL_ZERO) {
                const int t = clear_target(p, z, end);
                if (t >= 0) { set[t] = 1; gone[z] = 1; }
            }
        for (int j = i; j < end && rc == 0; j++) {
            const TlCall *c = &p->call[j];
            if (gone[j]) continue;
            if (c->op == TL_ZERO) {
                rc = group_launch(r, &g, stream, dry, &launches);
                note(r, launches, 1, 0.0, 4.0 * (double)c->n);
                if (!rc && !dry) rc = mark(r, launches, stream);
                if (!rc && !dry) rc = tlg_dev_zero(ptr(r, c->out, c->out_off), c->n, stream);
                if (!dry && launches < TL_MAXLAUNCH) r->lname[launches] = "k_zero";
                launches++;
                continue;
            }
            Span o, a, b;
            call_spans(c, &o, &a, &b);
            /* extend an mm_bt chain into the same dX */
            if (g.n > 0 && c->op == TL_MM_BT && !set[j]) {
                TlgGemmCall *last = &g.call[g.n - 1];
                if (last->op == 1 && last->nseg < 3 && last->C == ptr(r, c->out, c->out_off) &&
                    last->M == c->M && last->K == c->K) {
                    int clash = 0;
                    for (int k = 0; k < g.n; k++)
                        if (spans_overlap(a, g.wr[k]) || spans_overlap(b, g.wr[k])) clash = 1;
                    if (!clash) {
                        last->A[last->nseg] = ptr(r, c->a, c->a_off);
                        last->B[last->nseg] = ptr(r, c->b, c->b_off);
                        last->Nseg[last->nseg] = c->N;
                        last->nseg++;
                        g.rd[g.nrd++] = a;
                        g.rd[g.nrd++] = b;
                        continue;
                    }
                }
            }
            if (g.n == TL_GROUP_MAX || group_conflict(&g, c)) rc = group_launch(r, &g, stream, dry, &launches);
            if (rc) break;
            TlgGemmCall *k = &g.call[g.n];
            memset(k, 0, sizeof *k);
            k->op = c->op;
            k->beta = (c->op == TL_MM || set[j]) ? 0 : 1;
            k->C = ptr(r, c->out, c->out_off);
            k->M = c->M; k->K = c->K; k->N = c->N;
            k->nseg = 1;
            k->A[0] = ptr(r, c->a, c->a_off);
            k->B[0] = ptr(r, c->b, c->b_off);
            g.wr[g.n] = o;
            g.rd[g.nrd++] = a;
            g.rd[g.nrd++] = b;
            g.n++;
        }
        /* a clear the plan marks hoistable (nothing between the two runs
         * touches its range) rides along with this run's launch */
        if (!rc && g.n > 0 && end < p->ncall) {
            int e2 = end, all = 1;
            while (e2 < p->ncall && p->call[e2].run == p->call[end].run) e2++;
            for (int z = end; z < e2; z++)
                if (p->call[z].op != TL_ZERO || !p->call[z].hoist || p->call[z].n > (size_t)INT_MAX) all = 0;
            for (int z = end; all && z < e2 && g.n < TL_GROUP_MAX; z++) {
                const TlCall *c = &p->call[z];
                if (group_conflict(&g, c)) continue;
                Span o, a, b;
                call_spans(c, &o, &a, &b);
                TlgGemmCall *k = &g.call[g.n];
                memset(k, 0, sizeof *k);
                k->op = 3;
                k->C = ptr(r, c->out, c->out_off);
                k->M = (int)c->n;
                k->N = 1;
                g.wr[g.n++] = o;
                gone[z] = 1;
            }
        }
        if (!rc) rc = group_launch(r, &g, stream, dry, &launches);
        i = end;
    }
    /* the flush reduces the last launch's split partials (if any) */
    note(r, launches, 2, 0.0, 0.0);
    if (!rc && !dry) rc = mark(r, launches, stream);
    /* the flush launches a kernel only if split partials are pending */
    const int pending = dry ? 0 : tlg_dev_gemm_pending();
    if (!rc && !dry) rc = tlg_dev_gemm_flush(stream);
    if (!rc && !dry && launches < TL_MAXLAUNCH) r->lname[launches] = pending > 0 ? tlg_group_kernel() : NULL;
    if (!rc && !dry) rc = mark(r, launches + 1, stream);
    free(set);
    free(gone);
    if (rc) return rc;
    if (!dry) r->cur = (r->cur + 1) % r->pool;
    return dry ? launches : 0;
}

int tl_run_time_launches(TlRun *r, void **events, int nevents, void *stream)
{
    r->ev = events;
    r->nev = nevents;
    int rc = grouped(r, stream, 0);
    r->ev = NULL;
    r->nev = 0;
    return rc;
}

const char *tl_run_launch_kernel(TlRun *r, int k)
{
    if (k < 0 || k >= TL_MAXLAUNCH) return NULL;
    return r->lname[k];
}

int tl_run_launch_info(TlRun *r, int k, double *flops, double *bytes)
{
    if (k < 0 || k >= TL_MAXLAUNCH) return -1;
    *flops = r->lflops[k];
    *bytes = r->lbytes[k];
    return r->lkind[k];
}

int tl_run_step_grouped(TlRun *r, void *stream) { return grouped(r, stream, 0); }
int tl_run_grouped_launches(TlRun *r) { return grouped(r, NULL, 1); }

int tl_run_graph_build(TlRun *r, void *stream, int grouped_step)
{
    for (int c = 0; c < r->pool; c++) {
        if (r->graph[c]) { tlg_graph_destroy(r->graph[c]); r->graph[c] = NULL; }
        r->cur = c;
        int rc = tlg_graph_begin(stream);
        if (rc) return rc;
        if (grouped_step) {
            rc = grouped(r, stream, 0);
            r->cur = c;
        } else {
            for (int i = 0; i < r->plan->ncall && rc == 0; i++) rc = tl_run_call(r, i, stream);
        }
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

/* Per-launch tile and split choice by measurement: run `reps` timed steps
 * with every (configuration, split target) candidate pair applied to all
 * grouped launches, then give each launch the pair with the least time.
 * Numerically every candidate is a valid schedule of the same sums (the plan
 * tests cover each one).  A launch's split target also moves work into the
 * next launch (its partials are summed there), which the per-launch times
 * see as they come. */
int tl_run_autotune(TlRun *r, const int *cands, int ncands, int reps, void *stream)
{
    const int policy = 0;
    return tl_run_autotune_split(r, cands, ncands, &policy, 1, reps, stream);
}

int tl_run_autotune_split(TlRun *r, const int *cands, int ncands, const int *rts, int nrts, int reps,
                          void *stream)
{
    if (!r || !cands || ncands <= 0 || !rts || nrts <= 0 || reps <= 0) return -1;
    for (int s = 0; s < nrts; s++)
        if (rts[s] != 0 && rts[s] < 64) return -1;
    const int L = grouped(r, stream, 1);
    if (L < 0 || L + 2 > TL_MAXLAUNCH) return -1;
    double *best = malloc(sizeof(double) * (size_t)L);
    void **ev = malloc(sizeof(void *) * (size_t)(L + 2));
    int *pick = malloc(sizeof(int) * (size_t)L), *prt = malloc(sizeof(int) * (size_t)L);
    if (!best || !ev || !pick || !prt) { free(best); free(ev); free(pick); free(prt); return TLG_ENOMEM; }
    int rc = 0, made = 0;
    for (; made < L + 2; made++)
        if (!(ev[made] = tlg_event_create())) { rc = -1; break; }
    for (int k = 0; k < L; k++) { best[k] = 1e30; pick[k] = 0; prt[k] = 0; }
    for (int cs = 0; cs < ncands * nrts && !rc; cs++) {
        const int c = cs / nrts, rt = rts[cs % nrts];
        for (int k = 0; k < L; k++) { r->lcfg[k] = cands[c] + 1; r->lrt[k] = rt; }
        double *t = calloc((size_t)L, sizeof(double));
        if (!t) { rc = TLG_ENOMEM; break; }
        rc = tl_run_step_grouped(r, stream);                /* warm up this shape */
        for (int rep = 0; rep < reps && !rc; rep++) {
            rc = tl_run_time_launches(r, ev, L + 2, stream);
            if (!rc) rc = tlg_stream_sync(stream);
            for (int k = 0; k < L && !rc; k++) t[k] += tlg_event_elapsed_ms(ev[k], ev[k + 1]);
        }
        for (int k = 0; k < L && !rc; k++)
            if (r->lkind[k] == 0 && t[k] < best[k]) { best[k] = t[k]; pick[k] = cands[c] + 1; prt[k] = rt; }
        free(t);
    }
    for (int k = 0; k < L; k++) { r->lcfg[k] = rc ? 0 : pick[k]; r->lrt[k] = rc ? 0 : prt[k]; }
    for (int k = 0; k < made; k++) tlg_event_destroy(ev[k]);
    free(best); free(ev); free(pick); free(prt);
    return rc;
}

int tl_run_set_launch_config(TlRun *r, int k, int cfg)
{
    if (!r || k < 0 || k >= TL_MAXLAUNCH || cfg < -1) return -1;
    r->lcfg[k] = cfg + 1;
    return 0;
}

int tl_run_launch_config(TlRun *r, int k)
{
    if (!r || k < 0 || k >= TL_MAXLAUNCH) return -1;
    return r->lcfg[k] - 1;
}

int tl_run_set_launch_split(TlRun *r, int k, int rtarget)
{
    if (!r || k < 0 || k >= TL_MAXLAUNCH || (rtarget != 0 && rtarget < 64)) return -1;
    r->lrt[k] = rtarget;
    return 0;
}

int tl_run_launch_split(TlRun *r, int k)
{
    if (!r || k < 0 || k >= TL_MAXLAUNCH) return -1;
    return r->lrt[k];
}
