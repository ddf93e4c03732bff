
/* ref_seq_post.c -- appended after tinylm.c:539-1154 (oracle/Makefile).
 * TEST INFRASTRUCTURE ONLY.  tlref_train_log() runs the reference's own
 * forward + memset(G) + backward (as train_loop does, tinylm.c:2627-2629) on
 * a small dense model and returns its GEMM call list with every pointer
 * named by the buffer it lies in (P / G at map_weights offsets, or an Acts
 * field with a per-layer slice offset). */
#undef mm
#undef mm_bt
#undef mm_atb

static const char *tlref_names[] = {
    "P", "G", "a_in", "a_norm", "q", "k", "v", "att_ctx", "f_in", "f_norm", "g", "u",
    "x_final", "fn_norm", "logits", "probs", "dout", "dact", "dg", "du", "dfnorm", "dfin",
    "datt", "dq", "dk", "dv", "dnorm", "dain", "dlogits", "dfn", "?"};
const char *tlref_seq_name(int i) { return (i >= 0 && i < 31) ? tlref_names[i] : "?"; }

static void tlref_name(const float *p, const float *P, const float *G, size_t np, const Acts *a,
                       const Cfg *c, int *id, long long *off)
{
    const size_t N = a->N, D = c->D, KD = c->KD, F = c->F, V = c->V;
    *id = 30; *off = 0;
    if (p >= P && p < P + np) { *id = 0; *off = p - P; return; }
    if (p >= G && p < G + np) { *id = 1; *off = p - G; return; }
    float **per[] = {a->a_in, a->a_norm, a->q, a->k, a->v, a->att_ctx, a->f_in, a->f_norm, a->g, a->u};
    const size_t psz[] = {N * D, N * D, N * D, N * KD, N * KD, N * D, N * D, N * D, N * F, N * F};
    for (int f = 0; f < 10; f++)
        for (int l = 0; l < c->L; l++)
            if (p >= per[f][l] && p < per[f][l] + psz[f]) { *id = 2 + f; *off = (long long)(l * psz[f] + (p - per[f][l])); return; }
    const float *glob[] = {a->x_final, a->fn_norm, a->logits, a->probs, a->dout, a->dact, a->dg, a->du,
                           a->dfnorm, a->dfin, a->datt, a->dq, a->dk, a->dv, a->dnorm, a->dain, a->dlogits, a->dfn};
    const size_t gsz[] = {N * D, N * D, N * V, N * V, N * D, N * F, N * F, N * F, N * D, N * D, N * D,
                          N * D, N * KD, N * KD, N * D, N * D, N * V, N * D};
    for (int f = 0; f < 18; f++)
        if (p >= glob[f] && p < glob[f] + gsz[f]) { *id = 12 + f; *off = p - glob[f]; return; }
}

/* out[i*10 + 0..9] = op, out id, out off, a id, a off, b id, b off, M, K, N.
 * Returns the number of calls (at most cap). */
int tlref_train_log(int B, int T, int D, int H, int KV, int F, int V, int L, int n_mtp,
                    long long *out, int cap)
{
    Cfg c;
    memset(&c, 0, sizeof c);
    c.V = V; c.D = D; c.L = L; c.H = H; c.KV = KV; c.F = F; c.T = T; c.n_mtp = n_mtp;
    c.rope_base = 10000.0f;
    cfg_derive(&c);
    rope_init(&c, c.T);
    size_t np = param_count(&c);
    float *P = fz(np), *G = fz(np);
    Weights w, gr;
    map_weights(&c, P, &w);
    map_weights(&c, G, &gr);
    memset(&w.ng, 0, sizeof w.ng);
    memset(&gr.ng, 0, sizeof gr.ng);
    init_params(&c, &w);
    Acts *a = acts_new(&c, B);
    int N = B * T;
    int *tok = malloc(sizeof(int) * N), *tgt = malloc(sizeof(int) * N);
    for (int i = 0; i < N; i++) { tok[i] = (int)(xorshift() % V); tgt[i] = (int)(xorshift() % V); }
    int **tm = n_mtp ? malloc(sizeof(int *) * n_mtp) : NULL;
    for (int k = 0; k < n_mtp; k++) {
        tm[k] = malloc(sizeof(int) * N);
        for (int i = 0; i < N; i++) tm[k][i] = (int)(xorshift() % V);
    }
    tlref_ncalls = 0;
    forward(&c, &w, a, tok, tgt);
    memset(G, 0, sizeof(float) * np);
    backward(&c, &w, &gr, a, tok, tgt, tm);
    int n = tlref_ncalls < cap ? tlref_ncalls : cap;
    for (int i = 0; i < n; i++) {
        const TlrefCall *k = &tlref_calls[i];
        int id;
        long long off;
        long long *o = out + (size_t)i * 10;
        o[0] = k->op;
        tlref_name(k->o, P, G, np, a, &c, &id, &off); o[1] = id; o[2] = off;
        tlref_name(k->a, P, G, np, a, &c, &id, &off); o[3] = id; o[4] = off;
        tlref_name(k->b, P, G, np, a, &c, &id, &off); o[5] = id; o[6] = off;
        o[7] = k->M; o[8] = k->K; o[9] = k->N;
    }
    return n;
}

/* ---- the reference's own training-step functions (tinylm.c:539-1176) ----
 * Thin wrappers over the static functions so tests/golden/make_golden.py
 * and the CPU tests can record / compare their outputs. */
static Cfg tlref_mkcfg(int V, int D, int L, int H, int KV, int F, int T, int n_mtp, int n_exp, int win,
                       int full_every)
{
    Cfg c;
    memset(&c, 0, sizeof c);
    c.V = V; c.D = D; c.L = L; c.H = H; c.KV = KV; c.F = F; c.T = T; c.n_mtp = n_mtp; c.n_exp = n_exp;
    c.win = win; c.full_every = full_every;
    c.rope_base = 10000.0f;
    cfg_derive(&c);
    return c;
}
static void tlref_rope_reset(const Cfg *c, int maxpos)
{
    rope_max = 0;                       /* force rope_init to rebuild for this hd */
    rope_init(c, maxpos);
}
void tlref_rmsnorm_fwd(const float *x, const float *g, float *out, float *rinv, int rows, int D)
{ rmsnorm_fwd(x, g, out, rinv, rows, D); }
void tlref_rmsnorm_bwd(const float *x, const float *g, const float *rinv, const float *dy, float *dx, float *dg,
                       int rows, int D)
{ rmsnorm_bwd(x, g, rinv, dy, dx, dg, rows, D); }
/* rope_init's tables for head_dim hd (half = hd/2 floats per position). */
void tlref_rope_table(float *cs, float *sn, int maxpos, int hd)
{
    Cfg c = tlref_mkcfg(1, hd, 1, 1, 1, 1, maxpos, 0, 0, 0, 0);
    tlref_rope_reset(&c, maxpos);
    memcpy(cs, rope_cos, sizeof(float) * (size_t)maxpos * c.half);
    memcpy(sn, rope_sin, sizeof(float) * (size_t)maxpos * c.half);
}
void tlref_rope(float *buf, const int *pos, int rows, int nheads, int hd, int maxpos, int back)
{
    Cfg c = tlref_mkcfg(1, hd, 1, 1, 1, 1, maxpos, 0, 0, 0, 0);
    tlref_rope_reset(&c, maxpos);
    rope_apply(buf, pos, rows, nheads, hd, hd / 2, back);
}
/* attn_fwd / attn_bwd of one layer: q [B*T][H*hd], k, v [B*T][KV*hd]. */
static void tlref_attn_setup(Cfg *c, Acts *a, float **pq, float **pk, float **pv, float **pc, const float *q,
                             const float *k, const float *v, float *ctx, int B, int T, int H, int KV, int hd,
                             int win)
{
    *c = tlref_mkcfg(1, H * hd, 1, H, KV, 1, T, 0, 0, win, 0);
    memset(a, 0, sizeof *a);
    a->B = B; a->T = T; a->N = B * T;
    pq[0] = (float *)q; pk[0] = (float *)k; pv[0] = (float *)v; pc[0] = ctx;
    a->q = pq; a->k = pk; a->v = pv; a->att_ctx = pc;
}
void tlref_attn_fwd(const float *q, const float *k, const float *v, float *out, int B, int T, int H, int KV, int hd,
                    int win)
{
    Cfg c; Acts a; float *pq[1], *pk[1], *pv[1], *pc[1];
    tlref_attn_setup(&c, &a, pq, pk, pv, pc, q, k, v, out, B, T, H, KV, hd, win);
    attn_fwd(&c, &a, 0);
}
/* accumulates into dq, dk, dv (the reference's callers clear them first) */
void tlref_attn_bwd(const float *q, const float *k, const float *v, const float *datt, float *dq, float *dk,
                    float *dv, int B, int T, int H, int KV, int hd, int win)
{
    Cfg c; Acts a; float *pq[1], *pk[1], *pv[1], *pc[1];
    tlref_attn_setup(&c, &a, pq, pk, pv, pc, q, k, v, NULL, B, T, H, KV, hd, win);
    a.datt = (float *)datt; a.dq = dq; a.dk = dk; a.dv = dv;
    attn_bwd(&c, &a, 0);
}
void tlref_adamw(float *P, float *G, float *M, float *V, size_t n, float lr, float b1, float b2, float wd, int t,
                 float gscale)
{ adamw(P, G, M, V, n, lr, b1, b2, wd, t, gscale); }
float tlref_gradnorm(const float *G, size_t n) { return global_gradnorm(G, n); }

/* A whole model: parameter count, init_params from a seed, and one
 * forward + memset(G) + backward (train_loop, tinylm.c:2627-2629) with the
 * given tokens; returns the forward's loss.  tgt_mtp is n_mtp x N ints. */
size_t tlref_param_count(int V, int D, int L, int H, int KV, int F, int T, int n_mtp, int n_exp)
{
    Cfg c = tlref_mkcfg(V, D, L, H, KV, F, T, n_mtp, n_exp, 0, 0);
    return param_count(&c);
}
void tlref_init_params(float *P, unsigned long long seed, int V, int D, int L, int H, int KV, int F, int T,
                       int n_mtp, int n_exp)
{
    Cfg c = tlref_mkcfg(V, D, L, H, KV, F, T, n_mtp, n_exp, 0, 0);
    Weights w;
    map_weights(&c, P, &w);
    g_rng = seed;
    init_params(&c, &w);
}
/* acts_new has no counterpart that frees; this one releases what it took. */
static void tlref_acts_free(Acts *a, const Cfg *c)
{
    float **per[] = {a->a_in, a->a_norm, a->q, a->k, a->v, a->att_ctx, a->f_in, a->f_norm, a->g, a->u};
    for (int f = 0; f < 10; f++) {
        for (int l = 0; l < c->L; l++) free(per[f][l]);
        free(per[f]);
    }
    free(a->a_rinv); free(a->f_rinv); free(a->a_rinv_buf); free(a->f_rinv_buf);
    if (a->assign) {
        for (int l = 0; l < c->L; l++) { free(a->assign[l]); free(a->gate[l]); free(a->rprobs[l]); }
        free(a->assign); free(a->gate); free(a->rprobs);
    }
    float *glob[] = {a->x_final, a->fn_norm, a->fn_rinv, a->logits, a->probs, a->dout, a->dact, a->dg, a->du,
                     a->dfnorm, a->dfin, a->datt, a->dq, a->dk, a->dv, a->dnorm, a->dain, a->dlogits, a->dfn};
    for (int f = 0; f < 19; f++) free(glob[f]);
    free(a->pos);
    free(a);
}
float tlref_train_step(float *P, float *G, const int *tok, const int *tgt, const int *tgt_mtp, int B, int V, int D,
                       int L, int H, int KV, int F, int T, int n_mtp, int n_exp, int win, int full_every)
{
    Cfg c = tlref_mkcfg(V, D, L, H, KV, F, T, n_mtp, n_exp, win, full_every);
    tlref_rope_reset(&c, c.T);
    Weights w, gr;
    map_weights(&c, P, &w);
    map_weights(&c, G, &gr);
    memset(&w.ng, 0, sizeof w.ng);
    memset(&gr.ng, 0, sizeof gr.ng);
    Acts *a = acts_new(&c, B);
    const int N = B * T;
    int **tm = n_mtp ? malloc(sizeof(int *) * n_mtp) : NULL;
    for (int k = 0; k < n_mtp; k++) tm[k] = (int *)tgt_mtp + (size_t)k * N;
    tlref_ncalls = 0;                  /* the call log is not needed here */
    const float loss = forward(&c, &w, a, tok, tgt);
    memset(G, 0, sizeof(float) * param_count(&c));
    backward(&c, &w, &gr, a, tok, tgt, tm);
    free(tm);
    tlref_acts_free(a, &c);
    return loss;
}

/* forward()'s logits (tinylm.c:968-1018; no targets) for B sequences. */
void tlref_forward_logits(const float *P, const int *tok, float *logits, int B, int V, int D, int L, int H, int KV,
                          int F, int T, int n_exp, int win, int full_every)
{
    Cfg c = tlref_mkcfg(V, D, L, H, KV, F, T, 0, n_exp, win, full_every);
    tlref_rope_reset(&c, c.T);
    Weights w;
    map_weights(&c, (float *)P, &w);
    memset(&w.ng, 0, sizeof w.ng);
    Acts *a = acts_new(&c, B);
    forward(&c, &w, a, tok, NULL);
    memcpy(logits, a->logits, sizeof(float) * (size_t)B * T * V);
    tlref_acts_free(a, &c);
}
/* The decode path's KV-cache conversions and softmax exponential. */
void tlref_f2h(const float *x, unsigned short *h, int n) { for (int i = 0; i < n; i++) h[i] = f2h(x[i]); }
void tlref_h2f(const unsigned short *h, float *x, int n) { for (int i = 0; i < n; i++) x[i] = h2f(h[i]); }
void tlref_fast_expf(const float *x, float *y, int n) { for (int i = 0; i < n; i++) y[i] = fast_expf(x[i]); }
