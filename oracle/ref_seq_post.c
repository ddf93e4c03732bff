
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
