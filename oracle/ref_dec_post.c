/* ref_dec_post.c -- appended after the reference's decode attention
 * (oracle/Makefile, target _ref/libtlref_dec.so).  TEST INFRASTRUCTURE ONLY.
 *
 * tlref_dec_new() builds the reference's own decode state with gen_new (a
 * ring of W = T positions per layer; no weights, no int8 copies), and
 * tlref_dec_attn() runs one layer's attention step of forward_chunk
 * (tinylm.c:3759-3795) on given q / k / v rows: the hoisted kv_store of the m
 * new rows, then attn_body over every (row, kv-head) job with no split (NC =
 * 1, the path the reference calls bit-exact).  The ring's element type is
 * chosen the way the reference's CLI chooses it (TINYLM_KV, read by
 * gen_new); the decode pool stays serial (TINYLM_THREADS=1, before its first
 * use); the softmax exponential is fast_expf unless TINYLM_EXACT_EXP was set
 * before the first call. */
typedef struct { Cfg c; Gen *gn; } TlrefDec;

void *tlref_dec_new(int D, int H, int KV, int T, int L, int win, int full_every, int kvdt)
{
    setenv("TINYLM_THREADS", "1", 0);
    setenv("TINYLM_KV", kvdt ? "f16" : "f32", 1);
    TlrefDec *d = calloc(1, sizeof *d);
    if (!d) return NULL;
    memset(&d->c, 0, sizeof d->c);
    d->c.V = 1; d->c.D = D; d->c.L = L; d->c.H = H; d->c.KV = KV; d->c.F = 4; d->c.T = T;
    d->c.win = win; d->c.full_every = full_every;
    d->c.rope_base = 10000.0f;
    cfg_derive(&d->c);
    d->gn = gen_new(&d->c, NULL, 0);
    if (!d->gn) { free(d); return NULL; }
    return d;
}

/* ctx [m][D] of layer l for query rows q [m][D] at positions start_pos ..
 * start_pos + m - 1, whose new K / V rows (k, v [m][KD]) enter the ring first. */
int tlref_dec_attn(void *h, int l, const float *q, const float *k, const float *v, int m, int start_pos,
                   float *ctx)
{
    TlrefDec *d = (TlrefDec *)h;
    if (!d) return -1;
    const Cfg *c = &d->c;
    Gen *gn = d->gn;
    if (m < 1 || m > c->T || l < 0 || l >= c->L) return -1;
    const int D = c->D, KD = c->KD, KV = c->KV, hd = c->hd, W = c->T, grp = c->H / c->KV;
    memcpy(gn->q, q, sizeof(float) * (size_t)m * D);
    const int eff = cfg_lwin(c, l), wlim = (eff > 0 && eff < W) ? eff : W;
    const int dt = gn->kvdt, esz = kv_elem_sz(dt);
    for (int j = 0; j < m; j++) {
        const int slot = (start_pos + j) % W;
        kv_store(gn->Kc[l], gn->Ksc ? gn->Ksc[l] : NULL, slot, k + (size_t)j * KD, KD, KV, hd, dt);
        kv_store(gn->Vc[l], gn->Vsc ? gn->Vsc[l] : NULL, slot, v + (size_t)j * KD, KD, KV, hd, dt);
    }
    AttnJob aj = {c, gn, l, start_pos, wlim, W, 1, KV, grp, hd, D, KD, dt, esz, 1.0f / sqrtf((float)hd)};
    attn_body(&aj, 0, m * KV, 0);
    memcpy(ctx, gn->ctx, sizeof(float) * (size_t)m * D);
    return 0;
}

/* A whole model's decode state (V, F, experts, MTP heads, QK-norm; no int8
 * copies), for the pieces of forward_chunk and the speculative loop below. */
void *tlref_gen_new(int V, int D, int H, int KV, int F, int T, int L, int n_exp, int n_mtp, int qknorm, int kvdt)
{
    setenv("TINYLM_THREADS", "1", 0);
    setenv("TINYLM_KV", kvdt ? "f16" : "f32", 1);
    TlrefDec *d = calloc(1, sizeof *d);
    if (!d) return NULL;
    memset(&d->c, 0, sizeof d->c);
    d->c.V = V; d->c.D = D; d->c.L = L; d->c.H = H; d->c.KV = KV; d->c.F = F; d->c.T = T;
    d->c.n_exp = n_exp; d->c.n_mtp = n_mtp; d->c.qknorm = qknorm; d->c.topk = 1;
    d->c.rope_base = 10000.0f;
    cfg_derive(&d->c);
    d->gn = gen_new(&d->c, NULL, 0);
    if (!d->gn) { free(d); return NULL; }
    return d;
}

static void free_map(Weights *w)
{
    free(w->an1); free(w->wq); free(w->wk); free(w->wv); free(w->wo); free(w->an2); free(w->w1); free(w->w3);
    free(w->w2); free(w->wr); free(w->qn); free(w->kn); free(w->mtp);
}

/* qknorm_apply (tinylm.c:597-605) on rows x nheads heads of hd values. */
void tlref_qknorm(float *buf, const float *gain, int rows, int nheads, int hd)
{
    qknorm_apply(buf, gain, rows, nheads, hd);
}

/* The decode MoE layer l (moe_forward_q8's fp32 branch, :3433-3458) on N rows
 * of fnorm / fin with the flat parameters P (map_weights' layout). */
int tlref_dec_moe(void *h, float *P, int l, const float *fnorm, const float *fin, float *out, int N, int *assign,
                  float *gate, float *rprobs)
{
    TlrefDec *d = (TlrefDec *)h;
    if (!d || d->c.n_exp <= 0 || l < 0 || l >= d->c.L || N < 1) return -1;
    Weights w;
    map_weights(&d->c, P, &w);
    moe_forward_q8(&d->c, &w, d->gn, l, fnorm, fin, out, N, assign, gate, rprobs);
    free_map(&w);
    return 0;
}

/* MTP head k's greedy token from a final-normed row fn1 (mtp_argmax,
 * :3930-3936); its logits [V] go to logits. */
int tlref_mtp_argmax(void *h, float *P, const float *fn1, int k, float *logits)
{
    TlrefDec *d = (TlrefDec *)h;
    if (!d || k < 0 || k >= d->c.n_mtp) return -1;
    Weights w;
    map_weights(&d->c, P, &w);
    const int t = mtp_argmax(&d->c, &w, d->gn, fn1, k);
    memcpy(logits, d->gn->hlog, sizeof(float) * (size_t)d->c.V);
    free_map(&w);
    return t;
}
