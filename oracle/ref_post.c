
/* ref_post.c -- appended after the reference line ranges (oracle/Makefile).
 * TEST INFRASTRUCTURE ONLY: exports the reference's own static kernels under
 * tlref_* names so tests/golden/make_golden.py can record their outputs. */
void tlref_mm(float *Y, const float *X, const float *W, int M, int K, int N)
{ mm(Y, X, W, M, K, N); }
void tlref_mm_bt(float *dX, const float *dY, const float *W, int M, int K, int N)
{ mm_bt(dX, dY, W, M, K, N); }
void tlref_mm_atb(float *dW, const float *X, const float *dY, int M, int K, int N)
{ mm_atb(dW, X, dY, M, K, N); }
void tlref_seed(uint64_t s) { g_rng = s; }
float tlref_normal(void) { return rnd_normal(); }
void tlref_threads(int nt) { if (nt > 0) omp_set_num_threads(nt); }

/* One MoE layer with E routed experts and K=1 routing, through the reference's
 * own moe_forward / moe_backward (Weights arrays of length 1 = layer 0). */
static void tlref_moe_setup(Cfg *c, Weights *w, int D, int F, int E,
                            float *wr, float *w1, float *w3, float *w2,
                            float **p_wr, float **p_w1, float **p_w3, float **p_w2)
{
    memset(c, 0, sizeof(*c));
    c->D = D; c->F = F; c->n_exp = E; c->L = 1;
    memset(w, 0, sizeof(*w));
    p_wr[0] = wr; p_w1[0] = w1; p_w3[0] = w3; p_w2[0] = w2;
    w->wr = p_wr; w->w1 = p_w1; w->w3 = p_w3; w->w2 = p_w2;
}
void tlref_moe_forward(int N, int D, int F, int E, const float *fnorm, const float *fin,
                       float *out, float *wr, float *w1, float *w3, float *w2,
                       int *assign, float *gate, float *rprobs)
{
    Cfg c; Weights w; float *a[1], *b[1], *cc[1], *d[1];
    tlref_moe_setup(&c, &w, D, F, E, wr, w1, w3, w2, a, b, cc, d);
    moe_forward(&c, &w, 0, fnorm, fin, out, N, assign, gate, rprobs);
}
void tlref_moe_backward(int N, int D, int F, int E, const float *fnorm, const float *dout,
                        float *d_fnorm, float *wr, float *w1, float *w3, float *w2,
                        float *gwr, float *gw1, float *gw3, float *gw2,
                        const int *assign, const float *gate, const float *rprobs)
{
    Cfg c; Weights w, g; float *a[1], *b[1], *cc[1], *d[1], *ga[1], *gb[1], *gc[1], *gd[1];
    tlref_moe_setup(&c, &w, D, F, E, wr, w1, w3, w2, a, b, cc, d);
    tlref_moe_setup(&c, &g, D, F, E, gwr, gw1, gw3, gw2, ga, gb, gc, gd);
    moe_backward(&c, &w, &g, 0, fnorm, dout, d_fnorm, assign, gate, rprobs, N);
}

/* A plan's call list run in C (no interpreter between the calls), for the
 * CPU baseline of short calls such as the decode GEMVs: op 0 mm, 1 mm_bt,
 * 2 mm_atb, 3 memset of n floats; `reps` passes over the list. */
typedef struct { int op; float *out; const float *a, *b; int M, K, N; size_t n; } TlrefCall;
void tlref_run_calls(const TlrefCall *c, int n, int reps)
{
    for (int r = 0; r < reps; r++)
        for (int i = 0; i < n; i++) {
            switch (c[i].op) {
            case 0: mm(c[i].out, c[i].a, c[i].b, c[i].M, c[i].K, c[i].N); break;
            case 1: mm_bt(c[i].out, c[i].a, c[i].b, c[i].M, c[i].K, c[i].N); break;
            case 2: mm_atb(c[i].out, c[i].a, c[i].b, c[i].M, c[i].K, c[i].N); break;
            default: memset(c[i].out, 0, c[i].n * sizeof(float)); break;
            }
        }
}
