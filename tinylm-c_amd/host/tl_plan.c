/* tl_plan.c -- builds the reference's GEMM call sequences as plans.
 *
 * The call order, operands and (M, K, N) arguments follow tinylm.c line by
 * line (cited per call); buffers are named after the reference's Acts fields
 * and its flat P / G parameter layout.  Memsets are kept where they set the
 * base an accumulating GEMM adds into (tinylm.c:1015, :1047, :1104, :1113,
 * :1123, :1135, :3035) and for the memset(G) that precedes backward
 * (:2628).  Memsets followed by a setting `mm` (:1059, :1084) change no
 * result and are left out; memsets that feed only non-GEMM code
 * (:1090, :1127-1129) belong to that code.
 */
#include "tl_plan.h"
#include <stdlib.h>
#include <string.h>

void tl_weight_map(int V, int D, int KD, int F, int L, int n_mtp, int layer, TlWeightMap *m)
{
    /* map_weights for a dense FFN without QK-norm (tinylm.c:361-393):
     * emb | per layer: an1 wq wk wv wo an2 w1 w3 w2 | nf | mtp[k] */
    const size_t per = (size_t)D + (size_t)D * D + 2 * (size_t)D * KD + (size_t)D * D + (size_t)D
                     + 2 * (size_t)D * F + (size_t)F * D;
    m->emb = 0;
    m->an1 = (size_t)V * D + (size_t)layer * per;
    m->wq = m->an1 + D;
    m->wk = m->wq + (size_t)D * D;
    m->wv = m->wk + (size_t)D * KD;
    m->wo = m->wv + (size_t)D * KD;
    m->an2 = m->wo + (size_t)D * D;
    m->w1 = m->an2 + D;
    m->w3 = m->w1 + (size_t)D * F;
    m->w2 = m->w3 + (size_t)D * F;
    m->nf = (size_t)V * D + (size_t)L * per;
    m->mtp0 = m->nf + D;
    m->total = m->mtp0 + (size_t)n_mtp * D * D;
}

static int add_buf(TlPlan *p, const char *name, size_t floats, int init)
{
    if (p->nbuf >= TL_MAXBUF) return -1;
    TlBuf *b = &p->buf[p->nbuf];
    memset(b, 0, sizeof *b);
    strncpy(b->name, name, TL_NAMELEN - 1);
    b->floats = floats;
    b->init = init;
    return p->nbuf++;
}

int tl_plan_find(const TlPlan *p, const char *name)
{
    for (int i = 0; i < p->nbuf; i++)
        if (!strcmp(p->buf[i].name, name)) return i;
    return -1;
}

static TlCall *push(TlPlan *p)
{
    if (p->ncall == p->cap) {
        int cap = p->cap ? 2 * p->cap : 256;
        TlCall *c = realloc(p->call, sizeof(TlCall) * (size_t)cap);
        if (!c) return NULL;
        p->call = c;
        p->cap = cap;
    }
    TlCall *c = &p->call[p->ncall++];
    memset(c, 0, sizeof *c);
    return c;
}

/* The reference runs non-GEMM code here (norms, RoPE, attention, SwiGLU,
 * softmax, residual adds): the next GEMM starts a new run. */
static void glue(TlPlan *p) { p->run++; }

static int gemm(TlPlan *p, int op, int line, const char *what,
                int out, size_t oo, int a, size_t ao, int b, size_t bo, int M, int K, int N)
{
    TlCall *c = push(p);
    if (!c) return -1;
    c->op = op; c->line = line;
    strncpy(c->what, what, TL_NAMELEN - 1);
    c->out = out; c->out_off = oo;
    c->a = a; c->a_off = ao;
    c->b = b; c->b_off = bo;
    c->M = M; c->K = K; c->N = N;
    c->run = p->run;
    return 0;
}

static int zero(TlPlan *p, int line, const char *what, int out, size_t off, size_t n)
{
    TlCall *c = push(p);
    if (!c) return -1;
    c->op = TL_ZERO; c->line = line;
    strncpy(c->what, what, TL_NAMELEN - 1);
    c->out = out; c->out_off = off; c->n = n;
    c->a = c->b = -1;
    c->run = p->run;
    return 0;
}

void tl_plan_free(TlPlan *p)
{
    free(p->call);
    memset(p, 0, sizeof *p);
}

#define CHK(x) do { if ((x) < 0) { tl_plan_free(p); return -1; } } while (0)

int tl_plan_train(TlPlan *p, int R, int D, int KD, int F, int V, int L, int n_mtp)
{
    memset(p, 0, sizeof *p);
    if (R <= 0 || D <= 0 || KD <= 0 || F <= 0 || V <= 0 || L <= 0 || n_mtp < 0) return -1;
    p->R = R; p->D = D; p->KD = KD; p->F = F; p->V = V; p->L = L; p->n_mtp = n_mtp;
    TlWeightMap m0;
    tl_weight_map(V, D, KD, F, L, n_mtp, 0, &m0);
    const size_t RD = (size_t)R * D, RK = (size_t)R * KD, RF = (size_t)R * F, RV = (size_t)R * V;
    /* parameters / gradients: the flat buffers of tinylm.c:2739-2740 */
    const int P = add_buf(p, "P", m0.total, TL_INIT_WEIGHT);
    const int G = add_buf(p, "G", m0.total, TL_INIT_ZERO);
    /* per-layer activations (Acts, tinylm.c:654-696), L slices each */
    const int a_in = add_buf(p, "a_in", (size_t)L * RD, TL_INIT_ZERO);
    const int a_norm = add_buf(p, "a_norm", (size_t)L * RD, TL_INIT_ACT);
    const int q = add_buf(p, "q", (size_t)L * RD, TL_INIT_ZERO);
    const int k = add_buf(p, "k", (size_t)L * RK, TL_INIT_ZERO);
    const int v = add_buf(p, "v", (size_t)L * RK, TL_INIT_ZERO);
    const int att_ctx = add_buf(p, "att_ctx", (size_t)L * RD, TL_INIT_ACT);
    const int f_in = add_buf(p, "f_in", (size_t)L * RD, TL_INIT_ZERO);
    const int f_norm = add_buf(p, "f_norm", (size_t)L * RD, TL_INIT_ACT);
    const int g = add_buf(p, "g", (size_t)L * RF, TL_INIT_ZERO);
    const int u = add_buf(p, "u", (size_t)L * RF, TL_INIT_ZERO);
    /* step-wide buffers */
    const int x_final = add_buf(p, "x_final", RD, TL_INIT_ZERO);
    const int fn_norm = add_buf(p, "fn_norm", RD, TL_INIT_ACT);
    const int logits = add_buf(p, "logits", RV, TL_INIT_ZERO);
    const int dlogits = add_buf(p, "dlogits", RV, TL_INIT_GRAD);
    const int dout = add_buf(p, "dout", RD, TL_INIT_GRAD);
    const int dact = add_buf(p, "dact", RF, TL_INIT_ACT);   /* forward's act (:1004) */
    const int dg = add_buf(p, "dg", RF, TL_INIT_GRAD);
    const int du = add_buf(p, "du", RF, TL_INIT_ACT);       /* backward's act (:1099) */
    const int dfnorm = add_buf(p, "dfnorm", RD, TL_INIT_ZERO);
    const int dfin = add_buf(p, "dfin", RD, TL_INIT_GRAD);
    const int datt = add_buf(p, "datt", RD, TL_INIT_ZERO);
    const int dq = add_buf(p, "dq", RD, TL_INIT_GRAD);
    const int dk = add_buf(p, "dk", RK, TL_INIT_GRAD);
    const int dv = add_buf(p, "dv", RK, TL_INIT_GRAD);
    const int dnorm = add_buf(p, "dnorm", RD, TL_INIT_ZERO);
    const int dain = add_buf(p, "dain", RD, TL_INIT_GRAD);
    const int dfn = add_buf(p, "dfn", RD, TL_INIT_ZERO);
    if (dfn < 0) { tl_plan_free(p); return -1; }

    /* ---- forward, tinylm.c:978-1016 ---- */
    for (int l = 0; l < L; l++) {
        TlWeightMap w;
        tl_weight_map(V, D, KD, F, L, n_mtp, l, &w);
        const size_t ld = (size_t)l * RD, lk = (size_t)l * RK, lf = (size_t)l * RF;
        CHK(gemm(p, TL_MM, 981, "q", q, ld, a_norm, ld, P, w.wq, R, D, D));
        CHK(gemm(p, TL_MM, 982, "k", k, lk, a_norm, ld, P, w.wk, R, D, KD));
        CHK(gemm(p, TL_MM, 983, "v", v, lk, a_norm, ld, P, w.wv, R, D, KD));
        glue(p);                                    /* RoPE, attention :984-990 */
        CHK(gemm(p, TL_MM, 993, "o", f_in, ld, att_ctx, ld, P, w.wo, R, D, D));
        glue(p);                                    /* residual, rmsnorm :994-997 */
        CHK(gemm(p, TL_MM, 1002, "w1", g, lf, f_norm, ld, P, w.w1, R, D, F));
        CHK(gemm(p, TL_MM, 1003, "w3", u, lf, f_norm, ld, P, w.w3, R, D, F));
        glue(p);                                    /* silu(g)*u :1004-1006 */
        if (l + 1 < L) CHK(gemm(p, TL_MM, 1008, "w2", a_in, ld + RD, dact, 0, P, w.w2, R, F, D));
        else           CHK(gemm(p, TL_MM, 1008, "w2", x_final, 0, dact, 0, P, w.w2, R, F, D));
        glue(p);                                    /* residual :1009-1010, next rmsnorm */
    }
    CHK(zero(p, 1015, "logits", logits, 0, RV));
    CHK(gemm(p, TL_MM_BT, 1016, "logits", logits, 0, fn_norm, 0, P, m0.emb, R, V, D));

    glue(p);                                        /* softmax + CE :1017-1028 */
    /* ---- memset(G) then backward, tinylm.c:2628, :1072-1154 ---- */
    CHK(zero(p, 2628, "G", G, 0, m0.total));
    /* softmax / cross-entropy between the head GEMM and this memset touch
     * logits, dlogits and the loss only: the clear may run with the head */
    p->call[p->ncall - 1].hoist = 1;
    glue(p);                                        /* dlogits :1076-1082 */
    CHK(gemm(p, TL_MM, 1085, "dfn", dfn, 0, dlogits, 0, P, m0.emb, R, V, D));
    CHK(gemm(p, TL_MM_ATB, 1086, "dEmb", G, m0.emb, dlogits, 0, fn_norm, 0, R, V, D));
    /* MTP heads (mtp_grad, :1036-1069): t1=datt hk=dnorm dhk=dq dt1=dain
     * lg=logits dl=dlogits fn=fn_norm */
    for (int kk = 0; kk < n_mtp; kk++) {
        const size_t wk = m0.mtp0 + (size_t)kk * D * D;
        CHK(gemm(p, TL_MM, 1044, "mtp.t1", datt, 0, fn_norm, 0, P, wk, R, D, D));
        glue(p);                                    /* hk = fn + silu(t1) :1045-1046 */
        CHK(zero(p, 1047, "mtp.lg", logits, 0, RV));
        CHK(gemm(p, TL_MM_BT, 1048, "mtp.lg", logits, 0, dnorm, 0, P, m0.emb, R, V, D));
        glue(p);                                    /* softmax -> dl :1049-1057 */
        CHK(gemm(p, TL_MM_ATB, 1058, "mtp.dEmb", G, m0.emb, dlogits, 0, dnorm, 0, R, V, D));
        CHK(gemm(p, TL_MM, 1060, "mtp.dhk", dq, 0, dlogits, 0, P, m0.emb, R, V, D));
        glue(p);                                    /* dfn += dhk, dt1 :1061-1065 */
        CHK(gemm(p, TL_MM_ATB, 1066, "mtp.dWk", G, wk, fn_norm, 0, dain, 0, R, D, D));
        CHK(gemm(p, TL_MM_BT, 1067, "mtp.dfn", dfn, 0, dain, 0, P, wk, R, D, D));
    }
    for (int l = L - 1; l >= 0; l--) {
        TlWeightMap w;
        tl_weight_map(V, D, KD, F, L, n_mtp, l, &w);
        const size_t ld = (size_t)l * RD;
        glue(p);                                    /* rmsnorm_bwd / silu recompute :1091-1102 */
        CHK(gemm(p, TL_MM_ATB, 1103, "dW2", G, w.w2, du, 0, dout, 0, R, F, D));
        CHK(zero(p, 1104, "dact", dact, 0, RF));
        CHK(gemm(p, TL_MM_BT, 1105, "dact", dact, 0, dout, 0, P, w.w2, R, F, D));
        glue(p);                                    /* SwiGLU backward :1106-1112 */
        CHK(zero(p, 1113, "dfnorm", dfnorm, 0, RD));
        CHK(gemm(p, TL_MM_BT, 1114, "dfnorm.w1", dfnorm, 0, dg, 0, P, w.w1, R, D, F));
        CHK(gemm(p, TL_MM_BT, 1115, "dfnorm.w3", dfnorm, 0, du, 0, P, w.w3, R, D, F));
        CHK(gemm(p, TL_MM_ATB, 1116, "dW1", G, w.w1, f_norm, ld, dg, 0, R, D, F));
        CHK(gemm(p, TL_MM_ATB, 1117, "dW3", G, w.w3, f_norm, ld, du, 0, R, D, F));
        glue(p);                                    /* rmsnorm_bwd :1119-1121 */
        CHK(zero(p, 1123, "datt", datt, 0, RD));
        CHK(gemm(p, TL_MM_BT, 1124, "datt", datt, 0, dfin, 0, P, w.wo, R, D, D));
        CHK(gemm(p, TL_MM_ATB, 1125, "dWo", G, w.wo, att_ctx, ld, dfin, 0, R, D, D));
        glue(p);                                    /* attention + RoPE backward :1127-1133 */
        CHK(zero(p, 1135, "dnorm", dnorm, 0, RD));
        CHK(gemm(p, TL_MM_BT, 1136, "dnorm.q", dnorm, 0, dq, 0, P, w.wq, R, D, D));
        CHK(gemm(p, TL_MM_BT, 1137, "dnorm.k", dnorm, 0, dk, 0, P, w.wk, R, D, KD));
        CHK(gemm(p, TL_MM_BT, 1138, "dnorm.v", dnorm, 0, dv, 0, P, w.wv, R, D, KD));
        CHK(gemm(p, TL_MM_ATB, 1139, "dWq", G, w.wq, a_norm, ld, dq, 0, R, D, D));
        CHK(gemm(p, TL_MM_ATB, 1140, "dWk", G, w.wk, a_norm, ld, dk, 0, R, D, KD));
        CHK(gemm(p, TL_MM_ATB, 1141, "dWv", G, w.wv, a_norm, ld, dv, 0, R, D, KD));
    }
    return 0;
}

/* A decode projection mm(M, K, N) into `out` (set): as the reference calls it
 * (W [K][N]), or on the decode layout (W^T [N][K] at the same offset) as the
 * memset + mm_bt form with labels (M, N, K). */
static int dproj(TlPlan *p, int packed, int line, const char *what, int out, int in, int P, size_t wo, int M, int K,
                 int N)
{
    if (!packed) return gemm(p, TL_MM, line, what, out, 0, in, 0, P, wo, M, K, N);
    if (zero(p, line, what, out, 0, (size_t)M * N)) return -1;
    return gemm(p, TL_MM_BT, line, what, out, 0, in, 0, P, wo, M, N, K);
}

static int plan_decode(TlPlan *p, int M, int D, int KD, int F, int V, int L, int packed)
{
    memset(p, 0, sizeof *p);
    if (M <= 0 || D <= 0 || KD <= 0 || F <= 0 || V <= 0 || L <= 0) return -1;
    p->R = M; p->D = D; p->KD = KD; p->F = F; p->V = V; p->L = L;
    TlWeightMap m0;
    tl_weight_map(V, D, KD, F, L, 0, 0, &m0);
    /* Gen buffers (tinylm.c:3276-3289) */
    const int P = add_buf(p, "P", m0.total, TL_INIT_WEIGHT);
    const int xn = add_buf(p, "xn", (size_t)M * D, TL_INIT_ACT);
    const int q = add_buf(p, "q", (size_t)M * D, TL_INIT_ZERO);
    const int k = add_buf(p, "k", (size_t)M * KD, TL_INIT_ZERO);
    const int v = add_buf(p, "v", (size_t)M * KD, TL_INIT_ZERO);
    const int ctx = add_buf(p, "ctx", (size_t)M * D, TL_INIT_ACT);
    const int tmp = add_buf(p, "tmp", (size_t)M * D, TL_INIT_ZERO);
    const int g = add_buf(p, "g", (size_t)M * F, TL_INIT_ZERO);
    const int u = add_buf(p, "u", (size_t)M * F, TL_INIT_ACT);
    const int fn = add_buf(p, "fn", (size_t)M * D, TL_INIT_ACT);
    const int logits = add_buf(p, "logits", (size_t)M * V, TL_INIT_ZERO);
    if (logits < 0) { tl_plan_free(p); return -1; }
    for (int l = 0; l < L; l++) {
        TlWeightMap w;
        tl_weight_map(V, D, KD, F, L, 0, l, &w);
        CHK(dproj(p, packed, 3748, "q", q, xn, P, w.wq, M, D, D));
        CHK(dproj(p, packed, 3749, "k", k, xn, P, w.wk, M, D, KD));
        CHK(dproj(p, packed, 3750, "v", v, xn, P, w.wv, M, D, KD));
        glue(p);                                    /* RoPE, KV store, attention :3756-3810 */
        CHK(dproj(p, packed, 3812, "o", tmp, ctx, P, w.wo, M, D, D));
        glue(p);                                    /* residual, rmsnorm :3813-3815 */
        CHK(dproj(p, packed, 3821, "w1", g, xn, P, w.w1, M, D, F));
        CHK(dproj(p, packed, 3822, "w3", u, xn, P, w.w3, M, D, F));
        glue(p);                                    /* silu(g)*u :3823 */
        CHK(dproj(p, packed, 3824, "w2", tmp, u, P, w.w2, M, F, D));
        glue(p);                                    /* residual, next rmsnorm :3825 */
    }
    CHK(zero(p, 3035, "logits", logits, 0, (size_t)M * V));
    CHK(gemm(p, TL_MM_BT, 3035, "head", logits, 0, fn, 0, P, m0.emb, M, V, D));
    return 0;
}

int tl_plan_decode(TlPlan *p, int M, int D, int KD, int F, int V, int L)
{
    return plan_decode(p, M, D, KD, F, V, L, 0);
}

int tl_plan_decode_packed(TlPlan *p, int M, int D, int KD, int F, int V, int L)
{
    return plan_decode(p, M, D, KD, F, V, L, 1);
}

double tl_call_flops(const TlCall *c)
{
    if (c->op == TL_ZERO) return 0.0;
    return 2.0 * (double)c->M * (double)c->K * (double)c->N;
}

double tl_call_bytes(const TlCall *c)
{
    const double M = c->M, K = c->K, N = c->N;
    switch (c->op) {
    case TL_MM:     return 4.0 * (M * K + K * N + M * N);
    case TL_MM_BT:  return 4.0 * (M * N + K * N + 2.0 * M * K);
    case TL_MM_ATB: return 4.0 * (M * K + M * N + 2.0 * K * N);
    default:        return 4.0 * (double)c->n;
    }
}
