/* tl_oracle_step.c -- CPU oracle for the non-GEMM work of tinylm.c's
 * training step and a whole forward + backward step built on it.
 *
 * TEST INFRASTRUCTURE ONLY (see tl_oracle.h): restated from scratch from
 * the reference's arithmetic so that the device step (tltrain.h, tl_train.c)
 * can be compared with what tinylm.c computes on identical inputs.  Pinned
 * by tests/test_oracle.py against fixtures the reference's own compiled
 * functions wrote (tests/golden/step_*.npz), against fp64 / closed forms, and
 * against the reference itself when oracle/_ref is built.
 */
#include "tl_oracle.h"
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* ---- embedding, tinylm.c:972-976 / :1149-1153 ---------------------------- */
void orc_embed_fwd(float *out, const float *emb, const int *tok, int N, int D)
{
    for (int n = 0; n < N; n++) memcpy(out + (size_t)n * D, emb + (size_t)tok[n] * D, sizeof(float) * D);
}

void orc_embed_bwd(float *demb, const float *dout, const int *tok, int N, int D)
{
    for (int n = 0; n < N; n++) {                      /* in token order */
        float *row = demb + (size_t)tok[n] * D;
        const float *d = dout + (size_t)n * D;
        for (int i = 0; i < D; i++) row[i] += d[i];
    }
}

/* ---- rmsnorm, tinylm.c:540-588 ------------------------------------------- */
void orc_rmsnorm_fwd(const float *x, const float *g, float *out, float *rinv, int rows, int D)
{
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * D;
        float *o = out + (size_t)r * D;
        float ss = 0.0f;
        for (int i = 0; i < D; i++) ss += xr[i] * xr[i];
        const float s = 1.0f / sqrtf(ss / D + 1e-5f);
        rinv[r] = s;
        for (int i = 0; i < D; i++) o[i] = xr[i] * s * g[i];
    }
}

void orc_rmsnorm_bwd(const float *x, const float *g, const float *rinv, const float *dy, float *dx, float *dg,
                     int rows, int D)
{
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * D, *d = dy + (size_t)r * D;
        float *o = dx + (size_t)r * D;
        const float s = rinv[r];
        float c = 0.0f;
        for (int i = 0; i < D; i++) c += xr[i] * g[i] * d[i];
        const float coef = s * s * s / D * c;
        for (int i = 0; i < D; i++) o[i] += s * g[i] * d[i] - coef * xr[i];
    }
    /* dg: column sums over rows (the reference adds per-thread partials) */
#pragma omp parallel for schedule(static)
    for (int i = 0; i < D; i++) {
        float acc = 0.0f;
        for (int r = 0; r < rows; r++) acc += (x[(size_t)r * D + i] * rinv[r]) * dy[(size_t)r * D + i];
        dg[i] += acc;
    }
}

/* ---- RoPE, tinylm.c:605-651 ---------------------------------------------- */
void orc_rope_table(float *cs, float *sn, int maxpos, int hd, float base)
{
    const int half = hd / 2;
    for (int t = 0; t < maxpos; t++)
        for (int i = 0; i < half; i++) {
            const float inv = powf(base, -(2.0f * i) / hd);
            const float a = t * inv;
            cs[(size_t)t * half + i] = cosf(a);
            sn[(size_t)t * half + i] = sinf(a);
        }
}

void orc_rope(float *buf, const int *pos, int T, int rows, int nh, int hd, const float *cs, const float *sn,
              int back)
{
    const int half = hd / 2;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const int t = pos ? pos[r] : r % T;
        for (int h = 0; h < nh; h++) {
            float *v = buf + (size_t)r * nh * hd + (size_t)h * hd;
            for (int i = 0; i < half; i++) {
                const float c = cs[(size_t)t * half + i], s = sn[(size_t)t * half + i];
                const float a = v[i], b = v[i + half];
                if (back) { v[i] = a * c + b * s; v[i + half] = -a * s + b * c; }
                else      { v[i] = a * c - b * s; v[i + half] = b * c + a * s; }
            }
        }
    }
}

/* ---- attention, tinylm.c:699-783 (sliding window per cfg_lwin :64-68) ---- */
static int first_key(int t, int win) { return (win > 0 && t >= win) ? t - win + 1 : 0; }

void orc_attn_fwd(const float *q, const float *k, const float *v, float *out, int B, int T, int H, int KV, int hd,
                  int win)
{
    const int D = H * hd, KD = KV * hd, grp = H / KV;
    const float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel
    {
        float *w = malloc(sizeof(float) * (T > 0 ? T : 1));
#pragma omp for schedule(static)
        for (int bh = 0; bh < B * H; bh++) {
            const int b = bh / H, h = bh % H, kh = h / grp;
            for (int t = 0; t < T; t++) {
                const float *qr = q + (size_t)(b * T + t) * D + (size_t)h * hd;
                const int lo = first_key(t, win);
                float mx = -1e30f;
                for (int s = lo; s <= t; s++) {
                    const float *kr = k + (size_t)(b * T + s) * KD + (size_t)kh * hd;
                    float dot = 0.0f;
                    for (int d = 0; d < hd; d++) dot += qr[d] * kr[d];
                    w[s] = dot * scale;
                    if (w[s] > mx) mx = w[s];
                }
                float sum = 0.0f;
                for (int s = lo; s <= t; s++) { w[s] = expf(w[s] - mx); sum += w[s]; }
                const float inv = 1.0f / sum;
                float *o = out + (size_t)(b * T + t) * D + (size_t)h * hd;
                for (int d = 0; d < hd; d++) o[d] = 0.0f;
                for (int s = lo; s <= t; s++) {
                    const float p = w[s] * inv;
                    const float *vr = v + (size_t)(b * T + s) * KD + (size_t)kh * hd;
                    for (int d = 0; d < hd; d++) o[d] += p * vr[d];
                }
            }
        }
        free(w);
    }
}

void orc_attn_bwd(const float *q, const float *k, const float *v, const float *datt, float *dq, float *dk,
                  float *dv, int B, int T, int H, int KV, int hd, int win)
{
    const int D = H * hd, KD = KV * hd, grp = H / KV;
    const float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel
    {
        float *p = malloc(sizeof(float) * (T > 0 ? T : 1)), *dp = malloc(sizeof(float) * (T > 0 ? T : 1));
#pragma omp for schedule(static)
        for (int b = 0; b < B; b++)          /* per sequence: KV heads are shared across h */
            for (int h = 0; h < H; h++) {
                const int kh = h / grp;
                for (int t = 0; t < T; t++) {
                    const float *qr = q + (size_t)(b * T + t) * D + (size_t)h * hd;
                    const int lo = first_key(t, win);
                    float mx = -1e30f;
                    for (int s = lo; s <= t; s++) {
                        const float *kr = k + (size_t)(b * T + s) * KD + (size_t)kh * hd;
                        float dot = 0.0f;
                        for (int d = 0; d < hd; d++) dot += qr[d] * kr[d];
                        p[s] = dot * scale;
                        if (p[s] > mx) mx = p[s];
                    }
                    float sum = 0.0f;
                    for (int s = lo; s <= t; s++) { p[s] = expf(p[s] - mx); sum += p[s]; }
                    const float inv = 1.0f / sum;
                    for (int s = lo; s <= t; s++) p[s] *= inv;
                    const float *da = datt + (size_t)(b * T + t) * D + (size_t)h * hd;
                    for (int s = lo; s <= t; s++) {
                        const float *vr = v + (size_t)(b * T + s) * KD + (size_t)kh * hd;
                        float acc = 0.0f;
                        for (int d = 0; d < hd; d++) acc += da[d] * vr[d];
                        dp[s] = acc;
                        float *dvr = dv + (size_t)(b * T + s) * KD + (size_t)kh * hd;
                        for (int d = 0; d < hd; d++) dvr[d] += p[s] * da[d];
                    }
                    float pd = 0.0f;
                    for (int s = lo; s <= t; s++) pd += p[s] * dp[s];
                    float *dqr = dq + (size_t)(b * T + t) * D + (size_t)h * hd;
                    for (int s = lo; s <= t; s++) {
                        const float ds = p[s] * (dp[s] - pd) * scale;
                        const float *kr = k + (size_t)(b * T + s) * KD + (size_t)kh * hd;
                        float *dkr = dk + (size_t)(b * T + s) * KD + (size_t)kh * hd;
                        for (int d = 0; d < hd; d++) { dqr[d] += ds * kr[d]; dkr[d] += ds * qr[d]; }
                    }
                }
            }
        free(p);
        free(dp);
    }
}

/* ---- softmax + CE and its gradient, tinylm.c:1019-1028, :1076-1082,
 * :1051-1055: dl = softmax * scale, minus scale at the target; returns the
 * mean of -log(p[target] + 1e-12) (double sum, :1026). -------------------- */
double orc_xent(const float *logits, const int *tgt, float *dl, float scale, int N, int V)
{
    double loss = 0.0;
#pragma omp parallel for reduction(+ : loss) schedule(static)
    for (int n = 0; n < N; n++) {
        const float *lg = logits + (size_t)n * V;
        float *d = dl + (size_t)n * V;
        float mx = -1e30f;
        for (int i = 0; i < V; i++) if (lg[i] > mx) mx = lg[i];
        float sum = 0.0f;
        for (int i = 0; i < V; i++) { d[i] = expf(lg[i] - mx); sum += d[i]; }
        const float inv = 1.0f / sum;
        for (int i = 0; i < V; i++) d[i] = d[i] * inv;      /* probabilities */
        loss += -log((double)d[tgt[n]] + 1e-12);
        for (int i = 0; i < V; i++) d[i] = d[i] * scale;
        d[tgt[n]] -= scale;
    }
    return loss / N;
}

/* ---- gradient norm and AdamW, tinylm.c:1159-1176 ------------------------- */
float orc_gradnorm(const float *G, size_t n)
{
    double s = 0.0;
#pragma omp parallel for reduction(+ : s) schedule(static)
    for (long long i = 0; i < (long long)n; i++) s += (double)G[i] * G[i];
    return (float)sqrt(s);
}

void orc_adamw(float *P, const float *G, float *M, float *V, size_t n, float lr, float b1, float b2, float wd,
               int t, float gscale)
{
    const float bc1 = 1.0f - powf(b1, t), bc2 = 1.0f - powf(b2, t);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; i++) {
        const float g = G[i] * gscale;
        M[i] = b1 * M[i] + (1 - b1) * g;
        V[i] = b2 * V[i] + (1 - b2) * g * g;
        const float mh = M[i] / bc1, vh = V[i] / bc2;
        P[i] -= lr * (mh / (sqrtf(vh) + 1e-8f) + wd * P[i]);
    }
}

/* ---- a whole step ---------------------------------------------------------- */
static float silu(float z) { return z / (1.0f + expf(-z)); }
static float dsilu(float z)
{
    const float sg = 1.0f / (1.0f + expf(-z));
    return sg + z * sg * (1.0f - sg);
}
static float *zalloc(size_t n) { return calloc(n ? n : 1, sizeof(float)); }
static int layer_win(const OrcModel *m, int l)
{
    if (m->win <= 0) return 0;
    if (m->full_every > 0 && ((l + 1) % m->full_every) == 0) return 0;
    return m->win;
}

/* map_weights (tinylm.c:361-393) without QK-norm */
void orc_param_map(const OrcModel *m, int l, OrcLayerMap *o)
{
    const size_t D = m->D, hd = (size_t)(m->D / m->H), KD = (size_t)m->KV * hd, F = m->F,
                 E = m->n_exp > 0 ? m->n_exp : 1, QK = m->qknorm ? 2 * hd : 0;
    const size_t per = D + D * D + 2 * D * KD + D * D + QK + D + (m->n_exp > 0 ? D * m->n_exp : 0) + E * 3 * D * F;
    o->emb = 0;
    o->an1 = (size_t)m->V * D + (size_t)l * per;
    o->wq = o->an1 + D;
    o->wk = o->wq + D * D;
    o->wv = o->wk + D * KD;
    o->wo = o->wv + D * KD;
    o->qn = o->wo + D * D;                       /* QK-norm gains (hd each), when qknorm */
    o->kn = o->qn + (m->qknorm ? hd : 0);
    o->an2 = o->wo + D * D + QK;
    o->wr = o->an2 + D;
    o->w1 = o->wr + (m->n_exp > 0 ? D * m->n_exp : 0);
    o->w3 = o->w1 + E * D * F;
    o->w2 = o->w3 + E * D * F;
    o->nf = (size_t)m->V * D + (size_t)m->L * per;
    o->mtp0 = o->nf + D;
    o->total = o->mtp0 + (size_t)m->n_mtp * D * D;
}

/* forward (tinylm.c:968-1029), memset(G), backward (:1072-1154) with
 * mtp_grad (:1036-1069); returns the forward's loss. */
float orc_train_step(const OrcModel *m, int B, const float *P, float *G, const int *tok, const int *tgt,
                     const int *tgt_mtp)
{
    if (m->qknorm) return NAN;                   /* the reference refuses to train these (:2707-2713) */
    const int T = m->T, N = B * T, D = m->D, H = m->H, KV = m->KV, hd = D / H, KD = KV * hd, F = m->F,
              V = m->V, L = m->L, E = m->n_exp;
    const size_t ND = (size_t)N * D, NK = (size_t)N * KD, NF = (size_t)N * F, NV = (size_t)N * V;
    OrcLayerMap mp;
    orc_param_map(m, 0, &mp);
    const size_t np = mp.total;
    float *cs = zalloc((size_t)T * (hd / 2)), *sn = zalloc((size_t)T * (hd / 2));
    orc_rope_table(cs, sn, T, hd, m->rope_base);
    /* activations kept for the backward pass, per layer */
    float *a_in = zalloc(L * ND), *a_norm = zalloc(L * ND), *q = zalloc(L * ND), *k = zalloc(L * NK),
          *v = zalloc(L * NK), *ctx = zalloc(L * ND), *f_in = zalloc(L * ND), *f_norm = zalloc(L * ND),
          *g = zalloc(L * NF), *u = zalloc(L * NF), *a_rinv = zalloc((size_t)L * N), *f_rinv = zalloc((size_t)L * N);
    int *assign = E > 0 ? calloc((size_t)L * N, sizeof(int)) : NULL;
    float *gate = E > 0 ? zalloc((size_t)L * N) : NULL, *rprobs = E > 0 ? zalloc((size_t)L * N * E) : NULL;
    float *x_final = zalloc(ND), *fn = zalloc(ND), *fn_rinv = zalloc(N), *logits = zalloc(NV), *dl = zalloc(NV);
    float *dout = zalloc(ND), *act = zalloc(NF), *dg = zalloc(NF), *du = zalloc(NF), *dfnorm = zalloc(ND),
          *dfin = zalloc(ND), *datt = zalloc(ND), *dq = zalloc(ND), *dk = zalloc(NK), *dv = zalloc(NK),
          *dnorm = zalloc(ND), *dain = zalloc(ND), *dfn = zalloc(ND);

    /* forward */
    orc_embed_fwd(a_in, P + mp.emb, tok, N, D);
    for (int l = 0; l < L; l++) {
        OrcLayerMap w;
        orc_param_map(m, l, &w);
        float *xin = a_in + l * ND, *an = a_norm + l * ND, *ql = q + l * ND, *kl = k + l * NK, *vl = v + l * NK;
        float *cl = ctx + l * ND, *fi = f_in + l * ND, *fnl = f_norm + l * ND;
        orc_rmsnorm_fwd(xin, P + w.an1, an, a_rinv + (size_t)l * N, N, D);
        orc_mm(ql, an, P + w.wq, N, D, D);
        orc_mm(kl, an, P + w.wk, N, D, KD);
        orc_mm(vl, an, P + w.wv, N, D, KD);
        orc_rope(ql, NULL, T, N, H, hd, cs, sn, 0);
        orc_rope(kl, NULL, T, N, KV, hd, cs, sn, 0);
        orc_attn_fwd(ql, kl, vl, cl, B, T, H, KV, hd, layer_win(m, l));
        orc_mm(fi, cl, P + w.wo, N, D, D);
        for (size_t i = 0; i < ND; i++) fi[i] += xin[i];
        orc_rmsnorm_fwd(fi, P + w.an2, fnl, f_rinv + (size_t)l * N, N, D);
        float *out = l + 1 < L ? a_in + (l + 1) * ND : x_final;
        if (E > 0) {
            orc_moe_forward(N, D, F, E, fnl, fi, out, P + w.wr, P + w.w1, P + w.w3, P + w.w2,
                            assign + (size_t)l * N, gate + (size_t)l * N, rprobs + (size_t)l * N * E);
        } else {
            float *gl = g + l * NF, *ul = u + l * NF;
            orc_mm(gl, fnl, P + w.w1, N, D, F);
            orc_mm(ul, fnl, P + w.w3, N, D, F);
            for (size_t i = 0; i < NF; i++) act[i] = silu(gl[i]) * ul[i];
            orc_mm(out, act, P + w.w2, N, F, D);
            for (size_t i = 0; i < ND; i++) out[i] += fi[i];
        }
    }
    orc_rmsnorm_fwd(x_final, P + mp.nf, fn, fn_rinv, N, D);
    memset(logits, 0, NV * sizeof(float));
    orc_mm_bt(logits, fn, P + mp.emb, N, V, D);
    const float loss = (float)orc_xent(logits, tgt, dl, 1.0f / N, N, V);

    /* backward */
    memset(G, 0, np * sizeof(float));
    orc_mm(dfn, dl, P + mp.emb, N, V, D);
    orc_mm_atb(G + mp.emb, dl, fn, N, V, D);
    for (int h = 0; h < m->n_mtp; h++) {
        const float wk = 0.2f * powf(0.8f, (float)h);
        float *t1 = datt, *hk = dnorm, *dhk = dq, *dt1 = dain;
        const float *Wk = P + mp.mtp0 + (size_t)h * D * D;
        orc_mm(t1, fn, Wk, N, D, D);
        for (size_t i = 0; i < ND; i++) hk[i] = fn[i] + silu(t1[i]);
        memset(logits, 0, NV * sizeof(float));
        orc_mm_bt(logits, hk, P + mp.emb, N, V, D);
        (void)orc_xent(logits, tgt_mtp + (size_t)h * N, dl, wk / N, N, V);
        orc_mm_atb(G + mp.emb, dl, hk, N, V, D);
        memset(dhk, 0, ND * sizeof(float));
        orc_mm(dhk, dl, P + mp.emb, N, V, D);
        for (size_t i = 0; i < ND; i++) dfn[i] += dhk[i];
        for (size_t i = 0; i < ND; i++) dt1[i] = dhk[i] * dsilu(t1[i]);
        orc_mm_atb(G + mp.mtp0 + (size_t)h * D * D, fn, dt1, N, D, D);
        orc_mm_bt(dfn, dt1, Wk, N, D, D);
    }
    memset(dout, 0, ND * sizeof(float));
    orc_rmsnorm_bwd(x_final, P + mp.nf, fn_rinv, dfn, dout, G + mp.nf, N, D);
    for (int l = L - 1; l >= 0; l--) {
        OrcLayerMap w;
        orc_param_map(m, l, &w);
        float *xin = a_in + l * ND, *an = a_norm + l * ND, *ql = q + l * ND, *kl = k + l * NK, *vl = v + l * NK;
        float *cl = ctx + l * ND, *fi = f_in + l * ND, *fnl = f_norm + l * ND;
        if (E > 0) {
            orc_moe_backward(N, D, F, E, fnl, dout, dfnorm, P + w.wr, P + w.w1, P + w.w3, P + w.w2, G + w.wr,
                             G + w.w1, G + w.w3, G + w.w2, assign + (size_t)l * N, gate + (size_t)l * N,
                             rprobs + (size_t)l * N * E);
        } else {
            float *gl = g + l * NF, *ul = u + l * NF;
            for (size_t i = 0; i < NF; i++) du[i] = silu(gl[i]) * ul[i];
            orc_mm_atb(G + w.w2, du, dout, N, F, D);
            memset(act, 0, NF * sizeof(float));                /* d_act */
            orc_mm_bt(act, dout, P + w.w2, N, F, D);
            for (size_t i = 0; i < NF; i++) {
                const float z = gl[i], sg = 1.0f / (1.0f + expf(-z));
                dg[i] = act[i] * ul[i] * (sg + z * sg * (1.0f - sg));
                du[i] = act[i] * (z * sg);
            }
            memset(dfnorm, 0, ND * sizeof(float));
            orc_mm_bt(dfnorm, dg, P + w.w1, N, D, F);
            orc_mm_bt(dfnorm, du, P + w.w3, N, D, F);
            orc_mm_atb(G + w.w1, fnl, dg, N, D, F);
            orc_mm_atb(G + w.w3, fnl, du, N, D, F);
        }
        memcpy(dfin, dout, ND * sizeof(float));
        orc_rmsnorm_bwd(fi, P + w.an2, f_rinv + (size_t)l * N, dfnorm, dfin, G + w.an2, N, D);
        memset(datt, 0, ND * sizeof(float));
        orc_mm_bt(datt, dfin, P + w.wo, N, D, D);
        orc_mm_atb(G + w.wo, cl, dfin, N, D, D);
        memset(dq, 0, ND * sizeof(float));
        memset(dk, 0, NK * sizeof(float));
        memset(dv, 0, NK * sizeof(float));
        orc_attn_bwd(ql, kl, vl, datt, dq, dk, dv, B, T, H, KV, hd, layer_win(m, l));
        orc_rope(dq, NULL, T, N, H, hd, cs, sn, 1);
        orc_rope(dk, NULL, T, N, KV, hd, cs, sn, 1);
        memset(dnorm, 0, ND * sizeof(float));
        orc_mm_bt(dnorm, dq, P + w.wq, N, D, D);
        orc_mm_bt(dnorm, dk, P + w.wk, N, D, KD);
        orc_mm_bt(dnorm, dv, P + w.wv, N, D, KD);
        orc_mm_atb(G + w.wq, an, dq, N, D, D);
        orc_mm_atb(G + w.wk, an, dk, N, D, KD);
        orc_mm_atb(G + w.wv, an, dv, N, D, KD);
        memcpy(dain, dfin, ND * sizeof(float));
        orc_rmsnorm_bwd(xin, P + w.an1, a_rinv + (size_t)l * N, dnorm, dain, G + w.an1, N, D);
        memcpy(dout, dain, ND * sizeof(float));
    }
    orc_embed_bwd(G + mp.emb, dout, tok, N, D);

    float *all[] = {cs, sn, a_in, a_norm, q, k, v, ctx, f_in, f_norm, g, u, a_rinv, f_rinv, gate, rprobs,
                    x_final, fn, fn_rinv, logits, dl, dout, act, dg, du, dfnorm, dfin, datt, dq, dk, dv, dnorm,
                    dain, dfn};
    for (size_t i = 0; i < sizeof all / sizeof all[0]; i++) free(all[i]);
    free(assign);
    return loss;
}

/* init_params (tinylm.c:395-419): N(0, 0.02^2) draws in the reference's
 * order, residual projections (wo, w2) scaled by 1/sqrt(2L), gains 1, MTP
 * heads zero. */
void orc_init_params(const OrcModel *m, float *P, uint64_t seed)
{
    const size_t D = m->D, KD = (size_t)m->KV * (m->D / m->H), F = m->F, E = m->n_exp > 0 ? m->n_exp : 1;
    const float scaled = 0.02f / sqrtf(2.0f * m->L);
    OrcLayerMap w;
    orc_param_map(m, 0, &w);
    memset(P, 0, w.total * sizeof(float));
    orc_rng_seed(seed);
    orc_fill_normal(P + w.emb, (size_t)m->V * D, 0.02f);
    for (int l = 0; l < m->L; l++) {
        orc_param_map(m, l, &w);
        for (size_t i = 0; i < D; i++) { P[w.an1 + i] = 1.0f; P[w.an2 + i] = 1.0f; }
        orc_fill_normal(P + w.wq, D * D, 0.02f);
        orc_fill_normal(P + w.wk, D * KD, 0.02f);
        orc_fill_normal(P + w.wv, D * KD, 0.02f);
        orc_fill_normal(P + w.wo, D * D, scaled);
        if (m->qknorm)
            for (int i = 0; i < m->D / m->H; i++) { P[w.qn + i] = 1.0f; P[w.kn + i] = 1.0f; }
        orc_fill_normal(P + w.w1, E * D * F, 0.02f);
        orc_fill_normal(P + w.w3, E * D * F, 0.02f);
        orc_fill_normal(P + w.w2, E * F * D, scaled);
        if (m->n_exp > 0) orc_fill_normal(P + w.wr, D * m->n_exp, 0.02f);
    }
    for (size_t i = 0; i < D; i++) P[w.nf + i] = 1.0f;
}

/* ---- decode: forward_chunk (tinylm.c:3721-3830) with fp32 weights --------
 * KV ring cache of W positions per layer, stored as f32 or f16 (kv_store
 * :3236-3250, the f16 default of kv_dtype_env :3138-3146), attention over the
 * ring window with the unsplit attn_body path (:3639-3715: scores, max,
 * exp, normalise, then the weighted sum of V), the softmax exponential either
 * the reference's fast_expf (:3181-3191, its default) or expf. */
#include <immintrin.h>

/* fast_expf: clamp, x * log2(e) split into integer and fraction, 2^f by the
 * reference's degree-5 Horner polynomial, 2^k written into the exponent. */
float orc_fast_expf(float x)
{
    x = x < -87.0f ? -87.0f : (x > 88.0f ? 88.0f : x);
    const float t = x * 1.44269504088896f;
    const float k = floorf(t), f = t - k;
    const float p = 1.0f + f * (0.6931471805f + f * (0.2402265069f + f * (0.0555041087f +
                                                                        f * (0.0096181291f + f * 0.0013333558f))));
    const unsigned int bits = (unsigned int)(((int)k + 127) << 23);
    float two_k;
    memcpy(&two_k, &bits, 4);
    return p * two_k;
}
unsigned short orc_f2h(float f) { return _cvtss_sh(f, 0); }      /* IEEE round to nearest even */
float orc_h2f(unsigned short h) { return _cvtsh_ss(h); }

struct OrcDec {
    OrcModel m;
    int W, kvdt, exact, maxpos, nostore;
    void **K, **V;
    float *cs, *sn;
};

OrcDec *orc_dec_new(const OrcModel *m, int W, int kvdt, int exact_exp, int maxpos)
{
    OrcDec *d = calloc(1, sizeof *d);
    const int hd = m->D / m->H, KD = m->KV * hd, esz = kvdt ? 2 : 4;
    d->m = *m; d->W = W; d->kvdt = kvdt; d->exact = exact_exp; d->maxpos = maxpos;
    d->K = calloc(m->L, sizeof(void *));
    d->V = calloc(m->L, sizeof(void *));
    for (int l = 0; l < m->L; l++) {
        d->K[l] = calloc((size_t)W * KD, esz);
        d->V[l] = calloc((size_t)W * KD, esz);
    }
    d->cs = zalloc((size_t)maxpos * (hd / 2));
    d->sn = zalloc((size_t)maxpos * (hd / 2));
    orc_rope_table(d->cs, d->sn, maxpos, hd, m->rope_base);
    return d;
}

void orc_dec_set_ring(OrcDec *d, int l, const void *K, const void *V)
{
    const size_t bytes = (size_t)d->W * d->m.KV * (d->m.D / d->m.H) * (d->kvdt ? 2 : 4);
    memcpy(d->K[l], K, bytes);
    memcpy(d->V[l], V, bytes);
}

void orc_dec_set_store(OrcDec *d, int store) { d->nostore = !store; }
const void *orc_dec_ring(const OrcDec *d, int l, int v) { return v ? d->V[l] : d->K[l]; }

void orc_dec_free(OrcDec *d)
{
    if (!d) return;
    for (int l = 0; l < d->m.L; l++) { free(d->K[l]); free(d->V[l]); }
    free(d->K); free(d->V); free(d->cs); free(d->sn); free(d);
}

/* q . row with the row stored as f32 (sequential, dot_f :3086-3088) or f16
 * (eight fma lanes, then (l0..3 + l4..7) and two pairwise adds: kv_dot's F16C
 * path :3200-3207) */
static float dec_dot(const float *q, const void *row, int n, int kvdt)
{
    if (!kvdt) {
        const float *r = row;
        float s = 0.0f;
        for (int i = 0; i < n; i++) s += q[i] * r[i];
        return s;
    }
    const unsigned short *h = row;
    float acc[8] = {0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; j++) acc[j] = fmaf(q[i + j], orc_h2f(h[i + j]), acc[j]);
    const float l0 = acc[0] + acc[4], l1 = acc[1] + acc[5], l2 = acc[2] + acc[6], l3 = acc[3] + acc[7];
    float s = (l0 + l1) + (l2 + l3);
    for (; i < n; i++) s += q[i] * orc_h2f(h[i]);
    return s;
}
static float dec_val(const void *row, int i, int kvdt)
{
    return kvdt ? orc_h2f(((const unsigned short *)row)[i]) : ((const float *)row)[i];
}

/* One layer's decode attention for m rows at positions start..start+m-1:
 * the m new K / V rows go into the ring first (forward_chunk's hoisted
 * kv_store, :3765-3780), then every (row, head) attends over its window
 * (attn_body's unsplit path, :3639-3715); ctx [m][D]. */
void orc_dec_attn(OrcDec *d, int l, const float *q, const float *k, const float *v, int m, int start, float *ctx)
{
    const OrcModel *md = &d->m;
    const int D = md->D, H = md->H, KV = md->KV, hd = D / H, KD = KV * hd, W = d->W, grp = H / KV,
              esz = d->kvdt ? 2 : 4;
    const float scale = 1.0f / sqrtf((float)hd);
    float *pr = zalloc(W);
    int eff = layer_win(md, l), wlim = (eff > 0 && eff < W) ? eff : W;
    for (int j = 0; j < m && !d->nostore; j++) {   /* kv_store into the ring */
        const int slot = (start + j) % W;
        for (int i = 0; i < KD; i++) {
            if (d->kvdt) {
                ((unsigned short *)d->K[l])[(size_t)slot * KD + i] = orc_f2h(k[(size_t)j * KD + i]);
                ((unsigned short *)d->V[l])[(size_t)slot * KD + i] = orc_f2h(v[(size_t)j * KD + i]);
            } else {
                ((float *)d->K[l])[(size_t)slot * KD + i] = k[(size_t)j * KD + i];
                ((float *)d->V[l])[(size_t)slot * KD + i] = v[(size_t)j * KD + i];
            }
        }
    }
    for (int j = 0; j < m; j++)
        for (int h = 0; h < H; h++) {
            const int p = start + j, lo = p >= wlim ? p - wlim + 1 : 0, cnt = p - lo + 1, kh = h / grp;
            const float *qh = q + (size_t)j * D + (size_t)h * hd;
            float mx = -1e30f;
            for (int t = 0; t < cnt; t++) {
                const int slot = (lo + t) % W;
                const char *kr = (const char *)d->K[l] + ((size_t)slot * KD + (size_t)kh * hd) * esz;
                pr[t] = dec_dot(qh, kr, hd, d->kvdt) * scale;
                if (pr[t] > mx) mx = pr[t];
            }
            float s = 0.0f;
            for (int t = 0; t < cnt; t++) {
                pr[t] = d->exact ? expf(pr[t] - mx) : orc_fast_expf(pr[t] - mx);
                s += pr[t];
            }
            const float inv = s > 0 ? 1.0f / s : 0.0f;
            for (int t = 0; t < cnt; t++) pr[t] *= inv;
            float *acc = ctx + (size_t)j * D + (size_t)h * hd;
            for (int i = 0; i < hd; i++) acc[i] = 0.0f;
            for (int t = 0; t < cnt; t++) {
                const int slot = (lo + t) % W;
                const char *vr = (const char *)d->V[l] + ((size_t)slot * KD + (size_t)kh * hd) * esz;
                for (int i = 0; i < hd; i++) acc[i] = fmaf(pr[t], dec_val(vr, i, d->kvdt), acc[i]);
            }
        }
    free(pr);
}

void orc_qknorm(float *buf, const float *gain, int rows, int nheads, int hd)
{
    for (int r = 0; r < rows * nheads; r++) {
        float *v = buf + (size_t)r * hd;
        float ss = 0.0f;
        for (int i = 0; i < hd; i++) ss += v[i] * v[i];
        const float sc = 1.0f / sqrtf(ss / hd + 1e-5f);
        for (int i = 0; i < hd; i++) v[i] = v[i] * sc * gain[i];
    }
}

void orc_dec_moe(int N, int D, int F, int E, const float *fnorm, const float *fin, float *out, const float *wr,
                 const float *w1, const float *w3, const float *w2, int *assign, float *gate, float *rprobs)
{
    float *rt = zalloc((size_t)N * E), *X = zalloc((size_t)N * D), *g = zalloc((size_t)N * F),
          *u = zalloc((size_t)N * F), *y = zalloc((size_t)N * D);
    int *idx = calloc((size_t)N, sizeof(int));
    orc_mm(rt, fnorm, wr, N, D, E);
    for (int n = 0; n < N; n++) {                /* softmax, then the first maximum */
        const float *r = rt + (size_t)n * E;
        float *pr = rprobs + (size_t)n * E;
        float mx = -1e30f;
        for (int e = 0; e < E; e++) if (r[e] > mx) mx = r[e];
        float sm = 0.0f;
        for (int e = 0; e < E; e++) { pr[e] = expf(r[e] - mx); sm += pr[e]; }
        const float inv = 1.0f / sm;
        int best = 0;
        for (int e = 0; e < E; e++) { pr[e] *= inv; if (pr[e] > pr[best]) best = e; }
        assign[n] = best;
        gate[n] = pr[best];
    }
    memcpy(out, fin, sizeof(float) * (size_t)N * D);
    for (int e = 0; e < E; e++) {
        int ne = 0;
        for (int n = 0; n < N; n++) if (assign[n] == e) idx[ne++] = n;
        if (!ne) continue;
        for (int r = 0; r < ne; r++) memcpy(X + (size_t)r * D, fnorm + (size_t)idx[r] * D, sizeof(float) * D);
        orc_mm(g, X, w1 + (size_t)e * D * F, ne, D, F);
        orc_mm(u, X, w3 + (size_t)e * D * F, ne, D, F);
        for (size_t i = 0; i < (size_t)ne * F; i++) u[i] = silu(g[i]) * u[i];
        orc_mm(y, u, w2 + (size_t)e * F * D, ne, F, D);
        for (int r = 0; r < ne; r++) {
            const float gt = gate[idx[r]];
            float *o = out + (size_t)idx[r] * D;
            const float *yr = y + (size_t)r * D;
            for (int i = 0; i < D; i++) o[i] += gt * yr[i];
        }
    }
    free(rt); free(X); free(g); free(u); free(y); free(idx);
}

int orc_mtp_argmax(const OrcModel *md, const float *P, const float *fn1, int k, float *logits)
{
    const int D = md->D, V = md->V;
    OrcLayerMap w;
    orc_param_map(md, 0, &w);
    float *ht = zalloc(D), *hh = zalloc(D);
    orc_mm(ht, fn1, P + w.mtp0 + (size_t)k * D * D, 1, D, D);
    for (int i = 0; i < D; i++) hh[i] = fn1[i] + silu(ht[i]);
    memset(logits, 0, sizeof(float) * (size_t)V);
    orc_mm_bt(logits, hh, P + w.emb, 1, V, D);
    int best = 0;
    for (int i = 1; i < V; i++) if (logits[i] > logits[best]) best = i;
    free(ht); free(hh);
    return best;
}

/* m tokens at positions start..start+m-1; logits [m][V] (main head). */
void orc_dec_chunk(OrcDec *d, const float *P, const int *tok, int m, int start, float *logits)
{
    orc_dec_chunk_fn(d, P, tok, m, start, logits, NULL);
}

void orc_dec_chunk_fn(OrcDec *d, const float *P, const int *tok, int m, int start, float *logits, float *fn)
{
    const OrcModel *md = &d->m;
    const int D = md->D, H = md->H, KV = md->KV, hd = D / H, KD = KV * hd, F = md->F, V = md->V;
    OrcLayerMap w;
    orc_param_map(md, 0, &w);
    float *x = zalloc((size_t)m * D), *xn = zalloc((size_t)m * D), *q = zalloc((size_t)m * D),
          *k = zalloc((size_t)m * KD), *v = zalloc((size_t)m * KD), *ctx = zalloc((size_t)m * D),
          *tmp = zalloc((size_t)m * D), *g = zalloc((size_t)m * F), *u = zalloc((size_t)m * F),
          *rinv = zalloc(m);
    int *pos = calloc(m, sizeof(int));
    for (int j = 0; j < m; j++) {
        memcpy(x + (size_t)j * D, P + w.emb + (size_t)tok[j] * D, sizeof(float) * D);
        pos[j] = start + j;
    }
    for (int l = 0; l < md->L; l++) {
        orc_param_map(md, l, &w);
        orc_rmsnorm_fwd(x, P + w.an1, xn, rinv, m, D);
        orc_mm(q, xn, P + w.wq, m, D, D);
        orc_mm(k, xn, P + w.wk, m, D, KD);
        orc_mm(v, xn, P + w.wv, m, D, KD);
        if (md->qknorm) {                        /* :3752-3754 */
            orc_qknorm(q, P + w.qn, m, H, hd);
            orc_qknorm(k, P + w.kn, m, KV, hd);
        }
        orc_rope(q, pos, 1, m, H, hd, d->cs, d->sn, 0);
        orc_rope(k, pos, 1, m, KV, hd, d->cs, d->sn, 0);
        orc_dec_attn(d, l, q, k, v, m, start, ctx);
        orc_mm(tmp, ctx, P + w.wo, m, D, D);
        for (size_t i = 0; i < (size_t)m * D; i++) x[i] += tmp[i];
        orc_rmsnorm_fwd(x, P + w.an2, xn, rinv, m, D);
        if (md->n_exp > 0) {                      /* :3815-3818: out = tmp = x + ffn, then x = tmp */
            int *as = calloc((size_t)m, sizeof(int));
            float *gt = zalloc(m), *rp = zalloc((size_t)m * md->n_exp);
            orc_dec_moe(m, D, F, md->n_exp, xn, x, tmp, P + w.wr, P + w.w1, P + w.w3, P + w.w2, as, gt, rp);
            memcpy(x, tmp, sizeof(float) * (size_t)m * D);
            free(as); free(gt); free(rp);
            continue;
        }
        orc_mm(g, xn, P + w.w1, m, D, F);
        orc_mm(u, xn, P + w.w3, m, D, F);
        for (size_t i = 0; i < (size_t)m * F; i++) u[i] = silu(g[i]) * u[i];
        orc_mm(tmp, u, P + w.w2, m, F, D);
        for (size_t i = 0; i < (size_t)m * D; i++) x[i] += tmp[i];
    }
    orc_param_map(md, 0, &w);
    orc_rmsnorm_fwd(x, P + w.nf, xn, rinv, m, D);
    if (fn) memcpy(fn, xn, sizeof(float) * (size_t)m * D);
    memset(logits, 0, sizeof(float) * (size_t)m * V);
    orc_mm_bt(logits, xn, P + w.emb, m, V, D);
    float *all[] = {x, xn, q, k, v, ctx, tmp, g, u, rinv};
    for (size_t i = 0; i < sizeof all / sizeof all[0]; i++) free(all[i]);
    free(pos);
}
