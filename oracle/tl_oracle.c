/* tl_oracle.c -- CPU restatement of tinylm.c's fp32 GEMM primitives.
 *
 * TEST INFRASTRUCTURE ONLY (see tl_oracle.h).  The product path never links
 * this file; it exists so tests and the bench's CPU-baseline leg have the
 * reference arithmetic on the CPU.
 *
 * Why the loop nests mirror the reference's blocking: mm and mm_atb compute
 * every output element as ONE sequential multiply-add chain (over k for mm,
 * over m for mm_atb).  Keeping the same chain order -- and compiling with the
 * reference's flags (-O3 -ffast-math -funroll-loops -fopenmp, an FMA ISA) so
 * the multiply-adds contract to FMA the same way -- makes the restatement
 * bit-identical to tinylm.c for those two.  mm_bt is a dot product that
 * -ffast-math vectorises with reassociation; the 4-row blocking is kept so
 * the compiler sees the same reduction shape.
 */
#include "tl_oracle.h"
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <stdio.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_pool = 1;                       /* emulated tl_for workers (1 = off) */

void orc_set_pool(int nt) { g_pool = nt < 1 ? 1 : nt; }
int orc_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
void orc_set_threads(int nt) {
#ifdef _OPENMP
    if (nt > 0) omp_set_num_threads(nt);
#else
    (void)nt;
#endif
}

/* ------------------------------------------------------------------ mm --- */
/* One 4-row block b of Y = X W.  Rows are cleared, then every k adds
 * x[row][k] * W[k][:] into the row: per element, y = fma(x_k, w_k, y) for
 * k = 0..K-1 in order (tinylm.c:456-467).  A short final block runs the same
 * chain one row at a time (tinylm.c:468-476). */
static void mm_block_to(float *restrict Yb, int ldy, int ycol0, const float *restrict X, const float *restrict W,
                        int M, int K, int N, int b, int n0, int n1)
{
    /* rows r0 .. r0+3 of the block go to Yb + i*ldy, column n at n - ycol0 */
    const int r0 = b * 4;
    const int nr = (M - r0 < 4) ? (M - r0) : 4;
    if (nr == 4) {
        float *restrict ya = Yb - ycol0;
        float *restrict yb = ya + ldy;
        float *restrict yc = yb + ldy;
        float *restrict yd = yc + ldy;
        const float *restrict xa = X + (size_t)r0 * K;
        const float *restrict xb = xa + K;
        const float *restrict xc = xb + K;
        const float *restrict xd = xc + K;
        for (int n = n0; n < n1; n++) { ya[n] = 0.0f; yb[n] = 0.0f; yc[n] = 0.0f; yd[n] = 0.0f; }
        for (int k = 0; k < K; k++) {
            const float ca = xa[k], cb = xb[k], cc = xc[k], cd = xd[k];
            const float *restrict wk = W + (size_t)k * N;
            for (int n = n0; n < n1; n++) {
                const float w = wk[n];
                ya[n] += ca * w; yb[n] += cb * w; yc[n] += cc * w; yd[n] += cd * w;
            }
        }
        return;
    }
    for (int i = 0; i < nr; i++) {
        float *restrict y = Yb + (size_t)i * ldy - ycol0;
        const float *restrict x = X + (size_t)(r0 + i) * K;
        for (int n = n0; n < n1; n++) y[n] = 0.0f;
        for (int k = 0; k < K; k++) {
            const float c = x[k];
            const float *restrict wk = W + (size_t)k * N;
            for (int n = n0; n < n1; n++) y[n] += c * wk[n];
        }
    }
}
static void mm_block_cols(float *restrict Y, const float *restrict X, const float *restrict W,
                          int M, int K, int N, int b, int n0, int n1)
{
    mm_block_to(Y + (size_t)b * 4 * N, N, 0, X, W, M, K, N, b, n0, n1);
}
static void mm_block(float *restrict Y, const float *restrict X, const float *restrict W,
                     int M, int K, int N, int b)
{
    mm_block_cols(Y, X, W, M, K, N, b, 0, N);
}

/* The threaded GEMV variant of the CPU decode baseline (not the reference's
 * dispatch, which runs M <= 8 serially): M <= 8 calls split their outputs
 * over the OpenMP threads in contiguous ranges -- mm by column ranges of 16
 * floats, mm_bt by ranges of W rows that start at multiples of 4 -- and
 * every element keeps the reference's own chain, so the results equal the
 * serial ones.  Inside orc_run_calls the whole call list runs in one
 * parallel region (a barrier between calls), so no call pays for waking the
 * threads. */
static int g_gemv_split = 0;
void orc_set_gemv_split(int on) { g_gemv_split = on != 0; }

/* this thread's share [*lo, *hi) of n items in units of `unit` */
static void split_range(int n, int unit, int *lo, int *hi)
{
    int T = 1, t = 0;
#ifdef _OPENMP
    T = omp_get_num_threads();
    t = omp_get_thread_num();
#endif
    const int nu = (n + unit - 1) / unit;
    const int u0 = (int)((long long)nu * t / T), u1 = (int)((long long)nu * (t + 1) / T);
    *lo = u0 * unit;
    *hi = u1 * unit < n ? u1 * unit : n;
}

/* Dispatch rule of tinylm.c:444-448: a single block, or a live decode pool,
 * goes through tl_for (serial when the block count is below the worker count,
 * tinylm.c:239); otherwise OpenMP static over blocks. */
/* M <= 8 mm, this thread's column range (called by every thread of a region) */
static void mm_split_part(float *Y, const float *X, const float *W, int M, int K, int N)
{
    int n0, n1;
    split_range(N, 16, &n0, &n1);
    if (n0 >= n1) return;
    /* each block's rows accumulate in this thread's own buffer (neighbouring
     * threads' columns share cache lines of Y), then are copied out once */
    const int w = n1 - n0;
    float *t = malloc((size_t)4 * w * sizeof(float));
    if (!t) abort();
    for (int b = 0; b < (M + 3) / 4; b++) {
        const int nr = M - 4 * b < 4 ? M - 4 * b : 4;
        mm_block_to(t, w, n0, X, W, M, K, N, b, n0, n1);
        for (int i = 0; i < nr; i++) memcpy(Y + (size_t)(4 * b + i) * N + n0, t + (size_t)i * w, (size_t)w * sizeof(float));
    }
    free(t);
}

void orc_mm(float *Y, const float *X, const float *W, int M, int K, int N)
{
    const int nblk = (M + 3) / 4;
    if (g_gemv_split && M <= 8) {
        #pragma omp parallel
        mm_split_part(Y, X, W, M, K, N);
        return;
    }
    if (nblk == 1 || g_pool > 1) {
        if (g_pool <= 1 || nblk < g_pool) {
            for (int b = 0; b < nblk; b++) mm_block(Y, X, W, M, K, N, b);
            return;
        }
        #pragma omp parallel for schedule(static) num_threads(g_pool)
        for (int b = 0; b < nblk; b++) mm_block(Y, X, W, M, K, N, b);
        return;
    }
    #pragma omp parallel for schedule(static)
    for (int b = 0; b < nblk; b++) mm_block(Y, X, W, M, K, N, b);
}

/* --------------------------------------------------------------- mm_bt --- */
/* Row m of dX += dY W^T: four W rows at a time, each a dot product over n with
 * its own accumulator, added into dx once (tinylm.c:494-506). */
static void mmbt_rows(float *restrict dX, const float *restrict dY, const float *restrict W,
                      int K, int N, int m, int k0, int k1)
{
    const float *restrict g = dY + (size_t)m * N;
    float *restrict o = dX + (size_t)m * K;
    int k = k0;
    for (; k + 4 <= k1; k += 4) {
        const float *restrict wa = W + (size_t)k * N;
        const float *restrict wb = wa + N;
        const float *restrict wc = wb + N;
        const float *restrict wd = wc + N;
        float sa = 0.0f, sb = 0.0f, sc = 0.0f, sd = 0.0f;
        for (int n = 0; n < N; n++) {
            const float d = g[n];
            sa += d * wa[n]; sb += d * wb[n]; sc += d * wc[n]; sd += d * wd[n];
        }
        o[k] += sa; o[k + 1] += sb; o[k + 2] += sc; o[k + 3] += sd;
    }
    for (; k < k1; k++) {
        const float *restrict w = W + (size_t)k * N;
        float s = 0.0f;
        for (int n = 0; n < N; n++) s += g[n] * w[n];
        o[k] += s;
    }
}

static void mmbt_row(float *restrict dX, const float *restrict dY, const float *restrict W,
                     int K, int N, int m)
{
    mmbt_rows(dX, dY, W, K, N, m, 0, K);
}

/* tinylm.c:486-488: M==1 or a live pool -> tl_for over rows, else OpenMP. */
/* M <= 8 mm_bt, this thread's range of W rows (multiples of 4) */
static void mmbt_split_part(float *dX, const float *dY, const float *W, int M, int K, int N)
{
    int k0, k1;
    split_range(K, 4, &k0, &k1);
    for (int m = 0; k0 < k1 && m < M; m++) mmbt_rows(dX, dY, W, K, N, m, k0, k1);
}

void orc_mm_bt(float *dX, const float *dY, const float *W, int M, int K, int N)
{
    if (g_gemv_split && M <= 8) {
        #pragma omp parallel
        mmbt_split_part(dX, dY, W, M, K, N);
        return;
    }
    if (M == 1 || g_pool > 1) {
        if (g_pool <= 1 || M < g_pool) {
            for (int m = 0; m < M; m++) mmbt_row(dX, dY, W, K, N, m);
            return;
        }
        #pragma omp parallel for schedule(static) num_threads(g_pool)
        for (int m = 0; m < M; m++) mmbt_row(dX, dY, W, K, N, m);
        return;
    }
    #pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++) mmbt_row(dX, dY, W, K, N, m);
}

/* -------------------------------------------------------------- mm_atb --- */
/* dW += X^T dY.  Four dW rows (k0..k0+3) per task; m runs sequentially so each
 * dW element is one chain dw = fma(x[m][k], dy[m][n], dw) over m = 0..M-1,
 * starting from the caller's prefill (tinylm.c:515-536). */
void orc_mm_atb(float *dW, const float *X, const float *dY, int M, int K, int N)
{
    #pragma omp parallel for schedule(static)
    for (int k0 = 0; k0 < K; k0 += 4) {
        const int nk = (K - k0 < 4) ? (K - k0) : 4;
        if (nk == 4) {
            float *restrict da = dW + (size_t)k0 * N;
            float *restrict db = da + N;
            float *restrict dc = db + N;
            float *restrict dd = dc + N;
            for (int m = 0; m < M; m++) {
                const float *restrict x = X + (size_t)m * K;
                const float ca = x[k0], cb = x[k0 + 1], cc = x[k0 + 2], cd = x[k0 + 3];
                const float *restrict g = dY + (size_t)m * N;
                for (int n = 0; n < N; n++) {
                    const float d = g[n];
                    da[n] += ca * d; db[n] += cb * d; dc[n] += cc * d; dd[n] += cd * d;
                }
            }
        } else {
            for (int k = k0; k < k0 + nk; k++) {
                float *restrict dw = dW + (size_t)k * N;
                for (int m = 0; m < M; m++) {
                    const float c = X[(size_t)m * K + k];
                    const float *restrict g = dY + (size_t)m * N;
                    for (int n = 0; n < N; n++) dw[n] += c * g[n];
                }
            }
        }
    }
}

/* ------------------------------------------------------- fp64 oracles --- */
/* Textbook sums in double.  Loop orders stream rows (a double accumulator row
 * per output row) so the large configurations finish in seconds; every
 * product and partial sum is in double, so the order does not matter at the
 * fp32 precision the results are stored in. */
void orc_mm_f64(float *Y, const float *X, const float *W, int M, int K, int N)
{
    #pragma omp parallel
    {
        double *acc = malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
        #pragma omp for schedule(static)
        for (int m = 0; m < M; m++) {
            for (int n = 0; n < N; n++) acc[n] = 0.0;
            for (int k = 0; k < K; k++) {
                const double x = (double)X[(size_t)m * K + k];
                const float *w = W + (size_t)k * N;
                for (int n = 0; n < N; n++) acc[n] += x * (double)w[n];
            }
            for (int n = 0; n < N; n++) Y[(size_t)m * N + n] = (float)acc[n];
        }
        free(acc);
    }
}
void orc_mm_bt_f64(float *dX, const float *dY, const float *W, int M, int K, int N)
{
    #pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++)
        for (int k = 0; k < K; k++) {
            double s = (double)dX[(size_t)m * K + k];
            for (int n = 0; n < N; n++) s += (double)dY[(size_t)m * N + n] * (double)W[(size_t)k * N + n];
            dX[(size_t)m * K + k] = (float)s;
        }
}
void orc_mm_atb_f64(float *dW, const float *X, const float *dY, int M, int K, int N)
{
    #pragma omp parallel
    {
        double *acc = malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
        #pragma omp for schedule(static)
        for (int k = 0; k < K; k++) {
            for (int n = 0; n < N; n++) acc[n] = (double)dW[(size_t)k * N + n];
            for (int m = 0; m < M; m++) {
                const double x = (double)X[(size_t)m * K + k];
                const float *g = dY + (size_t)m * N;
                for (int n = 0; n < N; n++) acc[n] += x * (double)g[n];
            }
            for (int n = 0; n < N; n++) dW[(size_t)k * N + n] = (float)acc[n];
        }
        free(acc);
    }
}

/* ----------------------------------------------------------------- RNG --- */
/* xorshift64 with shifts 13, 7, 17; uniform from the top 53 bits; Box-Muller
 * cosine branch with u1 floored at 1e-9 (tinylm.c:127-134).  The default
 * state is the reference's initial g_rng. */
static uint64_t g_state = 1234567891011ULL;

void orc_rng_seed(uint64_t s) { g_state = s; }
uint64_t orc_rng_state(void) { return g_state; }
uint64_t orc_xorshift(void)
{
    uint64_t x = g_state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    g_state = x;
    return x;
}
static float uniform01(void) { return (float)(orc_xorshift() >> 11) * (1.0f / 9007199254740992.0f); }
float orc_rnd_normal(void)
{
    float a = uniform01();
    if (a < 1e-9f) a = 1e-9f;
    const float b = uniform01();
    return sqrtf(-2.0f * logf(a)) * cosf(6.28318530718f * b);
}
void orc_fill_normal(float *p, size_t n, float scale)
{
    for (size_t i = 0; i < n; i++) p[i] = scale * orc_rnd_normal();
}

/* ----------------------------------------------------------------- MoE --- */
static float silu(float z) { return z / (1.0f + expf(-z)); }

/* Rows of `src` listed in idx[0..ne-1], packed into dst. */
static void gather_rows(float *dst, const float *src, const int *idx, int ne, int D)
{
    for (int j = 0; j < ne; j++) memcpy(dst + (size_t)j * D, src + (size_t)idx[j] * D, sizeof(float) * D);
}

/* Router softmax over all E, then top-1 by strict-greater scan so ties keep
 * the lowest expert index (tinylm.c:814-827, :859-869).  out starts as the
 * residual fin; each expert e takes its tokens in ascending token order
 * (tinylm.c:876), runs silu(X W1) * (X W3) then W2, and adds gate*y back
 * (tinylm.c:877-889). */
void orc_moe_forward(int N, int D, int F, int E,
                     const float *fnorm, const float *fin, float *out,
                     const float *wr, const float *w1, const float *w3, const float *w2,
                     int *assign, float *gate, float *rprobs)
{
    float *logit = malloc(sizeof(float) * (size_t)N * E);
    float *xs = malloc(sizeof(float) * (size_t)N * D);
    float *g = malloc(sizeof(float) * (size_t)N * F);
    float *u = malloc(sizeof(float) * (size_t)N * F);
    float *y = malloc(sizeof(float) * (size_t)N * D);
    int *idx = malloc(sizeof(int) * (size_t)N);
    orc_mm(logit, fnorm, wr, N, D, E);
    for (int n = 0; n < N; n++) {
        const float *r = logit + (size_t)n * E;
        float *p = rprobs + (size_t)n * E;
        float mx = -1e30f;
        for (int e = 0; e < E; e++) if (r[e] > mx) mx = r[e];
        float s = 0.0f;
        for (int e = 0; e < E; e++) { p[e] = expf(r[e] - mx); s += p[e]; }
        const float inv = 1.0f / s;
        for (int e = 0; e < E; e++) p[e] *= inv;
        int best = -1; float bp = -1e30f;
        for (int e = 0; e < E; e++) if (p[e] > bp) { bp = p[e]; best = e; }
        assign[n] = best < 0 ? 0 : best;
        gate[n] = p[assign[n]];
    }
    memcpy(out, fin, sizeof(float) * (size_t)N * D);
    for (int e = 0; e < E; e++) {
        int ne = 0;
        for (int n = 0; n < N; n++) if (assign[n] == e) idx[ne++] = n;
        if (!ne) continue;
        gather_rows(xs, fnorm, idx, ne, D);
        orc_mm(g, xs, w1 + (size_t)e * D * F, ne, D, F);
        orc_mm(u, xs, w3 + (size_t)e * D * F, ne, D, F);
        for (size_t i = 0; i < (size_t)ne * F; i++) g[i] = silu(g[i]) * u[i];
        orc_mm(y, g, w2 + (size_t)e * F * D, ne, F, D);
        for (int j = 0; j < ne; j++) {
            const int n = idx[j];
            const float gt = gate[n];
            float *o = out + (size_t)n * D;
            const float *yy = y + (size_t)j * D;
            for (int d = 0; d < D; d++) o[d] += gt * yy[d];
        }
    }
    free(logit); free(xs); free(g); free(u); free(y); free(idx);
}

/* Backward of the above for K=1 (tinylm.c:895-947): per expert recompute the
 * forward, d_gate = <dout, y>, dy = gate*dout, then dW2, d_act, silu backward,
 * dW1/dW3 and dX (two accumulating mm_bt) scattered into d_fnorm; finally the
 * router softmax backward with the load-balance term 0.01*E*(cnt_e/N)/N and
 * the router GEMMs. */
void orc_moe_backward(int N, int D, int F, int E,
                      const float *fnorm, const float *dout, float *d_fnorm,
                      const float *wr, const float *w1, const float *w3, const float *w2,
                      float *gwr, float *gw1, float *gw3, float *gw2,
                      const int *assign, const float *gate, const float *rprobs)
{
    float *xs = malloc(sizeof(float) * (size_t)N * D);
    float *g = malloc(sizeof(float) * (size_t)N * F);
    float *u = malloc(sizeof(float) * (size_t)N * F);
    float *a = malloc(sizeof(float) * (size_t)N * F);
    float *y = malloc(sizeof(float) * (size_t)N * D);
    float *dy = malloc(sizeof(float) * (size_t)N * D);
    float *da = malloc(sizeof(float) * (size_t)N * F);
    float *dg = malloc(sizeof(float) * (size_t)N * F);
    float *du = malloc(sizeof(float) * (size_t)N * F);
    float *dx = malloc(sizeof(float) * (size_t)N * D);
    float *drt = malloc(sizeof(float) * (size_t)N * E);
    float *dgate = calloc((size_t)N, sizeof(float));
    int *idx = malloc(sizeof(int) * (size_t)N);
    int *cnt = calloc((size_t)E, sizeof(int));
    memset(d_fnorm, 0, sizeof(float) * (size_t)N * D);
    for (int e = 0; e < E; e++) {
        int ne = 0;
        for (int n = 0; n < N; n++) if (assign[n] == e) idx[ne++] = n;
        if (!ne) continue;
        const float *W1 = w1 + (size_t)e * D * F, *W3 = w3 + (size_t)e * D * F, *W2 = w2 + (size_t)e * F * D;
        gather_rows(xs, fnorm, idx, ne, D);
        orc_mm(g, xs, W1, ne, D, F);
        orc_mm(u, xs, W3, ne, D, F);
        for (size_t i = 0; i < (size_t)ne * F; i++) a[i] = silu(g[i]) * u[i];
        orc_mm(y, a, W2, ne, F, D);
        for (int j = 0; j < ne; j++) {
            const int n = idx[j];
            const float *o = dout + (size_t)n * D, *yy = y + (size_t)j * D;
            float s = 0.0f;
            for (int d = 0; d < D; d++) s += o[d] * yy[d];
            dgate[n] = s;
            float *t = dy + (size_t)j * D;
            for (int d = 0; d < D; d++) t[d] = gate[n] * o[d];
        }
        orc_mm_atb(gw2 + (size_t)e * F * D, a, dy, ne, F, D);
        memset(da, 0, sizeof(float) * (size_t)ne * F);
        orc_mm_bt(da, dy, W2, ne, F, D);
        for (size_t i = 0; i < (size_t)ne * F; i++) {
            const float z = g[i];
            const float sg = 1.0f / (1.0f + expf(-z));
            const float ds = sg + z * sg * (1.0f - sg);
            dg[i] = da[i] * u[i] * ds;
            du[i] = da[i] * (z * sg);
        }
        orc_mm_atb(gw1 + (size_t)e * D * F, xs, dg, ne, D, F);
        orc_mm_atb(gw3 + (size_t)e * D * F, xs, du, ne, D, F);
        memset(dx, 0, sizeof(float) * (size_t)ne * D);
        orc_mm_bt(dx, dg, W1, ne, D, F);
        orc_mm_bt(dx, du, W3, ne, D, F);
        for (int j = 0; j < ne; j++) {
            float *t = d_fnorm + (size_t)idx[j] * D;
            const float *s = dx + (size_t)j * D;
            for (int d = 0; d < D; d++) t[d] += s[d];
        }
    }
    for (int n = 0; n < N; n++) cnt[assign[n]]++;
    const float invN = 1.0f / (float)N;
    for (int n = 0; n < N; n++) {
        const float *p = rprobs + (size_t)n * E;
        float *d = drt + (size_t)n * E;
        float dp[64];
        for (int e = 0; e < E; e++) dp[e] = 0.01f * (float)E * ((float)cnt[e] * invN) * invN;
        dp[assign[n]] += dgate[n];
        float dot = 0.0f;
        for (int e = 0; e < E; e++) dot += p[e] * dp[e];
        for (int e = 0; e < E; e++) d[e] = p[e] * (dp[e] - dot);
    }
    orc_mm_bt(d_fnorm, drt, wr, N, D, E);
    orc_mm_atb(gwr, fnorm, drt, N, D, E);
    free(xs); free(g); free(u); free(a); free(y); free(dy); free(da); free(dg); free(du);
    free(dx); free(drt); free(dgate); free(idx); free(cnt);
}

void orc_run_calls(const OrcCall *c, int n, int reps)
{
    if (g_gemv_split) {
        /* the threaded decode variant: one region for the whole list, the
         * M <= 8 GEMVs split over its threads, everything else on one */
        #pragma omp parallel
        for (int r = 0; r < reps; r++)
            for (int i = 0; i < n; i++) {
                if (c[i].op == 0 && c[i].M <= 8) mm_split_part(c[i].out, c[i].a, c[i].b, c[i].M, c[i].K, c[i].N);
                else if (c[i].op == 1 && c[i].M <= 8)
                    mmbt_split_part(c[i].out, c[i].a, c[i].b, c[i].M, c[i].K, c[i].N);
                else {
                    #pragma omp single
                    {
                        switch (c[i].op) {
                        case 0: orc_mm(c[i].out, c[i].a, c[i].b, c[i].M, c[i].K, c[i].N); break;
                        case 1: orc_mm_bt(c[i].out, c[i].a, c[i].b, c[i].M, c[i].K, c[i].N); break;
                        case 2: orc_mm_atb(c[i].out, c[i].a, c[i].b, c[i].M, c[i].K, c[i].N); break;
                        default: memset(c[i].out, 0, c[i].n * sizeof(float)); break;
                        }
                    }
                }
                #pragma omp barrier
            }
        return;
    }
    for (int r = 0; r < reps; r++)
        for (int i = 0; i < n; i++) {
            switch (c[i].op) {
            case 0: orc_mm(c[i].out, c[i].a, c[i].b, c[i].M, c[i].K, c[i].N); break;
            case 1: orc_mm_bt(c[i].out, c[i].a, c[i].b, c[i].M, c[i].K, c[i].N); break;
            case 2: orc_mm_atb(c[i].out, c[i].a, c[i].b, c[i].M, c[i].K, c[i].N); break;
            default: memset(c[i].out, 0, c[i].n * sizeof(float)); break;
            }
        }
}
