/* tl_selftest.c -- a self-test of the -DUSE_HIP drop-in, in the spirit of
 * tinylm.c's own `selftest` command (tinylm.c:4750-4788): call mm, mm_bt and
 * mm_atb through their reference signatures on host buffers (so through the
 * seam in tl_mm_seam.c and the HIP kernels behind it) and compare with double
 * precision loops, reporting the normwise error max|err| / mean|ref|.
 *
 *   tl_selftest [M K N [seed]]      default: the reference's 201 131 259
 *
 * Exit status 0 when every result is within 1e-4 normwise, 1 otherwise.
 * The accumulating forms start from a random prefill, so the test also
 * checks that they add exactly once.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

void mm(float *restrict Y, const float *restrict X, const float *restrict W, int M, int K, int N);
void mm_bt(float *restrict dX, const float *restrict dY, const float *restrict W, int M, int K, int N);
void mm_atb(float *restrict dW, const float *restrict X, const float *restrict dY, int M, int K, int N);

/* splitmix64 -> two uniforms -> Box-Muller (this file's own generator) */
static uint64_t g_state;
static uint64_t next_u64(void)
{
    uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static float normal(void)
{
    double u1 = (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0);
    if (u1 < 1e-300) u1 = 1e-300;
    return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}
static float *rnd(size_t n, float scale)
{
    float *p = malloc(n * sizeof *p);
    if (!p) { fprintf(stderr, "out of memory\n"); exit(1); }
    for (size_t i = 0; i < n; i++) p[i] = scale * normal();
    return p;
}

/* max|got - ref| / mean|ref| */
static double normwise(const float *got, const double *ref, size_t n)
{
    double mx = 0.0, mean = 0.0;
    for (size_t i = 0; i < n; i++) {
        const double e = fabs((double)got[i] - ref[i]);
        if (e > mx || e != e) mx = e != e ? INFINITY : e;
        mean += fabs(ref[i]);
    }
    mean /= (double)(n ? n : 1);
    return mean > 0.0 ? mx / mean : mx;
}

int main(int argc, char **argv)
{
    int M = 201, K = 131, N = 259;
    uint64_t seed = 1234567891011ull;
    if (argc >= 4) { M = atoi(argv[1]); K = atoi(argv[2]); N = atoi(argv[3]); }
    if (argc >= 5) seed = strtoull(argv[4], NULL, 10);
    if (M <= 0 || K <= 0 || N <= 0) { fprintf(stderr, "usage: tl_selftest [M K N [seed]]\n"); return 2; }
    g_state = seed;
    const size_t MK = (size_t)M * K, KN = (size_t)K * N, MN = (size_t)M * N;
    float *X = rnd(MK, 1.0f), *W = rnd(KN, 1.0f), *dY = rnd(MN, 1.0f);
    float *Y = rnd(MN, 1.0f);                 /* garbage: mm must overwrite it */
    float *dX = rnd(MK, 1.0f), *dW = rnd(KN, 1.0f);
    double *rY = calloc(MN, sizeof *rY), *rX = malloc(MK * sizeof *rX), *rW = malloc(KN * sizeof *rW);
    if (!rY || !rX || !rW) { fprintf(stderr, "out of memory\n"); return 1; }
    for (size_t i = 0; i < MK; i++) rX[i] = dX[i];
    for (size_t i = 0; i < KN; i++) rW[i] = dW[i];

    /* double-precision references: Y = X W, dX += dY W^T, dW += X^T dY */
    for (int m = 0; m < M; m++)
        for (int k = 0; k < K; k++) {
            const double x = X[(size_t)m * K + k];
            for (int n = 0; n < N; n++) rY[(size_t)m * N + n] += x * W[(size_t)k * N + n];
        }
    for (int m = 0; m < M; m++)
        for (int k = 0; k < K; k++) {
            double s = 0.0;
            for (int n = 0; n < N; n++) s += (double)dY[(size_t)m * N + n] * W[(size_t)k * N + n];
            rX[(size_t)m * K + k] += s;
        }
    for (int m = 0; m < M; m++)
        for (int k = 0; k < K; k++) {
            const double x = X[(size_t)m * K + k];
            for (int n = 0; n < N; n++) rW[(size_t)k * N + n] += x * dY[(size_t)m * N + n];
        }

    mm(Y, X, W, M, K, N);
    mm_bt(dX, dY, W, M, K, N);
    mm_atb(dW, X, dY, M, K, N);

    const double eY = normwise(Y, rY, MN), eX = normwise(dX, rX, MK), eW = normwise(dW, rW, KN);
    const double tol = 1e-4;
    printf("selftest M=%d K=%d N=%d seed=%llu\n", M, K, N, (unsigned long long)seed);
    printf("  mm      normwise err %.3e %s\n", eY, eY <= tol ? "ok" : "FAIL");
    printf("  mm_bt   normwise err %.3e %s\n", eX, eX <= tol ? "ok" : "FAIL");
    printf("  mm_atb  normwise err %.3e %s\n", eW, eW <= tol ? "ok" : "FAIL");
    const int ok = eY <= tol && eX <= tol && eW <= tol;
    printf("%s\n", ok ? "PASS" : "FAIL");
    free(X); free(W); free(dY); free(Y); free(dX); free(dW); free(rY); free(rX); free(rW);
    return ok ? 0 : 1;
}
