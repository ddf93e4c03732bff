/* tl_oracle.h -- CPU oracle for the fp32 GEMM hot path of tinylm.c.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links this: only tests/,
 * __graft_entry__.smoke() (as the checker) and bench.py's cpu_baseline leg
 * load it.  It restates, from scratch, the arithmetic of the reference's
 * portable kernels so that a GPU result can be compared with what tinylm.c
 * computes on identical inputs.
 *
 * Pinning (how each function is checked, so a dropped term / wrong index /
 * transposed operand fails somewhere):
 *   orc_mm, orc_mm_bt, orc_mm_atb   golden fixtures written by the reference's
 *                                   own compiled kernels (tests/golden), the
 *                                   fp64 textbook loops below, and invariants
 *                                   (set vs accumulate, identity W, linearity).
 *   orc_*_f64                       closed-form textbook GEMM in double; checked
 *                                   against exact small-integer cases and brute
 *                                   force in tests/test_oracle.py.
 *   orc_rng_*                       the reference's xorshift/Box-Muller draw,
 *                                   pinned by the fixtures' stored inputs.
 *   orc_moe_*                       brute-force per-token expert evaluation in
 *                                   fp64 (tests/test_oracle.py) and the reference
 *                                   MoE compiled from its own source (fixtures).
 */
#ifndef TL_ORACLE_H
#define TL_ORACLE_H
#include <stdint.h>
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- the three primitives, same argument meaning as tinylm.c ---------- */
/* Y[M*N]  = X[M*K] @ W[K*N]          (set)         tinylm.c:438-478 */
void orc_mm(float *Y, const float *X, const float *W, int M, int K, int N);
/* dX[M*K] += dY[M*N] @ W[K*N]^T      (accumulate)  tinylm.c:480-508 */
void orc_mm_bt(float *dX, const float *dY, const float *W, int M, int K, int N);
/* dW[K*N] += X[M*K]^T @ dY[M*N]      (accumulate)  tinylm.c:510-537 */
void orc_mm_atb(float *dW, const float *X, const float *dY, int M, int K, int N);

/* Decode-pool dispatch emulation (tinylm.c:237-245, :446, :486).  nt<=1 is
 * the training setting (OpenMP), nt>1 emulates a live tl_for pool of nt
 * workers: ranges of fewer than nt items run serially on the caller. */
void orc_set_pool(int nt);
int  orc_threads(void);            /* OpenMP threads the oracle will use */
void orc_set_threads(int nt);      /* omp_set_num_threads */

/* ---- fp64 textbook references (the selftest pattern, tinylm.c:4764-4766),
 * extended with the accumulator prefill that mm_bt / mm_atb add into. ---- */
void orc_mm_f64(float *Y, const float *X, const float *W, int M, int K, int N);
void orc_mm_bt_f64(float *dX, const float *dY, const float *W, int M, int K, int N);
void orc_mm_atb_f64(float *dW, const float *X, const float *dY, int M, int K, int N);

/* ---- RNG: xorshift64 (13,7,17) + Box-Muller, tinylm.c:127-134 ---------- */
void     orc_rng_seed(uint64_t s);
uint64_t orc_rng_state(void);
uint64_t orc_xorshift(void);
float    orc_rnd_normal(void);
void     orc_fill_normal(float *p, size_t n, float scale);

/* ---- top-1 MoE (tinylm.c:814-827, :857-947), K=1 routing, no router bias.
 * fnorm[N*D], fin[N*D] -> out[N*D]; assign[N], gate[N], rprobs[N*E] written.
 * w1,w3: E x [D*F], w2: E x [F*D], wr: [D*E]; scratch handled internally. */
void orc_moe_forward(int N, int D, int F, int E,
                     const float *fnorm, const float *fin, float *out,
                     const float *wr, const float *w1, const float *w3, const float *w2,
                     int *assign, float *gate, float *rprobs);
/* dout[N*D] -> d_fnorm[N*D] (set); gw1/gw3/gw2/gwr accumulate. */
void orc_moe_backward(int N, int D, int F, int E,
                      const float *fnorm, const float *dout, float *d_fnorm,
                      const float *wr, const float *w1, const float *w3, const float *w2,
                      float *gwr, float *gw1, float *gw3, float *gw2,
                      const int *assign, const float *gate, const float *rprobs);

/* A plan's call list run in C (CPU baseline of short calls): op 0 mm,
 * 1 mm_bt, 2 mm_atb, 3 memset of n floats; `reps` passes over the list. */
typedef struct { int op; float *out; const float *a, *b; int M, K, N; size_t n; } OrcCall;
void orc_run_calls(const OrcCall *c, int n, int reps);

#ifdef __cplusplus
}
#endif
#endif
