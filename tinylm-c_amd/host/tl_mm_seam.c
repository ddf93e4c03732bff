/* tl_mm_seam.c -- the -DUSE_HIP drop-in of tinylm.c's three fp32 matmul
 * primitives, with the reference's names, signatures and semantics:
 *
 *   mm      Y[M*N]  =  X[M*K] @ W[K*N]      tinylm.c:438-449
 *   mm_bt   dX[M*K] += dY[M*N] @ W[K*N]^T   tinylm.c:480-489
 *   mm_atb  dW[K*N] += X[M*K]^T @ dY[M*N]   tinylm.c:510-537
 *
 * Inside tinylm.c the same three lines go into the existing bodies, next to
 * the USE_BLAS blocks (tinylm.c:441-443, :482-484, :512-514); this file is
 * that seam as a standalone translation unit, so the drop-in can be linked
 * and tested on its own.  There is deliberately no CPU body: without the HIP
 * library the build fails instead of silently computing on the host.
 */
#ifndef USE_HIP
#error "tl_mm_seam.c is the USE_HIP path only; build with -DUSE_HIP"
#endif
#include "../../include/tlgemm.h"

void mm(float *restrict Y, const float *restrict X, const float *restrict W, int M, int K, int N)
{
    tlg_sgemm_nn(Y, X, W, M, K, N);
}

void mm_bt(float *restrict dX, const float *restrict dY, const float *restrict W, int M, int K, int N)
{
    tlg_sgemm_nt_acc(dX, dY, W, M, K, N);
}

void mm_atb(float *restrict dW, const float *restrict X, const float *restrict dY, int M, int K, int N)
{
    tlg_sgemm_tn_acc(dW, X, dY, M, K, N);
}
