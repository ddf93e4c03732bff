// tlg_internal.h -- shared declarations of libtlgemm.so's translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include "../../include/tlgemm.h"

// Record a HIP failure as the thread's last error and return TLG_EHIP.
int tlg_fail_hip(hipError_t e, const char *what, const char *file, int line);
int tlg_fail(int code, const char *fmt, ...);

#define TLG_HIP(call)                                                        \
    do {                                                                     \
        hipError_t e_ = (call);                                              \
        if (e_ != hipSuccess) return tlg_fail_hip(e_, #call, __FILE__, __LINE__); \
    } while (0)

// Workspace for split reductions (64 MiB of partial sums), allocated by
// tlg_init: sized for the largest split plan the launchers make on the
// BASELINE shapes; a bigger plan falls back to fewer splits.
#define TLG_WS_FLOATS ((size_t)16 << 20)

// Library state shared by the kernels' launchers (tlg_api.hip owns it).
struct TlgState {
    int initialised;
    int device;
    hipStream_t stream;        // default stream for the host-pointer entries
    float *ws;                 // split-reduction partials
    size_t ws_floats;
};
extern TlgState g_tlg;
int tlg_ensure_init(void);

// Which operand layout a GEMM launch sees (see tlg_gemm.hip).
enum TlgKind { TLG_NN = 0, TLG_NT = 1, TLG_TN = 2 };

// C[Mo x No] (beta ? += : =) sum_r A(i,r) B(r,j) on `st`, with the operand
// layouts of `kind`:
//   NN: A(i,r) = A[i*lda + r], B(r,j) = B[r*ldb + j]    (mm)
//   NT: A(i,r) = A[i*lda + r], B(r,j) = B[j*ldb + r]    (mm_bt)
//   TN: A(i,r) = A[r*lda + i], B(r,j) = B[r*ldb + j]    (mm_atb)
int tlg_gemm_launch(TlgKind kind, const float *A, const float *B, float *C,
                    int Mo, int No, int R, int lda, int ldb, int ldc, int beta,
                    hipStream_t st);
int tlg_zero_launch(float *dst, size_t n, hipStream_t st);
int tlg_describe(TlgKind kind, int Mo, int No, int R, char *buf, int len, int *splits);
int tlg_group_launch(const TlgGemmCall *calls, int n, hipStream_t st);
int tlg_group_flush_launch(hipStream_t st);
int tlg_group_drain(hipStream_t st);
int tlg_group_flush_all(void);
int tlg_group_flush_stream(hipStream_t st);
int tlg_defer_colsum(const float *part, float *C, int splits, int No, int beta, hipStream_t st);

// One GEMM over every expert of a top-1 MoE layer whose token rows are
// grouped by expert: expert e owns rows [eoff[e], eoff[e+1]) of each row
// operand (eoff: E+1 ints in device memory).  Dimensions use the labels of
// the reference's primitives with M = the expert's row count:
//   op 0 (mm):     C[rows]  = A[rows] B_e                 B_e = B + e*es
//   op 1 (mm_bt):  C[rows] (beta)= sum_s A_s[rows] B_{s,e}^T  (nseg <= 2)
//   op 2 (mm_atb): C_e (beta)= A[rows]^T B[rows]          C_e = C + e*es
// Epilogues of an expert GEMM (TlgExpertCall.epi).
enum { TLG_EPI_STORE = 0, TLG_EPI_SWIGLU = 1, TLG_EPI_SWIGLU_BWD = 2, TLG_EPI_COMBINE = 3, TLG_EPI_ROWDOT = 4 };
struct TlgExpertCall {
    int op, beta;
    float *C;
    int K, N;
    int nseg;
    const float *A[2];
    const float *B[2];
    int Nseg[2];
    long long es;
    // fused forms (zero = none): A rows through amap; NN column pair B2
    // (requires epi SWIGLU); epilogue epi with its operands
    const int *amap, *omap;
    const float *B2;
    int epi;
    float *X1, *X2;
    const float *fin, *gate;
};
// carry: TLG_ECARRY_OUT holds this launch's expert slice reductions for the
// next expert launch over the same eoff, which takes them with TLG_ECARRY_IN
// (no other launch may come between; any other workspace user runs them).
// (flags: TLG_ECARRY_INOUT takes the held ones and holds its own; held
// reductions left over run in the next tlg_group_flush_launch)
enum { TLG_ECARRY_NONE = 0, TLG_ECARRY_OUT = 1, TLG_ECARRY_IN = 2, TLG_ECARRY_INOUT = 3 };
int tlg_expert_launch(const TlgExpertCall *calls, int n, const int *eoff, int E, int rows, hipStream_t st,
                      int carry = TLG_ECARRY_NONE);

// M <= 8 forms of mm / mm_bt (tlg_gemv.hip): weight-streaming GEMV kernels.
bool tlg_gemv_fits(TlgKind kind, int Mo);
int tlg_gemv_launch(TlgKind kind, const float *A, const float *B, float *C, int Mo, int No, int R, int lda,
                    int ldb, int ldc, int beta, hipStream_t st);
int tlg_gemv_group_launch(const TlgGemmCall *calls, int n, hipStream_t st);
const char *tlg_gemv_kernel_name(int M);
void tlg_gemv_describe(TlgKind kind, int Mo, int No, int R, char *buf, int len);
int tlg_gemv_init(void);
void tlg_gemv_release(void);

// Workgroup id -> logical work item, so that consecutive logical items land
// on the same XCD (the dispatcher deals workgroups round-robin over the 8
// XCDs and each XCD has its own L2).  A bijection on [0, nb).
__device__ __forceinline__ int xcd_remap(int b, int nb)
{
    const int per = nb >> 3, rem = nb & 7;
    const int x = b & 7, slot = b >> 3;
    const int base = (x < rem) ? x * (per + 1) : rem * (per + 1) + (x - rem) * per;
    return base + slot;
}

// The reference's fast_expf (tinylm.c:3181-3191): clamp, split x log2(e) into
// integer and fraction, 2^f by its degree-5 Horner polynomial, 2^k into the
// exponent.
__device__ __forceinline__ float tlg_fast_expf(float x)
{
    x = x < -87.0f ? -87.0f : (x > 88.0f ? 88.0f : x);
    const float t = x * 1.44269504088896f;
    const float k = floorf(t), f = t - k;
    const float p = 1.0f + f * (0.6931471805f + f * (0.2402265069f + f * (0.0555041087f +
                                                                        f * (0.0096181291f + f * 0.0013333558f))));
    return p * __uint_as_float((unsigned int)(((int)k + 127) << 23));
}
