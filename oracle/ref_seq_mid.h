
/* ref_seq_mid.h -- inserted by oracle/Makefile between tinylm.c:537 (end of
 * the three primitives) and tinylm.c:539 (start of the model code), when the
 * reference's forward/backward are compiled from their own lines.
 * TEST INFRASTRUCTURE ONLY: every mm / mm_bt / mm_atb call site after this
 * point is routed through a logger that records the call (operation, the
 * three pointers, M, K, N) and then runs the reference primitive itself. */
typedef struct { int op; const float *o, *a, *b; int M, K, N; } TlrefCall;
static TlrefCall *tlref_calls;
static int tlref_ncalls, tlref_capcalls;
static void tlref_log(int op, const float *o, const float *a, const float *b, int M, int K, int N)
{
    if (tlref_ncalls == tlref_capcalls) {
        tlref_capcalls = tlref_capcalls ? 2 * tlref_capcalls : 256;
        tlref_calls = realloc(tlref_calls, sizeof(TlrefCall) * (size_t)tlref_capcalls);
    }
    TlrefCall c = {op, o, a, b, M, K, N};
    tlref_calls[tlref_ncalls++] = c;
}
static void tlref_log_mm(float *restrict Y, const float *restrict X, const float *restrict W, int M, int K, int N)
{ tlref_log(0, Y, X, W, M, K, N); mm(Y, X, W, M, K, N); }
static void tlref_log_mm_bt(float *restrict dX, const float *restrict dY, const float *restrict W, int M, int K, int N)
{ tlref_log(1, dX, dY, W, M, K, N); mm_bt(dX, dY, W, M, K, N); }
static void tlref_log_mm_atb(float *restrict dW, const float *restrict X, const float *restrict dY, int M, int K, int N)
{ tlref_log(2, dW, X, dY, M, K, N); mm_atb(dW, X, dY, M, K, N); }
#define mm tlref_log_mm
#define mm_bt tlref_log_mm_bt
#define mm_atb tlref_log_mm_atb
