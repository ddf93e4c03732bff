/* tlgemm.h -- C ABI of libtlgemm.so, the MI355X (gfx950) implementation of
 * tinylm.c's three fp32 matmul primitives.
 *
 * Plain C: pointers, ints and sizes only.  HIP streams are passed as `void *`
 * (a hipStream_t; NULL = the null stream).
 *
 * Layout contract (identical to the reference): dense row-major fp32, leading
 * dimension = row width, any M, K, N >= 0, buffers never alias (the reference
 * marks every pointer `restrict`).  `mm` overwrites its output (beta = 0);
 * `mm_bt` and `mm_atb` add into theirs (beta = 1), exactly once per call.
 */
#ifndef TLGEMM_H
#define TLGEMM_H
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

/* Status codes of the int-returning entry points. */
#define TLG_OK       0
#define TLG_EINVAL  -1   /* bad argument (negative dimension, NULL pointer)  */
#define TLG_EHIP    -2   /* HIP runtime error; tlg_last_error() has the text */
#define TLG_ENOMEM  -3   /* device allocation failed                         */
#define TLG_ESTATE  -4   /* library not initialised / registry conflict      */

/* ---- lifetime ---------------------------------------------------------- */
/* Select `device`, create the library's default stream and workspace.  Safe
 * to call more than once.  No reference counterpart: tinylm.c needs no set-up
 * for its CPU kernels; the -DUSE_HIP seam calls this lazily. */
int  tlg_init(int device);
/* Free the workspace, every registered mirror and the default stream. */
void tlg_shutdown(void);
/* Text of the most recent error on this thread ("" if none). */
const char *tlg_last_error(void);

/* ---- drop-in, host pointers, synchronous ------------------------------- */
/* These keep the reference's signatures and its error behaviour (no status:
 * a failure prints the HIP error with file:line and aborts, where tinylm.c
 * exits on fatal errors, tinylm.c:137).  Operands that lie inside a range
 * given to tlg_register() are used in place on the device; all others are
 * copied in (and the output copied back) within the call.  The call returns
 * once the result is in host memory (or in the registered mirror). */

/* Y[M*N] = X[M*K] @ W[K*N]  (set).  Replaces mm(), tinylm.c:438-449. */
void tlg_sgemm_nn(float *Y, const float *X, const float *W, int M, int K, int N);
/* dX[M*K] += dY[M*N] @ W[K*N]^T  (accumulate).  Replaces mm_bt(), tinylm.c:480-489. */
void tlg_sgemm_nt_acc(float *dX, const float *dY, const float *W, int M, int K, int N);
/* dW[K*N] += X[M*K]^T @ dY[M*N]  (accumulate).  Replaces mm_atb(), tinylm.c:510-537. */
void tlg_sgemm_tn_acc(float *dW, const float *X, const float *dY, int M, int K, int N);

/* ---- host-buffer mirrors (device residency for long-lived buffers) ------ */
/* Give [host, host+bytes) a device mirror, initialised from host memory.
 * Intended for the flat parameter and gradient buffers (tinylm.c:2739-2740)
 * and any activation the caller keeps on the device.  Ranges must not
 * overlap.  No reference counterpart (the reference is host-only). */
int tlg_register(void *host, size_t bytes);
int tlg_unregister(void *host);
/* Copy host -> mirror (e.g. after the optimizer step) / mirror -> host (e.g.
 * gradients before the grad-norm).  `host` is the registered base pointer. */
int tlg_push(void *host);
int tlg_pull(void *host);
/* Device address that mirrors `host` (which may point inside a range), or
 * NULL if it is not registered. */
void *tlg_mirror(const void *host);

/* ---- device pointers, asynchronous on `stream` -------------------------- */
/* Same arithmetic as the drop-in entries on device-resident buffers; returns
 * TLG_OK once the kernels are enqueued.  These are what a device-resident
 * caller (the step drivers in tinylm-c_amd/host) uses. */
int tlg_dev_sgemm_nn(float *Y, const float *X, const float *W, int M, int K, int N, void *stream);
int tlg_dev_sgemm_nt_acc(float *dX, const float *dY, const float *W, int M, int K, int N, void *stream);
int tlg_dev_sgemm_tn_acc(float *dW, const float *X, const float *dY, int M, int K, int N, void *stream);
/* tlg_dev_sgemm_tn_acc without any device allocation.  No counterpart in the
 * reference: this is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arithmetic and kernels; the split-reduction partials go
 * to a fixed 16 MiB device array of the library (one per GPU, held until the
 * process ends) instead of the workspace tlg_init allocates, and the call
 * does not initialise the library.  Limit: K * N <= 2^21 floats (an 8 MiB
 * dW), else TLG_EINVAL; the split count is capped to what the array holds.
 * Calls that overlap on one GPU (two streams, two threads) share that array
 * and race; serialise them. */
int tlg_dev_sgemm_tn_acc_noalloc(float *dW, const float *X, const float *dY, int M, int K, int N, void *stream);
/* dst[0..n) = 0 on `stream`, by a fill kernel (never a memset node, so a
 * captured graph replays it correctly).  The reference's memset() before an
 * accumulating GEMM, e.g. tinylm.c:1015, :1104, :1113, :1123, :1134. */
int tlg_dev_zero(float *dst, size_t n, void *stream);

/* ---- grouped launches (device pointers, asynchronous) -------------------
 * The GEMMs a caller issues back to back with no other work in between --
 * e.g. the Q, K and V projections of one layer (tinylm.c:981-983), or the
 * dnorm chain and the Q/K/V weight gradients (tinylm.c:1135-1141) -- run as
 * one kernel launch.  No reference counterpart: this is what the device step
 * executor (tinylm-c_amd/host/tl_exec.c) uses to cut per-kernel overhead.
 *
 * A call is one primitive with the reference's arguments, or for mm_bt a
 * chain of up to 3 primitives accumulating into the same dX:
 *   dX (beta ? += : =) sum_s dY_s[M x N_s] @ W_s[K x N_s]^T
 * (N_0 = N).  beta = 0 turns "memset(C); mm_bt(C, ...)" into one call.
 * mm always sets.  op 3 clears C[0, M*N) (K, nseg and the operands are
 * ignored), so a memset can ride along with the GEMMs of a launch.  The calls
 * of one group must be independent (no call reads or writes what another
 * writes).  All operands must be 16-byte aligned with row widths that are
 * multiples of 4 (TLG_EINVAL otherwise).  When every call is an mm or mm_bt
 * with M <= 8 the group runs on the GEMV kernels instead.
 *
 * mm_atb calls with long reductions split them across workgroups; their
 * partial sums are added into C by the NEXT grouped launch on the stream
 * (the kernel boundary makes them visible) or by tlg_dev_gemm_flush, which
 * must be called before C is read.  Any single-call entry point flushes
 * first.  A launch on another stream first runs the queued sums on the
 * stream that wrote their partials (ordered after their producer); the
 * caller orders its consumers of C after that stream, as for any result. */
typedef struct {
    int op;                  /* 0 mm, 1 mm_bt, 2 mm_atb, 3 clear C[0, M*N) */
    int beta;                /* mm_bt / mm_atb: 1 add into C, 0 overwrite C */
    float *C;                /* Y, dX or dW */
    int M, K, N;             /* the primitive's arguments (N = N_0) */
    int nseg;                /* 1, or 2..3 for an mm_bt chain */
    const float *A[3];       /* X / dY_s / X  (first operand of segment s) */
    const float *B[3];       /* W / W_s  / dY (second operand of segment s) */
    int Nseg[3];             /* N_s for s >= 1 (mm_bt chains) */
    const float *R;          /* mm only, optional: C = R + X W, the residual add
                              * that follows mm in the reference (tinylm.c:994-995,
                              * :1009-1010) fused into the store; R [M x N] is
                              * read, not written, and may not alias C */
    /* mm_bt with beta 0 only, optional (both or neither): dotOut[i][b] =
     * sum_{c < 32} dX[i][32 b + c] dotB[i][32 b + c] for every 32-column block
     * b of dX (K % 32 == 0; dotB [M x K] 16-byte aligned, not C; dotOut
     * [M x K/32]), each a 16-term fma chain over c < 16, another over c >= 16,
     * then their sum.  The attention backward's D = dO . O per row and head
     * (tinylm.c:750-768) made in the O-projection backward that forms dO (no
     * counterpart). */
    const float *dotB;
    float *dotOut;
} TlgGemmCall;
int tlg_dev_gemm_group(const TlgGemmCall *calls, int n, void *stream);

/* The dense SwiGLU FFN's GEMMs with their elementwise neighbours fused (no
 * single reference counterpart).  swiglu_mm replaces mm(g, X, W1), mm(u, X,
 * W3) and act = silu(g) u (tinylm.c:1002-1006): X [M x K], W1 / W3 [K x N],
 * act [M x N]; g and u (may be NULL) receive the two products.  It is also
 * the backward's recompute of act (:1098-1100) when act is kept.
 * mm_bt_swiglu_bwd replaces memset(dact), mm_bt(dact, dY, W2, M, K, N) and
 * the SwiGLU backward (:1102-1109): dact = dY W2^T (dY [M x N], W2 [K x N]),
 * then in place g <- dact u silu'(g) (dg) and u <- dact silu(g) (du), g / u
 * [M x K].  Both flush or carry the pending split reductions of grouped
 * launches like any grouped launch. */
int tlg_dev_swiglu_mm(const float *X, const float *W1, const float *W3, float *act, float *g, float *u, int M, int K,
                      int N, void *stream);
int tlg_dev_mm_bt_swiglu_bwd(const float *dY, const float *W2, float *g, float *u, int M, int K, int N,
                             void *stream);
int tlg_dev_gemm_flush(void *stream);
/* Number of split reductions still pending (what a flush would launch),
 * the MoE backward's held expert reductions included. */
int tlg_dev_gemm_pending(void);
/* Kernel instance grouped launches use, as rocprofv3 names it. */
const char *tlg_group_kernel(void);
/* 1 if an M <= 8 launch (the GEMV kernels behind mm / mm_bt at M <= 8 and
 * tlg_dev_dec_gemv) ever timed out waiting for its split partial sums (its
 * outputs were then written as NaN), 0 if none did, -1 if the flag cannot be
 * read.  Synchronous.  No reference counterpart: a diagnostic of this
 * library's split reduction. */
int tlg_gemv_status(void);
/* Tuning hook: pin the tile configuration of grouped launches (an index of
 * the kernel's tile table; -1 = automatic: 64x64 tiles when a launch has at
 * least 3 x 256 of them, else 64x32 tiles whose wave pairs split each stage). */
int tlg_tune_group(int cfg);
/* Tuning hook: the automatic policy itself -- candidate tile configs (up to
 * 3, first that yields min_waves x 256 work items wins, else the last; ncands
 * 0 keeps the list), min_waves (<= 0 keeps it) and the target reduction
 * steps per split work item (0 keeps it).  Applies to later launches. */
int tlg_tune_group_policy(const int *cands, int ncands, double min_waves, int rtarget);
/* Tuning hook: pin the target reduction steps per work item of the split
 * (mm_atb) problems of later grouped launches: >= 64 splits every long
 * reduction into pieces of about that many steps; 0 restores the automatic
 * target (the launch's longest unsplit reduction, at least the policy's).
 * The split partials are summed in split order either way. */
int tlg_tune_group_split(int rtarget);
/* Tuning hook: the tile shape of the MoE expert launches (tlg_dev_moe_*):
 * cfg -1 = automatic (64x64 tiles of 16-step stages when a launch has about
 * 3 x 256 of them, else 64x32, else 32x32), or 3 (64x64), 18 (64x64, 16-step
 * stages), 14 (64x32), 15 (32x32), 22 (16-wave 64x64, whose waves split each
 * 64-step stage four ways) pinned;
 * sched 1 = each stage's fragment reads issued before its MFMAs, 2 = that
 * order with the outputs written by streaming stores, 0 = the compiler's
 * order, -1 = automatic (2 for the fused SwiGLU launches of dense rows, 1 for
 * MoE launches).  Applies to later launches. */
int tlg_tune_expert(int cfg, int sched);

/* ---- top-1 mixture-of-experts FFN --------------------------------------- */
/* The MoE layer of tinylm.c with K = 1 routing and no router bias (the
 * training default): N tokens of width D, E experts (1..64) of hidden width
 * F.  Weights as the reference stores them per layer: wr [D*E], w1 and w3
 * E x [D*F], w2 E x [F*D] (Weights.wr/w1/w3/w2 of one layer).  D and F must
 * be multiples of 4 and the float operands 16-byte aligned (wr, gwr excepted).
 *
 * Forward, replaces moe_forward (tinylm.c:857-891): router logits fnorm.wr,
 * softmax over all E into rprobs[N*E], top-1 expert assign[N] (strict-greater
 * argmax, ties to the lowest index, tinylm.c:814-827) with gate[N] =
 * rprobs[n][assign[n]], and out[n] = fin[n] + gate[n] * W2_e(silu(W1_e x) *
 * W3_e x) with x = fnorm[n].
 * Backward, replaces moe_backward (tinylm.c:895-947): from dout[N*D] and the
 * forward's assign/gate/rprobs, sets d_fnorm[N*D] and adds into gwr, gw1,
 * gw3, gw2 (expert GEMM grads, the router's softmax backward with the
 * 0.01 * E * (cnt_e / N) / N load-balance term, dWr).
 * Device-pointer forms enqueue on `stream` (asynchronous; scratch kept by the
 * library, grown on demand -- growing synchronizes the device, and calls on
 * different streams must not overlap).  Host-pointer forms are synchronous and abort on
 * error like the GEMM drop-ins; operands inside a registered range are used
 * in place. */
int  tlg_dev_moe_grouped_fwd(const float *fnorm, const float *fin, float *out, int N, int D, int F, int E,
                             const float *wr, const float *w1, const float *w3, const float *w2,
                             int *assign, float *gate, float *rprobs, void *stream);
int  tlg_dev_moe_grouped_bwd(const float *fnorm, const float *dout, float *d_fnorm, const int *assign,
                             const float *gate, const float *rprobs, int N, int D, int F, int E,
                             const float *wr, const float *w1, const float *w3, const float *w2,
                             float *gwr, float *gw1, float *gw3, float *gw2, void *stream);
/* Kept-state pair: no counterpart in the reference, whose moe_backward
 * recomputes the expert forward from fnorm (tinylm.c:906-914).  The forward
 * also stores, in a caller buffer of tlg_moe_keep_bytes(N, D, F, E) bytes
 * (16-byte aligned), the expert row index and the expert rows g, u, a and y
 * it computes anyway; the backward reads them instead of rebuilding the index
 * and recomputing W1 | W3 and W2 (3 of its launches), with the same results
 * bit for bit.  The backward overwrites g and u (they become dg and du), so
 * one kept state serves one backward, and its last summations (the router
 * gradient's column sum and the expert W1 / W3 gradients' slice sums) are
 * deferred like a split GEMM's reduction: gwr, gw1 and gw3 are complete after
 * the next grouped or expert launch on the stream, or tlg_dev_gemm_flush,
 * which runs them in one launch (gwr at return when it is not 16-byte
 * aligned).  For training steps
 * that can hold N (3F + D) floats per MoE layer until the backward. */
size_t tlg_moe_keep_bytes(int N, int D, int F, int E);   /* 0 for a bad shape */
int  tlg_dev_moe_grouped_fwd_keep(const float *fnorm, const float *fin, float *out, int N, int D, int F, int E,
                                  const float *wr, const float *w1, const float *w3, const float *w2,
                                  int *assign, float *gate, float *rprobs, void *keep, size_t keep_bytes,
                                  void *stream);
int  tlg_dev_moe_grouped_bwd_kept(const float *fnorm, const float *dout, float *d_fnorm, const int *assign,
                                  const float *gate, const float *rprobs, int N, int D, int F, int E,
                                  const float *wr, const float *w1, const float *w3, const float *w2,
                                  float *gwr, float *gw1, float *gw3, float *gw2, void *kept,
                                  size_t kept_bytes, void *stream);
void tlg_moe_grouped_fwd(const float *fnorm, const float *fin, float *out, int N, int D, int F, int E,
                         const float *wr, const float *w1, const float *w3, const float *w2,
                         int *assign, float *gate, float *rprobs);
void tlg_moe_grouped_bwd(const float *fnorm, const float *dout, float *d_fnorm, const int *assign,
                         const float *gate, const float *rprobs, int N, int D, int F, int E,
                         const float *wr, const float *w1, const float *w3, const float *w2,
                         float *gwr, float *gw1, float *gw3, float *gw2);

/* ---- runtime wrappers for C host code ---------------------------------- */
/* So the C step drivers (tinylm-c_amd/host) keep buffers and timing on the
 * device without including HIP headers.  No reference counterpart. */
void *tlg_dev_malloc(size_t bytes);                       /* NULL on failure */
/* Launches every queued reduction first (each on the stream its partials
 * were written on: they may read or write p), then frees p; hipFree waits for
 * the device.  Memory from another allocator must not be released while a
 * reduction queued by a grouped, expert or MoE launch may still touch it:
 * call tlg_dev_gemm_flush on that stream first. */
int   tlg_dev_free(void *p);
int   tlg_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream);
int   tlg_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream);
int   tlg_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream);
void *tlg_stream_create(void);                            /* default priority */
int   tlg_stream_destroy(void *stream);                   /* runs reductions queued on it first */
int   tlg_stream_sync(void *stream);
void *tlg_event_create(void);
int   tlg_event_destroy(void *ev);
int   tlg_event_record(void *ev, void *stream);
float tlg_event_elapsed_ms(void *start, void *stop);      /* < 0 on error */
/* dst[i] = scale * z_i, z_i ~ N(0,1) from a counter-based generator keyed by
 * (seed, i): splitmix64 -> two uniforms -> Box-Muller.  Deterministic for a
 * given (seed, n), independent of launch shape. */
int   tlg_dev_fill_normal(float *dst, size_t n, unsigned long long seed, float scale, void *stream);
/* Which kernel instance a device call of the primitive `op` (0 mm, 1 mm_bt,
 * 2 mm_atb) with reference arguments (M, K, N) and aligned operands launches,
 * written to buf as rocprofv3 names it (e.g. "k_gemm<64, 64, 32, 2, 1, true>"),
 * and how many workgroups share each output tile's reduction (*splits). */
int   tlg_kernel_name(int op, int M, int K, int N, char *buf, int len, int *splits);
/* Tuning hook: force tile configuration `cfg` (index into the kernel's tile
 * table, -1 = automatic choice) and `splits` reduction splits for every
 * following GEMM launch.  For sweeps only; results stay exact either way. */
int   tlg_tune_force(int cfg, int splits);
/* Measurement probes (no reference counterpart).  tlg_dev_copy: dst = src,
 * n floats (n % 4 == 0, 16-byte aligned) -- achievable HBM bandwidth and the
 * calibration kernel for HBM byte counters.  tlg_dev_mfma_peak: `blocks`
 * workgroups of 4 waves each issue 4*iters register-only fp32 MFMAs
 * (32x32x2, 4096 flop each) and write blocks*256 floats to out. */
int   tlg_dev_copy(float *dst, const float *src, size_t n, void *stream);
/* Achievable HBM read bandwidth: streams n floats of src (n % 4 == 0,
 * 16-byte aligned) and writes nothing but, in a case no finite input
 * reaches, sink[0]. */
int   tlg_dev_read(const float *src, size_t n, float *sink, void *stream);
int   tlg_dev_mfma_peak(float *out, int blocks, int iters, void *stream);
/* Stream capture into a HIP graph: begin, enqueue work, end -> executable
 * graph handle; replay with tlg_graph_launch. */
int   tlg_graph_begin(void *stream);
void *tlg_graph_end(void *stream);
int   tlg_graph_launch(void *graph, void *stream);
int   tlg_graph_destroy(void *graph);

#ifdef __cplusplus
}
#endif
#endif
