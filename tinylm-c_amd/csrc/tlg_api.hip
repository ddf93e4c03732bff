// tlg_api.hip -- the C ABI of libtlgemm.so (declared in include/tlgemm.h):
// lifetime, error text, host-buffer mirrors, the synchronous host-pointer
// drop-ins for mm / mm_bt / mm_atb and their asynchronous device twins.
#include "tlg_internal.h"
#include <mutex>
#include <vector>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

TlgState g_tlg = {0, 0, nullptr, nullptr, 0};

static thread_local char t_err[512];
static std::recursive_mutex g_mu;


int tlg_fail(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err, sizeof t_err, fmt, ap);
    va_end(ap);
    return code;
}

int tlg_fail_hip(hipError_t e, const char *what, const char *file, int line)
{
    return tlg_fail(TLG_EHIP, "%s:%d: %s failed: %s", file, line, what, hipGetErrorString(e));
}

extern "C" const char *tlg_last_error(void) { return t_err; }

static int init_locked(int device)
{
    if (g_tlg.initialised) return TLG_OK;
    int n = 0;
    TLG_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return tlg_fail(TLG_EINVAL, "tlg_init: device %d of %d", device, n);
    TLG_HIP(hipSetDevice(device));
    TLG_HIP(hipStreamCreateWithFlags(&g_tlg.stream, hipStreamNonBlocking));
    void *p = nullptr;
    if (hipMalloc(&p, TLG_WS_FLOATS * sizeof(float)) != hipSuccess)
        return tlg_fail(TLG_ENOMEM, "tlg_init: workspace of %zu bytes", TLG_WS_FLOATS * sizeof(float));
    g_tlg.ws = (float *)p;
    g_tlg.ws_floats = TLG_WS_FLOATS;
    int rc = tlg_gemv_init();
    if (rc) return rc;
    TLG_HIP(hipDeviceSynchronize());
    g_tlg.device = device;
    g_tlg.initialised = 1;
    return TLG_OK;
}

extern "C" int tlg_init(int device)
{
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    return init_locked(device);
}

int tlg_ensure_init(void)
{
    if (g_tlg.initialised) return TLG_OK;
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    return init_locked(0);
}

// ------------------------------------------------------------- mirrors --
struct Mirror { char *host; size_t bytes; char *dev; };
static std::vector<Mirror> g_mirrors;

static Mirror *find_mirror(const void *p, size_t need)
{
    const char *c = (const char *)p;
    for (auto &m : g_mirrors)
        if (c >= m.host && c < m.host + m.bytes) {
            if (c + need > m.host + m.bytes) return nullptr;
            return &m;
        }
    return nullptr;
}

extern "C" int tlg_register(void *host, size_t bytes)
{
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = init_locked(g_tlg.initialised ? g_tlg.device : 0);
    if (rc) return rc;
    if (!host || bytes == 0) return tlg_fail(TLG_EINVAL, "tlg_register: empty range");
    const char *h = (const char *)host;
    for (auto &m : g_mirrors)
        if (h < m.host + m.bytes && m.host < h + bytes)
            return tlg_fail(TLG_ESTATE, "tlg_register: range overlaps a registered range");
    void *d = nullptr;
    if (hipMalloc(&d, bytes) != hipSuccess) return tlg_fail(TLG_ENOMEM, "tlg_register: %zu bytes", bytes);
    hipError_t e = hipMemcpy(d, host, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) { (void)hipFree(d); return tlg_fail_hip(e, "hipMemcpy", __FILE__, __LINE__); }
    g_mirrors.push_back({(char *)host, bytes, (char *)d});
    return TLG_OK;
}

extern "C" int tlg_unregister(void *host)
{
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    for (size_t i = 0; i < g_mirrors.size(); i++)
        if (g_mirrors[i].host == (char *)host) {
            TLG_HIP(hipDeviceSynchronize());
            TLG_HIP(hipFree(g_mirrors[i].dev));
            g_mirrors.erase(g_mirrors.begin() + i);
            return TLG_OK;
        }
    return tlg_fail(TLG_ESTATE, "tlg_unregister: %p is not a registered base", host);
}

static int copy_mirror(void *host, bool to_dev)
{
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    for (auto &m : g_mirrors)
        if (m.host == (char *)host) {
            TLG_HIP(hipStreamSynchronize(g_tlg.stream));
            if (to_dev) TLG_HIP(hipMemcpy(m.dev, m.host, m.bytes, hipMemcpyHostToDevice));
            else        TLG_HIP(hipMemcpy(m.host, m.dev, m.bytes, hipMemcpyDeviceToHost));
            return TLG_OK;
        }
    return tlg_fail(TLG_ESTATE, "%p is not a registered base", host);
}

extern "C" int tlg_push(void *host) { return copy_mirror(host, true); }
extern "C" int tlg_pull(void *host) { return copy_mirror(host, false); }

extern "C" void *tlg_mirror(const void *host)
{
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    Mirror *m = find_mirror(host, 1);
    return m ? m->dev + ((const char *)host - m->host) : nullptr;
}

void tlg_shutdown_impl(void);
extern "C" void tlg_shutdown(void)
{
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    if (!g_tlg.initialised) return;
    (void)hipDeviceSynchronize();
    (void)tlg_group_drain(g_tlg.stream);       // queued reductions read the workspace
    (void)hipDeviceSynchronize();
    for (auto &m : g_mirrors) (void)hipFree(m.dev);
    g_mirrors.clear();
    tlg_shutdown_impl();
    (void)hipFree(g_tlg.ws);
    (void)hipStreamDestroy(g_tlg.stream);
    g_tlg = TlgState{0, 0, nullptr, nullptr, 0};
}

// ------------------------------------------------ host-pointer drop-ins --
// Staging buffers for operands that are not registered: grown on demand,
// kept for the life of the library.
struct Stage { void *p = nullptr; size_t bytes = 0; };
static Stage g_stage[16];

void tlg_moe_release(void);
void tlg_train_release(void);
void tlg_shutdown_impl(void)
{
    for (auto &s : g_stage) { (void)hipFree(s.p); s = Stage(); }
    tlg_moe_release();
    tlg_train_release();
    tlg_gemv_release();
}

static int stage_ptr(int slot, size_t bytes, void **out)
{
    Stage &s = g_stage[slot];
    if (s.bytes < bytes) {
        if (s.p) TLG_HIP(hipFree(s.p));
        s.p = nullptr; s.bytes = 0;
        if (hipMalloc(&s.p, bytes) != hipSuccess) return tlg_fail(TLG_ENOMEM, "staging %zu bytes", bytes);
        s.bytes = bytes;
    }
    *out = s.p;
    return TLG_OK;
}

// Device address for a host operand of `bytes`: the mirror when registered,
// else a staging slot (filled from the host when `upload`).
static int resolve(int slot, const void *host, size_t bytes, bool upload, void **dev, bool *mirrored)
{
    Mirror *m = find_mirror(host, bytes);
    if (m) { *dev = m->dev + ((const char *)host - m->host); *mirrored = true; return TLG_OK; }
    for (auto &mm : g_mirrors) {
        const char *c = (const char *)host;
        if (c >= mm.host && c < mm.host + mm.bytes)
            return tlg_fail(TLG_ESTATE, "operand runs past the end of its registered range");
    }
    *mirrored = false;
    int rc = stage_ptr(slot, bytes, dev);
    if (rc) return rc;
    if (upload) TLG_HIP(hipMemcpyAsync(*dev, host, bytes, hipMemcpyHostToDevice, g_tlg.stream));
    return TLG_OK;
}

// out[o_rows x o_cols] (beta) <- kind(A, B); A is a_elems floats, B b_elems.
static int host_gemm(TlgKind kind, float *out, const float *A, const float *B,
                     int M, int K, int N)
{
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = init_locked(g_tlg.initialised ? g_tlg.device : 0);
    if (rc) return rc;
    if (M < 0 || K < 0 || N < 0) return tlg_fail(TLG_EINVAL, "negative dimension");
    size_t nA, nB, nC;
    int Mo, No, R, lda, ldb, beta;
    switch (kind) {
    case TLG_NN: nA = (size_t)M * K; nB = (size_t)K * N; nC = (size_t)M * N;
                 Mo = M; No = N; R = K; lda = K; ldb = N; beta = 0; break;
    case TLG_NT: nA = (size_t)M * N; nB = (size_t)K * N; nC = (size_t)M * K;
                 Mo = M; No = K; R = N; lda = N; ldb = N; beta = 1; break;
    default:     nA = (size_t)M * K; nB = (size_t)M * N; nC = (size_t)K * N;
                 Mo = K; No = N; R = M; lda = K; ldb = N; beta = 1; break;
    }
    if (nC == 0) return TLG_OK;
    void *dA = nullptr, *dB = nullptr, *dC = nullptr;
    bool mA = false, mB = false, mC = false;
    if (nA) { rc = resolve(0, A, nA * 4, true, &dA, &mA); if (rc) return rc; }
    if (nB) { rc = resolve(1, B, nB * 4, true, &dB, &mB); if (rc) return rc; }
    rc = resolve(2, out, nC * 4, beta != 0, &dC, &mC);
    if (rc) return rc;
    rc = tlg_gemm_launch(kind, (const float *)dA, (const float *)dB, (float *)dC,
                         Mo, No, R, lda, ldb, No, beta, g_tlg.stream);
    if (rc) return rc;
    if (!mC) TLG_HIP(hipMemcpyAsync(out, dC, nC * 4, hipMemcpyDeviceToHost, g_tlg.stream));
    TLG_HIP(hipStreamSynchronize(g_tlg.stream));
    return TLG_OK;
}

// The reference's primitives return nothing and exit on fatal errors
// (tinylm.c:137); the drop-ins abort with the error text instead of
// returning wrong data.
static void die_on(int rc, const char *who)
{
    if (rc == TLG_OK) return;
    fprintf(stderr, "[tlgemm] %s: %s\n", who, t_err);
    fflush(stderr);
    abort();
}

extern "C" void tlg_sgemm_nn(float *Y, const float *X, const float *W, int M, int K, int N)
{ die_on(host_gemm(TLG_NN, Y, X, W, M, K, N), "tlg_sgemm_nn"); }
extern "C" void tlg_sgemm_nt_acc(float *dX, const float *dY, const float *W, int M, int K, int N)
{ die_on(host_gemm(TLG_NT, dX, dY, W, M, K, N), "tlg_sgemm_nt_acc"); }
extern "C" void tlg_sgemm_tn_acc(float *dW, const float *X, const float *dY, int M, int K, int N)
{ die_on(host_gemm(TLG_TN, dW, X, dY, M, K, N), "tlg_sgemm_tn_acc"); }

// ----------------------------------------------------- device twins --
extern "C" int tlg_dev_sgemm_nn(float *Y, const float *X, const float *W, int M, int K, int N, void *stream)
{
    if (M < 0 || K < 0 || N < 0) return tlg_fail(TLG_EINVAL, "negative dimension");
    return tlg_gemm_launch(TLG_NN, X, W, Y, M, N, K, K, N, N, 0, (hipStream_t)stream);
}
extern "C" int tlg_dev_sgemm_nt_acc(float *dX, const float *dY, const float *W, int M, int K, int N, void *stream)
{
    if (M < 0 || K < 0 || N < 0) return tlg_fail(TLG_EINVAL, "negative dimension");
    return tlg_gemm_launch(TLG_NT, dY, W, dX, M, K, N, N, N, K, 1, (hipStream_t)stream);
}
extern "C" int tlg_dev_sgemm_tn_acc(float *dW, const float *X, const float *dY, int M, int K, int N, void *stream)
{
    if (M < 0 || K < 0 || N < 0) return tlg_fail(TLG_EINVAL, "negative dimension");
    return tlg_gemm_launch(TLG_TN, X, dY, dW, K, N, M, K, N, N, 1, (hipStream_t)stream);
}
extern "C" int tlg_dev_zero(float *dst, size_t n, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    return tlg_zero_launch(dst, n, (hipStream_t)stream);
}

// ---------------------------------------------------- runtime wrappers --
extern "C" void *tlg_dev_malloc(size_t bytes)
{
    if (tlg_ensure_init()) return nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) {
        tlg_fail(TLG_ENOMEM, "tlg_dev_malloc: %zu bytes", bytes);
        return nullptr;
    }
    return p;
}
// Queued split reductions (and held expert ones) may read or write p: they
// are launched first, and hipFree waits for the device before releasing it.
extern "C" int tlg_dev_free(void *p)
{
    if (g_tlg.initialised) {
        const int rc = tlg_group_flush_all();
        if (rc) return rc;
    }
    TLG_HIP(hipFree(p));
    return TLG_OK;
}
extern "C" int tlg_memcpy_h2d(void *dst, const void *src, size_t bytes, void *stream)
{ TLG_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream)); return TLG_OK; }
extern "C" int tlg_memcpy_d2h(void *dst, const void *src, size_t bytes, void *stream)
{ TLG_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream)); return TLG_OK; }
extern "C" int tlg_memcpy_d2d(void *dst, const void *src, size_t bytes, void *stream)
{ TLG_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream)); return TLG_OK; }
extern "C" void *tlg_stream_create(void)
{
    if (tlg_ensure_init()) return nullptr;
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return nullptr;
    return s;
}
// Reductions queued on the stream (a grouped launch's split partials, the
// MoE backward's held sums) run on it before the handle is destroyed.
extern "C" int tlg_stream_destroy(void *s)
{
    if (g_tlg.initialised) {
        const int rc = tlg_group_flush_stream((hipStream_t)s);
        if (rc) return rc;
    }
    TLG_HIP(hipStreamDestroy((hipStream_t)s));
    return TLG_OK;
}
extern "C" int tlg_stream_sync(void *s) { TLG_HIP(hipStreamSynchronize((hipStream_t)s)); return TLG_OK; }
extern "C" void *tlg_event_create(void)
{
    if (tlg_ensure_init()) return nullptr;
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}
extern "C" int tlg_event_destroy(void *e) { TLG_HIP(hipEventDestroy((hipEvent_t)e)); return TLG_OK; }
extern "C" int tlg_event_record(void *e, void *s) { TLG_HIP(hipEventRecord((hipEvent_t)e, (hipStream_t)s)); return TLG_OK; }
extern "C" float tlg_event_elapsed_ms(void *a, void *b)
{
    float ms = -1.f;
    hipError_t e = hipEventElapsedTime(&ms, (hipEvent_t)a, (hipEvent_t)b);
    if (e != hipSuccess) { tlg_fail_hip(e, "hipEventElapsedTime", __FILE__, __LINE__); return -1.f; }
    return ms;
}
extern "C" int tlg_graph_begin(void *s)
{ TLG_HIP(hipStreamBeginCapture((hipStream_t)s, hipStreamCaptureModeThreadLocal)); return TLG_OK; }
extern "C" void *tlg_graph_end(void *s)
{
    hipGraph_t g = nullptr;
    hipGraphExec_t x = nullptr;
    hipError_t e = hipStreamEndCapture((hipStream_t)s, &g);
    if (e != hipSuccess) { tlg_fail_hip(e, "hipStreamEndCapture", __FILE__, __LINE__); return nullptr; }
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) { tlg_fail_hip(e, "hipGraphInstantiate", __FILE__, __LINE__); return nullptr; }
    return x;
}
extern "C" int tlg_graph_launch(void *g, void *s) { TLG_HIP(hipGraphLaunch((hipGraphExec_t)g, (hipStream_t)s)); return TLG_OK; }
extern "C" int tlg_graph_destroy(void *g) { TLG_HIP(hipGraphExecDestroy((hipGraphExec_t)g)); return TLG_OK; }

int tlg_fill_normal_launch(float *dst, size_t n, unsigned long long seed, float scale, hipStream_t st);
extern "C" int tlg_dev_fill_normal(float *dst, size_t n, unsigned long long seed, float scale, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    return tlg_fill_normal_launch(dst, n, seed, scale, (hipStream_t)stream);
}

extern "C" int tlg_kernel_name(int op, int M, int K, int N, char *buf, int len, int *splits)
{
    if (!buf || len <= 0) return tlg_fail(TLG_EINVAL, "tlg_kernel_name: no buffer");
    switch (op) {
    case 0: return tlg_describe(TLG_NN, M, N, K, buf, len, splits);
    case 1: return tlg_describe(TLG_NT, M, K, N, buf, len, splits);
    case 2: return tlg_describe(TLG_TN, K, N, M, buf, len, splits);
    default: return tlg_fail(TLG_EINVAL, "tlg_kernel_name: op %d", op);
    }
}

int tlg_copy_launch(float *dst, const float *src, size_t n, hipStream_t st);
int tlg_read_launch(const float *src, size_t n, float *sink, hipStream_t st);
int tlg_mfma_peak_launch(float *out, int blocks, int iters, hipStream_t st);
extern "C" int tlg_dev_copy(float *dst, const float *src, size_t n, void *stream)
{
    int rc = tlg_ensure_init();
    return rc ? rc : tlg_copy_launch(dst, src, n, (hipStream_t)stream);
}
extern "C" int tlg_dev_read(const float *src, size_t n, float *sink, void *stream)
{
    int rc = tlg_ensure_init();
    return rc ? rc : tlg_read_launch(src, n, sink, (hipStream_t)stream);
}
extern "C" int tlg_dev_mfma_peak(float *out, int blocks, int iters, void *stream)
{
    int rc = tlg_ensure_init();
    return rc ? rc : tlg_mfma_peak_launch(out, blocks, iters, (hipStream_t)stream);
}

extern "C" int tlg_dev_gemm_group(const TlgGemmCall *calls, int n, void *stream)
{
    if (n < 0 || (n > 0 && !calls)) return tlg_fail(TLG_EINVAL, "tlg_dev_gemm_group: bad call list");
    return tlg_group_launch(calls, n, (hipStream_t)stream);
}
extern "C" int tlg_dev_gemm_flush(void *stream)
{
    int rc = tlg_ensure_init();
    return rc ? rc : tlg_group_flush_launch((hipStream_t)stream);
}

int tlg_group_pending(void);
extern "C" int tlg_dev_gemm_pending(void) { return tlg_group_pending(); }

const char *tlg_group_kernel_name(void);
extern "C" const char *tlg_group_kernel(void) { return tlg_group_kernel_name(); }

// ------------------------------------------------ dense SwiGLU FFN pair --
// The dense FFN's GEMMs with their elementwise neighbours in the epilogue,
// run by the expert-batched launch with one expert owning every row.
static int ffn_check(const char *who, const float *A, const float *B, int M, int K, int N)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (M < 0 || K <= 0 || N <= 0 || K % 4 || N % 4 || !A || !B || ((uintptr_t)A & 15) || ((uintptr_t)B & 15))
        return tlg_fail(TLG_EINVAL, "%s: M=%d K=%d N=%d (widths %% 4 == 0, aligned operands)", who, M, K, N);
    return TLG_OK;
}

extern "C" int tlg_dev_swiglu_mm(const float *X, const float *W1, const float *W3, float *act, float *g, float *u,
                                 int M, int K, int N, void *stream)
{
    int rc = ffn_check("tlg_dev_swiglu_mm", X, W1, M, K, N);
    if (rc) return rc;
    if (!W3 || !act || ((uintptr_t)W3 & 15) || ((uintptr_t)act & 15) || ((uintptr_t)g & 15) || ((uintptr_t)u & 15))
        return tlg_fail(TLG_EINVAL, "tlg_dev_swiglu_mm: missing or unaligned operand");
    TlgExpertCall c;
    memset(&c, 0, sizeof c);
    c.op = 0; c.C = act; c.K = K; c.N = N; c.nseg = 1;
    c.A[0] = X; c.B[0] = W1; c.B2 = W3;
    c.epi = TLG_EPI_SWIGLU; c.X1 = g; c.X2 = u;
    return tlg_expert_launch(&c, 1, nullptr, 1, M, (hipStream_t)stream);
}

extern "C" int tlg_dev_mm_bt_swiglu_bwd(const float *dY, const float *W2, float *g, float *u, int M, int K, int N,
                                        void *stream)
{
    int rc = ffn_check("tlg_dev_mm_bt_swiglu_bwd", dY, W2, M, K, N);
    if (rc) return rc;
    if (!g || !u || ((uintptr_t)g & 15) || ((uintptr_t)u & 15))
        return tlg_fail(TLG_EINVAL, "tlg_dev_mm_bt_swiglu_bwd: missing or unaligned g / u");
    TlgExpertCall c;
    memset(&c, 0, sizeof c);
    c.op = 1; c.C = nullptr; c.K = K; c.N = N; c.nseg = 1;
    c.A[0] = dY; c.B[0] = W2;
    c.epi = TLG_EPI_SWIGLU_BWD; c.X1 = g; c.X2 = u;
    return tlg_expert_launch(&c, 1, nullptr, 1, M, (hipStream_t)stream);
}

// ------------------------------------------------------------- top-1 MoE --
int tlg_moe_fwd_launch(const float *fnorm, const float *fin, float *out, int N, int D, int F, int E,
                       const float *wr, const float *w1, const float *w3, const float *w2, int *assign,
                       float *gate, float *rprobs, void *keep, size_t keep_bytes, hipStream_t st);
int tlg_moe_bwd_launch(const float *fnorm, const float *dout, float *d_fnorm, const int *assign,
                       const float *gate, const float *rprobs, int N, int D, int F, int E, const float *wr,
                       const float *w1, const float *w3, const float *w2, float *gwr, float *gw1, float *gw3,
                       float *gw2, void *kept, size_t kept_bytes, hipStream_t st);

extern "C" int tlg_dev_moe_grouped_fwd(const float *fnorm, const float *fin, float *out, int N, int D, int F,
                                       int E, const float *wr, const float *w1, const float *w3,
                                       const float *w2, int *assign, float *gate, float *rprobs, void *stream)
{
    return tlg_moe_fwd_launch(fnorm, fin, out, N, D, F, E, wr, w1, w3, w2, assign, gate, rprobs, nullptr, 0,
                              (hipStream_t)stream);
}

extern "C" int tlg_dev_moe_grouped_bwd(const float *fnorm, const float *dout, float *d_fnorm,
                                       const int *assign, const float *gate, const float *rprobs, int N, int D,
                                       int F, int E, const float *wr, const float *w1, const float *w3,
                                       const float *w2, float *gwr, float *gw1, float *gw3, float *gw2,
                                       void *stream)
{
    return tlg_moe_bwd_launch(fnorm, dout, d_fnorm, assign, gate, rprobs, N, D, F, E, wr, w1, w3, w2, gwr, gw1,
                              gw3, gw2, nullptr, 0, (hipStream_t)stream);
}

extern "C" int tlg_dev_moe_grouped_fwd_keep(const float *fnorm, const float *fin, float *out, int N, int D,
                                            int F, int E, const float *wr, const float *w1, const float *w3,
                                            const float *w2, int *assign, float *gate, float *rprobs, void *keep,
                                            size_t keep_bytes, void *stream)
{
    if (!keep) return tlg_fail(TLG_EINVAL, "tlg_dev_moe_grouped_fwd_keep: NULL kept-state buffer");
    return tlg_moe_fwd_launch(fnorm, fin, out, N, D, F, E, wr, w1, w3, w2, assign, gate, rprobs, keep, keep_bytes,
                              (hipStream_t)stream);
}

extern "C" int tlg_dev_moe_grouped_bwd_kept(const float *fnorm, const float *dout, float *d_fnorm,
                                            const int *assign, const float *gate, const float *rprobs, int N,
                                            int D, int F, int E, const float *wr, const float *w1,
                                            const float *w3, const float *w2, float *gwr, float *gw1, float *gw3,
                                            float *gw2, void *kept, size_t kept_bytes, void *stream)
{
    if (!kept) return tlg_fail(TLG_EINVAL, "tlg_dev_moe_grouped_bwd_kept: NULL kept-state buffer");
    return tlg_moe_bwd_launch(fnorm, dout, d_fnorm, assign, gate, rprobs, N, D, F, E, wr, w1, w3, w2, gwr, gw1,
                              gw3, gw2, kept, kept_bytes, (hipStream_t)stream);
}

// Host-pointer operands of a MoE call: device addresses (mirror or staging
// slot) and which results go back to host memory at the end.
struct HostOps {
    int next = 0;
    struct Back { void *host, *dev; size_t bytes; } back[8];
    int nback = 0;
    int rc = TLG_OK;
    template <class P>
    P *get(P *host, size_t bytes, bool upload, bool download)
    {
        if (rc) return nullptr;
        void *dev = nullptr;
        bool mirrored = false;
        rc = resolve(next++, (const void *)host, bytes, upload, &dev, &mirrored);
        if (rc) return nullptr;
        if (download && !mirrored) back[nback++] = {(void *)host, dev, bytes};
        return (P *)dev;
    }
    int finish()
    {
        for (int k = 0; k < nback && !rc; k++)
            if (hipMemcpyAsync(back[k].host, back[k].dev, back[k].bytes, hipMemcpyDeviceToHost, g_tlg.stream) !=
                hipSuccess)
                rc = tlg_fail(TLG_EHIP, "MoE result copy");
        if (!rc && hipStreamSynchronize(g_tlg.stream) != hipSuccess) rc = tlg_fail(TLG_EHIP, "MoE stream sync");
        return rc;
    }
};

static int host_moe_fwd(const float *fnorm, const float *fin, float *out, int N, int D, int F, int E,
                        const float *wr, const float *w1, const float *w3, const float *w2, int *assign,
                        float *gate, float *rprobs)
{
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = init_locked(g_tlg.initialised ? g_tlg.device : 0);
    if (rc) return rc;
    if (N <= 0 || D <= 0 || F <= 0 || E <= 0) return N == 0 ? TLG_OK : tlg_fail(TLG_EINVAL, "MoE: bad shape");
    const size_t nd = (size_t)N * D * 4, wf = (size_t)E * D * F * 4;
    HostOps h;
    const float *dfn = h.get(fnorm, nd, true, false), *dfi = h.get(fin, nd, true, false);
    float *dout = h.get(out, nd, false, true);
    const float *dwr = h.get(wr, (size_t)D * E * 4, true, false);
    const float *d1 = h.get(w1, wf, true, false), *d3 = h.get(w3, wf, true, false), *d2 = h.get(w2, wf, true, false);
    int *das = h.get(assign, (size_t)N * 4, false, true);
    float *dg = h.get(gate, (size_t)N * 4, false, true), *dpr = h.get(rprobs, (size_t)N * E * 4, false, true);
    if (h.rc) return h.rc;
    rc = tlg_moe_fwd_launch(dfn, dfi, dout, N, D, F, E, dwr, d1, d3, d2, das, dg, dpr, nullptr, 0, g_tlg.stream);
    if (rc) return rc;
    return h.finish();
}

static int host_moe_bwd(const float *fnorm, const float *dout, float *d_fnorm, const int *assign,
                        const float *gate, const float *rprobs, int N, int D, int F, int E, const float *wr,
                        const float *w1, const float *w3, const float *w2, float *gwr, float *gw1, float *gw3,
                        float *gw2)
{
    std::lock_guard<std::recursive_mutex> lk(g_mu);
    int rc = init_locked(g_tlg.initialised ? g_tlg.device : 0);
    if (rc) return rc;
    if (N <= 0 || D <= 0 || F <= 0 || E <= 0) return N == 0 ? TLG_OK : tlg_fail(TLG_EINVAL, "MoE: bad shape");
    const size_t nd = (size_t)N * D * 4, wf = (size_t)E * D * F * 4;
    HostOps h;
    const float *dfn = h.get(fnorm, nd, true, false), *ddo = h.get(dout, nd, true, false);
    float *ddf = h.get(d_fnorm, nd, false, true);
    const int *das = h.get(assign, (size_t)N * 4, true, false);
    const float *dg = h.get(gate, (size_t)N * 4, true, false), *dpr = h.get(rprobs, (size_t)N * E * 4, true, false);
    const float *dwr = h.get(wr, (size_t)D * E * 4, true, false);
    const float *d1 = h.get(w1, wf, true, false), *d3 = h.get(w3, wf, true, false), *d2 = h.get(w2, wf, true, false);
    float *gr = h.get(gwr, (size_t)D * E * 4, true, true);
    float *g1 = h.get(gw1, wf, true, true), *g3 = h.get(gw3, wf, true, true), *g2 = h.get(gw2, wf, true, true);
    if (h.rc) return h.rc;
    rc = tlg_moe_bwd_launch(dfn, ddo, ddf, das, dg, dpr, N, D, F, E, dwr, d1, d3, d2, gr, g1, g3, g2, nullptr, 0,
                            g_tlg.stream);
    if (rc) return rc;
    return h.finish();
}

extern "C" void tlg_moe_grouped_fwd(const float *fnorm, const float *fin, float *out, int N, int D, int F, int E,
                                    const float *wr, const float *w1, const float *w3, const float *w2,
                                    int *assign, float *gate, float *rprobs)
{
    die_on(host_moe_fwd(fnorm, fin, out, N, D, F, E, wr, w1, w3, w2, assign, gate, rprobs), "tlg_moe_grouped_fwd");
}

extern "C" void tlg_moe_grouped_bwd(const float *fnorm, const float *dout, float *d_fnorm, const int *assign,
                                    const float *gate, const float *rprobs, int N, int D, int F, int E,
                                    const float *wr, const float *w1, const float *w3, const float *w2,
                                    float *gwr, float *gw1, float *gw3, float *gw2)
{
    die_on(host_moe_bwd(fnorm, dout, d_fnorm, assign, gate, rprobs, N, D, F, E, wr, w1, w3, w2, gwr, gw1, gw3,
                        gw2),
           "tlg_moe_grouped_bwd");
}
