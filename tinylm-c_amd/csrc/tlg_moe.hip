// tlg_moe.hip -- the top-1 mixture-of-experts FFN of tinylm.c on gfx950:
// routing, the per-expert row index, and the expert GEMMs as expert-batched
// grouped launches over rows grouped by expert.
//
// Reference: moe_forward tinylm.c:857-891, moe_backward :895-947, moe_route
// :814-827 (K = 1, no router bias), MOE_AUX :849.
//
// Data layout in HBM.  Token-order buffers are the caller's (fnorm, fin, out,
// dout, d_fnorm: N x D; rprobs N x E; assign, gate: N).  The library keeps
// one scratch arena with the expert-grouped ("sorted") rows: row i of Xg, g,
// u, a, y, dy, da holds token idx[i]; expert e owns sorted rows
// [eoff[e], eoff[e+1]) in ascending token order, the order in which the
// reference gathers them (:876).  pos[n] is token n's sorted row.
//
// Kernels (one pass each over the data they touch):
//   k_moe_route     router logits as the reference's own FMA chain over D
//                   (so the argmax sees the reference's logits bit for bit),
//                   softmax, strict-greater argmax (ties -> lowest expert)
//   k_moe_index     stable counting sort of the tokens by expert (one
//                   workgroup, wave ballots; no atomics)
//   k_gather_rows   Xg = fnorm[idx]
//   expert GEMMs    tlg_expert_launch (grouped MFMA tiles, every expert in
//                   one launch; the rows per expert stay on the device)
//   k_swiglu(_bwd)  a = silu(g) u and its backward
//   k_moe_combine   out[n] = fin[n] + gate[n] y[pos[n]]
//   k_moe_dgate     d_gate[n] = dout[n] . y[pos[n]],  dy = gate dout
//   k_moe_router_bwd  softmax backward with the load-balance term
//   k_moe_dfnorm    d_fnorm = dX[pos] + d_rt wr^T   (the router mm_bt, :944)
// and dWr += fnorm^T d_rt through the generic mm_atb launch (:945).
#include "tlg_internal.h"
#include <initializer_list>
#include <stdio.h>
#include <string.h>

#define TLG_MOE_MAXE 64          // the reference's dp[64] (:937)

// ------------------------------------------------------------ routing --
// MOE_TOK tokens per workgroup.  Logit (t, e) is the chain
//   l = 0; for d in 0..D-1: l = fma(x[t][d], wr[d][e], l)
// which is how the reference's mm evaluates each output (:462-466).  The
// token rows and router columns are staged in LDS (dynamic: `dch` columns of
// d at a time, all of D when it fits), so one round of loads serves the
// whole chain.
#define MOE_TOK 16
__global__ __launch_bounds__(256) void k_moe_route(const float *__restrict__ X, const float *__restrict__ Wr,
                                                   int N, int D, int E, int dch, float *__restrict__ rprobs,
                                                   int *__restrict__ assign, float *__restrict__ gate)
{
    extern __shared__ float lds_route[];
    float *xs = lds_route;                          // [MOE_TOK][dch + 1]
    float *wsm = xs + MOE_TOK * (dch + 1);          // [dch][E]
    float *lg = wsm + dch * E;                      // [MOE_TOK][E]
    const int n0 = blockIdx.x * MOE_TOK, tid = threadIdx.x;
    for (int p = tid; p < MOE_TOK * E; p += 256) lg[p] = 0.f;
    for (int d0 = 0; d0 < D; d0 += dch) {
        const int dn = min(dch, D - d0);
        __syncthreads();
        for (int p = tid; p < MOE_TOK * dch; p += 256) {
            const int t = p / dch, d = p - t * dch;
            xs[t * (dch + 1) + d] = (n0 + t < N && d < dn) ? X[(size_t)(n0 + t) * D + d0 + d] : 0.f;
        }
        for (int p = tid; p < dch * E; p += 256) {
            const int d = p / E;
            wsm[p] = d < dn ? Wr[(size_t)(d0 + d) * E + p % E] : 0.f;
        }
        __syncthreads();
        for (int p = tid; p < MOE_TOK * E; p += 256) {
            const int t = p / E, e = p % E;
            const float *xr = xs + t * (dch + 1);
            float l = lg[p];
            int d = 0;
            // the chain stays sequential; its LDS operands are fetched 8 ahead
            for (; d + 8 <= dn; d += 8) {
                float xv[8], wv[8];
#pragma unroll
                for (int u = 0; u < 8; u++) { xv[u] = xr[d + u]; wv[u] = wsm[(d + u) * E + e]; }
#pragma unroll
                for (int u = 0; u < 8; u++) l = fmaf(xv[u], wv[u], l);
            }
            for (; d < dn; d++) l = fmaf(xr[d], wsm[d * E + e], l);
            lg[p] = l;
        }
    }
    __syncthreads();
    const int t = tid, n = n0 + t;
    if (t >= MOE_TOK || n >= N) return;
    // softmax over all E (:862-867), then moe_route's slot 0 (:818-825)
    const float *r = lg + t * E;
    float *pr = rprobs + (size_t)n * E;
    float mx = -1e30f;
    for (int e = 0; e < E; e++) if (r[e] > mx) mx = r[e];
    float s = 0.f;
    for (int e = 0; e < E; e++) { const float v = expf(r[e] - mx); pr[e] = v; s += v; }
    const float inv = 1.0f / s;
    int best = -1;
    float bp = -1e30f;
    for (int e = 0; e < E; e++) {
        const float v = pr[e] * inv;
        pr[e] = v;
        if (v > bp) { bp = v; best = e; }
    }
    const int sel = best < 0 ? 0 : best;
    assign[n] = sel;
    gate[n] = pr[sel];
}

// LDS columns per round of k_moe_route: all of D when the staged rows and
// router columns fit in 48 KB, else 64.
static int route_dch(int D, int E)
{
    const size_t whole = (size_t)MOE_TOK * (D + 1) + (size_t)D * E + (size_t)MOE_TOK * E;
    return whole * 4 <= 48 * 1024 ? D : 64;
}
static size_t route_lds(int dch, int E)
{
    return 4 * ((size_t)MOE_TOK * (dch + 1) + (size_t)dch * E + (size_t)MOE_TOK * E);
}

// ------------------------------------------------------- expert index --
// Stable counting sort of tokens by expert in one workgroup of 16 waves.
// A wave finds each lane's rank among the lanes routed to the same expert
// with one ballot per expert; per-wave counts are scanned in wave order, so
// tokens keep ascending order inside each expert.  Tokens whose expert is
// out of range are left out (pos = -1).
__device__ __forceinline__ void wave_rank(int a, int E, int lane, int w, int (*wc)[TLG_MOE_MAXE], int *rank)
{
    for (int e = 0; e < E; e++) {
        const unsigned long long m = __ballot(a == e);
        if (a == e) *rank = __popcll(m & ((1ull << lane) - 1ull));
        if (lane == 0) wc[w][e] = __popcll(m);
    }
}

__global__ __launch_bounds__(1024) void k_moe_index(const int *__restrict__ assign, int N, int E,
                                                    int *__restrict__ idx, int *__restrict__ pos,
                                                    int *__restrict__ eoff)
{
    __shared__ int wc[16][TLG_MOE_MAXE];
    __shared__ int run[TLG_MOE_MAXE + 1];
    __shared__ int off[TLG_MOE_MAXE + 1];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    if (tid <= TLG_MOE_MAXE) run[tid] = 0;
    __syncthreads();
    // pass 1: tokens per expert
    for (int c0 = 0; c0 < N; c0 += 1024) {
        const int n = c0 + tid;
        const int a = n < N ? assign[n] : -1;
        int rank = 0;
        wave_rank(a, E, lane, w, wc, &rank);
        __syncthreads();
        if (tid < E) {
            int r = run[tid];
            for (int k = 0; k < 16; k++) r += wc[k][tid];
            run[tid] = r;
        }
        __syncthreads();
    }
    if (tid == 0) {
        int s = 0;
        for (int e = 0; e < E; e++) { off[e] = s; s += run[e]; }
        off[E] = s;
    }
    __syncthreads();
    if (tid <= E) { eoff[tid] = off[tid]; run[tid] = 0; }
    __syncthreads();
    // pass 2: placement in token order
    for (int c0 = 0; c0 < N; c0 += 1024) {
        const int n = c0 + tid;
        const int a = n < N ? assign[n] : -1;
        int rank = 0;
        wave_rank(a, E, lane, w, wc, &rank);
        __syncthreads();
        if (tid < E) {
            int r = run[tid];
            for (int k = 0; k < 16; k++) { const int c = wc[k][tid]; wc[k][tid] = r; r += c; }
            run[tid] = r;
        }
        __syncthreads();
        if (n < N) {
            const bool ok = a >= 0 && a < E;
            const int p = ok ? off[a] + wc[w][a] + rank : -1;
            pos[n] = p;
            if (ok) idx[p] = n;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------- elementwise --
typedef float f32x4 __attribute__((ext_vector_type(4)));

// dst[i] = src[idx[i]] for the eoff[E] routed rows (D % 4 == 0).
__global__ void k_gather_rows(const float *__restrict__ src, const int *__restrict__ idx,
                              const int *__restrict__ eoff, int E, int D, float *__restrict__ dst)
{
    const int d4 = D >> 2;
    const size_t total = (size_t)eoff[E] * d4;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += stride) {
        const size_t i = q / d4, c = q % d4;
        reinterpret_cast<f32x4 *>(dst)[i * d4 + c] =
            reinterpret_cast<const f32x4 *>(src)[(size_t)idx[i] * d4 + c];
    }
}

// a = silu(g) * u over the routed rows; silu(z) = z / (1 + e^-z) (:786).
__global__ void k_swiglu(const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ a,
                         const int *__restrict__ eoff, int E, int F)
{
    const size_t total = (size_t)eoff[E] * F;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const float z = g[i];
        a[i] = z / (1.0f + expf(-z)) * u[i];
    }
}

// In place: g <- da * u * silu'(g), u <- da * silu(g)  (:923-925).
__global__ void k_swiglu_bwd(float *__restrict__ g, float *__restrict__ u, const float *__restrict__ da,
                             const int *__restrict__ eoff, int E, int F)
{
    const size_t total = (size_t)eoff[E] * F;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const float z = g[i], uv = u[i], d = da[i];
        const float sg = 1.0f / (1.0f + expf(-z));
        const float si = z * sg;
        const float ds = sg + z * sg * (1.0f - sg);
        g[i] = d * uv * ds;
        u[i] = d * si;
    }
}

// out[n] = fin[n] + gate[n] * y[pos[n]]  (:870, :886-888); fin alone for a
// token with no expert.
__global__ void k_moe_combine(const float *__restrict__ fin, const float *__restrict__ y,
                              const int *__restrict__ pos, const float *__restrict__ gate, int N, int D,
                              float *__restrict__ out)
{
    const int d4 = D >> 2;
    const size_t total = (size_t)N * d4;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += stride) {
        const size_t n = q / d4, c = q % d4;
        const f32x4 f = reinterpret_cast<const f32x4 *>(fin)[q];
        const int p = pos[n];
        f32x4 o = f;
        if (p >= 0) {
            const float gt = gate[n];
            const f32x4 v = reinterpret_cast<const f32x4 *>(y)[(size_t)p * d4 + c];
            o[0] = fmaf(gt, v[0], f[0]); o[1] = fmaf(gt, v[1], f[1]);
            o[2] = fmaf(gt, v[2], f[2]); o[3] = fmaf(gt, v[3], f[3]);
        }
        reinterpret_cast<f32x4 *>(out)[q] = o;
    }
}

// One wave per routed row i (token n = idx[i]): d_gate[n] = dout[n] . y[i],
// dy[i] = gate[n] dout[n]  (:916-919).
__global__ __launch_bounds__(256) void k_moe_dgate(const float *__restrict__ dout, const float *__restrict__ y,
                                                   const int *__restrict__ idx, const int *__restrict__ eoff,
                                                   int E, int D, const float *__restrict__ gate,
                                                   float *__restrict__ dgate, float *__restrict__ dy)
{
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= eoff[E]) return;
    const int n = idx[i];
    const float *dr = dout + (size_t)n * D;
    const float *yr = y + (size_t)i * D;
    float *dyr = dy + (size_t)i * D;
    const float gt = gate[n];
    float s = 0.f;
    for (int d = lane; d < D; d += 64) {
        const float v = dr[d];
        s = fmaf(v, yr[d], s);
        dyr[d] = gt * v;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) dgate[n] = s;
}

// Router backward per token (:933-943): dp_e = 0.01 E (cnt_e / N) / N, plus
// d_gate on the chosen expert; d_rt = p (dp - p.dp).
__global__ void k_moe_router_bwd(const float *__restrict__ rprobs, const int *__restrict__ pos,
                                 const int *__restrict__ assign, const float *__restrict__ dgate,
                                 const int *__restrict__ eoff, int N, int E, float *__restrict__ drt)
{
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    const float invN = 1.0f / (float)N;
    const float auxw = 0.01f * (float)E;
    const int a = pos[n] >= 0 ? assign[n] : -1;
    const float dg = a >= 0 ? dgate[n] : 0.f;
    const float *pr = rprobs + (size_t)n * E;
    float dot = 0.f;
    for (int e = 0; e < E; e++) {
        float dp = auxw * ((float)(eoff[e + 1] - eoff[e]) * invN) * invN;
        if (e == a) dp += dg;
        dot = fmaf(pr[e], dp, dot);
    }
    float *dr = drt + (size_t)n * E;
    for (int e = 0; e < E; e++) {
        float dp = auxw * ((float)(eoff[e + 1] - eoff[e]) * invN) * invN;
        if (e == a) dp += dg;
        dr[e] = pr[e] * (dp - dot);
    }
}

// d_fnorm[n][d] = dX[pos[n]][d] + sum_e d_rt[n][e] wr[d][e]: the expert
// scatter (:928-930) after the memset (:900), then the router mm_bt (:944).
__global__ void k_moe_dfnorm(const float *__restrict__ dX, const int *__restrict__ pos,
                             const float *__restrict__ drt, const float *__restrict__ wr, int N, int D, int E,
                             float *__restrict__ dfn)
{
    const size_t total = (size_t)N * D;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += stride) {
        const size_t n = q / D, d = q % D;
        const int p = pos[n];
        const float x = p >= 0 ? dX[(size_t)p * D + d] : 0.f;
        const float *r = drt + n * E, *w = wr + d * E;
        float s = 0.f;
        for (int e = 0; e < E; e++) s = fmaf(r[e], w[e], s);
        dfn[q] = x + s;
    }
}

// -------------------------------------------------------------- scratch --
// One arena, grown on demand and kept until tlg_shutdown (like the
// reference's me_ensure, :840-848).  Growing it synchronizes the device, so
// the first call at a new size cannot be captured into a graph; calls on
// different streams must not overlap (they share the arena).
struct MoeScratch {
    int *idx, *pos, *eoff;
    float *dgate, *drt, *Xg, *y, *dy, *g, *u, *a, *da;
};
static void *g_moe_mem = nullptr;
static size_t g_moe_bytes = 0;

void tlg_moe_release(void)
{
    if (g_moe_mem) (void)hipFree(g_moe_mem);
    g_moe_mem = nullptr;
    g_moe_bytes = 0;
}

static int moe_scratch(int N, int D, int F, int E, MoeScratch *s)
{
    const size_t n = (size_t)N;
    const size_t sizes[12] = {n * 4, n * 4, (size_t)(TLG_MOE_MAXE + 1) * 4, n * 4, n * E * 4,
                              n * D * 4, n * D * 4, n * D * 4, n * F * 4, n * F * 4, n * F * 4, n * F * 4};
    size_t total = 0, offs[12];
    for (int k = 0; k < 12; k++) {
        offs[k] = total;
        total += (sizes[k] + 255) & ~(size_t)255;
    }
    if (total > g_moe_bytes) {
        // earlier launches may still read the old arena
        TLG_HIP(hipDeviceSynchronize());
        tlg_moe_release();
        if (hipMalloc(&g_moe_mem, total) != hipSuccess) {
            g_moe_mem = nullptr;
            return tlg_fail(TLG_ENOMEM, "MoE scratch of %zu bytes", total);
        }
        g_moe_bytes = total;
    }
    char *b = (char *)g_moe_mem;
    s->idx = (int *)(b + offs[0]);
    s->pos = (int *)(b + offs[1]);
    s->eoff = (int *)(b + offs[2]);
    s->dgate = (float *)(b + offs[3]);
    s->drt = (float *)(b + offs[4]);
    s->Xg = (float *)(b + offs[5]);
    s->y = (float *)(b + offs[6]);
    s->dy = (float *)(b + offs[7]);
    s->g = (float *)(b + offs[8]);
    s->u = (float *)(b + offs[9]);
    s->a = (float *)(b + offs[10]);
    s->da = (float *)(b + offs[11]);
    return TLG_OK;
}

// ------------------------------------------------------------ launches --
static inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }
static inline unsigned grid_for(size_t work, size_t per_block, unsigned cap)
{
    size_t b = (work + per_block - 1) / per_block;
    if (b < 1) b = 1;
    return (unsigned)(b > cap ? cap : b);
}

static int check_shape(int N, int D, int F, int E)
{
    if (N < 0 || D <= 0 || F <= 0) return tlg_fail(TLG_EINVAL, "MoE: N=%d D=%d F=%d", N, D, F);
    if (E < 1 || E > TLG_MOE_MAXE) return tlg_fail(TLG_EINVAL, "MoE: %d experts (1..%d)", E, TLG_MOE_MAXE);
    if (D % 4 || F % 4) return tlg_fail(TLG_EINVAL, "MoE: D=%d and F=%d must be multiples of 4", D, F);
    return TLG_OK;
}

#define MOE_PTRS_OK(...) moe_ptrs_ok({__VA_ARGS__})
static bool moe_ptrs_ok(std::initializer_list<const void *> ps)
{
    for (const void *p : ps)
        if (!p || !al16(p)) return false;
    return true;
}

// Per-expert row index of the routed tokens (idx, pos, eoff).
static int moe_index(const int *assign, int N, int E, const MoeScratch &s, hipStream_t st)
{
    hipLaunchKernelGGL(k_moe_index, dim3(1), dim3(1024), 0, st, assign, N, E, s.idx, s.pos, s.eoff);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

// g, u = Xg W1_e, Xg W3_e;  a = silu(g) u;  y = a W2_e  (:880-884 / :911-914)
static int moe_experts_fwd(const float *fnorm, int N, int D, int F, int E, const float *w1, const float *w3,
                           const float *w2, const MoeScratch &s, hipStream_t st)
{
    hipLaunchKernelGGL(k_gather_rows, dim3(grid_for((size_t)N * D / 4, 256, 4096)), dim3(256), 0, st, fnorm,
                       s.idx, s.eoff, E, D, s.Xg);
    TLG_HIP(hipGetLastError());
    TlgExpertCall c[2];
    memset(c, 0, sizeof c);
    c[0].op = 0; c[0].C = s.g; c[0].K = D; c[0].N = F; c[0].nseg = 1;
    c[0].A[0] = s.Xg; c[0].B[0] = w1; c[0].es = (long long)D * F;
    c[1] = c[0];
    c[1].C = s.u; c[1].B[0] = w3;
    int rc = tlg_expert_launch(c, 2, s.eoff, E, N, st);
    if (rc) return rc;
    hipLaunchKernelGGL(k_swiglu, dim3(grid_for((size_t)N * F, 256, 8192)), dim3(256), 0, st, s.g, s.u, s.a,
                       s.eoff, E, F);
    TLG_HIP(hipGetLastError());
    memset(c, 0, sizeof c);
    c[0].op = 0; c[0].C = s.y; c[0].K = F; c[0].N = D; c[0].nseg = 1;
    c[0].A[0] = s.a; c[0].B[0] = w2; c[0].es = (long long)F * D;
    return tlg_expert_launch(c, 1, s.eoff, E, N, st);
}

int tlg_moe_fwd_launch(const float *fnorm, const float *fin, float *out, int N, int D, int F, int E,
                       const float *wr, const float *w1, const float *w3, const float *w2, int *assign,
                       float *gate, float *rprobs, hipStream_t st)
{
    int rc = check_shape(N, D, F, E);
    if (rc) return rc;
    if (N == 0) return TLG_OK;
    if (!MOE_PTRS_OK(fnorm, fin, out, w1, w3, w2) || !wr || !assign || !gate || !rprobs)
        return tlg_fail(TLG_EINVAL, "MoE forward: NULL or misaligned (16-byte) pointer");
    if ((rc = tlg_ensure_init())) return rc;
    if ((rc = tlg_group_flush_launch(st))) return rc;
    MoeScratch s;
    if ((rc = moe_scratch(N, D, F, E, &s))) return rc;
    const int dch = route_dch(D, E);
    hipLaunchKernelGGL(k_moe_route, dim3((N + MOE_TOK - 1) / MOE_TOK), dim3(256), route_lds(dch, E), st, fnorm, wr,
                       N, D, E, dch, rprobs, assign, gate);
    TLG_HIP(hipGetLastError());
    if ((rc = moe_index(assign, N, E, s, st))) return rc;
    if ((rc = moe_experts_fwd(fnorm, N, D, F, E, w1, w3, w2, s, st))) return rc;
    hipLaunchKernelGGL(k_moe_combine, dim3(grid_for((size_t)N * D / 4, 256, 4096)), dim3(256), 0, st, fin, s.y,
                       s.pos, gate, N, D, out);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

int tlg_moe_bwd_launch(const float *fnorm, const float *dout, float *d_fnorm, const int *assign,
                       const float *gate, const float *rprobs, int N, int D, int F, int E, const float *wr,
                       const float *w1, const float *w3, const float *w2, float *gwr, float *gw1, float *gw3,
                       float *gw2, hipStream_t st)
{
    int rc = check_shape(N, D, F, E);
    if (rc) return rc;
    if (N == 0) return TLG_OK;
    if (!MOE_PTRS_OK(fnorm, dout, d_fnorm, w1, w3, w2, gw1, gw3, gw2) || !wr || !gwr || !assign || !gate ||
        !rprobs)
        return tlg_fail(TLG_EINVAL, "MoE backward: NULL or misaligned (16-byte) pointer");
    if ((rc = tlg_ensure_init())) return rc;
    if ((rc = tlg_group_flush_launch(st))) return rc;
    MoeScratch s;
    if ((rc = moe_scratch(N, D, F, E, &s))) return rc;
    if ((rc = moe_index(assign, N, E, s, st))) return rc;
    // recompute the forward of every expert (:910-914)
    if ((rc = moe_experts_fwd(fnorm, N, D, F, E, w1, w3, w2, s, st))) return rc;
    hipLaunchKernelGGL(k_moe_dgate, dim3((N + 3) / 4), dim3(256), 0, st, dout, s.y, s.idx, s.eoff, E, D, gate,
                       s.dgate, s.dy);
    TLG_HIP(hipGetLastError());
    // dW2_e += a^T dy ;  da = dy W2_e^T   (:921-922)
    TlgExpertCall c[3];
    memset(c, 0, sizeof c);
    c[0].op = 2; c[0].beta = 1; c[0].C = gw2; c[0].K = F; c[0].N = D; c[0].nseg = 1;
    c[0].A[0] = s.a; c[0].B[0] = s.dy; c[0].es = (long long)F * D;
    c[1].op = 1; c[1].beta = 0; c[1].C = s.da; c[1].K = F; c[1].N = D; c[1].nseg = 1;
    c[1].A[0] = s.dy; c[1].B[0] = w2; c[1].es = (long long)F * D;
    if ((rc = tlg_expert_launch(c, 2, s.eoff, E, N, st))) return rc;
    hipLaunchKernelGGL(k_swiglu_bwd, dim3(grid_for((size_t)N * F, 256, 8192)), dim3(256), 0, st, s.g, s.u, s.da,
                       s.eoff, E, F);
    TLG_HIP(hipGetLastError());
    // dW1_e += Xg^T dg ; dW3_e += Xg^T du ; dX = dg W1_e^T + du W3_e^T (:926-927)
    memset(c, 0, sizeof c);
    c[0].op = 2; c[0].beta = 1; c[0].C = gw1; c[0].K = D; c[0].N = F; c[0].nseg = 1;
    c[0].A[0] = s.Xg; c[0].B[0] = s.g; c[0].es = (long long)D * F;
    c[1] = c[0];
    c[1].C = gw3; c[1].B[0] = s.u;
    c[2].op = 1; c[2].beta = 0; c[2].C = s.y; c[2].K = D; c[2].N = F; c[2].nseg = 2;
    c[2].A[0] = s.g; c[2].B[0] = w1; c[2].A[1] = s.u; c[2].B[1] = w3; c[2].Nseg[1] = F;
    c[2].es = (long long)D * F;
    if ((rc = tlg_expert_launch(c, 3, s.eoff, E, N, st))) return rc;
    // router: softmax backward, d_fnorm, dWr  (:932-945)
    hipLaunchKernelGGL(k_moe_router_bwd, dim3((N + 255) / 256), dim3(256), 0, st, rprobs, s.pos, assign, s.dgate,
                       s.eoff, N, E, s.drt);
    TLG_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_moe_dfnorm, dim3(grid_for((size_t)N * D, 256, 8192)), dim3(256), 0, st, s.y, s.pos,
                       s.drt, wr, N, D, E, d_fnorm);
    TLG_HIP(hipGetLastError());
    return tlg_gemm_launch(TLG_TN, fnorm, s.drt, gwr, D, E, N, D, E, E, 1, st);
}
