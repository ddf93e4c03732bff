// tlg_train.hip -- the non-GEMM work of tinylm.c's training step on gfx950,
// so that a whole forward + backward + AdamW step stays in HBM: embedding
// gather/scatter, RMSNorm, RoPE, causal GQA attention (MFMA), the residual
// adds, SwiGLU, softmax cross-entropy, the MTP head's SiLU residual, the
// global gradient norm and AdamW.
//
// Reference (tinylm.c): embedding :972-976 / :1149-1153, rmsnorm_fwd
// :540-563, rmsnorm_bwd :565-588, rope_init / rope_apply :605-651,
// attn_fwd :699-732, attn_bwd :734-783, siluf :786, residual adds :994-995
// :1009-1010, SwiGLU :1005-1006 / :1100-1112, softmax-CE :1019-1028,
// dlogits :1076-1082, mtp_grad glue :1036-1069, adamw :1159-1170,
// global_gradnorm :1171-1176.
//
// Data layout in HBM: the reference's own (row-major [rows][width] activations,
// flat P / G with map_weights' offsets).  Attention additionally keeps, per
// layer, the log-sum-exp of each (row, head) softmax ([rows][H] floats) so
// the backward pass rebuilds P without a max/sum pass.
//
// Attention uses v_mfma_f32_32x32x2_f32 on 32 x 32 tiles with head_dim 32 (the
// width of every BASELINE model).  A wave works on 32 queries of one head
// (the workgroup's waves split the key blocks and merge in a fixed order).  The
// forward computes S^T = K Q^T, so in the MFMA result each lane holds one
// query (lane % 32) and 16 keys: the softmax max and sum are in-lane plus one
// exchange with lane ^ 32, and the same registers are the B operand of
// O^T = V^T P^T with no shuffle.  The backward uses the same trick for dQ
// (dS^T as the B operand) and the untransposed S for dK / dV (P and dS as the
// A operand, contracting over queries); dK / dV of the heads sharing a KV head
// are summed in a fixed order through LDS, so every result is deterministic.
#include "tlg_internal.h"
#include "../../include/tltrain.h"
#include <math.h>
#include <string.h>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// The attention loops that feed each MFMA one LDS element (P V, dS K, P^T dO,
// dS^T Q): left alone the compiler issues each read right before the MFMA
// that consumes it, so at two waves per SIMD every MFMA pair waits out an LDS
// round trip.  Called at the end of such a loop's scheduling region, this
// asks for every LDS read of the region first, then its MFMAs.
#ifndef TLG_ATT_SCHED
#define TLG_ATT_SCHED 1
#endif
__device__ __forceinline__ void at_reads_first()
{
#if TLG_ATT_SCHED
    __builtin_amdgcn_sched_group_barrier(0x100, 64, 0);    // LDS reads
    __builtin_amdgcn_sched_group_barrier(0x008, 64, 0);    // MFMAs
#endif
}

static inline unsigned grid_for(size_t work, size_t per_block, unsigned cap)
{
    size_t b = (work + per_block - 1) / per_block;
    if (b < 1) b = 1;
    return (unsigned)(b > cap ? cap : b);
}
static inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// -------------------------------------------------------------- scratch --
// One arena for the small per-call scratch (norm partials, attention's
// dO.O rows, loss rows, the embedding index); grown on demand and kept until
// tlg_shutdown.  Growing it synchronizes the device, so the first call at a
// new size cannot be captured into a graph; calls on different streams must
// not overlap.
static void *g_tr_mem = nullptr;
static size_t g_tr_bytes = 0;

void tlg_train_release(void)
{
    if (g_tr_mem) (void)hipFree(g_tr_mem);
    g_tr_mem = nullptr;
    g_tr_bytes = 0;
}

static int tr_scratch(size_t bytes, void **out)
{
    bytes = (bytes + 255) & ~(size_t)255;
    if (bytes > g_tr_bytes) {
        TLG_HIP(hipDeviceSynchronize());
        tlg_train_release();
        if (hipMalloc(&g_tr_mem, bytes) != hipSuccess) {
            g_tr_mem = nullptr;
            return tlg_fail(TLG_ENOMEM, "training scratch of %zu bytes", bytes);
        }
        g_tr_bytes = bytes;
    }
    *out = g_tr_mem;
    return TLG_OK;
}

static int begin(void)
{
    return tlg_ensure_init();
}

// ------------------------------------------------------------ embedding --
// out[n] = emb[tok[n]]; a row whose token is outside [0, V) becomes NaN.
__global__ void k_embed_fwd(const float *__restrict__ emb, const int *__restrict__ tok, int N, int D, int V,
                            float *__restrict__ out)
{
    const int d4 = D >> 2;
    const size_t total = (size_t)N * d4;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += (size_t)gridDim.x * blockDim.x) {
        const size_t n = q / d4, c = q % d4;
        const int t = tok[n];
        f32x4 v;
        if (t >= 0 && t < V) v = reinterpret_cast<const f32x4 *>(emb)[(size_t)t * d4 + c];
        else v = f32x4{NAN, NAN, NAN, NAN};
        reinterpret_cast<f32x4 *>(out)[q] = v;
    }
}

__global__ void k_fill_int(int *__restrict__ p, int n, int v)
{
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = v;
}

__global__ void k_tok_count(const int *__restrict__ tok, int N, int V, int *__restrict__ cnt)
{
    for (int n = blockIdx.x * blockDim.x + threadIdx.x; n < N; n += gridDim.x * blockDim.x) {
        const int t = tok[n];
        if (t >= 0 && t < V) atomicAdd(&cnt[t], 1);
    }
}

// Exclusive scan of cnt[V] into off[V+1] by one 1024-thread workgroup, and
// cur[] = off[] (the placement cursors).
__global__ __launch_bounds__(1024) void k_tok_scan(const int *__restrict__ cnt, int V, int *__restrict__ off,
                                                   int *__restrict__ cur)
{
    __shared__ int part[1024];
    const int t = threadIdx.x;
    const int per = (V + 1023) / 1024;
    const int lo = t * per, hi = min(V, lo + per);
    int s = 0;
    for (int i = lo; i < hi; i++) s += cnt[i];
    part[t] = s;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
        const int add = t >= o ? part[t - o] : 0;
        __syncthreads();
        part[t] += add;
        __syncthreads();
    }
    int run = part[t] - s;
    for (int i = lo; i < hi; i++) {
        off[i] = run;
        cur[i] = run;
        run += cnt[i];
    }
    if (t == 1023) off[V] = part[1023];
}

__global__ void k_tok_place(const int *__restrict__ tok, int N, int V, int *__restrict__ cur, int *__restrict__ idx)
{
    for (int n = blockIdx.x * blockDim.x + threadIdx.x; n < N; n += gridDim.x * blockDim.x) {
        const int t = tok[n];
        if (t >= 0 && t < V) idx[atomicAdd(&cur[t], 1)] = n;
    }
}

// demb[v] += dout[n] for the rows n with tok[n] == v, in increasing n, as the
// reference's sequential scatter does (so the sums are bit-identical).  One
// wave per vocabulary row; the bucket's rows are visited in order by
// selecting the smallest index above the last one.
__global__ __launch_bounds__(256) void k_embed_bwd(const float *__restrict__ dout, const int *__restrict__ off,
                                                   const int *__restrict__ idx, int V, int D,
                                                   float *__restrict__ demb)
{
    const int lane = threadIdx.x & 63;
    const int v = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (v >= V) return;
    const int b = off[v], k = off[v + 1] - b;
    float *de = demb + (size_t)v * D;
    int last = -1;
    for (int j = 0; j < k; j++) {
        int m = 0x7fffffff;
        for (int e = lane; e < k; e += 64) {
            const int n = idx[b + e];
            if (n > last && n < m) m = n;
        }
        for (int o = 32; o > 0; o >>= 1) m = min(m, __shfl_xor(m, o));
        const float *d = dout + (size_t)m * D;
        for (int i = lane; i < D; i += 64) de[i] += d[i];
        last = m;
    }
}

// The same scatter in one launch (D % 4 == 0, D <= 1024): workgroup b owns
// vocabulary rows [8b, 8b + 8), wave w rows 8b + w and 8b + w + 4.  A pass
// takes 4096 tokens: every thread loads its 16 ids at once, then per chunk
// of 256 ids the matching positions are appended, in token order, to a list
// in LDS (wave ballots and a prefix over the four waves; a pass cannot
// overflow the list); then each wave adds the dout rows of its entries in
// list order, four rows' loads in flight at a time.  Each vocabulary row
// receives its rows in increasing n starting from demb's value, as above.
#define EMB_VB 8
#define EMB_PASS 4096
template <int NV>
__global__ __launch_bounds__(256) void k_embed_bwd1(const float *__restrict__ dout, const int *__restrict__ tok,
                                                    int N, int D, int V, float *__restrict__ demb)
{
    __shared__ int lst[EMB_PASS];
    __shared__ int wcnt[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int v0 = blockIdx.x * EMB_VB, d4 = D >> 2, vend = min(v0 + EMB_VB, V);
    const f32x4 *dout4 = reinterpret_cast<const f32x4 *>(dout);
    f32x4 *de4 = reinterpret_cast<f32x4 *>(demb);
    f32x4 acc[2][NV];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int v = min(v0 + wave + 4 * r, V - 1);
#pragma unroll
        for (int j = 0; j < NV; j++) acc[r][j] = de4[(size_t)v * d4 + min(lane + 64 * j, d4 - 1)];
    }
    for (int p0 = 0; p0 < N; p0 += EMB_PASS) {
        int tk[EMB_PASS / 256];
#pragma unroll
        for (int c = 0; c < EMB_PASS / 256; c++) {
            const int n = p0 + c * 256 + tid;
            tk[c] = tok[min(n, N - 1)];
            if (n >= N) tk[c] = -1;
        }
        int cnt = 0;
#pragma unroll
        for (int c = 0; c < EMB_PASS / 256; c++) {
            const int t = tk[c];
            const bool m = t >= v0 && t < vend;
            const unsigned long long bal = __ballot(m);
            if (lane == 0) wcnt[wave] = __popcll(bal);
            __syncthreads();
            int off = cnt, tot = cnt;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const int k = wcnt[w];
                off += w < wave ? k : 0;
                tot += k;
            }
            if (m) lst[off + __popcll(bal & ((1ull << lane) - 1ull))] = ((p0 + c * 256 + tid) << 3) | (t - v0);
            cnt = tot;
            __syncthreads();
        }
        for (int e0 = 0; e0 < cnt; e0 += 64) {
            const int e = e0 + lane;
            const int ent = e < cnt ? lst[e] : 0;
            unsigned long long mb = __ballot(e < cnt && ((ent & 7) & 3) == wave);
            while (mb) {
                int nn[4], rr[4];
                bool ok[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    ok[k] = mb != 0;
                    const int b = ok[k] ? __ffsll((long long)mb) - 1 : 0;
                    if (ok[k]) mb &= mb - 1;
                    const int en = __shfl(ent, b);
                    nn[k] = ok[k] ? en >> 3 : 0;
                    rr[k] = (en & 7) >> 2;
                }
                f32x4 rv[4][NV];
#pragma unroll
                for (int k = 0; k < 4; k++)
#pragma unroll
                    for (int j = 0; j < NV; j++) rv[k][j] = dout4[(size_t)nn[k] * d4 + min(lane + 64 * j, d4 - 1)];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    if (!ok[k]) break;
#pragma unroll
                    for (int j = 0; j < NV; j++) {
                        if (rr[k]) acc[1][j] += rv[k][j];
                        else acc[0][j] += rv[k][j];
                    }
                }
            }
        }
        __syncthreads();                            // the list is refilled next pass
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int v = v0 + wave + 4 * r;
        if (v >= V) continue;
#pragma unroll
        for (int j = 0; j < NV; j++)
            if (lane + 64 * j < d4) de4[(size_t)v * d4 + lane + 64 * j] = acc[r][j];
    }
}

// -------------------------------------------------------------- rmsnorm --
// One wave per row: s = 1 / sqrt(sum(x^2) / D + 1e-5), out = x * s * g.  With
// NV > 0 the row stays in registers between the sum and the output (NV float4
// columns per lane, D <= 256 NV; loads use clamped, in-bounds indices, columns
// past D are masked at use); NV = 0 takes any D and reads the row twice.  Both
// forms add the same terms in the same order.
// With tok (NV > 0 only): row r is the embedding row x[tok[r]] (x = the
// table of V rows; NaN for a token outside [0, V), as k_embed_fwd), also
// stored to xout[r] -- the embedding gather (:972-976) and the first norm in
// one pass.
template <int NV>
__global__ __launch_bounds__(256) void k_rms_fwd(const float *__restrict__ x, const float *__restrict__ g,
                                                 float *__restrict__ out, float *__restrict__ rinv, int rows, int D,
                                                 const int *__restrict__ tok = nullptr, int V = 0,
                                                 float *__restrict__ xout = nullptr)
{
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int d4 = D >> 2;
    int tr = r;
    bool bad = false;
    if (NV > 0 && tok) {
        tr = tok[r];
        bad = tr < 0 || tr >= V;
        if (bad) tr = 0;
    }
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(x + (size_t)tr * D);
    const f32x4 *g4 = reinterpret_cast<const f32x4 *>(g);
    f32x4 *orow = reinterpret_cast<f32x4 *>(out + (size_t)r * D);
    float ms = 0.f;
    if constexpr (NV == 0) {
        for (int i = lane; i < d4; i += 64) {
            const f32x4 v = xr[i];
            ms += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        for (int o = 32; o > 0; o >>= 1) ms += __shfl_xor(ms, o);
        const float s = 1.0f / sqrtf(ms / (float)D + 1e-5f);
        if (lane == 0 && rinv) rinv[r] = s;
        for (int i = lane; i < d4; i += 64) {
            const f32x4 v = xr[i], w = g4[i];
            orow[i] = f32x4{v.x * s * w.x, v.y * s * w.y, v.z * s * w.z, v.w * s * w.w};
        }
    } else {
        f32x4 xa[NV], gv[NV];
#pragma unroll
        for (int j = 0; j < NV; j++) {
            xa[j] = xr[min(lane + 64 * j, d4 - 1)];
            gv[j] = g4[min(lane + 64 * j, d4 - 1)];
        }
        if (tok) {
            f32x4 *xo = reinterpret_cast<f32x4 *>(xout + (size_t)r * D);
#pragma unroll
            for (int j = 0; j < NV; j++) {
                if (bad) xa[j] = f32x4{NAN, NAN, NAN, NAN};
                if (lane + 64 * j < d4) xo[lane + 64 * j] = xa[j];
            }
        }
#pragma unroll
        for (int j = 0; j < NV; j++)
            if (lane + 64 * j < d4) {
                const f32x4 v = xa[j];
                ms += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
        for (int o = 32; o > 0; o >>= 1) ms += __shfl_xor(ms, o);
        const float s = 1.0f / sqrtf(ms / (float)D + 1e-5f);
        if (lane == 0 && rinv) rinv[r] = s;
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int i = lane + 64 * j;
            if (i < d4) {
                const f32x4 v = xa[j], w = gv[j];
                orow[i] = f32x4{v.x * s * w.x, v.y * s * w.y, v.z * s * w.z, v.w * s * w.w};
            }
        }
    }
}

// dx = base + s g dy - (s^3 / D) (x . g dy) x (base = dx_in, or 0 when
// dx_in is null; dx_in may be dx itself) for RMS_ROWS rows per
// workgroup (one wave per row, RMS_ROWS / 4 rows per wave); the workgroup's
// share of dg = sum_r x s dy goes to part[blockIdx.x][D] (summed in a fixed
// order by k_rms_dg or a deferred column sum).  NV float4 columns per lane;
// a wave issues the loads of RB rows before it reduces any of them, so the
// rows' load latencies overlap instead of adding up (loads use clamped,
// in-bounds indices; rows past `rows` and columns past D are masked at use).
#define RMS_ROWS 16
#define RMS_MAXV 8            // float4 columns per lane: D <= 64 * 4 * 8
template <int NV>
__global__ __launch_bounds__(256) void k_rms_bwd(const float *__restrict__ x, const float *__restrict__ g,
                                                 const float *__restrict__ rinv, const float *__restrict__ dy,
                                                 const float *dx_in, float *dx, int rows, int D,
                                                 float *__restrict__ part)
{
    constexpr int PER = RMS_ROWS / 4;                 // rows per wave
    constexpr int RB = NV >= PER ? 1 : PER / NV;      // rows in flight per wave
    __shared__ f32x4 red[3][64 * NV];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d4 = D >> 2;
    const f32x4 *g4 = reinterpret_cast<const f32x4 *>(g);
    f32x4 gv[NV], acc[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        gv[j] = g4[min(lane + 64 * j, d4 - 1)];
        acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int r0 = blockIdx.x * RMS_ROWS + wave;
#pragma unroll
    for (int p = 0; p < PER; p += RB) {
        f32x4 xa[RB][NV], da[RB][NV], ba[RB][NV];
        float s[RB], c[RB];
#pragma unroll
        for (int b = 0; b < RB; b++) {
            const size_t r = (size_t)min(r0 + 4 * (p + b), rows - 1);
            s[b] = rinv[r];
#pragma unroll
            for (int j = 0; j < NV; j++) {
                const size_t i = r * d4 + min(lane + 64 * j, d4 - 1);
                xa[b][j] = reinterpret_cast<const f32x4 *>(x)[i];
                da[b][j] = reinterpret_cast<const f32x4 *>(dy)[i];
                ba[b][j] = dx_in ? reinterpret_cast<const f32x4 *>(dx_in)[i] : f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
#pragma unroll
        for (int b = 0; b < RB; b++) {
            c[b] = 0.f;
#pragma unroll
            for (int j = 0; j < NV; j++) {
                const f32x4 a = xa[b][j], w = gv[j], d = da[b][j];
                if (lane + 64 * j < d4) c[b] += a.x * w.x * d.x + a.y * w.y * d.y + a.z * w.z * d.z + a.w * w.w * d.w;
            }
        }
        for (int o = 32; o > 0; o >>= 1)
#pragma unroll
            for (int b = 0; b < RB; b++) c[b] += __shfl_xor(c[b], o);
#pragma unroll
        for (int b = 0; b < RB; b++) {
            const int r = r0 + 4 * (p + b);
            if (r >= rows) break;
            const float sb = s[b], coef = sb * sb * sb / (float)D * c[b];
            f32x4 *xo = reinterpret_cast<f32x4 *>(dx + (size_t)r * D);
#pragma unroll
            for (int j = 0; j < NV; j++) {
                const int i = lane + 64 * j;
                if (i < d4) {
                    const f32x4 a = xa[b][j], w = gv[j], d = da[b][j], base = ba[b][j];
                    f32x4 o;
                    o.x = base.x + (sb * w.x * d.x - coef * a.x);
                    o.y = base.y + (sb * w.y * d.y - coef * a.y);
                    o.z = base.z + (sb * w.z * d.z - coef * a.z);
                    o.w = base.w + (sb * w.w * d.w - coef * a.w);
                    xo[i] = o;
                    acc[j].x += a.x * sb * d.x;
                    acc[j].y += a.y * sb * d.y;
                    acc[j].z += a.z * sb * d.z;
                    acc[j].w += a.w * sb * d.w;
                }
            }
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int j = 0; j < NV; j++) red[wave - 1][j * 64 + lane] = acc[j];
    }
    __syncthreads();
    if (wave == 0) {
        f32x4 *pr = reinterpret_cast<f32x4 *>(part + (size_t)blockIdx.x * D);
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const int i = lane + 64 * j;
            if (i < d4) {
                f32x4 t = acc[j];
                for (int w = 0; w < 3; w++) t += red[w][j * 64 + lane];
                pr[i] = t;
            }
        }
    }
}

// dg += sum over the nblk partial rows, one wave per float4 column: lane l
// adds partials l, l + 64, ... in order, then a fixed butterfly.
__global__ __launch_bounds__(256) void k_rms_dg(const float *__restrict__ part, int nblk, int D,
                                                float *__restrict__ dg)
{
    const int lane = threadIdx.x & 63;
    const int c = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (c >= (D >> 2)) return;
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int b = lane; b < nblk; b += 64) s += reinterpret_cast<const f32x4 *>(part + (size_t)b * D)[c];
    for (int o = 32; o > 0; o >>= 1) {
        s.x += __shfl_xor(s.x, o);
        s.y += __shfl_xor(s.y, o);
        s.z += __shfl_xor(s.z, o);
        s.w += __shfl_xor(s.w, o);
    }
    if (lane == 0) reinterpret_cast<f32x4 *>(dg)[c] += s;
}

// ----------------------------------------------------------------- rope --
// In place on [rows][nh * hd]: the pair (v[i], v[i + hd/2]) of each head is
// rotated by the angle of row r's position (pos[r], or r % T when pos is
// null); back = 1 applies the transpose (the backward pass).  Positions
// outside the table turn the row into NaN.
__global__ void k_rope(float *__restrict__ buf, const int *__restrict__ pos, int T, int rows, int nh, int hd,
                       const float *__restrict__ cs, const float *__restrict__ sn, int maxpos, int back)
{
    const int half = hd >> 1;
    const size_t total = (size_t)rows * nh * half;
    for (size_t q = (size_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += (size_t)gridDim.x * blockDim.x) {
        const int i = (int)(q % half);
        const size_t rh = q / half;
        const int h = (int)(rh % nh);
        const size_t r = rh / nh;
        const int t = pos ? pos[r] : (int)(r % T);
        float *v = buf + r * nh * hd + (size_t)h * hd;
        if (t < 0 || t >= maxpos) {
            v[i] = NAN;
            v[i + half] = NAN;
            continue;
        }
        const float c = cs[(size_t)t * half + i], s = sn[(size_t)t * half + i];
        const float a = v[i], b = v[i + half];
        if (!back) {
            v[i] = a * c - b * s;
            v[i + half] = b * c + a * s;
        } else {
            v[i] = a * c + b * s;
            v[i + half] = -a * s + b * c;
        }
    }
}

// The same on four consecutive pairs per thread (hd / 2 a multiple of 4,
// 16-byte aligned rows and tables).
__global__ void k_rope4(float *__restrict__ buf, const int *__restrict__ pos, int T, int rows, int nh, int hd,
                        const float *__restrict__ cs, const float *__restrict__ sn, int maxpos, int back)
{
    const int half = hd >> 1, h4 = half >> 2, per_row = nh * h4;
    const int total = rows * per_row;
    for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < total; q += gridDim.x * blockDim.x) {
        const int r = q / per_row, rem = q - r * per_row;
        const int h = rem / h4, i = (rem - h * h4) * 4;
        const int t = pos ? pos[r] : r % T;
        f32x4 *va = reinterpret_cast<f32x4 *>(buf + (size_t)r * nh * hd + h * hd + i);
        f32x4 *vb = reinterpret_cast<f32x4 *>(buf + (size_t)r * nh * hd + h * hd + half + i);
        if (t < 0 || t >= maxpos) {
            *va = f32x4{NAN, NAN, NAN, NAN};
            *vb = f32x4{NAN, NAN, NAN, NAN};
            continue;
        }
        const f32x4 c = *reinterpret_cast<const f32x4 *>(cs + (size_t)t * half + i);
        const f32x4 sv = *reinterpret_cast<const f32x4 *>(sn + (size_t)t * half + i);
        const f32x4 a = *va, b = *vb;
        if (!back) {
            *va = a * c - b * sv;
            *vb = b * c + a * sv;
        } else {
            *va = a * c + b * sv;
            *vb = -a * sv + b * c;
        }
    }
}

// ------------------------------------------------------------ attention --
#define AT_HD 32
// Row (within a 32 x 32 tile) of register r of lane l in the MFMA result.
__device__ __forceinline__ int at_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// 16 contiguous floats from p (16-byte aligned), or zeros when !ok.  p must
// be a valid address either way (callers clamp the row): every load in the
// attention kernels is issued unconditionally and masked afterwards, so the
// compiler counts outstanding loads exactly and a prefetch is not waited for
// at the first branch join after it.
__device__ __forceinline__ void ld16(const float *p, bool ok, float (&o)[16])
{
    const f32x4 *q = reinterpret_cast<const f32x4 *>(p);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const f32x4 t = q[k];
        o[4 * k] = ok ? t.x : 0.f;
        o[4 * k + 1] = ok ? t.y : 0.f;
        o[4 * k + 2] = ok ? t.z : 0.f;
        o[4 * k + 3] = ok ? t.w : 0.f;
    }
}

// Key s is visible from query q: causal, inside the sequence, and inside
// the sliding window when win > 0 (s >= q - win + 1, attn_fwd's lo).
__device__ __forceinline__ bool at_visible(int s, int q, int T, int win)
{
    return s <= q && q < T && (win <= 0 || s > q - win);
}

// Key block kb is visible in full from every valid query of block qb: below
// the diagonal block and, with a window, inside it for the block's last
// query (then also for every earlier one).  Such blocks need no mask.
__device__ __forceinline__ bool at_full(int kb, int qb, int win)
{
    return kb < qb && (win <= 0 || kb * 32 > qb * 32 + 31 - win);
}

// First key block any query of block qb can see.
__device__ __forceinline__ int at_kb0(int qb, int win)
{
    if (win <= 0) return 0;
    const int lo = qb * 32 - win + 1;
    return lo > 0 ? lo / 32 : 0;
}

// K of block kb in the MFMA A layout (row s0 + lane % 32, 16 dims from
// 16 * (lane / 32)) and V in the transposed-B layout (row s0 + at_row(r),
// dim lane % 32); zeros past T.
__device__ __forceinline__ void at_load_kv(const float *kb_, const float *vb_, int kb, int T, int KD, int lane,
                                           float (&kv)[16], float (&vv)[16])
{
    const int s0 = kb * 32, sl = s0 + (lane & 31);
    ld16(kb_ + (size_t)(sl < T ? sl : 0) * KD + 16 * (lane >> 5), sl < T, kv);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int s = s0 + at_row(r, lane);
        const float x = vb_[(size_t)min(s, T - 1) * KD + (lane & 31)];
        vv[r] = s < T ? x : 0.f;
    }
}

// One workgroup per (b, h, 32-query block), heaviest blocks (latest
// queries) first; its four waves take the visible key blocks in turn
// (kb = kb0 + wave, + 4, ...) and their partial softmax states are merged
// in wave order through LDS.  out = softmax(q k^T * scale) v per head (GQA:
// head h reads KV head h / (H / KV)); lse = log2 of the softmax's
// denominator sum_s 2^(s * scale * log2 e) per (row, head), which the
// backward kernels turn back into P with one exp2 per score.
#define AT_W 4
__global__ __launch_bounds__(256) void k_attn_fwd(const float *__restrict__ q, const float *__restrict__ k,
                                                  const float *__restrict__ v, float *__restrict__ out,
                                                  float *__restrict__ lse, int B, int T, int H, int KV, int win,
                                                  float scale)
{
    __shared__ float sm_o[AT_W - 1][16][64];
    __shared__ float sm_m[AT_W - 1][64], sm_l[AT_W - 1][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nqb = (T + 31) >> 5;
    const int item = blockIdx.x;
    const int qb = nqb - 1 - item / (B * H);
    const int bh = item % (B * H);
    const int b = bh / H, h = bh % H, kvh = h / (H / KV);
    const int D = H * AT_HD, KD = KV * AT_HD;
    const int lq = lane & 31, hh = lane >> 5;
    const int qi = qb * 32 + lq;
    const bool qok = qi < T;
    float qv[16];
    ld16(q + (size_t)(b * T + (qok ? qi : 0)) * D + h * AT_HD + 16 * hh, qok, qv);
    const float *kb_ = k + (size_t)b * T * KD + kvh * AT_HD;
    const float *vb_ = v + (size_t)b * T * KD + kvh * AT_HD;
    f32x16 o;
#pragma unroll
    for (int r = 0; r < 16; r++) o[r] = 0.f;
    // scores in the base-2 domain: p = 2^(s * scale * log2(e) - m)
    const float c2 = scale * 1.44269504088896341f;
    float m = -INFINITY, l = 0.f;
    float kn[16], vn[16];                       // next block's K / V (prefetched)
    // block indices clamp to qb: loads past the wave's last block re-read it
    int kb = at_kb0(qb, win) + wave;
    at_load_kv(kb_, vb_, min(kb, qb), T, KD, lane, kn, vn);
    for (; kb <= qb; kb += AT_W) {
        const int s0 = kb * 32;
        float kv[16], vv[16];
#pragma unroll
        for (int j = 0; j < 16; j++) { kv[j] = kn[j]; vv[j] = vn[j]; }
        at_load_kv(kb_, vb_, min(kb + AT_W, qb), T, KD, lane, kn, vn);
        f32x16 st;
#pragma unroll
        for (int r = 0; r < 16; r++) st[r] = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) st = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[j], qv[j], st, 0, 0, 0);
        // st[r] = S^T[s0 + at_row(r)][qi]
        float sc[16], bm = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int s = s0 + at_row(r, lane);
            sc[r] = at_visible(s, qi, T, win) ? st[r] * c2 : -INFINITY;
            bm = fmaxf(bm, sc[r]);
        }
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        const float mn = fmaxf(m, bm);
        const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mn);
        float ps = 0.f, p[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            p[r] = sc[r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sc[r] - mn);
            ps += p[r];
        }
        l = l * alpha + ps;
#pragma unroll
        for (int r = 0; r < 16; r++) o[r] *= alpha;
        // O^T[d][q] += sum_s V[s][d] P^T[s][q]
#pragma unroll
        for (int r = 0; r < 16; r++) o = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[r], p[r], o, 0, 0, 0);
        m = mn;
    }
    if (wave > 0) {
        sm_m[wave - 1][lane] = m;
        sm_l[wave - 1][lane] = l;
#pragma unroll
        for (int r = 0; r < 16; r++) sm_o[wave - 1][r][lane] = o[r];
    }
    __syncthreads();
    if (wave != 0 || !qok) return;
    float M = m;
    for (int w = 0; w < AT_W - 1; w++) M = fmaxf(M, sm_m[w][lane]);
    const float a0 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
    l *= a0;
#pragma unroll
    for (int r = 0; r < 16; r++) o[r] *= a0;
    for (int w = 0; w < AT_W - 1; w++) {
        const float mw = sm_m[w][lane];
        const float aw = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
        l += sm_l[w][lane] * aw;
#pragma unroll
        for (int r = 0; r < 16; r++) o[r] += sm_o[w][r][lane] * aw;
    }
    l += __shfl_xor(l, 32);
    const float inv = 1.0f / l;
    float *orow = out + (size_t)(b * T + qi) * D + h * AT_HD;
#pragma unroll
    for (int g4 = 0; g4 < 4; g4++)
        *reinterpret_cast<f32x4 *>(orow + 8 * g4 + 4 * hh) =
            f32x4{o[4 * g4] * inv, o[4 * g4 + 1] * inv, o[4 * g4 + 2] * inv, o[4 * g4 + 3] * inv};
    if (hh == 0) lse[(size_t)(b * T + qi) * H + h] = M + __builtin_amdgcn_logf(l);
}

// K and V of block kb in the A layout, and K again in the transposed-B
// layout (for dQ = dS K); zeros past T.
__device__ __forceinline__ void at_load_kvk(const float *kb_, const float *vb_, int kb, int T, int KD, int lane,
                                            float (&kv)[16], float (&vv)[16], float (&kk)[16])
{
    const int s0 = kb * 32, sl = s0 + (lane & 31);
    ld16(kb_ + (size_t)(sl < T ? sl : 0) * KD + 16 * (lane >> 5), sl < T, kv);
    ld16(vb_ + (size_t)(sl < T ? sl : 0) * KD + 16 * (lane >> 5), sl < T, vv);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int s = s0 + at_row(r, lane);
        const float x = kb_[(size_t)min(s, T - 1) * KD + (lane & 31)];
        kk[r] = s < T ? x : 0.f;
    }
}

// dQ, one workgroup per (b, h, 32-query block), its waves taking the key
// blocks in turn and summing their partial dQ in wave order; also writes
// Dq = dO . O per (row, head) for k_attn_bwd_dkv.  dS = P (dP - Dq) scale
// (attn_bwd's dsc), dQ = dS K.
__global__ __launch_bounds__(256) void k_attn_bwd_dq(const float *__restrict__ q, const float *__restrict__ k,
                                                     const float *__restrict__ v, const float *__restrict__ o,
                                                     const float *__restrict__ dout, const float *__restrict__ lse,
                                                     float *__restrict__ Dq, float *__restrict__ dq, int B, int T,
                                                     int H, int KV, int win, float scale)
{
    __shared__ float sm_a[AT_W - 1][16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nqb = (T + 31) >> 5;
    const int item = blockIdx.x;
    const int qb = nqb - 1 - item / (B * H);
    const int bh = item % (B * H);
    const int b = bh / H, h = bh % H, kvh = h / (H / KV);
    const int D = H * AT_HD, KD = KV * AT_HD;
    const int lq = lane & 31, hh = lane >> 5;
    const int qi = qb * 32 + lq;
    const bool qok = qi < T;
    const size_t qoff = (size_t)(b * T + (qok ? qi : 0)) * D + h * AT_HD + 16 * hh;
    float qv[16], dov[16], ov[16];
    ld16(q + qoff, qok, qv);
    ld16(dout + qoff, qok, dov);
    ld16(o + qoff, qok, ov);
    float dd = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) dd += dov[j] * ov[j];
    dd += __shfl_xor(dd, 32);
    const size_t rh = (size_t)(b * T + (qok ? qi : 0)) * H + h;
    if (qok && hh == 0 && wave == 0) Dq[rh] = dd;
    const float lsv = lse[rh];
    const float ls = qok ? lsv : 0.f;
    const float *kb_ = k + (size_t)b * T * KD + kvh * AT_HD;
    const float *vb_ = v + (size_t)b * T * KD + kvh * AT_HD;
    const float c2 = scale * 1.44269504088896341f;
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.f;
    float kn[16], vn[16], kkn[16];              // next block (prefetched)
    int kb = at_kb0(qb, win) + wave;
    at_load_kvk(kb_, vb_, min(kb, qb), T, KD, lane, kn, vn, kkn);
    for (; kb <= qb; kb += AT_W) {
        const int s0 = kb * 32;
        float kv[16], vv[16], kk[16];
#pragma unroll
        for (int j = 0; j < 16; j++) { kv[j] = kn[j]; vv[j] = vn[j]; kk[j] = kkn[j]; }
        at_load_kvk(kb_, vb_, min(kb + AT_W, qb), T, KD, lane, kn, vn, kkn);
        f32x16 st, dp;
#pragma unroll
        for (int r = 0; r < 16; r++) { st[r] = 0.f; dp[r] = 0.f; }
#pragma unroll
        for (int j = 0; j < 16; j++) {
            st = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[j], qv[j], st, 0, 0, 0);
            dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[j], dov[j], dp, 0, 0, 0);
        }
        float ds[16];
        if (at_full(kb, qb, win)) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float p = __builtin_amdgcn_exp2f(st[r] * c2 - ls);
                ds[r] = p * (dp[r] - dd) * scale;
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int s = s0 + at_row(r, lane);
                if (at_visible(s, qi, T, win)) {
                    const float p = __builtin_amdgcn_exp2f(st[r] * c2 - ls);
                    ds[r] = p * (dp[r] - dd) * scale;
                } else {
                    ds[r] = 0.f;
                }
            }
        }
        // dQ^T[d][q] += sum_s K[s][d] dS^T[s][q]
#pragma unroll
        for (int r = 0; r < 16; r++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[r], ds[r], acc, 0, 0, 0);
    }
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < 16; r++) sm_a[wave - 1][r][lane] = acc[r];
    }
    __syncthreads();
    if (wave != 0 || !qok) return;
    for (int w = 0; w < AT_W - 1; w++) {
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] += sm_a[w][r][lane];
    }
    float *orow = dq + (size_t)(b * T + qi) * D + h * AT_HD;
#pragma unroll
    for (int g4 = 0; g4 < 4; g4++)
        *reinterpret_cast<f32x4 *>(orow + 8 * g4 + 4 * hh) =
            f32x4{acc[4 * g4], acc[4 * g4 + 1], acc[4 * g4 + 2], acc[4 * g4 + 3]};
}

// rope_apply on an A fragment (lane (row, half) holds dims 16 half + i of the
// row at position t): the partner dims are in lane ^ 32.
__device__ __forceinline__ void at_rot_a(float (&x)[16], int t, int lane, const float *__restrict__ cs,
                                         const float *__restrict__ sn)
{
    const bool hi = lane >= 32;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const f32x4 c = *reinterpret_cast<const f32x4 *>(cs + (size_t)t * 16 + 4 * k);
        const f32x4 s = *reinterpret_cast<const f32x4 *>(sn + (size_t)t * 16 + 4 * k);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float me = x[4 * k + i], pa = __shfl_xor(me, 32);
            x[4 * k + i] = hi ? me * c[i] + pa * s[i] : me * c[i] - pa * s[i];
        }
    }
}

// rope_apply (back = 0) or its transpose (back = 1) on one element per lane:
// dim d = lane % 32 of a row at position t, the partner dim in lane ^ 16.
__device__ __forceinline__ float at_rot_1(float x, int t, int lane, const float *__restrict__ cs,
                                          const float *__restrict__ sn, bool back)
{
    const int i = lane & 15;
    const bool hi = (lane & 16) != 0;
    const float c = cs[(size_t)t * 16 + i], s = sn[(size_t)t * 16 + i], pa = __shfl_xor(x, 16);
    // forward: lo' = lo c - hi s, hi' = hi c + lo s; back: lo = lo' c + hi' s, hi = hi' c - lo' s
    const float sg = (hi != back) ? 1.f : -1.f;
    return x * c + sg * pa * s;
}

// dK, dV: one workgroup per (b, kv head, 32-key block), first key blocks
// (most queries) first.  Its eight waves share the (head, query block) pairs
// that see the block; each accumulates dV = P^T dO and dK = dS^T Q for its
// pairs, and the partials are summed in wave order through LDS.
#define AT_KW 8
__global__ __launch_bounds__(512) void k_attn_bwd_dkv(const float *__restrict__ q, const float *__restrict__ k,
                                                      const float *__restrict__ v, const float *__restrict__ dout,
                                                      const float *__restrict__ lse, const float *__restrict__ Dq,
                                                      float *__restrict__ dk, float *__restrict__ dv, int B, int T,
                                                      int H, int KV, int win, float scale)
{
    __shared__ float red[AT_KW - 1][2][16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nkb = (T + 31) >> 5;
    const int item = blockIdx.x;
    const int kb = item / (B * KV);
    const int bkv = item % (B * KV);
    const int b = bkv / KV, kvh = bkv % KV, G = H / KV;
    const int D = H * AT_HD, KD = KV * AT_HD;
    const int lq = lane & 31, hh = lane >> 5;
    const int s0 = kb * 32, sl = s0 + lq;
    const bool sok = sl < T;
    const size_t koff = (size_t)(b * T + (sok ? sl : 0)) * KD + kvh * AT_HD + 16 * hh;
    float kv[16], vv[16];
    ld16(k + koff, sok, kv);
    ld16(v + koff, sok, vv);
    int qb_last = nkb - 1;
    if (win > 0) qb_last = min(qb_last, (s0 + 31 + win - 1) >> 5);
    const int npairs = G * (qb_last - kb + 1);
    const float c2 = scale * 1.44269504088896341f;
    f32x16 ak, av;
#pragma unroll
    for (int r = 0; r < 16; r++) { ak[r] = 0.f; av[r] = 0.f; }
    for (int pi = wave; pi < npairs; pi += AT_KW) {
        const int h = kvh * G + pi % G;
        const int q0 = (kb + pi / G) * 32;
        const int ql = q0 + lq;
        const bool qok = ql < T;
        const size_t qoff = (size_t)(b * T + (qok ? ql : 0)) * D + h * AT_HD + 16 * hh;
        float qa[16], da[16], dob[16], qbv[16], lr[16], dr[16];
        ld16(q + qoff, qok, qa);
        ld16(dout + qoff, qok, da);
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int qq = q0 + at_row(r, lane);
            const bool ok = qq < T;
            const size_t off = (size_t)(b * T + (ok ? qq : 0)) * D + h * AT_HD + lq;
            const size_t rh = (size_t)(b * T + (ok ? qq : 0)) * H + h;
            const float x0 = dout[off], x1 = q[off], x2 = lse[rh], x3 = Dq[rh];
            dob[r] = ok ? x0 : 0.f;
            qbv[r] = ok ? x1 : 0.f;
            lr[r] = ok ? x2 : 0.f;
            dr[r] = ok ? x3 : 0.f;
        }
        f32x16 st, dp;
#pragma unroll
        for (int r = 0; r < 16; r++) { st[r] = 0.f; dp[r] = 0.f; }
#pragma unroll
        for (int j = 0; j < 16; j++) {
            st = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[j], kv[j], st, 0, 0, 0);
            dp = __builtin_amdgcn_mfma_f32_32x32x2f32(da[j], vv[j], dp, 0, 0, 0);
        }
        // st[r] = S[q0 + at_row(r)][sl], dp likewise
        float pp[16], ds[16];
        // a fully visible pair still masks queries past T (their lse / Dq
        // rows are clamped copies, not zeros)
        if (at_full(kb, q0 >> 5, win) && q0 + 32 <= T) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                pp[r] = __builtin_amdgcn_exp2f(st[r] * c2 - lr[r]);
                ds[r] = pp[r] * (dp[r] - dr[r]) * scale;
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int qq = q0 + at_row(r, lane);
                if (at_visible(sl, qq, T, win)) {
                    pp[r] = __builtin_amdgcn_exp2f(st[r] * c2 - lr[r]);
                    ds[r] = pp[r] * (dp[r] - dr[r]) * scale;
                } else {
                    pp[r] = 0.f;
                    ds[r] = 0.f;
                }
            }
        }
        // dV[s][d] += sum_q P[q][s] dO[q][d];  dK[s][d] += sum_q dS[q][s] Q[q][d]
#pragma unroll
        for (int r = 0; r < 16; r++) {
            av = __builtin_amdgcn_mfma_f32_32x32x2f32(pp[r], dob[r], av, 0, 0, 0);
            ak = __builtin_amdgcn_mfma_f32_32x32x2f32(ds[r], qbv[r], ak, 0, 0, 0);
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            red[wave - 1][0][r][lane] = ak[r];
            red[wave - 1][1][r][lane] = av[r];
        }
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        float a = ak[r], c = av[r];
        for (int w = 0; w < AT_KW - 1; w++) {
            a += red[w][0][r][lane];
            c += red[w][1][r][lane];
        }
        const int s = s0 + at_row(r, lane);
        if (s < T) {
            const size_t off = (size_t)(b * T + s) * KD + kvh * AT_HD + lq;
            dk[off] = a;
            dv[off] = c;
        }
    }
}

// ------------------------------------------------ GQA-group attention --
// Forward and dQ for H / KV a multiple of 4.  One workgroup of 4 A4_KS waves
// per (b, KV head, group of 4 query heads, 32-query block), latest blocks
// first: wave w takes head w % 4 of the group and every A4_KS-th key block
// from w / 4.
// The four heads read the same K / V, so the workgroup stages up to A4_CH
// key blocks at a time in LDS and every wave streams its blocks from there
// with no barrier between blocks (the waves sharing a SIMD drift out of
// phase, so one's softmax overlaps the others' MFMAs); the key splits of
// each head merge through LDS in fixed order.  With ROPE the kernels take q
// and k before rope_apply (tinylm.c:621-651) and rotate them while staging
// -- pair (x[i], x[i + 16]) of a head by the row's position -- so no rotated
// copy reaches HBM; dQ is rotated back before it is stored.
#define A4_LD 36        // LDS row stride of a staged 32 x 32 block (16-byte rows)
#define A4_CH 8         // key blocks staged at once (K + V: 72 KB)
#define A4_KS 2         // key splits per head: 4 heads x 2 splits = 8 waves (4 measured slower)
#define A4_CH2 6        // key blocks staged at once by the 2-head forward items (K + V: 54 KB)
#define A4_FNH 2        // heads per forward item (4 or 2)

// One staging task: dims [4c, 4c + 4) and [16 + 4c, 16 + 4c + 4) of one
// 32-dim head row, rotated by position t when ROPE and `rot`, zeroed when !ok.
template <bool ROPE>
struct A4Task {
    f32x4 a, b, c, s;
    __device__ __forceinline__ void load(const float *__restrict__ row, int c4, int t, bool rot,
                                         const float *__restrict__ cs, const float *__restrict__ sn)
    {
        a = *reinterpret_cast<const f32x4 *>(row + 4 * c4);
        b = *reinterpret_cast<const f32x4 *>(row + 16 + 4 * c4);
        if (ROPE && rot) {
            c = *reinterpret_cast<const f32x4 *>(cs + (size_t)t * 16 + 4 * c4);
            s = *reinterpret_cast<const f32x4 *>(sn + (size_t)t * 16 + 4 * c4);
        }
    }
    __device__ __forceinline__ void rotate(bool rot)
    {
        if (ROPE && rot) {
            const f32x4 x = a * c - b * s, y = b * c + a * s;
            a = x;
            b = y;
        }
    }
    __device__ __forceinline__ void store(float *__restrict__ L, int c4, bool ok) const
    {
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<f32x4 *>(L + 4 * c4) = ok ? a : z;
        *reinterpret_cast<f32x4 *>(L + 16 + 4 * c4) = ok ? b : z;
    }
};

// Item -> (b, kvh, first head h0 of the group, qb), latest query blocks first.
__device__ __forceinline__ void a4_item(int item, int B, int H, int KV, int nqb, int *b, int *kvh, int *h0, int *qb)
{
    const int G = H / KV, HG = G / 4, per = B * KV * HG;
    *qb = nqb - 1 - item / per;
    int r = item % per;
    const int hg = r % HG;
    r /= HG;
    *kvh = r % KV;
    *b = r / KV;
    *h0 = *kvh * G + hg * 4;
}

// Forward item -> (b, kvh, first head h0 of its NH heads, qb).  NH = 4: as
// a4_item.  NH = 2 (two workgroups per CU): the latest query blocks first for
// the first half of the items, then the earliest first, so with items dealt
// round-robin over the CUs one CU's two items see about nqb + 1 key blocks
// together (query block nqb - 1 - j beside j).
template <int NH>
__device__ __forceinline__ void a4f_item(int item, int B, int H, int KV, int nqb, int *b, int *kvh, int *h0,
                                         int *qb)
{
    const int G = H / KV, HG = G / NH, per = B * KV * HG, qhi = (nqb + 1) >> 1;
    if (NH == 4 || item < qhi * per) *qb = nqb - 1 - item / per;
    else *qb = (item - qhi * per) / per;
    int r = item % per;
    const int hg = r % HG;
    r /= HG;
    *kvh = r % KV;
    *b = r / KV;
    *h0 = *kvh * G + hg * NH;
}

// Stage key blocks c0 .. c0 + nb - 1 of (b, kvh): K (rotated with ROPE) into
// Ks[blk][32][A4_LD], V into Vs.  Task = (K or V, block, row, c4), two per
// thread per round with all their loads issued first.
template <bool ROPE>
__device__ __forceinline__ void a4_stage_kv(float *Ks, float *Vs, const float *k, const float *v, int b, int kvh,
                                            int T, int KV, int c0, int nb, const float *cs, const float *sn)
{
    const int ntask = nb * 32 * 4 * 2;           // per block: 32 rows x 4 c4, K and V
    const int nt = blockDim.x;
    for (int t0 = threadIdx.x; t0 < ntask; t0 += 2 * nt) {
        A4Task<ROPE> tk[2];
        bool ok[2], isk[2];
        int slot[2], c4v[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int t = min(t0 + nt * u, ntask - 1);
            const int kv_ = t & 1, rest = t >> 1;             // K / V interleaved
            const int c4 = rest & 3, x = (rest >> 2) & 31, blk = rest >> 7;
            const int s = (c0 + blk) * 32 + x, sc = min(s, T - 1);
            isk[u] = kv_ == 0;
            ok[u] = s < T;
            slot[u] = (blk * 32 + x) * A4_LD;
            c4v[u] = c4;
            tk[u].load((isk[u] ? k : v) + (size_t)(b * T + sc) * (KV * AT_HD) + kvh * AT_HD, c4, sc, isk[u], cs, sn);
        }
#pragma unroll
        for (int u = 0; u < 2; u++) {
            if (t0 + nt * u >= ntask) break;
            tk[u].rotate(isk[u]);
            tk[u].store((isk[u] ? Ks : Vs) + slot[u], c4v[u], ok[u]);
        }
    }
}

// Q of the group's 4 heads for query block qb into Qs[4][32][A4_LD]
// (rotated with ROPE), one task per thread.
template <bool ROPE>
__device__ __forceinline__ void a4_stage_q(float *Qs, const float *q, int b, int h0, int qb, int T, int H,
                                           const float *cs, const float *sn)
{
    const int tid = threadIdx.x, hs = tid >> 7, x = (tid & 127) >> 2, c4 = tid & 3;
    const int qr = qb * 32 + x, qc = min(qr, T - 1);
    const size_t off = (size_t)(b * T + qc) * (H * AT_HD) + (h0 + hs) * AT_HD;
    A4Task<ROPE> tq;
    tq.load(q + off, c4, qc, true, cs, sn);
    tq.rotate(true);
    tq.store(Qs + (hs * 32 + x) * A4_LD, c4, qr < T);
}

// 16 floats of row `row` of a staged block from column 16 * half (the MFMA
// A / B fragment of lane (row, half)).
__device__ __forceinline__ void a4_frag(const float *L, int row, int half, float (&o)[16])
{
    const float *p = L + row * A4_LD + 16 * half;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const f32x4 t = *reinterpret_cast<const f32x4 *>(p + 4 * k);
        o[4 * k] = t.x; o[4 * k + 1] = t.y; o[4 * k + 2] = t.z; o[4 * k + 3] = t.w;
    }
}

template <bool ROPE, int NH>
__global__ __launch_bounds__(512) void k_attn_fwd4(const float *__restrict__ q, const float *__restrict__ k,
                                                   const float *__restrict__ v, float *__restrict__ out,
                                                   float *__restrict__ lse, int B, int T, int H, int KV, int win,
                                                   float scale, const float *__restrict__ cs,
                                                   const float *__restrict__ sn)
{
    // NH heads per item, KS = 8 / NH key splits per head (8 waves), CH key
    // blocks staged at once; K and V staging in one array: its whole extent
    // is the merge area later
    constexpr int KS = 8 / NH, CH = NH == 4 ? A4_CH : A4_CH2;
    __shared__ __attribute__((aligned(16))) float KVs[2 * CH * 32 * A4_LD], Qs[NH * 32 * A4_LD];
    static_assert(2 * CH * 32 * A4_LD >= NH * (KS - 1) * 18 * 64, "merge area");
    float *Ks = KVs, *Vs = KVs + CH * 32 * A4_LD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hs = wave % NH, ks = wave / NH;
    const int nqb = (T + 31) >> 5;
    int b, kvh, h0, qb;
    a4f_item<NH>(blockIdx.x, B, H, KV, nqb, &b, &kvh, &h0, &qb);
    const int h = h0 + hs, D = H * AT_HD;
    const int lq = lane & 31, hh = lane >> 5;
    const int qi = qb * 32 + lq;
    const int kb0 = at_kb0(qb, win);

    if (tid < NH * 128) a4_stage_q<ROPE>(Qs, q, b, h0, qb, T, H, cs, sn);
    const float c2 = scale * 1.44269504088896341f;
    float qv[16];
    f32x16 o;
#pragma unroll
    for (int r = 0; r < 16; r++) o[r] = 0.f;
    float m = -INFINITY, l = 0.f;
    for (int c0 = kb0; c0 <= qb; c0 += CH) {
        const int nb = min(CH, qb - c0 + 1);
        if (c0 > kb0) __syncthreads();          // the previous chunk is read
        a4_stage_kv<ROPE>(Ks, Vs, k, v, b, kvh, T, KV, c0, nb, cs, sn);
        __syncthreads();
        if (c0 == kb0) a4_frag(Qs + hs * 32 * A4_LD, lq, hh, qv);
        for (int kb = c0 + ks; kb < c0 + nb; kb += KS) {
            const float *Kb = Ks + (kb - c0) * 32 * A4_LD, *Vb = Vs + (kb - c0) * 32 * A4_LD;
            float kv[16];
            a4_frag(Kb, lq, hh, kv);
            f32x16 st;
#pragma unroll
            for (int r = 0; r < 16; r++) st[r] = 0.f;
#pragma unroll
            for (int i = 0; i < 16; i++) st = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[i], qv[i], st, 0, 0, 0);
            // st[r] = S^T[kb * 32 + at_row(r)][qi]; only blocks on the
            // diagonal or the window edge are masked
            float p[16], bm = -INFINITY;
            const bool full = at_full(kb, qb, win);
            if (full) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    p[r] = st[r] * c2;
                    bm = fmaxf(bm, p[r]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    p[r] = at_visible(kb * 32 + at_row(r, lane), qi, T, win) ? st[r] * c2 : -INFINITY;
                    bm = fmaxf(bm, p[r]);
                }
            }
            bm = fmaxf(bm, __shfl_xor(bm, 32));
            const float mn = fmaxf(m, bm);
            const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mn);
            float ps = 0.f;
            if (full) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    p[r] = __builtin_amdgcn_exp2f(p[r] - mn);
                    ps += p[r];
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    p[r] = p[r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(p[r] - mn);
                    ps += p[r];
                }
            }
            l = l * alpha + ps;
#pragma unroll
            for (int r = 0; r < 16; r++) o[r] *= alpha;
            // O^T[d][q] += sum_s V[s][d] P^T[s][q]
#pragma unroll
            for (int r = 0; r < 16; r++)
                o = __builtin_amdgcn_mfma_f32_32x32x2f32(Vb[at_row(r, lane) * A4_LD + lq], p[r], o, 0, 0, 0);
            at_reads_first();
            m = mn;
        }
    }
    __syncthreads();
    // the other key splits' states join split 0's in split order (the K / V
    // area is free by now)
    float *mg = Ks + hs * (KS - 1) * 18 * 64;
    if (ks > 0) {
        float *mine = mg + (ks - 1) * 18 * 64;
#pragma unroll
        for (int r = 0; r < 16; r++) mine[r * 64 + lane] = o[r];
        mine[16 * 64 + lane] = m;
        mine[17 * 64 + lane] = l;
    }
    __syncthreads();
    if (ks > 0 || qi >= T) return;
    float M = m;
#pragma unroll
    for (int w = 0; w < KS - 1; w++) M = fmaxf(M, mg[w * 18 * 64 + 16 * 64 + lane]);
    const float a0 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
    l *= a0;
#pragma unroll
    for (int r = 0; r < 16; r++) o[r] *= a0;
#pragma unroll
    for (int w = 0; w < KS - 1; w++) {
        const float *th = mg + w * 18 * 64;
        const float mw = th[16 * 64 + lane];
        const float aw = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
        l += th[17 * 64 + lane] * aw;
#pragma unroll
        for (int r = 0; r < 16; r++) o[r] += th[r * 64 + lane] * aw;
    }
    l += __shfl_xor(l, 32);
    const float inv = 1.0f / l;
#pragma unroll
    for (int r = 0; r < 16; r++) o[r] *= inv;
    float *orow = out + (size_t)(b * T + qi) * D + h * AT_HD;
#pragma unroll
    for (int g4 = 0; g4 < 4; g4++)
        *reinterpret_cast<f32x4 *>(orow + 8 * g4 + 4 * hh) = f32x4{o[4 * g4], o[4 * g4 + 1], o[4 * g4 + 2], o[4 * g4 + 3]};
    if (hh == 0) lse[(size_t)(b * T + qi) * H + h] = M + __builtin_amdgcn_logf(l);
}

// dQ for the same items; also writes Dq = dO . O per (row, head) for the
// dK / dV kernel.
// dS = P (dP - Dq) scale, dQ = dS K (attn_bwd, :750-768).
#define A4_DQ_LDS (2 * A4_CH * 32 * A4_LD + 4 * 32 * A4_LD)    // K, V staging + Q of 4 heads

// One dQ item (a4_item's numbering) on `lds` (A4_DQ_LDS floats).  WDQ: also
// store Dq (else it was computed before and the dK / dV items may read it).
template <bool ROPE, bool WDQ>
__device__ __forceinline__ void attn_dq4_item(float *__restrict__ lds, int item, const float *__restrict__ q,
                                              const float *__restrict__ k, const float *__restrict__ v,
                                              const float *__restrict__ o, const float *__restrict__ dout,
                                              const float *__restrict__ lse, float *__restrict__ Dq,
                                              float *__restrict__ dq, int B, int T, int H, int KV, int win,
                                              float scale, const float *__restrict__ cs,
                                              const float *__restrict__ sn)
{
    // K and V staging in one array: its whole extent is the merge area later
    float *KVs = lds, *Qs = lds + 2 * A4_CH * 32 * A4_LD;
    static_assert(2 * A4_CH * 32 * A4_LD >= 4 * (A4_KS - 1) * 18 * 64, "merge area");
    float *Ks = KVs, *Vs = KVs + A4_CH * 32 * A4_LD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hs = wave & 3, ks = wave >> 2;
    const int nqb = (T + 31) >> 5;
    int b, kvh, h0, qb;
    a4_item(item, B, H, KV, nqb, &b, &kvh, &h0, &qb);
    const int h = h0 + hs, D = H * AT_HD;
    const int lq = lane & 31, hh = lane >> 5;
    const int qi = qb * 32 + lq;
    const bool qok = qi < T;
    const int kb0 = at_kb0(qb, win);

    const size_t qoff = (size_t)(b * T + (qok ? qi : T - 1)) * D + h * AT_HD + 16 * hh;
    float dov[16], ov[16];
    ld16(dout + qoff, qok, dov);
    ld16(o + qoff, qok, ov);
    const size_t rh = (size_t)(b * T + (qok ? qi : T - 1)) * H + h;
    const float lsv = lse[rh];
    if (tid < 512) a4_stage_q<ROPE>(Qs, q, b, h0, qb, T, H, cs, sn);
    float dd = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) dd += dov[i] * ov[i];
    dd += __shfl_xor(dd, 32);
    if (WDQ && qok && hh == 0 && ks == 0) Dq[rh] = dd;
    const float ls = qok ? lsv : 0.f;
    const float c2 = scale * 1.44269504088896341f;
    float qv[16];
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.f;
    for (int c0 = kb0; c0 <= qb; c0 += A4_CH) {
        const int nb = min(A4_CH, qb - c0 + 1);
        if (c0 > kb0) __syncthreads();
        a4_stage_kv<ROPE>(Ks, Vs, k, v, b, kvh, T, KV, c0, nb, cs, sn);
        __syncthreads();
        if (c0 == kb0) a4_frag(Qs + hs * 32 * A4_LD, lq, hh, qv);
        for (int kb = c0 + ks; kb < c0 + nb; kb += A4_KS) {
            const float *Kb = Ks + (kb - c0) * 32 * A4_LD, *Vb = Vs + (kb - c0) * 32 * A4_LD;
            float kv[16], vv[16];
            a4_frag(Kb, lq, hh, kv);
            a4_frag(Vb, lq, hh, vv);
            f32x16 st, dp;
#pragma unroll
            for (int r = 0; r < 16; r++) { st[r] = 0.f; dp[r] = 0.f; }
#pragma unroll
            for (int i = 0; i < 16; i++) {
                st = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[i], qv[i], st, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[i], dov[i], dp, 0, 0, 0);
            }
            float ds[16];
            if (at_full(kb, qb, win)) {
#pragma unroll
                for (int r = 0; r < 16; r++)
                    ds[r] = __builtin_amdgcn_exp2f(st[r] * c2 - ls) * (dp[r] - dd) * scale;
            } else {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const float pr = __builtin_amdgcn_exp2f(st[r] * c2 - ls);
                    ds[r] = at_visible(kb * 32 + at_row(r, lane), qi, T, win) ? pr * (dp[r] - dd) * scale : 0.f;
                }
            }
            // dQ^T[d][q] += sum_s K[s][d] dS^T[s][q]
#pragma unroll
            for (int r = 0; r < 16; r++)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(Kb[at_row(r, lane) * A4_LD + lq], ds[r], acc, 0, 0, 0);
            at_reads_first();
        }
    }
    __syncthreads();
    float *mg = Ks + hs * (A4_KS - 1) * 16 * 64;
    if (ks > 0) {
#pragma unroll
        for (int r = 0; r < 16; r++) mg[((ks - 1) * 16 + r) * 64 + lane] = acc[r];
    }
    __syncthreads();
    if (ks > 0 || !qok) return;
#pragma unroll
    for (int w = 0; w < A4_KS - 1; w++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] += mg[(w * 16 + r) * 64 + lane];
    if (ROPE) {
        // rope_apply's transpose: lane holds dims 8 g + 4 hh + i and the
        // same +16 (registers 4 g + i and 4 (g + 2) + i)
#pragma unroll
        for (int g4 = 0; g4 < 2; g4++) {
            const int d = 8 * g4 + 4 * hh;
            const f32x4 c = *reinterpret_cast<const f32x4 *>(cs + (size_t)qi * 16 + d);
            const f32x4 sn4 = *reinterpret_cast<const f32x4 *>(sn + (size_t)qi * 16 + d);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float a = acc[4 * g4 + i], bb = acc[4 * (g4 + 2) + i];
                acc[4 * g4 + i] = a * c[i] + bb * sn4[i];
                acc[4 * (g4 + 2) + i] = -a * sn4[i] + bb * c[i];
            }
        }
    }
    float *orow = dq + (size_t)(b * T + qi) * D + h * AT_HD;
#pragma unroll
    for (int g4 = 0; g4 < 4; g4++)
        *reinterpret_cast<f32x4 *>(orow + 8 * g4 + 4 * hh) =
            f32x4{acc[4 * g4], acc[4 * g4 + 1], acc[4 * g4 + 2], acc[4 * g4 + 3]};
}

template <bool ROPE>
__global__ __launch_bounds__(64 * 4 * A4_KS) void k_attn_dq4(const float *__restrict__ q, const float *__restrict__ k,
                                                  const float *__restrict__ v, const float *__restrict__ o,
                                                  const float *__restrict__ dout, const float *__restrict__ lse,
                                                  float *__restrict__ Dq, float *__restrict__ dq, int B, int T, int H,
                                                  int KV, int win, float scale, const float *__restrict__ cs,
                                                  const float *__restrict__ sn)
{
    __shared__ __attribute__((aligned(16))) float lds[A4_DQ_LDS];
    attn_dq4_item<ROPE, true>(lds, blockIdx.x, q, k, v, o, dout, lse, Dq, dq, B, T, H, KV, win, scale, cs, sn);
}

// dK / dV for H / KV a multiple of 4.  One workgroup of 8 waves per (b, KV
// head, 32-key block), first key blocks first.  Per step the workgroup
// stages two query blocks of one group of 4 heads in LDS -- q (rotated with
// ROPE), dO, and the rows' lse and Dq, loaded as whole rows -- with the next
// step's loads in flight during this step's MFMAs; wave w takes head w % 4
// and query block w / 4 of the pair.  Its dV = P^T dO and dK = dS^T Q sum
// over its pairs in registers, the 8 waves' sums add in wave order through
// LDS (so every head of the KV group and every query block is summed in a
// fixed order; each thread of the workgroup sums a share of the outputs),
// and dK is rotated back before it is stored.
#define A4_DKV_ST (2 * 4 * 32 * A4_LD)          // one staged array: 2 query blocks x 4 heads x 32 rows

template <bool ROPE>
struct Dkv4Stage {
    A4Task<ROPE> tq[2];       // q rows, query block 0 / 1 of the pair
    f32x4 da[2][2];           // dO rows (the two halves of the head row)
    f32x4 ld;                 // lse or Dq of one row, 4 heads
    bool okq[2], okl;

    // thread task: (head hs, row x, c4) of both query blocks; threads < 128
    // also one lse / Dq float4 (query block tid >> 6, lse or Dq, row)
    __device__ __forceinline__ void load(const float *q, const float *dout, const float *lse, const float *Dq,
                                         int b, int h0, int T, int H, int qb0, int qb_last, const float *cs,
                                         const float *sn)
    {
        const int tid = threadIdx.x, hs = tid >> 7, x = (tid & 127) >> 2, c4 = tid & 3;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int qb = min(qb0 + u, qb_last), qr = qb * 32 + x, qc = min(qr, T - 1);
            okq[u] = qr < T && qb0 + u <= qb_last;
            const size_t off = (size_t)(b * T + qc) * (H * AT_HD) + (h0 + hs) * AT_HD;
            tq[u].load(q + off, c4, qc, true, cs, sn);
            da[u][0] = *reinterpret_cast<const f32x4 *>(dout + off + 4 * c4);
            da[u][1] = *reinterpret_cast<const f32x4 *>(dout + off + 16 + 4 * c4);
        }
        const int u = (tid >> 6) & 1, isd = (tid >> 5) & 1, xr = tid & 31;
        const int qb = min(qb0 + u, qb_last), qr = qb * 32 + xr, qc = min(qr, T - 1);
        okl = qr < T && qb0 + u <= qb_last;
        ld = *reinterpret_cast<const f32x4 *>((isd ? Dq : lse) + (size_t)(b * T + qc) * H + h0);
    }
    __device__ __forceinline__ void store(float *Qs, float *Ds, float *LDs)
    {
        const int tid = threadIdx.x, hs = tid >> 7, x = (tid & 127) >> 2, c4 = tid & 3;
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int row = ((u * 4 + hs) * 32 + x) * A4_LD;
            tq[u].rotate(true);
            tq[u].store(Qs + row, c4, okq[u]);
            *reinterpret_cast<f32x4 *>(Ds + row + 4 * c4) = okq[u] ? da[u][0] : z;
            *reinterpret_cast<f32x4 *>(Ds + row + 16 + 4 * c4) = okq[u] ? da[u][1] : z;
        }
        if (tid < 128) {
            const int u = (tid >> 6) & 1, isd = (tid >> 5) & 1, xr = tid & 31;
            *reinterpret_cast<f32x4 *>(LDs + ((isd * 2 + u) * 32 + xr) * 4) = okl ? ld : z;
        }
    }
};

#define A4_DKV_LDS (2 * A4_DKV_ST + 2 * 2 * 32 * 4)

// One dK / dV item (key block item / (B KV), first ones first) on `Sm`
// (A4_DKV_LDS floats): staged q, dO (2 query blocks x 4 heads) and lse / Dq;
// the wave sums at the end reuse it.
template <bool ROPE>
__device__ __forceinline__ void attn_dkv4_item(float *__restrict__ Sm, int item, const float *__restrict__ q,
                                               const float *__restrict__ k, const float *__restrict__ v,
                                               const float *__restrict__ dout, const float *__restrict__ lse,
                                               const float *__restrict__ Dq, float *__restrict__ dk,
                                               float *__restrict__ dv, int B, int T, int H, int KV, int win,
                                               float scale, const float *__restrict__ cs,
                                               const float *__restrict__ sn)
{
    static_assert(2 * A4_DKV_ST >= 8 * 2 * 16 * 64, "wave sums fit the staging area");
    float *Qs = Sm, *Ds = Sm + A4_DKV_ST, *LDs = Sm + 2 * A4_DKV_ST;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, hs = wave & 3, qs = wave >> 2;
    const int nkb = (T + 31) >> 5;
    const int kb = item / (B * KV), bkv = item % (B * KV);
    const int b = bkv / KV, kvh = bkv % KV, G = H / KV, HG = G / 4;
    const int KD = KV * AT_HD;
    const int lq = lane & 31, hh = lane >> 5;
    const int s0 = kb * 32, sl = s0 + lq;
    const bool sok = sl < T;
    int qb_last = nkb - 1;
    if (win > 0) qb_last = min(qb_last, (s0 + 31 + win - 1) >> 5);
    const int nch = (qb_last - kb + 2) >> 1, nsteps = HG * nch;

    Dkv4Stage<ROPE> stg;
    stg.load(q, dout, lse, Dq, b, kvh * G, T, H, kb, qb_last, cs, sn);
    const size_t koff = (size_t)(b * T + (sok ? sl : T - 1)) * KD + kvh * AT_HD + 16 * hh;
    float kv[16], vv[16];
    ld16(k + koff, sok, kv);
    ld16(v + koff, sok, vv);
    if (ROPE) at_rot_a(kv, sok ? sl : T - 1, lane, cs, sn);
    const float c2 = scale * 1.44269504088896341f;
    f32x16 ak, av;
#pragma unroll
    for (int r = 0; r < 16; r++) { ak[r] = 0.f; av[r] = 0.f; }
    for (int st = 0; st < nsteps; st++) {
        const int qb = kb + 2 * (st % nch) + qs;
        stg.store(Qs, Ds, LDs);
        __syncthreads();
        {   // the next step's rows in flight (the last step re-reads its own)
            const int nx = min(st + 1, nsteps - 1);
            stg.load(q, dout, lse, Dq, b, kvh * G + (nx / nch) * 4, T, H, kb + 2 * (nx % nch), qb_last, cs, sn);
        }
        if (qb <= qb_last) {
            const float *Qw = Qs + (qs * 4 + hs) * 32 * A4_LD, *Dw = Ds + (qs * 4 + hs) * 32 * A4_LD;
            const float *Lw = LDs + qs * 32 * 4, *Pw = LDs + (2 + qs) * 32 * 4;
            float qa[16], da[16];
            a4_frag(Qw, lq, hh, qa);
            a4_frag(Dw, lq, hh, da);
            f32x16 sc, dp;
#pragma unroll
            for (int r = 0; r < 16; r++) { sc[r] = 0.f; dp[r] = 0.f; }
#pragma unroll
            for (int i = 0; i < 16; i++) {
                sc = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[i], kv[i], sc, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x2f32(da[i], vv[i], dp, 0, 0, 0);
            }
            // sc[r] = S[qb * 32 + at_row(r)][sl], dp likewise
            const bool full = at_full(kb, qb, win);
            float pp[16], ds[16];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int x = at_row(r, lane);
                const float lr = Lw[x * 4 + hs], dr = Pw[x * 4 + hs];
                const bool vis = full || at_visible(sl, qb * 32 + x, T, win);
                const float p = __builtin_amdgcn_exp2f(sc[r] * c2 - lr);
                pp[r] = vis ? p : 0.f;
                ds[r] = vis ? p * (dp[r] - dr) * scale : 0.f;
            }
            // dV[s][d] += sum_q P[q][s] dO[q][d];  dK[s][d] += sum_q dS[q][s] Q[q][d]
#if TLG_ATT_SCHED
            __builtin_amdgcn_sched_barrier(0);      // this loop is a region of its own
#endif
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int x = at_row(r, lane);
                av = __builtin_amdgcn_mfma_f32_32x32x2f32(pp[r], Dw[x * A4_LD + lq], av, 0, 0, 0);
                ak = __builtin_amdgcn_mfma_f32_32x32x2f32(ds[r], Qw[x * A4_LD + lq], ak, 0, 0, 0);
            }
            at_reads_first();
        }
        __syncthreads();
    }
    // the 8 waves' sums, in wave order, spread over the workgroup: thread t
    // adds dK's pair of columns (d, d + 16) of MFMA register t / 32 (the RoPE
    // pair, rotated back together) and two of dV's values
    float *red = Sm;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        red[((wave * 2 + 0) * 16 + r) * 64 + lane] = ak[r];
        red[((wave * 2 + 1) * 16 + r) * 64 + lane] = av[r];
    }
    __syncthreads();
    const size_t obase = (size_t)b * T * KD + kvh * AT_HD;
    {
        const int r = tid >> 5, lp = tid & 31;
        const int l0 = (lp & 15) | ((lp & 16) << 1), l1 = l0 | 16;     // same row, columns d and d + 16
        float a0 = red[(0 * 16 + r) * 64 + l0], a1 = red[(0 * 16 + r) * 64 + l1];
#pragma unroll
        for (int w = 1; w < 8; w++) {
            a0 += red[((w * 2) * 16 + r) * 64 + l0];
            a1 += red[((w * 2) * 16 + r) * 64 + l1];
        }
        const int s = s0 + at_row(r, l0);
        if (ROPE) {
            // rope_apply's transpose of the pair: lo = lo' c + hi' s, hi = hi' c - lo' s
            const int t = min(s, T - 1), i = l0 & 15;
            const float c = cs[(size_t)t * 16 + i], sv = sn[(size_t)t * 16 + i];
            const float lo = a0 * c + a1 * sv, hi = a1 * c - a0 * sv;
            a0 = lo;
            a1 = hi;
        }
        if (s < T) {
            dk[obase + (size_t)s * KD + (l0 & 31)] = a0;
            dk[obase + (size_t)s * KD + (l1 & 31)] = a1;
        }
    }
#pragma unroll
    for (int k2 = 0; k2 < 2; k2++) {
        const int e = tid + 512 * k2, r = e >> 6, l = e & 63;
        float c = red[(16 + r) * 64 + l];
#pragma unroll
        for (int w = 1; w < 8; w++) c += red[((w * 2 + 1) * 16 + r) * 64 + l];
        const int s = s0 + at_row(r, l);
        if (s < T) dv[obase + (size_t)s * KD + (l & 31)] = c;
    }
}

// Dq[row][h] = dO[row][h] . O[row][h] (attn_bwd's per-row term, tinylm.c:750-768)
// in the dQ item's order: the two 16-term halves, then their sum.  Eight lanes
// per (row, head), lane q holding float4 q of both rows, so a wave's loads are
// 1 KB contiguous; each half's chain passes through its four lanes in order
// (lane q continues the sum lane q - 1 ended with).
__global__ __launch_bounds__(256) void k_attn_delta(const float *__restrict__ dout, const float *__restrict__ o,
                                                    float *__restrict__ Dq, int n)
{
    const int q = threadIdx.x & 7;
    const int t = (blockIdx.x * 256 + threadIdx.x) >> 3;     // (row, head) = row * H + h
    const size_t tc = (size_t)min(t, n - 1);                 // every lane takes part in the shuffles
    const f32x4 x = reinterpret_cast<const f32x4 *>(dout)[tc * (AT_HD / 4) + q];
    const f32x4 y = reinterpret_cast<const f32x4 *>(o)[tc * (AT_HD / 4) + q];
    float d = 0.f;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const float in = __shfl_up(d, 1, 4);
        if ((q & 3) == s) {
            float c = s ? in : 0.f;
            c += x[0] * y[0];
            c += x[1] * y[1];
            c += x[2] * y[2];
            c += x[3] * y[3];
            d = c;
        }
    }
    const float h0 = __shfl_up(d, 4, 8);
    if (q == 7 && t < n) Dq[t] = h0 + d;
}

// dQ and dK / dV in one launch, after k_attn_delta: workgroups
// 0 .. nkb B KV - 1 take the dK / dV items (first key blocks first, the
// longest), the rest the dQ items (last query blocks first, the longest).
// The two kinds are long at opposite ends of the causal triangle, so CUs
// freed by short dK / dV items start the long dQ items while the long dK /
// dV items still run (as two launches: dQ 22 us, dK / dV 30 us per m3
// layer).
template <bool ROPE>
__global__ __launch_bounds__(512) void k_attn_bwd4(const float *__restrict__ q, const float *__restrict__ k,
                                                   const float *__restrict__ v, const float *__restrict__ o,
                                                   const float *__restrict__ dout, const float *__restrict__ lse,
                                                   const float *__restrict__ Dq, float *__restrict__ dq,
                                                   float *__restrict__ dk, float *__restrict__ dv, int B, int T,
                                                   int H, int KV, int win, float scale,
                                                   const float *__restrict__ cs, const float *__restrict__ sn)
{
    static_assert(64 * 4 * A4_KS == 512, "both item kinds run 8 waves");
    __shared__ __attribute__((aligned(16))) float lds[A4_DQ_LDS > A4_DKV_LDS ? A4_DQ_LDS : A4_DKV_LDS];
    const int ndkv = ((T + 31) >> 5) * B * KV;
    if ((int)blockIdx.x < ndkv)
        attn_dkv4_item<ROPE>(lds, blockIdx.x, q, k, v, dout, lse, Dq, dk, dv, B, T, H, KV, win, scale, cs, sn);
    else
        attn_dq4_item<ROPE, false>(lds, blockIdx.x - ndkv, q, k, v, o, dout, lse, nullptr, dq, B, T, H, KV, win,
                                   scale, cs, sn);
}

// ----------------------------------------------------------- elementwise --
enum { EW_ADD = 0, EW_SWIGLU = 1, EW_SWIGLU_BWD = 2, EW_SILU_RES = 3, EW_SILU_BWD = 4 };

// ADD:        y += x
// SWIGLU:     y = silu(a) * b                     silu(z) = z / (1 + e^-z)
// SWIGLU_BWD: y = dact * b * silu'(a), y2 = dact * silu(a)   (dact = x)
// SILU_RES:   y = x + silu(a)                     (MTP's hk = fn + silu(t1))
// SILU_BWD:   y = x * silu'(a)                    (MTP's dt1)
__global__ void k_ew(int op, size_t n, float *__restrict__ y, float *__restrict__ y2, const float *__restrict__ x,
                     const float *__restrict__ a, const float *__restrict__ bb)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        switch (op) {
        case EW_ADD: y[i] += x[i]; break;
        case EW_SWIGLU: {
            const float z = a[i];
            y[i] = z / (1.0f + expf(-z)) * bb[i];
            break;
        }
        case EW_SWIGLU_BWD: {
            const float z = a[i], d = x[i];
            const float sg = 1.0f / (1.0f + expf(-z));
            const float si = z * sg, ds = sg + z * sg * (1.0f - sg);
            y[i] = d * bb[i] * ds;
            y2[i] = d * si;
            break;
        }
        case EW_SILU_RES: {
            const float z = a[i];
            y[i] = x[i] + z / (1.0f + expf(-z));
            break;
        }
        default: {
            const float z = a[i];
            const float sg = 1.0f / (1.0f + expf(-z));
            y[i] = x[i] * (sg + z * sg * (1.0f - sg));
            break;
        }
        }
    }
}

// ---------------------------------------------------- softmax + CE rows --
// One wave per row of logits[N][V]: p = softmax(row), dl = p * scale with
// scale subtracted at the target; rowloss[r] = -log(p[target] + 1e-12) in
// double when rowloss is given.  A target outside [0, V) gives a NaN loss.
__global__ __launch_bounds__(256) void k_xent(const float *__restrict__ logits, const int *__restrict__ tgt,
                                              float *__restrict__ dl, double *__restrict__ rowloss, float scale,
                                              int N, int V)
{
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= N) return;
    const float *lg = logits + (size_t)r * V;
    float mx = -INFINITY;
    for (int i = lane; i < V; i += 64) mx = fmaxf(mx, lg[i]);
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float sum = 0.f;
    for (int i = lane; i < V; i += 64) sum += expf(lg[i] - mx);
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    const float inv = 1.0f / sum;
    const int t = tgt[r];
    float *d = dl + (size_t)r * V;
    for (int i = lane; i < V; i += 64) {
        const float p = expf(lg[i] - mx) * inv;
        float g = p * scale;
        if (i == t) {
            g -= scale;
            if (rowloss) rowloss[r] = -log((double)p + 1e-12);
        }
        d[i] = g;
    }
    if (rowloss && lane == 0 && (t < 0 || t >= V)) rowloss[r] = NAN;
}

// The same with the row held in registers (V % 4 == 0, V <= 256 * XV):
// one read of the logits, and each e^(l - max) evaluated once and used for
// both the sum and the probability, as the reference's loop does.
#define XENT_XV 8
__global__ __launch_bounds__(256) void k_xent_reg(const float *__restrict__ logits, const int *__restrict__ tgt,
                                                  float *__restrict__ dl, double *__restrict__ rowloss, float scale,
                                                  int N, int V)
{
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= N) return;
    const int v4 = V >> 2;
    const f32x4 *lg = reinterpret_cast<const f32x4 *>(logits + (size_t)r * V);
    f32x4 x[XENT_XV];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < XENT_XV; j++) {
        const int i = lane + 64 * j;
        x[j] = i < v4 ? lg[i] : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        mx = fmaxf(mx, fmaxf(fmaxf(x[j].x, x[j].y), fmaxf(x[j].z, x[j].w)));
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < XENT_XV; j++) {
        x[j] = f32x4{expf(x[j].x - mx), expf(x[j].y - mx), expf(x[j].z - mx), expf(x[j].w - mx)};
        sum += (x[j].x + x[j].y) + (x[j].z + x[j].w);
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    const float inv = 1.0f / sum;
    const int t = tgt[r];
    f32x4 *d = reinterpret_cast<f32x4 *>(dl + (size_t)r * V);
#pragma unroll
    for (int j = 0; j < XENT_XV; j++) {
        const int i = lane + 64 * j;
        if (i >= v4) continue;
        const f32x4 p = x[j] * inv;
        f32x4 g = p * scale;
        if ((t >> 2) == i) {
            const int c = t & 3;
            const float pt = c == 0 ? p.x : c == 1 ? p.y : c == 2 ? p.z : p.w;
            if (c == 0) g.x -= scale;
            else if (c == 1) g.y -= scale;
            else if (c == 2) g.z -= scale;
            else g.w -= scale;
            if (rowloss) rowloss[r] = -log((double)pt + 1e-12);
        }
        d[i] = g;
    }
    if (rowloss && lane == 0 && (t < 0 || t >= V)) rowloss[r] = NAN;
}

// Sum of n doubles by one workgroup in a fixed order; out = (float)(sum / n).
// the mean of rowloss[0, n) by 1024 threads: strided per-thread sums, then a
// fixed tree over them (s: 1024 doubles of LDS)
__device__ __forceinline__ void sum_loss_1024(const double *__restrict__ rowloss, int n, float *__restrict__ out,
                                              double *s)
{
    double a = 0.0;
    for (int i = threadIdx.x; i < n; i += 1024) a += rowloss[i];
    s[threadIdx.x] = a;
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) s[threadIdx.x] += s[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = (float)(s[0] / n);
}

__global__ __launch_bounds__(1024) void k_sum_loss(const double *__restrict__ rowloss, int n, float *__restrict__ out)
{
    __shared__ double s[1024];
    sum_loss_1024(rowloss, n, out, s);
}

// ------------------------------------------------------ gradnorm, AdamW --
#define GN_BLOCKS 1024
// n4: the float4 columns of G read as float4 (n / 4 when G is 16-byte
// aligned, else 0); elements from 4 n4 on are read one by one.
__global__ __launch_bounds__(256) void k_sumsq(const float *__restrict__ G, size_t n, size_t n4,
                                               double *__restrict__ part)
{
    __shared__ double s[256];
    double a = 0.0;
    const f32x4 *G4 = reinterpret_cast<const f32x4 *>(G);
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)GN_BLOCKS * 256) {
        const f32x4 v = G4[i];
        a += (double)v.x * v.x;
        a += (double)v.y * v.y;
        a += (double)v.z * v.z;
        a += (double)v.w * v.w;
    }
    for (size_t i = 4 * n4 + (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)GN_BLOCKS * 256) {
        const double g = G[i];
        a += g * g;
    }
    s[threadIdx.x] = a;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) s[threadIdx.x] += s[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = s[0];
}

// With rowloss: also loss[0] = the mean of rowloss[0, n), exactly as
// k_sum_loss forms it (after the norm, in the same LDS).
__global__ __launch_bounds__(1024) void k_norm_final(const double *__restrict__ part, float *__restrict__ norm,
                                                     const double *__restrict__ rowloss, int n,
                                                     float *__restrict__ loss)
{
    __shared__ double s[1024];
    s[threadIdx.x] = part[threadIdx.x];
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) s[threadIdx.x] += s[threadIdx.x + o];
        __syncthreads();
    }
    if (threadIdx.x == 0) norm[0] = (float)sqrt(s[0]);
    if (!rowloss) return;
    __syncthreads();                      // s[0] is read before the loss sum reuses s
    sum_loss_1024(rowloss, n, loss, s);
}

// hyper = {lr, b1, b2, wd, bc1, bc2}; gscale = 1 / norm when norm > 1.
__global__ __launch_bounds__(256) void k_adamw(float *__restrict__ P, const float *__restrict__ G,
                                               float *__restrict__ M, float *__restrict__ Vv, size_t n,
                                               const float *__restrict__ hyper, const float *__restrict__ norm)
{
    const float lr = hyper[0], b1 = hyper[1], b2 = hyper[2], wd = hyper[3], bc1 = hyper[4], bc2 = hyper[5];
    float gs = 1.0f;
    if (norm) {
        const float gn = norm[0];
        gs = gn > 1.0f ? 1.0f / gn : 1.0f;
    }
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float g = G[i] * gs;
        const float m = b1 * M[i] + (1 - b1) * g;
        const float vv = b2 * Vv[i] + (1 - b2) * g * g;
        M[i] = m;
        Vv[i] = vv;
        const float mh = m / bc1, vh = vv / bc2;
        P[i] -= lr * (mh / (sqrtf(vh) + 1e-8f) + wd * P[i]);
    }
}

// ============================================================== entries ==
#define ST(s) ((hipStream_t)(s))
#define LAUNCH_CHECK() TLG_HIP(hipGetLastError())

extern "C" int tlg_dev_embed_fwd(float *out, const float *emb, const int *tok, int N, int D, int V, void *stream)
{
    int rc = begin();
    if (rc) return rc;
    if (N < 0 || D <= 0 || V <= 0 || D % 4 || !al16(out) || !al16(emb))
        return tlg_fail(TLG_EINVAL, "embed_fwd: N=%d D=%d V=%d (D %% 4 == 0, aligned rows)", N, D, V);
    if (N == 0) return TLG_OK;
    hipLaunchKernelGGL(k_embed_fwd, dim3(grid_for((size_t)N * D / 4, 256, 8192)), dim3(256), 0, ST(stream), emb,
                       tok, N, D, V, out);
    LAUNCH_CHECK();
    return TLG_OK;
}

extern "C" int tlg_dev_embed_bwd(float *demb, const float *dout, const int *tok, int N, int D, int V, void *stream)
{
    int rc = begin();
    if (rc) return rc;
    if (N < 0 || D <= 0 || V <= 0) return tlg_fail(TLG_EINVAL, "embed_bwd: N=%d D=%d V=%d", N, D, V);
    if (N == 0) return TLG_OK;
    const int nv = (D / 4 + 63) / 64;
    // the one-launch form has each of the V / 8 workgroups scan all N ids
    // (V N / 2 bytes of id reads in all): beyond V N = 2^26 (32 MB of scans,
    // ~10x the m3 step's 2048 x 4096) the counting sort, which reads each id
    // a fixed number of times, takes over
    if (D % 4 == 0 && nv <= 4 && al16(demb) && al16(dout) && N < (1 << 28) && (long long)V * N <= (1LL << 26)) {
        const dim3 grid((V + EMB_VB - 1) / EMB_VB);
        hipStream_t st = ST(stream);
        if (nv == 1) hipLaunchKernelGGL(k_embed_bwd1<1>, grid, dim3(256), 0, st, dout, tok, N, D, V, demb);
        else if (nv == 2) hipLaunchKernelGGL(k_embed_bwd1<2>, grid, dim3(256), 0, st, dout, tok, N, D, V, demb);
        else hipLaunchKernelGGL(k_embed_bwd1<4>, grid, dim3(256), 0, st, dout, tok, N, D, V, demb);
        LAUNCH_CHECK();
        return TLG_OK;
    }
    void *ws;
    const size_t vb = ((size_t)(V + 1) * 4 + 255) & ~(size_t)255;
    if ((rc = tr_scratch(3 * vb + (size_t)N * 4, &ws))) return rc;
    int *cnt = (int *)ws, *off = (int *)((char *)ws + vb), *cur = (int *)((char *)ws + 2 * vb);
    int *idx = (int *)((char *)ws + 3 * vb);
    hipStream_t st = ST(stream);
    hipLaunchKernelGGL(k_fill_int, dim3(grid_for(V, 256, 1024)), dim3(256), 0, st, cnt, V, 0);
    hipLaunchKernelGGL(k_tok_count, dim3(grid_for(N, 256, 1024)), dim3(256), 0, st, tok, N, V, cnt);
    hipLaunchKernelGGL(k_tok_scan, dim3(1), dim3(1024), 0, st, cnt, V, off, cur);
    hipLaunchKernelGGL(k_tok_place, dim3(grid_for(N, 256, 1024)), dim3(256), 0, st, tok, N, V, cur, idx);
    hipLaunchKernelGGL(k_embed_bwd, dim3((V + 3) / 4), dim3(256), 0, st, dout, off, idx, V, D, demb);
    LAUNCH_CHECK();
    return TLG_OK;
}

extern "C" int tlg_dev_rmsnorm_fwd(const float *x, const float *g, float *out, float *rinv, int rows, int D,
                                   void *stream)
{
    int rc = begin();
    if (rc) return rc;
    if (rows < 0 || D <= 0 || D % 4 || !al16(x) || !al16(g) || !al16(out))
        return tlg_fail(TLG_EINVAL, "rmsnorm_fwd: rows=%d D=%d (D %% 4 == 0, aligned rows)", rows, D);
    if (rows == 0) return TLG_OK;
    const dim3 grid((rows + 3) / 4);
    const int nv = (D / 4 + 63) / 64;
    if (nv <= 1)
        hipLaunchKernelGGL(k_rms_fwd<1>, grid, dim3(256), 0, ST(stream), x, g, out, rinv, rows, D,
                           (const int *)nullptr, 0, (float *)nullptr);
    else if (nv <= 2)
        hipLaunchKernelGGL(k_rms_fwd<2>, grid, dim3(256), 0, ST(stream), x, g, out, rinv, rows, D,
                           (const int *)nullptr, 0, (float *)nullptr);
    else if (nv <= 4)
        hipLaunchKernelGGL(k_rms_fwd<4>, grid, dim3(256), 0, ST(stream), x, g, out, rinv, rows, D,
                           (const int *)nullptr, 0, (float *)nullptr);
    else if (nv <= 8)
        hipLaunchKernelGGL(k_rms_fwd<8>, grid, dim3(256), 0, ST(stream), x, g, out, rinv, rows, D,
                           (const int *)nullptr, 0, (float *)nullptr);
    else
        hipLaunchKernelGGL(k_rms_fwd<0>, grid, dim3(256), 0, ST(stream), x, g, out, rinv, rows, D,
                           (const int *)nullptr, 0, (float *)nullptr);
    LAUNCH_CHECK();
    return TLG_OK;
}

extern "C" int tlg_dev_embed_rmsnorm_fwd(const float *emb, const int *tok, int V, float *x, const float *g, float *out,
                                         float *rinv, int N, int D, void *stream)
{
    int rc = begin();
    if (rc) return rc;
    const int nv = (D / 4 + 63) / 64;
    if (N < 0 || D <= 0 || D % 4 || V <= 0 || !tok || !al16(emb) || !al16(x) || !al16(g) || !al16(out))
        return tlg_fail(TLG_EINVAL, "embed_rmsnorm_fwd: N=%d D=%d V=%d (D %% 4 == 0, aligned rows)", N, D, V);
    if (N == 0) return TLG_OK;
    if (nv > 8) {        // rows wider than 2048: the two passes
        if ((rc = tlg_dev_embed_fwd(x, emb, tok, N, D, V, stream))) return rc;
        return tlg_dev_rmsnorm_fwd(x, g, out, rinv, N, D, stream);
    }
    const dim3 grid((N + 3) / 4);
    hipStream_t st = ST(stream);
    if (nv <= 1)
        hipLaunchKernelGGL(k_rms_fwd<1>, grid, dim3(256), 0, st, emb, g, out, rinv, N, D, tok, V, x);
    else if (nv <= 2)
        hipLaunchKernelGGL(k_rms_fwd<2>, grid, dim3(256), 0, st, emb, g, out, rinv, N, D, tok, V, x);
    else if (nv <= 4)
        hipLaunchKernelGGL(k_rms_fwd<4>, grid, dim3(256), 0, st, emb, g, out, rinv, N, D, tok, V, x);
    else
        hipLaunchKernelGGL(k_rms_fwd<8>, grid, dim3(256), 0, st, emb, g, out, rinv, N, D, tok, V, x);
    LAUNCH_CHECK();
    return TLG_OK;
}

static void rms_bwd_launch(const float *x, const float *g, const float *rinv, const float *dy, const float *dx_in,
                           float *dx, int rows, int D, float *part, int nblk, hipStream_t st)
{
    const int nv = (D / 4 + 63) / 64;
    if (nv <= 1)
        hipLaunchKernelGGL(k_rms_bwd<1>, dim3(nblk), dim3(256), 0, st, x, g, rinv, dy, dx_in, dx, rows, D, part);
    else if (nv <= 2)
        hipLaunchKernelGGL(k_rms_bwd<2>, dim3(nblk), dim3(256), 0, st, x, g, rinv, dy, dx_in, dx, rows, D, part);
    else if (nv <= 4)
        hipLaunchKernelGGL(k_rms_bwd<4>, dim3(nblk), dim3(256), 0, st, x, g, rinv, dy, dx_in, dx, rows, D, part);
    else
        hipLaunchKernelGGL(k_rms_bwd<8>, dim3(nblk), dim3(256), 0, st, x, g, rinv, dy, dx_in, dx, rows, D, part);
}

extern "C" int tlg_dev_rmsnorm_bwd(const float *x, const float *g, const float *rinv, const float *dy,
                                   const float *dx_in, float *dx, float *dg, int rows, int D, void *stream)
{
    int rc = begin();
    if (rc) return rc;
    if (rows < 0 || D <= 0 || D % 4 || D > 256 * RMS_MAXV || !al16(x) || !al16(g) || !al16(dy) || !al16(dx) ||
        !al16(dg) || (dx_in && !al16(dx_in)))
        return tlg_fail(TLG_EINVAL, "rmsnorm_bwd: rows=%d D=%d (D %% 4 == 0, D <= %d, aligned rows)", rows, D,
                        256 * RMS_MAXV);
    if (rows == 0) return TLG_OK;
    const int nblk = (rows + RMS_ROWS - 1) / RMS_ROWS;
    void *ws;
    if ((rc = tr_scratch((size_t)nblk * D * 4, &ws))) return rc;
    hipStream_t st = ST(stream);
    rms_bwd_launch(x, g, rinv, dy, dx_in, dx, rows, D, (float *)ws, nblk, st);
    hipLaunchKernelGGL(k_rms_dg, dim3((D / 4 + 3) / 4), dim3(256), 0, st, (const float *)ws, nblk, D, dg);
    LAUNCH_CHECK();
    return TLG_OK;
}

extern "C" int tlg_dev_rmsnorm_bwd_defer(const float *x, const float *g, const float *rinv, const float *dy,
                                         const float *dx_in, float *dx, float *dg, int rows, int D, float *part,
                                         size_t part_floats, void *stream)
{
    int rc = begin();
    if (rc) return rc;
    if (rows < 0 || D <= 0 || D % 4 || D > 256 * RMS_MAXV || !al16(x) || !al16(g) || !al16(dy) || !al16(dx) ||
        !al16(dg) || (dx_in && !al16(dx_in)) || !part || !al16(part))
        return tlg_fail(TLG_EINVAL, "rmsnorm_bwd_defer: rows=%d D=%d (D %% 4 == 0, D <= %d, aligned rows)", rows,
                        D, 256 * RMS_MAXV);
    if (rows == 0) return TLG_OK;
    const int nblk = (rows + RMS_ROWS - 1) / RMS_ROWS;
    if (part_floats < (size_t)nblk * D)
        return tlg_fail(TLG_EINVAL, "rmsnorm_bwd_defer: partials need %zu floats, have %zu", (size_t)nblk * D,
                        part_floats);
    hipStream_t st = ST(stream);
    // a column sum still queued on these partials lands before they are rewritten
    if ((rc = tlg_defer_colsum(part, dg, nblk, D, 1, st))) return rc;
    rms_bwd_launch(x, g, rinv, dy, dx_in, dx, rows, D, part, nblk, st);
    LAUNCH_CHECK();
    return TLG_OK;
}

extern "C" int tlg_dev_rope(float *buf, const int *pos, int T, int rows, int nheads, int hd, const float *cos_t,
                            const float *sin_t, int maxpos, int back, void *stream)
{
    int rc = begin();
    if (rc) return rc;
    if (rows < 0 || nheads <= 0 || hd <= 0 || hd % 2 || maxpos <= 0 || (!pos && T <= 0))
        return tlg_fail(TLG_EINVAL, "rope: rows=%d nheads=%d hd=%d T=%d maxpos=%d", rows, nheads, hd, T, maxpos);
    if (rows == 0) return TLG_OK;
    const size_t total = (size_t)rows * nheads * (hd / 2);
    if ((hd / 2) % 4 == 0 && total / 4 < (1u << 30) && al16(buf) && al16(cos_t) && al16(sin_t))
        hipLaunchKernelGGL(k_rope4, dim3(grid_for(total / 4, 256, 8192)), dim3(256), 0, ST(stream), buf, pos, T,
                           rows, nheads, hd, cos_t, sin_t, maxpos, back);
    else
        hipLaunchKernelGGL(k_rope, dim3(grid_for(total, 256, 8192)), dim3(256), 0, ST(stream), buf, pos, T, rows,
                           nheads, hd, cos_t, sin_t, maxpos, back);
    LAUNCH_CHECK();
    return TLG_OK;
}

static int attn_check(const char *who, int B, int T, int H, int KV, int hd)
{
    if (B < 0 || T < 0 || H <= 0 || KV <= 0 || H % KV || hd != AT_HD)
        return tlg_fail(TLG_EINVAL, "%s: B=%d T=%d H=%d KV=%d hd=%d (head_dim 32, H %% KV == 0)", who, B, T, H, KV,
                        hd);
    return TLG_OK;
}

// Forward: the GQA-group kernel when H / KV is a multiple of 4, else one
// workgroup per (b, head, query block).  Rope tables (cs, sn) given: q and k
// are pre-rope (group kernel only).
static int attn_fwd_launch(const float *q, const float *k, const float *v, float *out, float *lse, int B, int T,
                           int H, int KV, int hd, int win, const float *cs, const float *sn, void *stream)
{
    int rc = begin();
    if (rc || (rc = attn_check("attn_fwd", B, T, H, KV, hd))) return rc;
    if (!al16(q) || !al16(k) || !al16(v) || !al16(out) || !lse)
        return tlg_fail(TLG_EINVAL, "attn_fwd: unaligned operand or no lse buffer");
    const bool g4 = (H / KV) % 4 == 0;
    if (cs && (!g4 || !al16(cs) || !al16(sn)))
        return tlg_fail(TLG_EINVAL, "attn_fwd_rope: needs H / KV a multiple of 4 and 16-byte aligned tables");
    if (B == 0 || T == 0) return TLG_OK;
    const float scale = 1.0f / sqrtf((float)hd);
    const int nqb = (T + 31) / 32;
    if (g4) {
        const dim3 grid(B * KV * (H / KV / A4_FNH) * nqb);
        if (cs)
            hipLaunchKernelGGL((k_attn_fwd4<true, A4_FNH>), grid, dim3(512), 0, ST(stream), q, k, v, out, lse, B, T, H,
                               KV, win, scale, cs, sn);
        else
            hipLaunchKernelGGL((k_attn_fwd4<false, A4_FNH>), grid, dim3(512), 0, ST(stream), q, k, v, out, lse, B, T, H,
                               KV, win, scale, nullptr, nullptr);
    } else {
        hipLaunchKernelGGL(k_attn_fwd, dim3(B * H * nqb), dim3(64 * AT_W), 0, ST(stream), q, k, v, out, lse, B, T, H,
                           KV, win, scale);
    }
    LAUNCH_CHECK();
    return TLG_OK;
}

// Dq_in: the per-row term D = dO . O [B*T][H], formed by the caller (the
// O-projection backward's block-dot epilogue); NULL: k_attn_delta forms it.
static int attn_bwd_launch(const float *q, const float *k, const float *v, const float *out, const float *lse,
                           const float *datt, float *dq, float *dk, float *dv, int B, int T, int H, int KV, int hd,
                           int win, const float *cs, const float *sn, void *stream, const float *Dq_in = nullptr)
{
    int rc = begin();
    if (rc || (rc = attn_check("attn_bwd", B, T, H, KV, hd))) return rc;
    if (!al16(q) || !al16(k) || !al16(v) || !al16(out) || !al16(datt) || !al16(dq) || !lse || !dk || !dv)
        return tlg_fail(TLG_EINVAL, "attn_bwd: unaligned or missing operand");
    const bool g4 = (H / KV) % 4 == 0;
    if (cs && (!g4 || !al16(cs) || !al16(sn)))
        return tlg_fail(TLG_EINVAL, "attn_bwd_rope: needs H / KV a multiple of 4 and 16-byte aligned tables");
    if (B == 0 || T == 0) return TLG_OK;
    // workspace: Dq [B*T][H]
    void *ws;
    if ((rc = tr_scratch((size_t)B * T * H * 4, &ws))) return rc;
    const float scale = 1.0f / sqrtf((float)hd);
    const int nqb = (T + 31) / 32;
    hipStream_t st = ST(stream);
    float *Dq = (float *)ws;
    // the group dK / dV items read lse rows as float4 (4 heads)
    if (g4 && cs && !al16(lse)) return tlg_fail(TLG_EINVAL, "attn_bwd_rope: lse must be 16-byte aligned");
    if (Dq_in && !(g4 && al16(lse)))
        return tlg_fail(TLG_EINVAL, "attn_bwd: a given D needs H / KV a multiple of 4 and an aligned lse");
    if (g4 && al16(lse)) {
        // Dq first (unless given); then the dK / dV and dQ items of every
        // group in one launch
        if (Dq_in)
            Dq = const_cast<float *>(Dq_in);
        else
            hipLaunchKernelGGL(k_attn_delta, dim3((B * T * H + 31) / 32), dim3(256), 0, st, datt, out, Dq,
                               B * T * H);
        const dim3 grid(nqb * B * KV + B * KV * (H / KV / 4) * nqb);
        if (cs)
            hipLaunchKernelGGL(k_attn_bwd4<true>, grid, dim3(512), 0, st, q, k, v, out, datt, lse, (const float *)Dq,
                               dq, dk, dv, B, T, H, KV, win, scale, cs, sn);
        else
            hipLaunchKernelGGL(k_attn_bwd4<false>, grid, dim3(512), 0, st, q, k, v, out, datt, lse,
                               (const float *)Dq, dq, dk, dv, B, T, H, KV, win, scale, nullptr, nullptr);
        LAUNCH_CHECK();
        return TLG_OK;
    }
    if (g4)        // no rope tables here (they need an aligned lse)
        hipLaunchKernelGGL(k_attn_dq4<false>, dim3(B * KV * (H / KV / 4) * nqb), dim3(256 * A4_KS), 0, st, q, k, v,
                           out, datt, lse, Dq, dq, B, T, H, KV, win, scale, nullptr, nullptr);
    else
        hipLaunchKernelGGL(k_attn_bwd_dq, dim3(B * H * nqb), dim3(64 * AT_W), 0, st, q, k, v, out, datt, lse, Dq, dq,
                           B, T, H, KV, win, scale);
    hipLaunchKernelGGL(k_attn_bwd_dkv, dim3(nqb * B * KV), dim3(64 * AT_KW), 0, st, q, k, v, datt, lse,
                       (const float *)Dq, dk, dv, B, T, H, KV, win, scale);
    LAUNCH_CHECK();
    return TLG_OK;
}

extern "C" int tlg_dev_attn_fwd(const float *q, const float *k, const float *v, float *out, float *lse, int B, int T,
                                int H, int KV, int hd, int win, void *stream)
{
    return attn_fwd_launch(q, k, v, out, lse, B, T, H, KV, hd, win, nullptr, nullptr, stream);
}

extern "C" int tlg_dev_attn_bwd(const float *q, const float *k, const float *v, const float *out, const float *lse,
                                const float *datt, float *dq, float *dk, float *dv, int B, int T, int H, int KV,
                                int hd, int win, void *stream)
{
    return attn_bwd_launch(q, k, v, out, lse, datt, dq, dk, dv, B, T, H, KV, hd, win, nullptr, nullptr, stream);
}

extern "C" int tlg_dev_attn_fwd_rope(const float *q, const float *k, const float *v, float *out, float *lse, int B,
                                     int T, int H, int KV, int hd, int win, const float *cos_t, const float *sin_t,
                                     void *stream)
{
    if (!cos_t || !sin_t) return tlg_fail(TLG_EINVAL, "attn_fwd_rope: no rope tables");
    return attn_fwd_launch(q, k, v, out, lse, B, T, H, KV, hd, win, cos_t, sin_t, stream);
}

extern "C" int tlg_dev_attn_bwd_rope(const float *q, const float *k, const float *v, const float *out,
                                     const float *lse, const float *datt, float *dq, float *dk, float *dv, int B,
                                     int T, int H, int KV, int hd, int win, const float *cos_t, const float *sin_t,
                                     void *stream)
{
    if (!cos_t || !sin_t) return tlg_fail(TLG_EINVAL, "attn_bwd_rope: no rope tables");
    return attn_bwd_launch(q, k, v, out, lse, datt, dq, dk, dv, B, T, H, KV, hd, win, cos_t, sin_t, stream);
}

extern "C" int tlg_dev_attn_bwd_rope_d(const float *q, const float *k, const float *v, const float *out,
                                       const float *lse, const float *datt, const float *D, float *dq, float *dk,
                                       float *dv, int B, int T, int H, int KV, int hd, int win, const float *cos_t,
                                       const float *sin_t, void *stream)
{
    if (!cos_t || !sin_t || !D) return tlg_fail(TLG_EINVAL, "attn_bwd_rope_d: no rope tables or no D");
    return attn_bwd_launch(q, k, v, out, lse, datt, dq, dk, dv, B, T, H, KV, hd, win, cos_t, sin_t, stream, D);
}

static int ew(int op, size_t n, float *y, float *y2, const float *x, const float *a, const float *b, void *stream)
{
    int rc = begin();
    if (rc) return rc;
    if (n == 0) return TLG_OK;
    hipLaunchKernelGGL(k_ew, dim3(grid_for(n, 256, 16384)), dim3(256), 0, ST(stream), op, n, y, y2, x, a, b);
    LAUNCH_CHECK();
    return TLG_OK;
}

extern "C" int tlg_dev_add(float *y, const float *x, size_t n, void *stream)
{
    return ew(EW_ADD, n, y, nullptr, x, nullptr, nullptr, stream);
}
extern "C" int tlg_dev_swiglu_fwd(float *act, const float *g, const float *u, size_t n, void *stream)
{
    return ew(EW_SWIGLU, n, act, nullptr, nullptr, g, u, stream);
}
extern "C" int tlg_dev_swiglu_bwd(const float *dact, const float *g, const float *u, float *dg, float *du, size_t n,
                                  void *stream)
{
    return ew(EW_SWIGLU_BWD, n, dg, du, dact, g, u, stream);
}
extern "C" int tlg_dev_silu_res(float *hk, const float *fn, const float *t1, size_t n, void *stream)
{
    return ew(EW_SILU_RES, n, hk, nullptr, fn, t1, nullptr, stream);
}
extern "C" int tlg_dev_silu_bwd(float *dt1, const float *dhk, const float *t1, size_t n, void *stream)
{
    return ew(EW_SILU_BWD, n, dt1, nullptr, dhk, t1, nullptr, stream);
}

static int xent_launch(const float *logits, const int *tgt, float *dlogits, double *rows, float *loss, float scale,
                       int N, int V, void *stream)
{
    int rc = begin();
    if (rc) return rc;
    if (N < 0 || V <= 0) return tlg_fail(TLG_EINVAL, "xent: N=%d V=%d", N, V);
    if (N == 0) return TLG_OK;
    if (loss && !rows) {
        void *ws;
        if ((rc = tr_scratch((size_t)N * 8, &ws))) return rc;
        rows = (double *)ws;
    }
    hipStream_t st = ST(stream);
    if (V % 4 == 0 && V <= 256 * XENT_XV && al16(logits) && al16(dlogits))
        hipLaunchKernelGGL(k_xent_reg, dim3((N + 3) / 4), dim3(256), 0, st, logits, tgt, dlogits, rows, scale, N, V);
    else
        hipLaunchKernelGGL(k_xent, dim3((N + 3) / 4), dim3(256), 0, st, logits, tgt, dlogits, rows, scale, N, V);
    if (loss) hipLaunchKernelGGL(k_sum_loss, dim3(1), dim3(1024), 0, st, (const double *)rows, N, loss);
    LAUNCH_CHECK();
    return TLG_OK;
}

extern "C" int tlg_dev_xent(const float *logits, const int *tgt, float *dlogits, float *loss, float scale, int N,
                            int V, void *stream)
{
    return xent_launch(logits, tgt, dlogits, nullptr, loss, scale, N, V, stream);
}

extern "C" int tlg_dev_xent_rows(const float *logits, const int *tgt, float *dlogits, double *rows, float scale,
                                 int N, int V, void *stream)
{
    if (!rows) return tlg_fail(TLG_EINVAL, "xent_rows: no row buffer");
    return xent_launch(logits, tgt, dlogits, rows, nullptr, scale, N, V, stream);
}

extern "C" int tlg_dev_gradnorm(const float *G, size_t n, float *norm, void *stream)
{
    int rc = begin();
    if (rc) return rc;
    void *ws;
    if ((rc = tr_scratch(GN_BLOCKS * 8, &ws))) return rc;
    hipStream_t st = ST(stream);
    hipLaunchKernelGGL(k_sumsq, dim3(GN_BLOCKS), dim3(256), 0, st, G, n, al16(G) ? n / 4 : 0, (double *)ws);
    hipLaunchKernelGGL(k_norm_final, dim3(1), dim3(1024), 0, st, (const double *)ws, norm, nullptr, 0, nullptr);
    LAUNCH_CHECK();
    return TLG_OK;
}

extern "C" int tlg_dev_gradnorm_loss(const float *G, size_t n, float *norm, const double *rows, int N, float *loss,
                                     void *stream)
{
    int rc = begin();
    if (rc) return rc;
    if (!rows || !loss || N <= 0) return tlg_fail(TLG_EINVAL, "gradnorm_loss: rows, loss and N > 0 required");
    void *ws;
    if ((rc = tr_scratch(GN_BLOCKS * 8, &ws))) return rc;
    hipStream_t st = ST(stream);
    hipLaunchKernelGGL(k_sumsq, dim3(GN_BLOCKS), dim3(256), 0, st, G, n, al16(G) ? n / 4 : 0, (double *)ws);
    hipLaunchKernelGGL(k_norm_final, dim3(1), dim3(1024), 0, st, (const double *)ws, norm, rows, N, loss);
    LAUNCH_CHECK();
    return TLG_OK;
}

extern "C" int tlg_dev_adamw(float *P, const float *G, float *M, float *V, size_t n, const float *hyper,
                             const float *norm, void *stream)
{
    int rc = begin();
    if (rc) return rc;
    if (!hyper) return tlg_fail(TLG_EINVAL, "adamw: hyper is required");
    if (n == 0) return TLG_OK;
    hipLaunchKernelGGL(k_adamw, dim3(grid_for(n, 256, 16384)), dim3(256), 0, ST(stream), P, G, M, V, n, hyper, norm);
    LAUNCH_CHECK();
    return TLG_OK;
}
