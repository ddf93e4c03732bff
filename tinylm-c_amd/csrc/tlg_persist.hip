// tlg_persist.hip -- n greedy single-token decode steps in ONE launch on gfx950.
//
// tinylm.c generates token after token with forward_chunk (:3721-3830) and
// argmax_v (:3844).  At M = 1 each GEMV moves 0.1-3 MB, which HBM delivers in
// well under a microsecond, while every dependent kernel launch costs several:
// a graph of 43 launches per token is bound by the gaps between them.  Here one
// workgroup per CU stays resident for the whole run (a cooperative launch
// guarantees they are all resident at once) and the workgroups hand each
// phase's outputs to each other through memory:
//
//   work items of a token, in phase order; item i belongs to workgroup i % NB
//     layer l:  H attention items   (RMSNorm, the head's Q and its group's K, V
//                                    columns, RoPE, ring store, attention)
//               D/32 O items        (32 output columns of ctx . Wo)
//               F/16 SwiGLU items   (16 columns of RMSNorm(x) . W1 and . W3,
//                                    then silu(g) * u)
//               D/32 W2 items       (32 columns of act . W2)
//     head:     V/8 items           (8 vocabulary rows of fn . emb^T and their
//                                    first maximum), item j to workgroup j % NB
//   exchange  every output element is a 64-bit word (value | tag << 32) written
//             with an agent-scope relaxed atomic store (global_store sc1: it goes
//             to the device-coherent level, not only the XCD's L2); a consumer
//             reads the words it needs with agent-scope atomic loads until all of
//             them carry its phase's tag.  Tags count phases over launches
//             (state[3]), so a stale word never matches.  Per layer four
//             exchanges (ctx, O out, act, W2 out), per token one more (argmax
//             candidates, double-buffered by token parity).
//   residual  every workgroup keeps x in LDS and adds each O / W2 output row to
//             it in the same order, so all copies are bit-identical; RMSNorm is
//             computed where it is needed.
//   prefetch  nothing an item reads from memory except its inputs waits on the
//             critical path: after finishing an item a workgroup loads the
//             weight panel and RMSNorm gain of its next one into registers
//             (about 256 items later, 2-3 layers ahead); the RoPE factors of
//             the position come at the token's start; the ring rows of the
//             keys before the position half a layer before the attention.
//             Token i reads weight copy (copy0 + i) % pool.
//   KV ring   ring rows are read with agent-scope atomic loads (another
//             workgroup, possibly on another XCD, wrote them), 8 (f16) or 16
//             (f32) threads per row so a load instruction covers whole rows,
//             and the new row is stored the same way; the writer waits for
//             those stores to complete before it publishes its ctx, so every
//             later reader, which depends on that ctx, sees the row.
//
// No dependency points forward (an item only waits for earlier phases), so the
// run always progresses; every wait is bounded (0.5 s of the real-time
// counter), after which the workgroup raises an abort flag that ends every
// other wait too, and the kernel returns.
//
// Reference arithmetic followed: rmsnorm_fwd :540-548 (1/sqrt(ss/D + 1e-5),
// x * s * g), rope_apply :645-651 with rope_init's tables, kv_store :3236-3250
// (f16 round to nearest even or f32), attn_body :3639-3715 (scores q.k hd^-1/2,
// fast_expf :3181-3191 or expf, normalise then sum p_t v_t), SwiGLU silu(g) * u
// with silu(z) = z / (1 + e^-z) (:786, :3821-3823), residual adds :3818, :3824,
// the head mm_bt :3829-3830 and argmax_v :3844.  Sums run in a fixed order of
// their own (the same in every workgroup and launch), not the reference's.
#include "tlg_internal.h"
#include "../../include/tldecode.h"
#include <math.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned long long u64;
typedef unsigned int u32;

#define PD_T 512            // threads per workgroup (8 waves, 2 per SIMD)
#define PD_NW 8
#define PD_MAXQ 6           // row slices of a K = D panel: D / 64 with D <= 384
#define PD_MAXFQ 16         // row slices of a K = F panel: F / 64 with F <= 1024
#define PD_WB 18            // f32x4 per thread of the weight panel: 3 * PD_MAXQ
#define PD_MAXD 384
#define PD_MAXF 1024
#define PD_MAXW 256         // ring positions
#define PD_MAXHI 512        // head items V / 8
#define PD_SPIN 50000000ull // 0.5 s of the 100 MHz real-time counter

static_assert(PD_WB >= 3 * PD_MAXQ && PD_WB >= PD_MAXFQ, "weight panel");
static_assert(PD_MAXD <= PD_T, "one gain element per thread");

// Exchange area (64-bit words): control words, then per layer ctx [D], O out
// [D], act [F], W2 out [D], then the argmax candidates [2][V/8][2].
struct PdLayout {
    size_t ctrl, ctx, yo, act, y2, cand, total;
};
__host__ __device__ static inline PdLayout pd_layout(int V, int D, int L, int F)
{
    PdLayout o;
    size_t p = 0;
    o.ctrl = p;  p += 8;
    o.ctx = p;   p += (size_t)L * D;
    o.yo = p;    p += (size_t)L * D;
    o.act = p;   p += (size_t)L * F;
    o.y2 = p;    p += (size_t)L * D;
    o.cand = p;  p += (size_t)2 * (V / 8) * 2;
    o.total = p;
    return o;
}

// Every access of this kernel goes through global-address-space pointers:
// flat loads would also count against lgkmcnt, so each LDS barrier would wait
// for the weight prefetches in flight.
#define GAS __attribute__((address_space(1)))
template <class T> __device__ __forceinline__ GAS T *gp(T *p) { return (GAS T *)p; }

__device__ __forceinline__ u64 pd_ld(const u64 *p)
{
    return __hip_atomic_load(gp(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void pd_st(u64 *p, u64 v)
{
    __hip_atomic_store(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 pd_word(float v, u32 tag) { return ((u64)tag << 32) | (u64)__float_as_uint(v); }

// A pointer every thread holds the same value of (read from LDS, say), moved
// to scalar registers so addresses are a scalar base plus a 32-bit offset.
template <class T> __device__ __forceinline__ T *pd_uni(T *p)
{
    const u64 v = (u64)(uintptr_t)p;
    const u32 lo = __builtin_amdgcn_readfirstlane((u32)v), hi = __builtin_amdgcn_readfirstlane((u32)(v >> 32));
    return (T *)(uintptr_t)(((u64)hi << 32) | lo);
}
template <class T> __device__ __forceinline__ T pd_at(const void *base, u32 byteoff)
{
    return *reinterpret_cast<const GAS T *>(reinterpret_cast<const GAS char *>(gp(base)) + byteoff);
}

// Wait until this wave's stores have completed (vmcnt counts stores on gfx9).
__device__ __forceinline__ void pd_wait_stores()
{
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);        // vmcnt(0) expcnt(7) lgkmcnt(15)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Wait until the n words src[0..n) carry `tag`; then dst[e] = (ADD ? dst[e] +
// : ) their values, and with NORM (x += delta, n <= PD_T) the norm parts of the
// new x for gain element gn (pd_norm_parts into xn, sw) before the closing
// barrier.  Called by every thread; false after an abort.  Each wave
// polls its own words (thread tid: words tid + PD_T k) until they all carry
// the tag, deciding with a wave vote, so the poll loop has no barrier; lane 0
// checks the abort flag and the time limit every 8th round; one barrier at the
// end joins the waves.
__device__ __forceinline__ void pd_norm_parts(float xv, float gj, float *xg, int D, float *sw);
template <int KPL, int ADD, int NORM = 0>
__device__ bool pd_fetch(const u64 *src, int n, u32 tag, float *dst, u32 *abortp, float gn = 0.f,
                         float *xn = nullptr, float *sw = nullptr)
{
    static_assert(!NORM || (KPL == 1 && ADD), "the norm parts follow x += delta");
    const int tid = threadIdx.x;
    const u64 t0 = wall_clock64();
    u64 w[KPL];
    int stop = 0;
    for (int it = 0;; it++) {
#pragma unroll
        for (int k = 0; k < KPL; k++)
            w[k] = pd_ld(reinterpret_cast<const u64 *>(reinterpret_cast<const char *>(src) +
                                                        8u * (u32)min(tid + PD_T * k, n - 1)));
        int bad = 0;
#pragma unroll
        for (int k = 0; k < KPL; k++) bad |= (tid + PD_T * k < n) && (u32)(w[k] >> 32) != tag;
        if (__ballot(bad) == 0ull) break;
        if ((it & 7) == 7) {
            int s = 0;
            if ((tid & 63) == 0)
                s = __hip_atomic_load(gp(abortp), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u ||
                    wall_clock64() - t0 > PD_SPIN;
            if (__ballot(s) != 0ull) { stop = 1; break; }
        }
    }
    if (!stop) {
        float nv = 0.f;
#pragma unroll
        for (int k = 0; k < KPL; k++) {
            const int e = tid + PD_T * k;
            if (e < n) {
                nv = ADD ? dst[e] + __uint_as_float((u32)w[k]) : __uint_as_float((u32)w[k]);
                dst[e] = nv;
            }
        }
        if (NORM) pd_norm_parts(nv, gn, xn, n, sw);
    }
    if (__syncthreads_or(stop)) {
        if (tid == 0) __hip_atomic_store(gp(abortp), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    return true;
}

// Cross-lane steps on the VALU (DPP) rather than through LDS permutes, which
// wait one at a time: row_shr scans within 16-lane rows, then row_bcast:15 /
// :31 carry the rows upward; lane 63 ends with the total, read back as a
// scalar.  A fixed order, the same in every wave.
template <int CTRL, int ROWMASK> __device__ __forceinline__ float pd_dpp(float fill, float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(x), CTRL, ROWMASK, 0xf,
                                                      false));
}
__device__ __forceinline__ float pd_wave_sum(float x)
{
    x += pd_dpp<0x111, 0xf>(0.f, x);          // row_shr:1
    x += pd_dpp<0x112, 0xf>(0.f, x);          // row_shr:2
    x += pd_dpp<0x114, 0xf>(0.f, x);          // row_shr:4
    x += pd_dpp<0x118, 0xf>(0.f, x);          // row_shr:8
    x += pd_dpp<0x142, 0xa>(0.f, x);          // row_bcast:15 into rows 1, 3
    x += pd_dpp<0x143, 0xc>(0.f, x);          // row_bcast:31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}
// The maximum (sum) over a wave's key groups when the NW lanes of a key hold
// the same value: the two keys of a 16-lane row (NW = 8) meet by row_ror:8,
// then the four rows by lane reads.
__device__ __forceinline__ float pd_lane(float v, int l)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
template <int NW> __device__ __forceinline__ float pd_keys_max(float v)
{
    if (NW == 8) v = fmaxf(v, pd_dpp<0x128, 0xf>(-INFINITY, v));
    return fmaxf(fmaxf(pd_lane(v, 0), pd_lane(v, 16)), fmaxf(pd_lane(v, 32), pd_lane(v, 48)));
}
template <int NW> __device__ __forceinline__ float pd_keys_sum(float v)
{
    if (NW == 8) v += pd_dpp<0x128, 0xf>(0.f, v);
    return (pd_lane(v, 0) + pd_lane(v, 16)) + (pd_lane(v, 32) + pd_lane(v, 48));
}

// RMSNorm folded into the GEMV that follows it: xg[j] = x[j] g[j] (thread j
// holds x[j] in xv and g[j] in gj) and the waves' sums of x^2, made visible by
// the caller's next barrier; the GEMV's column sums are then scaled by s =
// pd_norm_scale(sw, D).  (The reference normalises first, x * s * g, then
// multiplies; the two differ only in fp32 rounding.)  Called by whole waves.
__device__ __forceinline__ void pd_norm_parts(float xv, float gj, float *xg, int D, float *sw)
{
    const int tid = threadIdx.x;
    const float xj = tid < D ? xv : 0.f;
    if (tid < D) xg[tid] = xj * gj;
    const float ss = pd_wave_sum(xj * xj);
    if ((tid & 63) == 0) sw[tid >> 6] = ss;
}
// s = 1 / sqrt(sum x^2 / D + 1e-5) (rmsnorm_fwd, tinylm.c:546) from the waves'
// sums; the hardware reciprocal square root, within 2 ulp of the reference's
// square root then divide.
__device__ __forceinline__ float pd_norm_scale(const float *sw, int D)
{
    float tot = sw[0];
#pragma unroll
    for (int w = 1; w < PD_NW; w++) tot += sw[w];
    return rsqrtf(tot / (float)D + 1e-5f);
}

// Column-panel GEMV.  Thread (c4 = tid & 7, rg = tid >> 3) holds
// w[i] = W[(rg + 64 i) * N + col0 + 4 c4 .. + 3] for rows rg + 64 i < K
// (rows past K load row K - 1, unused: every element is written, so the panel
// stays in registers).
template <int MAXI>
__device__ __forceinline__ void pd_load_cols(f32x4 *w, const float *__restrict__ W, int N, int col0, int K)
{
    const int c4 = threadIdx.x & 7, rg = threadIdx.x >> 3;
#pragma unroll
    for (int i = 0; i < MAXI; i++)
        w[i] = pd_at<f32x4>(W, 4u * ((u32)min(rg + 64 * i, K - 1) * (u32)N + (u32)(col0 + 4 * c4)));
}

// The rows of vin that thread tid's panel entries meet (rg + 64 i, clamped), read
// once for several panels; pd_dot_r is pd_dot on them.
template <int MAXI> __device__ __forceinline__ void pd_rows(const float *vin, int K, float (&xv)[MAXI])
{
    const int rg = threadIdx.x >> 3;
#pragma unroll
    for (int i = 0; i < MAXI; i++) xv[i] = vin[min(rg + 64 * i, K - 1)];
}
template <int MAXI> __device__ __forceinline__ f32x4 pd_dot_r(const float (&xv)[MAXI], const f32x4 *w, int K)
{
    const int rg = threadIdx.x >> 3;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < MAXI; i++) {
        const bool in = K == 64 * MAXI || rg + 64 * i < K;
        acc.x = in ? fmaf(xv[i], w[i].x, acc.x) : acc.x;
        acc.y = in ? fmaf(xv[i], w[i].y, acc.y) : acc.y;
        acc.z = in ? fmaf(xv[i], w[i].z, acc.z) : acc.z;
        acc.w = in ? fmaf(xv[i], w[i].w, acc.w) : acc.w;
    }
    return acc;
}

template <int MAXI>
__device__ __forceinline__ f32x4 pd_dot(const float *vin, const f32x4 *w, int K)
{
    // branch-free: every row's LDS read is issued at once.  K = 64 MAXI (every
    // BASELINE shape) needs no guard; otherwise rows past K read row K - 1 and
    // are not added.
    const int rg = threadIdx.x >> 3;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (K == 64 * MAXI) {
#pragma unroll
        for (int i = 0; i < MAXI; i++) {
            const float xv = vin[rg + 64 * i];
            acc.x = fmaf(xv, w[i].x, acc.x);
            acc.y = fmaf(xv, w[i].y, acc.y);
            acc.z = fmaf(xv, w[i].z, acc.z);
            acc.w = fmaf(xv, w[i].w, acc.w);
        }
        return acc;
    }
#pragma unroll
    for (int i = 0; i < MAXI; i++) {
        const bool in = rg + 64 * i < K;
        const float xv = vin[min(rg + 64 * i, K - 1)];
        acc.x = in ? fmaf(xv, w[i].x, acc.x) : acc.x;
        acc.y = in ? fmaf(xv, w[i].y, acc.y) : acc.y;
        acc.z = in ? fmaf(xv, w[i].z, acc.z) : acc.z;
        acc.w = in ? fmaf(xv, w[i].w, acc.w) : acc.w;
    }
    return acc;
}

// The 64 row groups' partials of one panel: the two row groups of a 16-lane
// row meet with row_ror:8 (lane ^ 8), then the 32 row pairs go through LDS
// (red: 32 x 8 f32x4) and pd_colsum_half adds them.
#define PD_RED (PD_T / 16 * 8)
__device__ __forceinline__ void pd_colsum_put(f32x4 acc, f32x4 *red)
{
    const int tid = threadIdx.x;
    acc.x += pd_dpp<0x128, 0xf>(0.f, acc.x);
    acc.y += pd_dpp<0x128, 0xf>(0.f, acc.y);
    acc.z += pd_dpp<0x128, 0xf>(0.f, acc.z);
    acc.w += pd_dpp<0x128, 0xf>(0.f, acc.w);
    if ((tid & 8) == 0) red[(tid >> 4) * 8 + (tid & 7)] = acc;
}
// Column col's sum read by two lanes (2 k, 2 k + 1): lane h adds row pairs
// 16 h .. 16 h + 15 as two in-order chains of 8, (r0 + r1) or (r2 + r3), and
// one quad_perm exchange forms (r0 + r1) + (r2 + r3) in both lanes.
__device__ __forceinline__ float pd_colsum_half(const f32x4 *red, int col)
{
    const int h = threadIdx.x & 1;
    const float *rf = reinterpret_cast<const float *>(red);
    float v[16];
#pragma unroll
    for (int g = 0; g < 16; g++) v[g] = rf[32 * (16 * h + g) + col];
    float r0 = v[0], r1 = v[8];
#pragma unroll
    for (int g = 1; g < 8; g++) {
        r0 += v[g];
        r1 += v[8 + g];
    }
    const float r = r0 + r1;
    return r + pd_dpp<0xB1, 0xf>(0.f, r);         // quad_perm [1, 0, 3, 2]: the other half
}
// Which column lane t of a 64-lane group reads: column t / 2 (PAIRS 0), or for
// t = 4 p + 2 m + h column p + 16 m (PAIRS 1: the columns i, i + 16 of a RoPE
// pair or of a SwiGLU W1 / W3 pair sit in one quad, the partner at lane ^ 2).
template <int PAIRS> __device__ __forceinline__ int pd_half_col(int t)
{
    return PAIRS ? ((t >> 2) & 15) + 16 * ((t >> 1) & 1) : (t >> 1) & 31;
}
__device__ __forceinline__ float pd_pair_other(float v)
{
    return pd_dpp<0x4E, 0xf>(0.f, v);             // quad_perm [2, 3, 0, 1]: lane ^ 2
}
// one panel: the lanes of wave 0 get the sum of column pd_half_col<PAIRS>(tid)
template <int PAIRS> __device__ __forceinline__ float pd_colsum(f32x4 acc, f32x4 *red)
{
    pd_colsum_put(acc, red);
    __syncthreads();
    return threadIdx.x < 64 ? pd_colsum_half(red, pd_half_col<PAIRS>(threadIdx.x)) : 0.f;
}

// The weight panel of layer item g (index within a token) in thread order and
// the RMSNorm gain element of thread tid (items that normalise x):
//   attention (k < NA): Wq columns of head k, Wk and Wv columns of its KV head
//     at panel offsets 0, PD_MAXQ, 2 PD_MAXQ; gain an1
//   O: Wo columns; SwiGLU: threads c4 < 4 the W1 columns 16 c + 4 c4 .. + 3,
//     c4 >= 4 the same columns of W3; gain an2; W2: W2 columns (K = F)
// Every kind writes the whole panel, so it stays in registers.
__device__ __forceinline__ void pd_load_item(f32x4 (&wb)[PD_WB], float &gn, const float *__restrict__ P, int g,
                                             int NPL, int NA, int NO, int NS, size_t lay0, size_t per, int D, int KD,
                                             int F, int grp, int qk)
{
    const int l = g / NPL, k = g % NPL;
    const size_t an1 = lay0 + (size_t)l * per, wq = an1 + D, wk = wq + (size_t)D * D, wv = wk + (size_t)D * KD,
                 wo = wv + (size_t)D * KD, an2 = wo + (size_t)D * D + qk, w1 = an2 + D, w3 = w1 + (size_t)D * F,
                 w2 = w3 + (size_t)D * F;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    const int tid = threadIdx.x, c4 = tid & 7;
    const u32 gof = 4u * (u32)min(tid, D - 1);
    if (k < NA) {
        const int gq = k / grp;
        pd_load_cols<PD_MAXQ>(wb, P + wq, D, k * 32, D);
        pd_load_cols<PD_MAXQ>(wb + PD_MAXQ, P + wk, KD, gq * 32, D);
        pd_load_cols<PD_MAXQ>(wb + 2 * PD_MAXQ, P + wv, KD, gq * 32, D);
        gn = pd_at<float>(P + an1, gof);
    } else if (k < NA + NO) {
        pd_load_cols<PD_MAXQ>(wb, P + wo, D, (k - NA) * 32, D);
#pragma unroll
        for (int i = PD_MAXQ; i < PD_WB; i++) wb[i] = z;
        gn = 0.f;
    } else if (k < NA + NO + NS) {
        // columns 16 c .. 16 c + 15 of W1 (c4 < 4) and of W3 (c4 >= 4): thread
        // c4 reads the float4 at 16 c + 4 (c4 & 3); pd_load_cols' 4 c4 offset is
        // taken back by col0
        const int c = k - NA - NO;
        const float *W = c4 < 4 ? P + w1 : P + w3;
        pd_load_cols<PD_MAXQ>(wb, W, F, 16 * c - 4 * (c4 & 4), D);
#pragma unroll
        for (int i = PD_MAXQ; i < PD_WB; i++) wb[i] = z;
        gn = pd_at<float>(P + an2, gof);
    } else {
        pd_load_cols<PD_MAXFQ>(wb, P + w2, D, (k - NA - NO - NS) * 32, F);
#pragma unroll
        for (int i = PD_MAXFQ; i < PD_WB; i++) wb[i] = z;
        gn = 0.f;
    }
}

// Head item j: wave r holds vocabulary row 8 j + r, thread c = tid & 63 the
// float4s c and c + 64 of it (those below D / 4).
__device__ __forceinline__ void pd_load_head(f32x4 (&hb)[2], const float *__restrict__ emb, int j, int D)
{
    const int tid = threadIdx.x;
    const float *rows = emb + (size_t)8 * j * D;
#pragma unroll
    for (int i = 0; i < 2; i++)
        hb[i] = pd_at<f32x4>(rows, 4u * ((u32)(tid >> 6) * (u32)D + 4u * (u32)min((tid & 63) + 64 * i, D / 4 - 1)));
}

// Ring rows of 32 elements as 64-bit words: NW per row (8 f16, 16 f32), EPW
// elements per word; thread (key slot tid / NW, word tid % NW).
template <int F16> struct PdRing;
template <> struct PdRing<1> {
    typedef _Float16 E;
    static constexpr int NW = 8, EPW = 4, LOG2NW = 3;
    __device__ static float get(u64 w, int e)
    {
        return (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> (16 * e)));
    }
    __device__ static float round(float v) { return (float)(_Float16)v; }
    __device__ static u64 pack(const float *v)
    {
        u64 r = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) r |= (u64)__builtin_bit_cast(unsigned short, (_Float16)v[c]) << (16 * c);
        return r;
    }
};
template <> struct PdRing<0> {
    typedef float E;
    static constexpr int NW = 16, EPW = 2, LOG2NW = 4;
    __device__ static float get(u64 w, int e) { return __uint_as_float((u32)(w >> (32 * e))); }
    __device__ static float round(float v) { return v; }
    __device__ static u64 pack(const float *v)
    {
        return (u64)__float_as_uint(v[0]) | ((u64)__float_as_uint(v[1]) << 32);
    }
};
#define PD_MAXR 8           // key rounds: PD_MAXW / (PD_T / NW), 8 for f32 (4 for f16)

// The visible window of `pos` in layer l: positions lo .. pos, cnt of them.
__device__ __forceinline__ void pd_window(const TlgDecPersist &a, int l, int pos, int *lo, int *cnt)
{
    int wl = a.win;
    if (wl <= 0 || (a.full_every > 0 && ((l + 1) % a.full_every) == 0)) wl = 0;   // cfg_lwin :64-68
    const int wlim = (wl > 0 && wl < a.W) ? wl : a.W;
    *lo = pos >= wlim ? pos - wlim + 1 : 0;
    *cnt = pos - *lo + 1;
}

// Ring words of the keys before `pos` (the window's first cnt - 1 keys) for
// KV head kvh of layer l: round r, thread (key slot, word); K words if LK, V
// words if LV.
template <int F16, int LK, int LV>
__device__ __forceinline__ void pd_ring_load(u64 (&kw)[PD_MAXR], u64 (&vw)[PD_MAXR], const void *Kc, const void *Vc,
                                             int kvh, int KD, int W, int lo, int cnt)
{
    typedef PdRing<F16> R;
    constexpr int KPR = PD_T / R::NW, MAXR = PD_MAXW / KPR;
    const int tid = threadIdx.x, key0 = tid >> R::LOG2NW, wd = tid & (R::NW - 1);
    const u32 rowb = (u32)KD * (u32)sizeof(typename R::E);          // bytes per ring row
    const char *Kb = pd_uni(reinterpret_cast<const char *>(Kc) + (size_t)kvh * 32 * sizeof(typename R::E));
    const char *Vb = pd_uni(reinterpret_cast<const char *>(Vc) + (size_t)kvh * 32 * sizeof(typename R::E));
    // every round loads (keys past the window reload an earlier slot, unused):
    // straight-line loads are issued back to back, with no wait between them
#pragma unroll
    for (int r = 0; r < MAXR; r++) {
        const int t = min(key0 + KPR * r, max(cnt - 2, 0));
        const u32 off = (u32)((lo + t) % W) * rowb + 8u * (u32)wd;
        if (LK) kw[r] = pd_ld(reinterpret_cast<const u64 *>(Kb + off));
        if (LV) vw[r] = pd_ld(reinterpret_cast<const u64 *>(Vb + off));
    }
}

struct PdShared {
    float x[PD_MAXD], xn[PD_MAXD], in[PD_MAXF];
    f32x4 red[3][PD_RED];
    float sw[2 * PD_NW];
    float q[32], k[32], v[32], ctxw[PD_T / 16][32];
    u64 key[PD_T];
    float lg[8];
    int tok;
    const float *P[16];                 // the launch's pointer tables, indexed at run time
    void *Kc[TLG_PD_MAXL], *Vc[TLG_PD_MAXL];
};

// argmax_v order as one unsigned key: larger value first, then the lower index
__device__ __forceinline__ u64 pd_argkey(float v, u32 i)
{
    u32 b = __float_as_uint(v + 0.0f);                          // -0 as +0: equal values tie
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);           // order-preserving map of the float
    return ((u64)b << 32) | (u64)(~i);
}

// The first maximum over the argmax candidates of a token (argmax_v: ties to
// the lowest index; no candidate above -inf gives token 0, as the reference's
// scan does) into sh.tok: each wave's largest key by DPP, then the 8 waves'
// through LDS.  false after an abort.
// The maximum of the lanes' unsigned words (row_shr scan, then row_bcast),
// every lane gets it; 0 is the identity.
__device__ __forceinline__ u32 pd_wave_umax(u32 x)
{
    x = max(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false));
    x = max(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false));
    x = max(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false));
    x = max(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false));
    x = max(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false));
    x = max(x, (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false));
    return (u32)__builtin_amdgcn_readlane((int)x, 63);
}
__device__ __forceinline__ bool pd_argmax(PdShared &sh, const u64 *cand, int NHI, u32 tag, u32 *abortp)
{
    const int tid = threadIdx.x;
    if (!pd_fetch<2, 0>(cand, 2 * NHI, tag, sh.in, abortp)) return false;
    u64 kx = 0;
    if (tid < NHI) {
        const u32 i = __float_as_uint(sh.in[2 * tid + 1]);
        kx = i == 0x7fffffffu ? 0 : pd_argkey(sh.in[2 * tid], i);
    }
    // a wave's largest key: its largest high word, then the largest low word
    // among the lanes holding that high word; then the 8 waves' keys via LDS
    const u32 hm = pd_wave_umax((u32)(kx >> 32));
    const u32 lm = pd_wave_umax((u32)(kx >> 32) == hm ? (u32)kx : 0u);
    if ((tid & 63) == 0) sh.key[tid >> 6] = ((u64)hm << 32) | lm;
    __syncthreads();
    if (tid == 0) {
        u64 m = sh.key[0];
#pragma unroll
        for (int w = 1; w < PD_NW; w++) m = max(m, sh.key[w]);
        sh.tok = m == 0 ? 0 : (int)(~(u32)m);
    }
    __syncthreads();
    return true;
}

// One attention item (layer l, query head h) at position pos, after the norm
// parts of x (sh.xn, sh.sw; gain an1): the head's q and its KV head's k, v
// from the panel in wb scaled by the norm's s, RoPE
// (this thread's factors rc, rs for pair (tid >> 2) & 15), the ring store (by the
// group's first head), softmax attention over the window with the ring words
// kw / vw already loaded (f32 rings: vw loaded here), then ctx_h published
// with `tag`.
template <int F16>
__device__ __forceinline__ void pd_attention(PdShared &sh, const f32x4 (&wb)[PD_WB], float rc, float rs,
                                             u64 (&kw)[PD_MAXR], u64 (&vw)[PD_MAXR], const TlgDecPersist &a,
                                             int l, int h, int pos, int D, int KD, int grp, const float *qkn,
                                             u64 *ctxout, u32 tag)
{
    typedef PdRing<F16> R;
    constexpr int NW = R::NW, KPR = PD_T / NW, MAXR = PD_MAXW / KPR;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvh = h / grp, key0 = tid >> R::LOG2NW, wd = tid & (NW - 1);
    int lo, cnt;
    pd_window(a, l, pos, &lo, &cnt);
    const float sn = pd_norm_scale(sh.sw, D);        // read before the softmax reuses sw
    {
        float xv[PD_MAXQ];
        pd_rows<PD_MAXQ>(sh.xn, D, xv);
        pd_colsum_put(pd_dot_r<PD_MAXQ>(xv, wb, D), sh.red[0]);
        pd_colsum_put(pd_dot_r<PD_MAXQ>(xv, wb + PD_MAXQ, D), sh.red[1]);
        pd_colsum_put(pd_dot_r<PD_MAXQ>(xv, wb + 2 * PD_MAXQ, D), sh.red[2]);
    }
    if (!F16) {                          // f32 rings: V words now, for register room
        u64 none[PD_MAXR];
        pd_ring_load<F16, 0, 1>(none, vw, sh.Kc[l], sh.Vc[l], kvh, KD, a.W, lo, cnt);
    }
    __syncthreads();
    // q, k, v columns (thread 32 m + i: column i of q, k, v for m = 0, 1, 2);
    // RoPE of q and the new k (rope_apply's pairs (i, i + 16), the partner
    // column from the lane i ^ 16); new k and v in the ring's format
    if (tid < 192) {                     // wave m reads panel m, pairs (i, i + 16) in quads
        const int m = tid >> 6, i = pd_half_col<1>(tid);
        float c = pd_colsum_half(sh.red[m], i) * sn;
        if (qkn && m < 2) {
            // QK-norm (qknorm_apply, tinylm.c:597-605, before RoPE :3752-3754) of
            // q (wave 0) and the new k (wave 1): v s gain, s = 1 / sqrt(sum v^2 /
            // hd + 1e-5); each column sits in two lanes, one of them counted
            const float ss = pd_wave_sum((tid & 1) ? 0.f : c * c);
            c = c * (1.0f / sqrtf(ss / 32.0f + 1e-5f)) * gp(qkn)[32 * m + i];
        }
        const float o = pd_pair_other(c);
        const bool inpos = pos >= 0 && pos < a.maxpos;
        const float rot = inpos ? (i < 16 ? c * rc - o * rs : c * rc + o * rs) : NAN;
        if ((tid & 1) == 0) {
            if (m == 0) sh.q[i] = rot;
            else if (m == 1) sh.k[i] = R::round(rot);
            else sh.v[i] = R::round(c);
        }
    }
    __syncthreads();
    const bool writer = (h % grp) == 0;
    if (writer && tid < 2 * NW) {                              // ring slot pos % W
        const int w = tid & (NW - 1);
        char *row = reinterpret_cast<char *>(tid < NW ? sh.Kc[l] : sh.Vc[l]) +
                    ((size_t)(pos % a.W) * KD + (size_t)kvh * 32) * sizeof(typename R::E);
        pd_st(reinterpret_cast<u64 *>(row) + w, R::pack((tid < NW ? sh.k : sh.v) + R::EPW * w));
    }
    // key t = key0 + KPR r; t < cnt - 1 come from the ring words loaded, the new
    // row t = cnt - 1 (round nr, key slot ns) is spliced into its threads' words
    const int nr = (cnt - 1) / KPR, ns = (cnt - 1) % KPR;
    const bool newslot = key0 == ns;
    const u64 knew = R::pack(sh.k + R::EPW * wd);
#pragma unroll
    for (int r = 0; r < MAXR; r++) kw[r] = (newslot && r == nr) ? knew : kw[r];
    // scores: the NW threads of a key sum their words' partial dots
    const float scale = 1.0f / sqrtf(32.0f);
    float qv[R::EPW];
#pragma unroll
    for (int e = 0; e < R::EPW; e++) qv[e] = sh.q[R::EPW * wd + e];
    float sc[MAXR];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < MAXR; r++) {
        const int t = key0 + KPR * r;
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < R::EPW; e++) part = fmaf(qv[e], R::get(kw[r], e), part);
        // the NW lanes of the key: butterflies inside quads (quad_perm), then the
        // two quads of an 8-lane group (row_ror:n reads lane (i - n) mod 16, so
        // lanes 0-3 of the group take row_ror:12, lanes 4-7 row_ror:4), for f32
        // the two halves of the 16-lane row (row_ror:8)
        part += pd_dpp<0xB1, 0xf>(0.f, part);
        part += pd_dpp<0x4E, 0xf>(0.f, part);
        {
            const float r4 = pd_dpp<0x124, 0xf>(0.f, part), r12 = pd_dpp<0x12C, 0xf>(0.f, part);
            part += (lane & 4) ? r4 : r12;
        }
        if (NW == 16) part += pd_dpp<0x128, 0xf>(0.f, part);
        sc[r] = t < cnt ? part * scale : -INFINITY;
        mx = fmaxf(mx, sc[r]);
    }
    // softmax: the maximum M over the waves first (fast_expf's error depends on
    // its argument, so every p_t is exp(s_t - M) as the reference forms it);
    // the sum and the unnormalised context then meet at one barrier, and the
    // context is divided by the sum at the end
    mx = pd_keys_max<NW>(mx);
    if (lane == 0) sh.sw[wave] = mx;
    __syncthreads();
    mx = sh.sw[0];
#pragma unroll
    for (int w = 1; w < PD_NW; w++) mx = fmaxf(mx, sh.sw[w]);
    float sum = 0.f;
#pragma unroll
    for (int r = 0; r < MAXR; r++) {
        const int t = key0 + KPR * r;
        const float e = a.exact ? expf(sc[r] - mx) : tlg_fast_expf(sc[r] - mx);
        sc[r] = t < cnt ? e : 0.f;
        sum += sc[r];
    }
    sum = pd_keys_sum<NW>(sum);
    if (lane == 0) sh.sw[PD_NW + wave] = sum;
    // ctx[d] = sum_t p_t v_t[d]: thread (key slot, word) over its keys, then the
    // key slots of a word: shuffles in the wave, the rows through LDS
    // (keys t >= cnt hold clamped ring words, masked off)
    const u64 vnew = R::pack(sh.v + R::EPW * wd);
#pragma unroll
    for (int r = 0; r < MAXR; r++) vw[r] = (newslot && r == nr) ? vnew : vw[r];
    float acc[R::EPW];
#pragma unroll
    for (int e = 0; e < R::EPW; e++) acc[e] = 0.f;
#pragma unroll
    for (int r = 0; r < MAXR; r++) {
        const int t = key0 + KPR * r;
#pragma unroll
        for (int e = 0; e < R::EPW; e++) acc[e] = t < cnt ? fmaf(sc[r], R::get(vw[r], e), acc[e]) : acc[e];
    }
    // the key slots of a word: for f16 the two slots of a 16-lane row meet with
    // row_ror:8, then each row's partials go through LDS, added in row order
    const int row = tid >> 4;
#pragma unroll
    for (int e = 0; e < R::EPW; e++) {
        if (NW == 8) acc[e] += pd_dpp<0x128, 0xf>(0.f, acc[e]);
        if ((tid & 15) < NW) sh.ctxw[row][R::EPW * wd + e] = acc[e];
    }
    __syncthreads();
    if (tid < 64) {                      // lanes 2 d, 2 d + 1: rows 0-15 and 16-31 of ctx[d]
        float tot = sh.sw[PD_NW];
#pragma unroll
        for (int w = 1; w < PD_NW; w++) tot += sh.sw[PD_NW + w];
        const int d = tid >> 1, r0 = 16 * (tid & 1);
        float c0 = sh.ctxw[r0][d], c1 = sh.ctxw[r0 + 8][d];
#pragma unroll
        for (int rr = 1; rr < 8; rr++) {
            c0 += sh.ctxw[r0 + rr][d];
            c1 += sh.ctxw[r0 + 8 + rr][d];
        }
        float cx = c0 + c1;
        cx += pd_dpp<0xB1, 0xf>(0.f, cx);             // quad_perm [1, 0, 3, 2]: the other half
        cx *= tot > 0.f ? __builtin_amdgcn_rcpf(tot) : 0.f;
        if (writer) pd_wait_stores();                          // the ring row first
        if ((tid & 1) == 0) pd_st(ctxout + d, pd_word(cx, tag));
    }
    __syncthreads();
}

// An O or W2 item: the 32 columns of the panel in wb against in[0..K), out[c]
// = their sums, published with `tag`.
template <int MAXI>
__device__ __forceinline__ void pd_gemv_item(PdShared &sh, const float *in, const f32x4 (&wb)[PD_WB], int K, u64 *out,
                                             u32 tag)
{
    const int tid = threadIdx.x;
    const float r = pd_colsum<0>(pd_dot<MAXI>(in, wb, K), sh.red[0]);
    if (tid < 64 && (tid & 1) == 0) pd_st(out + (tid >> 1), pd_word(r, tag));
    __syncthreads();
}

// A SwiGLU item (after the norm parts of the layer's second norm): the 16 W1 and
// the 16 W3 columns of the panel against xn, scaled by the norm's s, then
// out[c] = silu(W1 col) * (W3 col) (:786, :3821-3823), published with `tag`.
__device__ __forceinline__ void pd_swiglu_item(PdShared &sh, const f32x4 (&wb)[PD_WB], int D, u64 *out, u32 tag)
{
    const int tid = threadIdx.x;
    // lanes 4 p, 4 p + 1 of wave 0 hold W1 column p, lanes 4 p + 2, 4 p + 3 its W3 column
    const float sn = pd_norm_scale(sh.sw, D);
    const float r = pd_colsum<1>(pd_dot<PD_MAXQ>(sh.xn, wb, D), sh.red[0]) * sn;
    const float u = pd_pair_other(r);
    // silu(r) = r / (1 + e^-r) with the hardware exp2 and reciprocal (a few ulp
    // from the reference's expf and divide)
    const float e = __builtin_amdgcn_exp2f(-r * 1.44269504088896f);
    if (tid < 64 && (tid & 3) == 0) pd_st(out + (tid >> 2), pd_word(r * __builtin_amdgcn_rcpf(1.0f + e) * u, tag));
    __syncthreads();
}

template <int F16>
__global__ __launch_bounds__(PD_T, 1) void k_dec_persist(TlgDecPersist a, int n)
{
    __shared__ PdShared sh;
    const int tid = threadIdx.x;
    // workgroup b runs on XCD b % 8 (round-robin dispatch); items are owned by the
    // virtual index b' = (b % 8) NB / 8 + b / 8, so consecutive items (a layer's
    // attention and O items, its W2 items) share an XCD, whose exchanges are
    // shorter than across XCDs
    const int NB = gridDim.x,
              b = (NB % 8) ? (int)blockIdx.x : (int)(blockIdx.x % 8u) * (NB / 8) + (int)(blockIdx.x / 8u);
    const int D = a.D, F = a.F, V = a.V, L = a.L, H = a.H, KD = a.KV * 32, grp = a.H / a.KV;
    const int NA = H, NO = D / 32, NS = F / 16, NPL = NA + NO + NS + D / 32, NLI = L * NPL, NHI = V / 8;
    const u32 NPH = 4u * (u32)L + 1u;
    const int qk = a.qknorm ? 64 : 0;                 // the QK-norm gains qn, kn (hd = 32 each) after wo
    const size_t per = (size_t)D + (size_t)D * D + 2 * (size_t)D * KD + (size_t)D * D + qk + D + 3 * (size_t)D * F;
    const size_t lay0 = (size_t)V * D;
    u64 *xb = reinterpret_cast<u64 *>(a.xbuf);
    const PdLayout lay = pd_layout(V, D, L, F);
    u32 *abortp = reinterpret_cast<u32 *>(xb + lay.ctrl);
    const int pos0 = gp(a.state)[0];
    const u32 base = (u32)gp(a.state)[3];
    int tok = gp(a.state)[2];
    if (b >= NLI && b >= NHI) return;
    if (tid == 0) {                      // constant indices: scalar kernel-argument loads
#pragma unroll
        for (int i = 0; i < 16; i++) sh.P[i] = a.P[i];
#pragma unroll
        for (int i = 0; i < TLG_PD_MAXL; i++) { sh.Kc[i] = a.Kc[i]; sh.Vc[i] = a.Vc[i]; }
    }
    __syncthreads();

    // this workgroup's items: layer items g = b, b + NB, ... < NLI of every
    // token (panel and gain prefetched one item ahead into wb, gn), head items
    // j = b, b + NB, ... < NHI (the first prefetched at the token's start)
    f32x4 wb[PD_WB];
    float gn = 0.f;
    f32x4 hb[2];
    u64 kw[PD_MAXR], vw[PD_MAXR];
    if (b < NLI)
        pd_load_item(wb, gn, pd_uni(sh.P[a.copy0 % a.pool]), b, NPL, NA, NO, NS, lay0, per, D, KD, F, grp, qk);
    // this workgroup's first attention item in layer l (query head), or -1
    auto attn_head = [&](int l) -> int {
        const int s = l * NPL, g = s + ((b - s) % NB + NB) % NB;
        return g < s + NA ? g - s : -1;
    };

    for (int t = 0; t < n; t++) {
        const float *P = pd_uni(sh.P[(a.copy0 + t) % a.pool]);
        const int pos = pos0 + t;
        const u32 tag0 = base + (u32)t * NPH + 1u;            // tag of phase 0 of this token
        // ---- token start: the previous step's greedy token, x = emb[tok]
        if (t > 0) {
            if (!pd_argmax(sh, xb + lay.cand + (size_t)((t - 1) & 1) * NHI * 2, NHI, tag0 - 1u, abortp)) return;
            tok = sh.tok;
            if (b == 0 && tid == 0 && a.toks_out) gp(a.toks_out)[t - 1] = tok;
        }
        {   // x = emb[tok], with the norm parts for the first item's gain (attention: an1)
            const float xv = (tok >= 0 && tok < V) ? gp(P)[(size_t)min(tid, D - 1) + (size_t)tok * D] : NAN;
            if (tid < D) sh.x[tid] = xv;
            pd_norm_parts(xv, gn, sh.xn, D, sh.sw);
        }
        pd_load_head(hb, P, min(b, NHI - 1), D);
        const float hg = pd_at<float>(P + lay0 + (size_t)L * per, 4u * (u32)min(tid, D - 1));
        const bool inpos = pos >= 0 && pos < a.maxpos;
        // RoPE factors of pair (tid >> 2) & 15, the pair this thread's quad reads
        const float rc = inpos ? gp(a.cs)[(size_t)pos * 16 + ((tid >> 2) & 15)] : 0.f;
        const float rs = inpos ? gp(a.sn)[(size_t)pos * 16 + ((tid >> 2) & 15)] : 0.f;
        {   // ring words of layer 0's attention
            const int h = attn_head(0);
            int lo, cnt;
            pd_window(a, 0, pos, &lo, &cnt);
            if (h >= 0) pd_ring_load<F16, 1, F16>(kw, vw, sh.Kc[0], sh.Vc[0], h / grp, KD, a.W, lo, cnt);
        }
        __syncthreads();

        for (int l = 0; l < L; l++) {
            const int g0 = l * NPL;
            const u32 tl = tag0 + 4u * (u32)l;                  // ctx, O out, act, W2 out: tl .. tl + 3
            u64 *ctx = xb + lay.ctx + (size_t)l * D, *yo = xb + lay.yo + (size_t)l * D;
            u64 *act = xb + lay.act + (size_t)l * F, *y2 = xb + lay.y2 + (size_t)l * D;
            // first item index >= g0 + k0 that belongs to this workgroup
#define PD_FIRST(k0) ((g0 + (k0)) + ((b - (g0 + (k0))) % NB + NB) % NB)
// the next item's panel (past the last token: a harmless reload, so that wb is
// always overwritten)
#define PD_NEXT(g)                                                                                           \
    do {                                                                                                     \
        const int ng_ = (g) + NB < NLI ? (g) + NB : b, nt_ = min((g) + NB < NLI ? t : t + 1, n - 1);          \
        pd_load_item(wb, gn, pd_uni(sh.P[(a.copy0 + nt_) % a.pool]), ng_, NPL, NA, NO, NS, lay0, per, D, KD, F, \
                     grp, qk);                                                                               \
    } while (0)

            for (int g = PD_FIRST(0); g < g0 + NA; g += NB) {
                if (g != PD_FIRST(0)) {      // a second attention item in this layer: its ring words,
                    int lo, cnt;             // and the norm parts again (the first one's softmax used sw)
                    pd_window(a, l, pos, &lo, &cnt);
                    pd_ring_load<F16, 1, F16>(kw, vw, sh.Kc[l], sh.Vc[l], (g - g0) / grp, KD, a.W, lo, cnt);
                    pd_norm_parts(sh.x[min(tid, D - 1)], gn, sh.xn, D, sh.sw);
                    __syncthreads();
                }
                pd_attention<F16>(sh, wb, rc, rs, kw, vw, a, l, g - g0, pos, D, KD, grp,
                                  qk ? P + lay0 + (size_t)l * per + D + 2 * (size_t)D * D + 2 * (size_t)D * KD
                                     : nullptr,
                                  ctx + (size_t)(g - g0) * 32, tl);
                PD_NEXT(g);
            }
            for (int g = PD_FIRST(NA); g < g0 + NA + NO; g += NB) {        // O: ctx . Wo
                if (!pd_fetch<1, 0>(ctx, D, tl, sh.in, abortp)) return;
                pd_gemv_item<PD_MAXQ>(sh, sh.in, wb, D, yo + (size_t)(g - g0 - NA) * 32, tl + 1u);
                PD_NEXT(g);
            }
            // x += O out, with the norm parts for the next item's gain (SwiGLU: an2)
            if (!pd_fetch<1, 1, 1>(yo, D, tl + 1u, sh.x, abortp, gn, sh.xn, sh.sw)) return;
            if (l + 1 < L) {                 // ring words of the next layer's attention, early
                const int h = attn_head(l + 1);
                int lo, cnt;
                pd_window(a, l + 1, pos, &lo, &cnt);
                if (h >= 0)
                    pd_ring_load<F16, 1, F16>(kw, vw, sh.Kc[l + 1], sh.Vc[l + 1], h / grp, KD, a.W, lo, cnt);
            }
            for (int g = PD_FIRST(NA + NO); g < g0 + NA + NO + NS; g += NB) {    // silu(xn . W1) * (xn . W3)
                pd_swiglu_item(sh, wb, D, act + (size_t)(g - g0 - NA - NO) * 16, tl + 2u);
                PD_NEXT(g);
            }
            for (int g = PD_FIRST(NA + NO + NS); g < g0 + NPL; g += NB) {       // act . W2
                if (!pd_fetch<2, 0>(act, F, tl + 2u, sh.in, abortp)) return;
                pd_gemv_item<PD_MAXFQ>(sh, sh.in, wb, F, y2 + (size_t)(g - g0 - NA - NO - NS) * 32, tl + 3u);
                PD_NEXT(g);
            }
            // x += W2 out, with the norm parts for the next item's gain (attention: an1;
            // after the last layer the head's final-norm gain)
            if (!pd_fetch<1, 1, 1>(y2, D, tl + 3u, sh.x, abortp, l + 1 < L ? gn : hg, sh.xn, sh.sw)) return;
#undef PD_FIRST
#undef PD_NEXT
        }

        // ---- head: 8 vocabulary rows per item against x g (final-norm gain), scaled
        // by the norm's s, and their first maximum
        if (b < NHI) {
            const u32 th = tag0 + 4u * (u32)L;
            u64 *cand = xb + lay.cand + (size_t)(t & 1) * NHI * 2;
            const float s = pd_norm_scale(sh.sw, D);        // norm parts from the last x fetch
            for (int j = b; j < NHI; j += NB) {
                f32x4 hw[2] = {hb[0], hb[1]};
                if (j != b) pd_load_head(hw, P, j, D);
                const int r = tid >> 6, c = tid & 63;
                float acc = 0.f;
#pragma unroll
                for (int i = 0; i < 2; i++)
                    if (4 * (c + 64 * i) < D) {
                        const f32x4 f = *reinterpret_cast<const f32x4 *>(sh.xn + 4 * (c + 64 * i));
                        acc = fmaf(f.x, hw[i].x, acc);
                        acc = fmaf(f.y, hw[i].y, acc);
                        acc = fmaf(f.z, hw[i].z, acc);
                        acc = fmaf(f.w, hw[i].w, acc);
                    }
                acc = pd_wave_sum(acc) * s;
                if (c == 0) {
                    sh.lg[r] = acc;
                    gp(a.logits)[(size_t)8 * j + r] = acc;
                }
                __syncthreads();
                if (tid == 0) {
                    float bv = -INFINITY;
                    int bi = 0x7fffffff;
                    for (int rr = 0; rr < 8; rr++)
                        if (sh.lg[rr] > bv) { bv = sh.lg[rr]; bi = 8 * j + rr; }
                    pd_st(cand + (size_t)2 * j, pd_word(bv, th));
                    pd_st(cand + (size_t)2 * j + 1, ((u64)th << 32) | (u64)(u32)bi);
                }
                __syncthreads();
            }
        }
    }

    // ---- the last step's greedy token and the state for the next launch
    if (b == 0) {
        const u32 th = base + (u32)n * NPH;                    // head tag of token n - 1
        if (!pd_argmax(sh, xb + lay.cand + (size_t)((n - 1) & 1) * NHI * 2, NHI, th, abortp)) return;
        if (tid == 0) {
            const int tk = sh.tok;
            if (a.toks_out) gp(a.toks_out)[n - 1] = tk;
            GAS int *st = gp(a.state);
            st[0] = pos0 + n;
            st[1] = 1;
            st[2] = tk;
            st[3] = (int)(base + (u32)n * NPH);
            gp(a.tok)[0] = tk;
        }
    }
}

// ================================================================ chunks ==
// forward_chunk at m = MR rows (tinylm.c:3721-3830) for n chunks of MR
// consecutive positions whose tokens are given (prefill; the verification
// chunk of speculative decoding, :3989), in ONE cooperative launch.  The M
// rows share every weight load, so a step streams the same 52.7 MB (the
// configs[3] model) for MR tokens.
//
// Phases of a layer (item i of a chunk to workgroup i % NB, as above):
//   QKV  (D + 2 KD) / 32 items  32 columns of [Wq | Wk | Wv] (one head) for
//                                the MR rows of RMSNorm(x); RoPE on q and k;
//                                the k and v items store the MR new ring rows
//                                of their KV head (kv_store, :3775-3780) and
//                                publish them in the ring's precision
//   ATT  H * MR items            head h, row j (ordered by KV head, then row,
//                                then head): softmax attention of q_j over
//                                the window of position pos + j (attn_body,
//                                :3639-3715): ring keys before pos, the
//                                chunk's new keys pos .. pos + j, and -- as the
//                                reference's hoisted stores leave the ring --
//                                a window key whose slot a later row of the
//                                chunk wrote reads that row's key
//   O    D / 32                  32 columns of ctx . Wo, every row
//   SW   F / 16                  RMSNorm(x) . W1 and . W3, 16 columns each,
//                                silu(g) * u
//   W2   D / 32                  32 columns of act . W2
//   head V / 8 items per chunk   8 vocabulary rows against the final-normed
//                                rows, their first maximum per row
// Every workgroup adds the O and W2 outputs of every layer into its own copy
// of the MR residual rows (same order everywhere, bit-identical copies).  A
// chunk starts once the previous chunk's argmax candidates are all there, so
// chunk t + 1 reads ring rows chunk t completed, and no exchange word is
// rewritten while a workgroup of the previous chunk may still read it.
#define PC_MAXMR 8
#define PC_MAXQKV (3 * PD_MAXD)     // D + 2 KD with KD <= D

struct PcLayout {
    size_t ctrl, qkv, ctx, yo, act, y2, cand, total;
};
__host__ __device__ static inline PcLayout pc_layout(int V, int D, int KD, int L, int F, int MR)
{
    PcLayout o;
    size_t p = 0;
    o.ctrl = p; p += 8;
    o.qkv = p;  p += (size_t)L * MR * (D + 2 * KD);
    o.ctx = p;  p += (size_t)L * MR * D;
    o.yo = p;   p += (size_t)L * MR * D;
    o.act = p;  p += (size_t)L * MR * F;
    o.y2 = p;   p += (size_t)L * MR * D;
    o.cand = p; p += (size_t)2 * MR * (V / 8) * 2;
    o.total = p;
    return o;
}

template <int MR> struct PcShared {
    float x[MR][PD_MAXD], xn[MR][PD_MAXD];
    float in[MR * PD_MAXF];
    f32x4 red[MR][PD_RED];
    float sw[MR][PD_NW];
    float col[MR][64];                  // an item's column results (q / k / v, SwiGLU g and u)
    float q[32], kn[MR][32], vn[MR][32];
    float ctxw[PD_T / 16][32];
    float sm[2 * PD_NW];
    u64 key[PD_NW];
    float lg[MR][8];
    int tok[MR];
    const float *P[16];
    void *Kc[TLG_PD_MAXL], *Vc[TLG_PD_MAXL];
};

// The norm parts of the MR rows of x (tid < D holds element tid of every row)
// for gain element gj: xg[j][tid] = x[j][tid] g and the waves' sums of x^2
// (sw[j][wave]); made visible by the caller's next barrier.
template <int MR>
__device__ __forceinline__ void pc_norm_parts(const float (&x)[MR][PD_MAXD], float gj, float (&xg)[MR][PD_MAXD],
                                              int D, float (&sw)[MR][PD_NW])
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < MR; j++) {
        const float xv = tid < D ? x[j][tid] : 0.f;
        if (tid < D) xg[j][tid] = xv * gj;
        const float ss = pd_wave_sum(xv * xv);
        if ((tid & 63) == 0) sw[j][tid >> 6] = ss;
    }
}

// Column panel against the MR rows of vin (row stride PD_MAXD, or F for the
// W2 input): thread (c4, rg) sums rows rg + 64 i of its 4 columns for every
// row, then pd_colsum_put per row.  After the caller's barrier, red[j] holds
// row j's partials.
template <int MAXI, int MR>
__device__ __forceinline__ void pc_panel(const float *vin, int ldv, const f32x4 *w, int K, f32x4 (*red)[PD_RED])
{
    const int rg = threadIdx.x >> 3;
    // two rows at a time: all the rows' activations at once would need MR x
    // MAXI registers next to the panel's
#pragma unroll 2
    for (int j = 0; j < MR; j++) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < MAXI; i++) {
            const bool in = K == 64 * MAXI || rg + 64 * i < K;
            const float xv = vin[j * ldv + min(rg + 64 * i, K - 1)];
            acc.x = in ? fmaf(xv, w[i].x, acc.x) : acc.x;
            acc.y = in ? fmaf(xv, w[i].y, acc.y) : acc.y;
            acc.z = in ? fmaf(xv, w[i].z, acc.z) : acc.z;
            acc.w = in ? fmaf(xv, w[i].w, acc.w) : acc.w;
        }
        pd_colsum_put(acc, red[j]);
    }
}

// Wait until the n words at src + idx(e), e < n, carry `tag`, then dst[e] =
// their values (KPL words per thread).  Like pd_fetch, for gathered words.
template <int KPL, class IDX>
__device__ bool pc_gather(const u64 *src, int n, IDX idx, u32 tag, float *dst, u32 *abortp)
{
    const int tid = threadIdx.x;
    const u64 t0 = wall_clock64();
    u64 w[KPL];
    int stop = 0;
    for (int it = 0;; it++) {
#pragma unroll
        for (int k = 0; k < KPL; k++) w[k] = pd_ld(src + idx(min(tid + PD_T * k, n - 1)));
        int bad = 0;
#pragma unroll
        for (int k = 0; k < KPL; k++) bad |= (tid + PD_T * k < n) && (u32)(w[k] >> 32) != tag;
        if (__ballot(bad) == 0ull) break;
        if ((it & 7) == 7) {
            int s = 0;
            if ((tid & 63) == 0)
                s = __hip_atomic_load(gp(abortp), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u ||
                    wall_clock64() - t0 > PD_SPIN;
            if (__ballot(s) != 0ull) { stop = 1; break; }
        }
    }
    if (!stop) {
#pragma unroll
        for (int k = 0; k < KPL; k++)
            if (tid + PD_T * k < n) dst[tid + PD_T * k] = __uint_as_float((u32)w[k]);
    }
    if (__syncthreads_or(stop)) {
        if (tid == 0) __hip_atomic_store(gp(abortp), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    return true;
}

// x[j] += the MR x D words of src (row-major), the norm parts for gain gj
// after; false after an abort.
template <int MR>
__device__ bool pc_add_rows(PcShared<MR> &sh, const u64 *src, int D, u32 tag, float gj, u32 *abortp)
{
    constexpr int KPL = (MR * PD_MAXD + PD_T - 1) / PD_T;
    if (!pd_fetch<KPL, 0>(src, MR * D, tag, sh.in, abortp)) return false;
    const int tid = threadIdx.x;
    if (tid < D)
#pragma unroll
        for (int j = 0; j < MR; j++) sh.x[j][tid] += sh.in[j * D + tid];
    pc_norm_parts<MR>(sh.x, gj, sh.xn, D, sh.sw);
    __syncthreads();
    return true;
}

// The first maximum of each row's argmax candidates (2 words per head item:
// value, index) into sh.tok[j]; false after an abort.
template <int MR>
__device__ bool pc_argmax(PcShared<MR> &sh, const u64 *cand, int NHI, u32 tag, u32 *abortp)
{
    const int tid = threadIdx.x;
    if (!pd_fetch<(2 * MR * PD_MAXHI + PD_T - 1) / PD_T, 0>(cand, 2 * MR * NHI, tag, sh.in, abortp))
        return false;
#pragma unroll 1
    for (int j = 0; j < MR; j++) {
        u64 kx = 0;
        if (tid < NHI) {
            const u32 i = __float_as_uint(sh.in[(j * NHI + tid) * 2 + 1]);
            kx = i == 0x7fffffffu ? 0 : pd_argkey(sh.in[(j * NHI + tid) * 2], i);
        }
        const u32 hm = pd_wave_umax((u32)(kx >> 32));
        const u32 lm = pd_wave_umax((u32)(kx >> 32) == hm ? (u32)kx : 0u);
        if ((tid & 63) == 0) sh.key[tid >> 6] = ((u64)hm << 32) | lm;
        __syncthreads();
        if (tid == 0) {
            u64 m = sh.key[0];
#pragma unroll
            for (int w = 1; w < PD_NW; w++) m = max(m, sh.key[w]);
            sh.tok[j] = m == 0 ? 0 : (int)(~(u32)m);
        }
        __syncthreads();
    }
    return true;
}

// Attention of row j (position p = pos + j) of query head h, layer l: the
// ring words kw / vw of the window's keys before pos are loaded (pd_ring_load
// with key count cnt - j ... see the caller); sh.q holds q_j, sh.kn / sh.vn the
// chunk's new rows of the head's KV head.  ctx_j of the head is published.
template <int F16, int MR>
__device__ __forceinline__ void pc_attention(PcShared<MR> &sh, u64 (&kw)[PD_MAXR], u64 (&vw)[PD_MAXR],
                                             const TlgDecPersist &a, int pos, int j, int lo, int cnt, u64 *ctxout,
                                             u32 tag)
{
    typedef PdRing<F16> R;
    constexpr int NW = R::NW, KPR = PD_T / NW, MAXR = PD_MAXW / KPR;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int key0 = tid >> R::LOG2NW, wd = tid & (NW - 1);
    // key t = lo + key0 + KPR r (window order).  Position tp = lo + t: a new
    // row (tp >= pos) or a slot a later row of the chunk overwrote (tp <
    // pos - W + MR) reads that row of the chunk; every other key its ring word
    float qv[R::EPW];
#pragma unroll
    for (int e = 0; e < R::EPW; e++) qv[e] = sh.q[R::EPW * wd + e];
    const float scale = 1.0f / sqrtf(32.0f);
    float sc[MAXR];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < MAXR; r++) {
        const int t = key0 + KPR * r, tp = lo + t;
        const int nr = tp >= pos ? tp - pos : tp - pos + a.W;      // chunk row of the key, if any
        if (t < cnt && nr >= 0 && nr < MR) {
            kw[r] = R::pack(&sh.kn[nr][R::EPW * wd]);
            vw[r] = R::pack(&sh.vn[nr][R::EPW * wd]);
        }
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < R::EPW; e++) part = fmaf(qv[e], R::get(kw[r], e), part);
        part += pd_dpp<0xB1, 0xf>(0.f, part);
        part += pd_dpp<0x4E, 0xf>(0.f, part);
        {
            const float r4 = pd_dpp<0x124, 0xf>(0.f, part), r12 = pd_dpp<0x12C, 0xf>(0.f, part);
            part += (lane & 4) ? r4 : r12;
        }
        if (NW == 16) part += pd_dpp<0x128, 0xf>(0.f, part);
        sc[r] = t < cnt ? part * scale : -INFINITY;
        mx = fmaxf(mx, sc[r]);
    }
    mx = pd_keys_max<NW>(mx);
    if (lane == 0) sh.sm[wave] = mx;
    __syncthreads();
    mx = sh.sm[0];
#pragma unroll
    for (int w = 1; w < PD_NW; w++) mx = fmaxf(mx, sh.sm[w]);
    float sum = 0.f;
#pragma unroll
    for (int r = 0; r < MAXR; r++) {
        const int t = key0 + KPR * r;
        const float e = a.exact ? expf(sc[r] - mx) : tlg_fast_expf(sc[r] - mx);
        sc[r] = t < cnt ? e : 0.f;
        sum += sc[r];
    }
    sum = pd_keys_sum<NW>(sum);
    if (lane == 0) sh.sm[PD_NW + wave] = sum;
    float acc[R::EPW];
#pragma unroll
    for (int e = 0; e < R::EPW; e++) acc[e] = 0.f;
#pragma unroll
    for (int r = 0; r < MAXR; r++) {
        const int t = key0 + KPR * r;
#pragma unroll
        for (int e = 0; e < R::EPW; e++) acc[e] = t < cnt ? fmaf(sc[r], R::get(vw[r], e), acc[e]) : acc[e];
    }
    const int row = tid >> 4;
#pragma unroll
    for (int e = 0; e < R::EPW; e++) {
        if (NW == 8) acc[e] += pd_dpp<0x128, 0xf>(0.f, acc[e]);
        if ((tid & 15) < NW) sh.ctxw[row][R::EPW * wd + e] = acc[e];
    }
    __syncthreads();
    if (tid < 64) {
        float tot = sh.sm[PD_NW];
#pragma unroll
        for (int w = 1; w < PD_NW; w++) tot += sh.sm[PD_NW + w];
        const int d = tid >> 1, r0 = 16 * (tid & 1);
        float c0 = sh.ctxw[r0][d], c1 = sh.ctxw[r0 + 8][d];
#pragma unroll
        for (int rr = 1; rr < 8; rr++) {
            c0 += sh.ctxw[r0 + rr][d];
            c1 += sh.ctxw[r0 + 8 + rr][d];
        }
        float cx = c0 + c1;
        cx += pd_dpp<0xB1, 0xf>(0.f, cx);
        cx = tot > 0.f ? (a.exact ? cx / tot : cx * __builtin_amdgcn_rcpf(tot)) : 0.f;
        if ((tid & 1) == 0) pd_st(ctxout + d, pd_word(cx, tag));
    }
    __syncthreads();
}

// Item counts of a chunk layer at MR rows.  Every GEMV phase has one item per
// (column block, row) -- SW items take RS rows -- so the VALU work of an item
// stays that of a single row and the MR rows spread over MR times as many
// workgroups; the items of one column block are consecutive (one XCD), so
// the panel they all read comes from that XCD's L2 after the first.
struct PcItems {
    int NQ, NQI, NA, NOI, RS, NSI, NWI, NPL;
    __device__ PcItems(int MR, int D, int KD, int H, int F)
    {
        NQ = (D + 2 * KD) / 32;
        NQI = NQ * MR;
        NA = H * MR;
        NOI = (D / 32) * MR;
        RS = MR >= 4 ? MR / 4 : 1;
        NSI = (F / 16) * (MR / RS);
        NWI = (D / 32) * MR;
        NPL = NQI + NA + NOI + NSI + NWI;
    }
};

// The weight panel of chunk item g (index within a chunk's layer items):
// QKV: 32 columns of Wq (q heads), Wk or Wv (KV heads); O: Wo; SW: W1 | W3
// (threads c4 < 4 / >= 4); W2 (K = F); ATT items load no panel.  The RMSNorm
// gain element of thread tid for items that normalise x.
__device__ __forceinline__ void pc_load_item(f32x4 (&wb)[PD_MAXFQ], float &gn, const float *__restrict__ P, int g,
                                             const PcItems &it, int MR, int H, int KV, size_t lay0, size_t per,
                                             int D, int KD, int F)
{
    const int l = g / it.NPL, k = g % it.NPL;
    const size_t an1 = lay0 + (size_t)l * per, wq = an1 + D, wk = wq + (size_t)D * D, wv = wk + (size_t)D * KD,
                 wo = wv + (size_t)D * KD, an2 = wo + (size_t)D * D, w1 = an2 + D, w3 = w1 + (size_t)D * F,
                 w2 = w3 + (size_t)D * F;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    const int tid = threadIdx.x, c4 = tid & 7;
    const u32 gof = 4u * (u32)min(tid, D - 1);
    gn = 0.f;
    if (k < it.NQI) {
        const int c = k / MR;
        if (c < H) pd_load_cols<PD_MAXQ>(wb, P + wq, D, c * 32, D);
        else if (c < H + KV) pd_load_cols<PD_MAXQ>(wb, P + wk, KD, (c - H) * 32, D);
        else pd_load_cols<PD_MAXQ>(wb, P + wv, KD, (c - H - KV) * 32, D);
        gn = pd_at<float>(P + an1, gof);
    } else if (k < it.NQI + it.NA) {
#pragma unroll
        for (int i = 0; i < PD_MAXQ; i++) wb[i] = z;
    } else if (k < it.NQI + it.NA + it.NOI) {
        pd_load_cols<PD_MAXQ>(wb, P + wo, D, ((k - it.NQI - it.NA) / MR) * 32, D);
    } else if (k < it.NQI + it.NA + it.NOI + it.NSI) {
        const int c = (k - it.NQI - it.NA - it.NOI) / (MR / it.RS);
        const float *W = c4 < 4 ? P + w1 : P + w3;
        pd_load_cols<PD_MAXQ>(wb, W, F, 16 * c - 4 * (c4 & 4), D);
        gn = pd_at<float>(P + an2, gof);
    } else {
        pd_load_cols<PD_MAXFQ>(wb, P + w2, D, ((k - it.NQI - it.NA - it.NOI - it.NSI) / MR) * 32, F);
        return;
    }
#pragma unroll
    for (int i = PD_MAXQ; i < PD_MAXFQ; i++) wb[i] = z;
}

// The 32 column sums of panel row j after pc_panel<..., 1> into red[0]:
// wave 0's lanes 2 i, 2 i + 1 get column i (PAIRS 0), or the SwiGLU pairing
// (PAIRS 1); the caller's barrier precedes.
template <int PAIRS> __device__ __forceinline__ float pc_cols(const f32x4 *red)
{
    return threadIdx.x < 64 ? pd_colsum_half(red, pd_half_col<PAIRS>(threadIdx.x)) : 0.f;
}

template <int F16, int MR>
__global__ __launch_bounds__(PD_T, 1) void k_dec_chunk(TlgDecPersist a, const int *toks_in, int n)
{
    typedef PdRing<F16> R;
    __shared__ PcShared<MR> sh;
    const int tid = threadIdx.x;
    const int NB = gridDim.x,
              b = (NB % 8) ? (int)blockIdx.x : (int)(blockIdx.x % 8u) * (NB / 8) + (int)(blockIdx.x / 8u);
    const int D = a.D, F = a.F, V = a.V, L = a.L, H = a.H, KV = a.KV, KD = a.KV * 32, grp = a.H / a.KV;
    const int QN = D + 2 * KD;
    const PcItems it(MR, D, KD, H, F);
    const int NPL = it.NPL, NLI = L * NPL, NHI = V / 8;
    const u32 NPH = 5u * (u32)L + 1u;
    const size_t per = (size_t)D + (size_t)D * D + 2 * (size_t)D * KD + (size_t)D * D + D + 3 * (size_t)D * F;
    const size_t lay0 = (size_t)V * D;
    u64 *xb = reinterpret_cast<u64 *>(a.xbuf);
    const PcLayout lay = pc_layout(V, D, KD, L, F, MR);
    u32 *abortp = reinterpret_cast<u32 *>(xb + lay.ctrl);
    const int pos0 = gp(a.state)[0];
    const u32 base = (u32)gp(a.state)[3];
    if (b >= NLI && b >= NHI) return;
    if (tid == 0) {
#pragma unroll
        for (int i = 0; i < 16; i++) sh.P[i] = a.P[i];
#pragma unroll
        for (int i = 0; i < TLG_PD_MAXL; i++) { sh.Kc[i] = a.Kc[i]; sh.Vc[i] = a.Vc[i]; }
    }
    __syncthreads();

    f32x4 wb[PD_MAXFQ];
    float gn = 0.f;
    u64 kw[PD_MAXR], vw[PD_MAXR];
    if (b < NLI) pc_load_item(wb, gn, pd_uni(sh.P[a.copy0 % a.pool]), b, it, MR, H, KV, lay0, per, D, KD, F);

    for (int t = 0; t < n; t++) {
        const float *P = pd_uni(sh.P[(a.copy0 + t) % a.pool]);
        const int pos = pos0 + t * MR;
        const u32 tag0 = base + (u32)t * NPH + 1u;
        if (t > 0) {            // the previous chunk's head is complete: its greedy tokens
            if (!pc_argmax<MR>(sh, xb + lay.cand + (size_t)((t - 1) & 1) * MR * NHI * 2, NHI, tag0 - 1u, abortp))
                return;
            if (b == 0 && tid < MR && a.toks_out) gp(a.toks_out)[(size_t)(t - 1) * MR + tid] = sh.tok[tid];
        }
        // x = emb[token] for the MR rows, norm parts for the first item's gain
        if (tid < D)
#pragma unroll
            for (int j = 0; j < MR; j++) {
                const int tk = gp(toks_in)[(size_t)t * MR + j];
                sh.x[j][tid] = (tk >= 0 && tk < V) ? gp(P)[(size_t)tk * D + tid] : NAN;
            }
        __syncthreads();
        pc_norm_parts<MR>(sh.x, gn, sh.xn, D, sh.sw);
        __syncthreads();
        const float hg = pd_at<float>(P + lay0 + (size_t)L * per, 4u * (u32)min(tid, D - 1));

        for (int l = 0; l < L; l++) {
            const int g0 = l * NPL;
            const u32 tl = tag0 + 5u * (u32)l;              // qkv, ctx, yo, act, y2: tl .. tl + 4
            u64 *qkv = xb + lay.qkv + (size_t)l * MR * QN, *ctx = xb + lay.ctx + (size_t)l * MR * D;
            u64 *yo = xb + lay.yo + (size_t)l * MR * D, *act = xb + lay.act + (size_t)l * MR * F;
            u64 *y2 = xb + lay.y2 + (size_t)l * MR * D;
            const int kA = it.NQI, kO = kA + it.NA, kS = kO + it.NOI, kW = kS + it.NSI;
#define PC_FIRST(k0) ((g0 + (k0)) + ((b - (g0 + (k0))) % NB + NB) % NB)
#define PC_NEXT(g)                                                                                            \
    do {                                                                                                      \
        const int ng_ = (g) + NB < NLI ? (g) + NB : b, nt_ = min((g) + NB < NLI ? t : t + 1, n - 1);           \
        pc_load_item(wb, gn, pd_uni(sh.P[(a.copy0 + nt_) % a.pool]), ng_, it, MR, H, KV, lay0, per, D, KD, F); \
    } while (0)
            // ---- QKV: 32 columns of one head, one row
            for (int g = PC_FIRST(0); g < g0 + kA; g += NB) {
                const int c = (g - g0) / MR, j = (g - g0) % MR, p = pos + j;  // c < H: q; < H + KV: k; else v
                pc_panel<PD_MAXQ, 1>(&sh.xn[j][0], PD_MAXD, wb, D, sh.red);
                __syncthreads();
                if (tid < 64) {
                    float s = 0.f;
#pragma unroll
                    for (int w = 0; w < PD_NW; w++) s += sh.sw[j][w];
                    const float v = pc_cols<0>(sh.red[0]) * rsqrtf(s / (float)D + 1e-5f);
                    if ((tid & 1) == 0) sh.col[0][tid >> 1] = v;
                }
                __syncthreads();
                if (tid < 32) {                              // RoPE (q, k), ring precision (k, v)
                    const int i = tid;
                    const float cv = sh.col[0][i], o = sh.col[0][i ^ 16];
                    float r = cv;
                    if (c < H + KV) {
                        const bool inpos = p >= 0 && p < a.maxpos;
                        const float rc = inpos ? gp(a.cs)[(size_t)p * 16 + (i & 15)] : 0.f;
                        const float rs = inpos ? gp(a.sn)[(size_t)p * 16 + (i & 15)] : 0.f;
                        r = inpos ? (i < 16 ? cv * rc - o * rs : cv * rc + o * rs) : NAN;
                    }
                    if (c >= H) r = R::round(r);
                    sh.col[0][32 + i] = r;
                }
                __syncthreads();
                if (c >= H && tid < R::NW) {                 // the ring row of position p (kv_store)
                    const int kvh = c < H + KV ? c - H : c - H - KV;
                    char *row = reinterpret_cast<char *>(c < H + KV ? sh.Kc[l] : sh.Vc[l]) +
                                ((size_t)(p % a.W) * KD + (size_t)kvh * 32) * sizeof(typename R::E);
                    pd_st(reinterpret_cast<u64 *>(row) + tid, R::pack(&sh.col[0][32 + R::EPW * tid]));
                    pd_wait_stores();
                }
                __syncthreads();
                if (tid < 32) {
                    const int off = c < H ? c * 32 : c < H + KV ? D + (c - H) * 32 : D + KD + (c - H - KV) * 32;
                    pd_st(qkv + (size_t)j * QN + off + tid, pd_word(sh.col[0][32 + tid], tl));
                }
                PC_NEXT(g);
            }
            // ---- ATT: head h, row j
            for (int g = PC_FIRST(kA); g < g0 + kO; g += NB) {
                // items (KV head, row, head of the group) in that order: the rows and
                // heads reading one KV head's ring window are consecutive (one XCD)
                const int ka = g - g0 - kA, kvh = ka / (MR * grp), j = (ka / grp) % MR;
                const int h = kvh * grp + ka % grp, p = pos + j;
                int lo, cnt;
                pd_window(a, l, p, &lo, &cnt);
                // ring words of the window's keys (those of the chunk's rows are
                // replaced in pc_attention); issued before the wait for this chunk's rows
                pd_ring_load<F16, 1, 1>(kw, vw, sh.Kc[l], sh.Vc[l], kvh, KD, a.W, lo, cnt + 1);
                // q_j of head h, then the chunk's k and v rows of KV head kvh
                auto qi = [&](int e) -> size_t {
                    if (e < 32) return (size_t)j * QN + h * 32 + e;
                    e -= 32;
                    const int r = e / 64, w = e % 64;
                    return (size_t)r * QN + D + (w < 32 ? 0 : KD) + kvh * 32 + (w & 31);
                };
                if (!pc_gather<(32 + MR * 64 + PD_T - 1) / PD_T>(qkv, 32 + MR * 64, qi, tl, sh.in, abortp)) return;
                if (tid < 32) sh.q[tid] = sh.in[tid];
                if (tid < MR * 64) {
                    const int r = tid / 64, w = tid % 64;
                    if (w < 32) sh.kn[r][w] = sh.in[32 + tid];
                    else sh.vn[r][w - 32] = sh.in[32 + tid];
                }
                __syncthreads();
                pc_attention<F16, MR>(sh, kw, vw, a, pos, j, lo, cnt, ctx + (size_t)j * D + h * 32, tl + 1u);
                PC_NEXT(g);
            }
            // ---- O: 32 columns of ctx_j . Wo
            for (int g = PC_FIRST(kO); g < g0 + kS; g += NB) {
                const int c = (g - g0 - kO) / MR, j = (g - g0 - kO) % MR;
                if (!pd_fetch<(PD_MAXD + PD_T - 1) / PD_T, 0>(ctx + (size_t)j * D, D, tl + 1u, sh.in, abortp)) return;
                pc_panel<PD_MAXQ, 1>(sh.in, D, wb, D, sh.red);
                __syncthreads();
                const float v = pc_cols<0>(sh.red[0]);
                if (tid < 64 && (tid & 1) == 0) pd_st(yo + (size_t)j * D + c * 32 + (tid >> 1), pd_word(v, tl + 2u));
                __syncthreads();
                PC_NEXT(g);
            }
            // every workgroup: x += O out, norm parts for the SwiGLU gain (an2)
            if (!pc_add_rows<MR>(sh, yo, D, tl + 2u, gn, abortp)) return;
            // ---- SW: silu(xn . W1) * (xn . W3), 16 columns, RS rows
            for (int g = PC_FIRST(kS); g < g0 + kW; g += NB) {
                const int c = (g - g0 - kS) / (MR / it.RS), j0 = ((g - g0 - kS) % (MR / it.RS)) * it.RS;
                pc_panel<PD_MAXQ, (MR >= 4 ? MR / 4 : 1)>(&sh.xn[j0][0], PD_MAXD, wb, D, sh.red);
                __syncthreads();
                for (int jj = tid >> 6; jj < it.RS; jj += PD_NW) {
                    const int j = j0 + jj;
                    float s = 0.f;
#pragma unroll
                    for (int w = 0; w < PD_NW; w++) s += sh.sw[j][w];
                    const float sn = rsqrtf(s / (float)D + 1e-5f);
                    const float r = pd_colsum_half(sh.red[jj], pd_half_col<1>(tid & 63)) * sn;
                    const float u = pd_pair_other(r);
                    float sg;
                    if (a.exact) sg = r / (1.0f + expf(-r));
                    else sg = r * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-r * 1.44269504088896f));
                    if (((tid & 63) & 3) == 0)
                        pd_st(act + (size_t)j * F + c * 16 + ((tid & 63) >> 2), pd_word(sg * u, tl + 3u));
                }
                __syncthreads();
                PC_NEXT(g);
            }
            // ---- W2: 32 columns of act_j . W2 (K = F)
            for (int g = PC_FIRST(kW); g < g0 + NPL; g += NB) {
                const int c = (g - g0 - kW) / MR, j = (g - g0 - kW) % MR;
                if (!pd_fetch<(PD_MAXF + PD_T - 1) / PD_T, 0>(act + (size_t)j * F, F, tl + 3u, sh.in, abortp)) return;
                pc_panel<PD_MAXFQ, 1>(sh.in, F, wb, F, sh.red);
                __syncthreads();
                const float v = pc_cols<0>(sh.red[0]);
                if (tid < 64 && (tid & 1) == 0) pd_st(y2 + (size_t)j * D + c * 32 + (tid >> 1), pd_word(v, tl + 4u));
                __syncthreads();
                PC_NEXT(g);
            }
            // every workgroup: x += W2 out, norm parts for the next gain (an1, or
            // the final norm's after the last layer)
            if (!pc_add_rows<MR>(sh, y2, D, tl + 4u, l + 1 < L ? gn : hg, abortp)) return;
#undef PC_FIRST
#undef PC_NEXT
        }

        // ---- head: 8 vocabulary rows per item against the MR final-normed rows
        if (b < NHI) {
            const u32 th = tag0 + 5u * (u32)L;
            u64 *cand = xb + lay.cand + (size_t)(t & 1) * MR * NHI * 2;
            for (int hj = b; hj < NHI; hj += NB) {
                f32x4 hw[2];
                pd_load_head(hw, P, hj, D);
                const int r = tid >> 6, c = tid & 63;
#pragma unroll 2
                for (int j = 0; j < MR; j++) {
                    float s = 0.f;
#pragma unroll
                    for (int w = 0; w < PD_NW; w++) s += sh.sw[j][w];
                    const float sn = rsqrtf(s / (float)D + 1e-5f);
                    float acc = 0.f;
#pragma unroll
                    for (int i = 0; i < 2; i++)
                        if (4 * (c + 64 * i) < D) {
                            const f32x4 f = *reinterpret_cast<const f32x4 *>(&sh.xn[j][4 * (c + 64 * i)]);
                            acc = fmaf(f.x, hw[i].x, acc);
                            acc = fmaf(f.y, hw[i].y, acc);
                            acc = fmaf(f.z, hw[i].z, acc);
                            acc = fmaf(f.w, hw[i].w, acc);
                        }
                    acc = pd_wave_sum(acc) * sn;
                    if (c == 0) {
                        sh.lg[j][r] = acc;
                        if (t == n - 1) gp(a.logits)[(size_t)j * V + 8 * hj + r] = acc;
                    }
                }
                __syncthreads();
                if (tid < MR) {
                    float bv = -INFINITY;
                    int bi = 0x7fffffff;
                    for (int rr = 0; rr < 8; rr++)
                        if (sh.lg[tid][rr] > bv) { bv = sh.lg[tid][rr]; bi = 8 * hj + rr; }
                    pd_st(cand + ((size_t)tid * NHI + hj) * 2, pd_word(bv, th));
                    pd_st(cand + ((size_t)tid * NHI + hj) * 2 + 1, ((u64)th << 32) | (u64)(u32)bi);
                }
                __syncthreads();
            }
        }
    }

    // ---- the last chunk's greedy tokens and the state for the next launch
    if (b == 0) {
        const u32 th = base + (u32)n * NPH;
        if (!pc_argmax<MR>(sh, xb + lay.cand + (size_t)((n - 1) & 1) * MR * NHI * 2, NHI, th, abortp)) return;
        if (tid < MR && a.toks_out) gp(a.toks_out)[(size_t)(n - 1) * MR + tid] = sh.tok[tid];
        if (tid == 0) {
            const int tk = sh.tok[MR - 1];
            GAS int *st = gp(a.state);
            st[0] = pos0 + n * MR;
            st[1] = 1;
            st[2] = tk;
            st[3] = (int)(base + (u32)n * NPH);
            gp(a.tok)[0] = tk;
        }
    }
}

// ============================================================== entries ==
extern "C" size_t tlg_dec_persist_xbytes(int V, int D, int L, int F)
{
    if (V <= 0 || D <= 0 || L <= 0 || F <= 0) return 0;
    // the single-token layout or the chunk layout at 8 rows (KD <= D), whichever is larger
    const size_t a = pd_layout(V, D, L, F).total, c = pc_layout(V, D, D, L, F, PC_MAXMR).total;
    return (a > c ? a : c) * sizeof(u64);
}

static int g_pd_cus = 0;

extern "C" int tlg_dev_dec_persist(const TlgDecPersist *a, int n, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (!a || n <= 0 || a->pool <= 0 || a->pool > 16 || a->copy0 < 0 || a->H <= 0 || a->KV <= 0 ||
        a->H % a->KV || a->D != 32 * a->H || a->D > PD_MAXD || a->F <= 0 || a->F % 32 || a->F > PD_MAXF ||
        a->V <= 0 || a->V % 8 || a->V / 8 > PD_MAXHI || a->L <= 0 || a->L > TLG_PD_MAXL || a->W <= 0 ||
        a->W > PD_MAXW || a->maxpos <= 0 || !a->cs || !a->sn || !a->logits || !a->state || !a->tok || !a->xbuf ||
        (a->qknorm != 0 && a->qknorm != 1))
        return tlg_fail(TLG_EINVAL,
                        "dec_persist: n=%d V=%d D=%d L=%d H=%d KV=%d F=%d W=%d pool=%d (head_dim 32, D <= %d, "
                        "F %% 32 == 0 and F <= %d, V %% 8 == 0 and V <= %d, W <= %d, L <= %d, qknorm 0 or 1)",
                        n, a ? a->V : 0, a ? a->D : 0, a ? a->L : 0, a ? a->H : 0, a ? a->KV : 0, a ? a->F : 0,
                        a ? a->W : 0, a ? a->pool : 0, PD_MAXD, PD_MAXF, 8 * PD_MAXHI, PD_MAXW, TLG_PD_MAXL);
    for (int c = 0; c < a->pool; c++)
        if (!a->P[c] || ((uintptr_t)a->P[c] & 15u)) return tlg_fail(TLG_EINVAL, "dec_persist: weight copy %d", c);
    for (int l = 0; l < a->L; l++)
        if (!a->Kc[l] || !a->Vc[l] || ((uintptr_t)a->Kc[l] & 63u) || ((uintptr_t)a->Vc[l] & 63u))
            return tlg_fail(TLG_EINVAL, "dec_persist: cache of layer %d", l);
    if ((uintptr_t)a->xbuf & 15u) return tlg_fail(TLG_EINVAL, "dec_persist: xbuf alignment");
    if (!g_pd_cus) {
        int cus = 0;
        TLG_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, g_tlg.device));
        g_pd_cus = cus;
    }
    const int nli = a->L * (a->H + 2 * (a->D / 32) + a->F / 16), nhi = a->V / 8;
    int nb = nli > nhi ? nli : nhi;
    if (nb > g_pd_cus) nb = g_pd_cus;
    const void *fn = a->f16 ? (const void *)k_dec_persist<1> : (const void *)k_dec_persist<0>;
    int per_cu = 0;
    TLG_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, PD_T, 0));
    if (per_cu < 1) return tlg_fail(TLG_EHIP, "dec_persist: the kernel does not fit on a CU");
    TlgDecPersist args = *a;
    int nn = n;
    void *kargs[] = {&args, &nn};
    TLG_HIP(hipLaunchCooperativeKernel(fn, dim3(nb), dim3(PD_T), kargs, 0, (hipStream_t)stream));
    return TLG_OK;
}

extern "C" int tlg_dev_dec_chunks(const TlgDecPersist *a, int m, const int *toks, int n, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (!a || n <= 0 || !toks || !(m == 1 || m == 2 || m == 4 || m == 8) || a->pool <= 0 || a->pool > 16 ||
        a->copy0 < 0 || a->H <= 0 || a->KV <= 0 || a->H % a->KV || a->D != 32 * a->H || a->D > PD_MAXD ||
        a->F <= 0 || a->F % 32 || a->F > PD_MAXF || a->V <= 0 || a->V % 8 || a->V / 8 > PD_MAXHI || a->L <= 0 ||
        a->L > TLG_PD_MAXL || a->W < m || a->W > PD_MAXW || a->maxpos <= 0 || !a->cs || !a->sn || !a->logits ||
        !a->state || !a->tok || !a->xbuf)
        return tlg_fail(TLG_EINVAL,
                        "dec_chunks: m=%d n=%d V=%d D=%d L=%d H=%d KV=%d F=%d W=%d (m in 1, 2, 4, 8; head_dim 32, "
                        "D <= %d, F %% 32 == 0 and F <= %d, V %% 8 == 0 and V <= %d, m <= W <= %d, L <= %d)",
                        m, n, a ? a->V : 0, a ? a->D : 0, a ? a->L : 0, a ? a->H : 0, a ? a->KV : 0, a ? a->F : 0,
                        a ? a->W : 0, PD_MAXD, PD_MAXF, 8 * PD_MAXHI, PD_MAXW, TLG_PD_MAXL);
    for (int c = 0; c < a->pool; c++)
        if (!a->P[c] || ((uintptr_t)a->P[c] & 15u)) return tlg_fail(TLG_EINVAL, "dec_chunks: weight copy %d", c);
    for (int l = 0; l < a->L; l++)
        if (!a->Kc[l] || !a->Vc[l] || ((uintptr_t)a->Kc[l] & 63u) || ((uintptr_t)a->Vc[l] & 63u))
            return tlg_fail(TLG_EINVAL, "dec_chunks: cache of layer %d", l);
    if ((uintptr_t)a->xbuf & 15u) return tlg_fail(TLG_EINVAL, "dec_chunks: xbuf alignment");
    if (a->qknorm) return tlg_fail(TLG_EINVAL, "dec_chunks: QK-norm models run on the graph step (tl_decode_chunk)");
    if (!g_pd_cus) {
        int cus = 0;
        TLG_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, g_tlg.device));
        g_pd_cus = cus;
    }
    const int rs = m >= 4 ? m / 4 : 1;
    const int npl = (a->H + (a->D + 2 * a->KV * 32) / 32 + 2 * (a->D / 32)) * m + (a->F / 16) * (m / rs);
    const int nli = a->L * npl, nhi = a->V / 8;
    int nb = nli > nhi ? nli : nhi;
    if (nb > g_pd_cus) nb = g_pd_cus;
    const void *fn = nullptr;
    switch (m) {
    case 1: fn = a->f16 ? (const void *)k_dec_chunk<1, 1> : (const void *)k_dec_chunk<0, 1>; break;
    case 2: fn = a->f16 ? (const void *)k_dec_chunk<1, 2> : (const void *)k_dec_chunk<0, 2>; break;
    case 4: fn = a->f16 ? (const void *)k_dec_chunk<1, 4> : (const void *)k_dec_chunk<0, 4>; break;
    default: fn = a->f16 ? (const void *)k_dec_chunk<1, 8> : (const void *)k_dec_chunk<0, 8>; break;
    }
    int per_cu = 0;
    TLG_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, PD_T, 0));
    if (per_cu < 1) return tlg_fail(TLG_EHIP, "dec_chunks: the kernel does not fit on a CU");
    TlgDecPersist args = *a;
    const int *tk = toks;
    int nn = n;
    void *kargs[] = {&args, &tk, &nn};
    TLG_HIP(hipLaunchCooperativeKernel(fn, dim3(nb), dim3(PD_T), kargs, 0, (hipStream_t)stream));
    return TLG_OK;
}

extern "C" int tlg_dec_persist_status(void *xbuf, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (!xbuf) return tlg_fail(TLG_EINVAL, "dec_persist_status: xbuf");
    u32 flag = 0;
    TLG_HIP(hipMemcpyAsync(&flag, xbuf, sizeof flag, hipMemcpyDeviceToHost, (hipStream_t)stream));
    TLG_HIP(hipStreamSynchronize((hipStream_t)stream));
    if (flag) return tlg_fail(TLG_EHIP, "dec_persist: a workgroup's wait for its inputs expired (launch aborted)");
    return TLG_OK;
}
