// tlg_decode.hip -- the non-GEMM work of tinylm.c's decode step on gfx950:
// the token embedding at the decode position, the KV ring-cache store, the
// attention of a few new rows over the ring window, and the greedy argmax
// that feeds the next step -- all driven by a small device-side state, so a
// whole token step can be captured once and replayed.
//
// Reference (tinylm.c): forward_chunk :3721-3830 (embedding :3727-3728,
// ring store :3775-3780, attention :3795-3815), kv_store :3236-3250 (f32 /
// f16 elements), attn_body :3639-3715 (unsplit path: scores, max, exp,
// normalise, weighted sum of V), fast_expf :3181-3191, argmax_v :3844.
//
// Data layout in HBM: the K and V caches of a layer are [W][KV*hd] rows of
// f32 or f16 (IEEE binary16, round to nearest even as the reference's F16C
// conversion); position p lives in slot p % W.
#include "tlg_internal.h"
#include "../../include/tldecode.h"
#include <math.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));

static inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// state[0] = first position of the next chunk, state[1] = rows of the next
// chunk, state[2] = last greedy token.
// x[j] = emb[tok[j]], pos[j] = state[0] + j (or start + j when state is null).
__global__ void k_dec_embed(const float *__restrict__ emb, const int *__restrict__ tok,
                            const int *__restrict__ state, int start, int m, int D, int V, float *__restrict__ x,
                            int *__restrict__ pos)
{
    const int p0 = state ? state[0] : start;
    const int d4 = D >> 2;
    for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < m * d4; q += gridDim.x * blockDim.x) {
        const int j = q / d4, c = q - j * d4;
        const int t = tok[j];
        reinterpret_cast<f32x4 *>(x)[q] = (t >= 0 && t < V) ? reinterpret_cast<const f32x4 *>(emb)[(size_t)t * d4 + c]
                                                            : f32x4{NAN, NAN, NAN, NAN};
        if (c == 0) pos[j] = p0 + j;
    }
}

// Ring store of the m new rows of K and V (after RoPE) into slot pos % W.
__global__ void k_kv_store(const float *__restrict__ k, const float *__restrict__ v, const int *__restrict__ pos,
                           int m, int KD, int W, int f16, void *__restrict__ Kc, void *__restrict__ Vc)
{
    for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < m * KD; q += gridDim.x * blockDim.x) {
        const int j = q / KD, i = q - j * KD;
        const size_t dst = (size_t)(pos[j] % W) * KD + i;
        if (f16) {
            reinterpret_cast<_Float16 *>(Kc)[dst] = (_Float16)k[q];
            reinterpret_cast<_Float16 *>(Vc)[dst] = (_Float16)v[q];
        } else {
            reinterpret_cast<float *>(Kc)[dst] = k[q];
            reinterpret_cast<float *>(Vc)[dst] = v[q];
        }
    }
}

#define DEC_MAXW 4096
#define DEC_HD 32
#define DEC_MAXM 8

// Cache element type of an f16 (1) or f32 (0) cache.
template <int F16> struct KvT { typedef float T; };
template <> struct KvT<1> { typedef _Float16 T; };
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// 8 elements of a K row from a generic pointer (cache row in HBM, or a new
// row in LDS): one 16-byte load for f16, two for f32.
template <int F16> struct KRaw;
template <> struct KRaw<1> {
    h8 v;
    __device__ __forceinline__ void load(const _Float16 *p) { v = *reinterpret_cast<const h8 *>(p); }
    __device__ __forceinline__ float operator[](int c) const { return (float)v[c]; }
};
template <> struct KRaw<0> {
    f32x4 a, b;
    __device__ __forceinline__ void load(const float *p)
    {
        a = *reinterpret_cast<const f32x4 *>(p);
        b = *reinterpret_cast<const f32x4 *>(p + 4);
    }
    __device__ __forceinline__ float operator[](int c) const { return c < 4 ? a[c] : b[c - 4]; }
};

// 4 elements of a V row (one 8- or 16-byte load), kept raw until used.
template <int F16> struct VRaw;
template <> struct VRaw<1> {
    h4 v;
    __device__ __forceinline__ void load(const _Float16 *p) { v = *reinterpret_cast<const h4 *>(p); }
    __device__ __forceinline__ float operator[](int c) const { return (float)v[c]; }
};
template <> struct VRaw<0> {
    f32x4 v;
    __device__ __forceinline__ void load(const float *p) { v = *reinterpret_cast<const f32x4 *>(p); }
    __device__ __forceinline__ float operator[](int c) const { return v[c]; }
};

// The decode attention of one (row j, KV head): a workgroup of 4 ATT_SPLIT
// waves; wave w = ATT_SPLIT hs + sp takes the heads g = hs, hs + 4, ... of the
// GQA group and the sp-th part of the visible positions lo .. lo + cnt - 1;
// the parts of a head meet through LDS (the softmax max, then its sum, then
// the weighted sums in part order), so the result is the unsplit
// attention of attn_body (normalise, then sum p_t V_t).  Every load that
// depends only on the positions -- the first head's query, the new rows and
// their RoPE angles, the query's angles, the first key / value batch of the
// wave's part -- is issued before anything waits.
//
// NEW = 1 (tlg_dev_dec_rope_attn): q and the m new K rows arrive before RoPE;
// the workgroup rotates the new K rows of its KV head and keeps them with
// their V rows in LDS, in the cache's format (f16-rounded for an f16 cache),
// and stores row j's into slot pos[j] % W.  A key whose slot this chunk
// writes ((slot - pos[0]) mod W < m: the reference stores every new row
// before any attention, :3775-3780) comes from those LDS rows, every other
// key from the cache, so no workgroup reads a slot another one writes.
// NEW = 0 (tlg_dev_dec_attn): q is rotated and every row is in the cache.
//   scores  lanes over keys; the 32-dim dot in eight fma lanes then pairwise
//           sums (kv_dot's F16C order), times hd^-1/2
//   softmax fast_expf (the reference default, :3181-3191) or expf
//   output  lane = (key stream s = lane / 8, dims 4 (lane % 8) .. + 3): each
//           stream walks keys s, s + 8, ... of the part, then the 8
//           streams are summed (shuffles, fixed order).
#define ATT_SPLIT 2                 // key splits per head
#define ATT_WAVES (4 * ATT_SPLIT)   // 4 heads of the GQA group at a time
template <int F16, int NEW>
__device__ __forceinline__ void attn_wg(const float *__restrict__ q, const float *__restrict__ kin,
                                        const float *__restrict__ vin, const int *__restrict__ pos,
                                        const float *__restrict__ cs, const float *__restrict__ sn, int maxpos,
                                        void *__restrict__ Kc, void *__restrict__ Vc, int m, int H, int KV, int W,
                                        int wlim, int exact, float *__restrict__ ctx, float *sp,
                                        typename KvT<F16>::T *kn, typename KvT<F16>::T *vn, float *wm, float *ws,
                                        f32x4 *wacc)
{
    typedef typename KvT<F16>::T E;
    constexpr int half = DEC_HD / 2, VU = (F16 ? 64 : 32) / ATT_SPLIT;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int hs = wave / ATT_SPLIT, spl = wave % ATT_SPLIT;
    const int j = blockIdx.x / KV, kvh = blockIdx.x % KV, grp = H / KV;
    const int D = H * DEC_HD, KD = KV * DEC_HD;
    const float scale = 1.0f / sqrtf((float)DEC_HD);
    // the new rows sit at consecutive positions p0 + jj (forward_chunk's)
    const int p0 = pos[0], p = NEW ? p0 + j : pos[j];
    const int lo = p >= wlim ? p - wlim + 1 : 0, cnt = p - lo + 1;
    const int s0 = lo % W, r0 = NEW ? ((p0 % W) + W) % W : 0, mm = NEW ? m : 0;
    const int chunk = (cnt + ATT_SPLIT - 1) / ATT_SPLIT, tb = spl * chunk, te = min(cnt, tb + chunk);
    const E *Kb = reinterpret_cast<const E *>(Kc) + (size_t)kvh * DEC_HD;
    const E *Vb = reinterpret_cast<const E *>(Vc) + (size_t)kvh * DEC_HD;
    const int sidx = lane >> 3, d0 = (lane & 7) * 4;
    const bool inpos = p >= 0 && p < maxpos;
    float *pr = sp + (size_t)hs * W;

    // ring slot of visible key t (0 <= t < cnt <= W) and its new-row index
    auto slot_of = [&](int t) { const int s = s0 + t; return s >= W ? s - W : s; };
    auto new_of = [&](int slot) { const int d = slot - r0; return d < 0 ? d + W : d; };
    auto krow = [&](int t) -> const E * {
        const int slot = slot_of(t), jn = new_of(slot);
        return jn < mm ? kn + jn * DEC_HD : Kb + (size_t)slot * KD;
    };
    auto vrow = [&](int t) -> const E * {
        const int slot = slot_of(t), jn = new_of(slot);
        return jn < mm ? vn + jn * DEC_HD : Vb + (size_t)slot * KD;
    };

    // ---- loads that depend only on the positions, all issued together
    float qv[DEC_HD];
    auto load_q = [&](int g) {
        const int gc = min(g, grp - 1);
        const f32x4 *q4 = reinterpret_cast<const f32x4 *>(q + (size_t)j * D + (size_t)(kvh * grp + gc) * DEC_HD);
#pragma unroll
        for (int c = 0; c < DEC_HD / 4; c++) {
            const f32x4 t = q4[c];
            qv[4 * c] = t.x; qv[4 * c + 1] = t.y; qv[4 * c + 2] = t.z; qv[4 * c + 3] = t.w;
        }
    };
    load_q(hs);
    const int e = threadIdx.x;                         // new-row element of this thread
    float ka = 0.f, kb = 0.f, kc = 0.f, ks = 0.f, vx = 0.f;
    float cq[half], sq[half];
    if (NEW) {
        if (e < m * half) {
            const int jj = e / half, i = e % half;
            const int t = min(max(p0 + jj, 0), maxpos - 1);
            const float *kr = kin + (size_t)jj * KD + (size_t)kvh * DEC_HD;
            ka = kr[i];
            kb = kr[i + half];
            kc = cs[(size_t)t * half + i];
            ks = sn[(size_t)t * half + i];
        }
        if (e < m * DEC_HD) vx = vin[(size_t)(e / DEC_HD) * KD + (size_t)kvh * DEC_HD + e % DEC_HD];
        const int pc = inpos ? p : 0;
#pragma unroll
        for (int i = 0; i < half; i++) {
            cq[i] = cs[(size_t)pc * half + i];
            sq[i] = sn[(size_t)pc * half + i];
        }
    }
    KRaw<F16> kk[DEC_HD / 8];
    VRaw<F16> vv[VU];
    {
        const E *row = Kb + (size_t)slot_of(min(tb + lane, cnt - 1)) * KD;
#pragma unroll
        for (int i = 0; i < DEC_HD / 8; i++) kk[i].load(row + 8 * i);
#pragma unroll
        for (int u = 0; u < VU; u++)
            vv[u].load(Vb + (size_t)slot_of(min(tb + 8 * u + sidx, cnt - 1)) * KD + d0);
    }
    if (NEW) {
        // the new rows of the KV head, rotated (rope_apply's pairs (i, i + hd/2))
        if (e < m * half) {
            const int jj = e / half, i = e % half, t = p0 + jj;
            float a_ = NAN, b_ = NAN;
            if (t >= 0 && t < maxpos) {
                a_ = ka * kc - kb * ks;
                b_ = kb * kc + ka * ks;
            }
            kn[jj * DEC_HD + i] = (E)a_;
            kn[jj * DEC_HD + i + half] = (E)b_;
        }
        if (e < m * DEC_HD) vn[e] = (E)vx;
    }
    __syncthreads();
    if (NEW) {
        if (threadIdx.x < DEC_HD) {                   // this row's ring slot
            const size_t dst = (size_t)(p % W) * KD + (size_t)kvh * DEC_HD + threadIdx.x;
            reinterpret_cast<E *>(Kc)[dst] = kn[j * DEC_HD + threadIdx.x];
            reinterpret_cast<E *>(Vc)[dst] = vn[j * DEC_HD + threadIdx.x];
        }
        // keys in slots this chunk writes: the new rows
        {
            const int jn = new_of(slot_of(min(tb + lane, cnt - 1)));
            if (jn < m)
#pragma unroll
                for (int i = 0; i < DEC_HD / 8; i++) kk[i].load(kn + jn * DEC_HD + 8 * i);
        }
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int jn = new_of(slot_of(min(tb + 8 * u + sidx, cnt - 1)));
            if (jn < m) vv[u].load(vn + jn * DEC_HD + d0);
        }
    }

    // every wave runs the same rounds (the barriers are workgroup-wide)
    for (int g = hs, round = 0; round < (grp + 3) / 4; g += 4, round++) {
        const bool live = g < grp;
        if (round > 0) load_q(g);
        if (NEW) {
#pragma unroll
            for (int i = 0; i < half; i++) {
                const float a = qv[i], b = qv[i + half];
                qv[i] = inpos ? a * cq[i] - b * sq[i] : NAN;
                qv[i + half] = inpos ? b * cq[i] + a * sq[i] : NAN;
            }
        }
        float mx = -1e30f;
        if (live) {
            for (int t0 = tb; t0 < te; t0 += 64) {
                if (t0 > tb || round > 0) {
                    const E *row = krow(min(t0 + lane, cnt - 1));
#pragma unroll
                    for (int i = 0; i < DEC_HD / 8; i++) kk[i].load(row + 8 * i);
                }
                float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < DEC_HD / 8; i++)
#pragma unroll
                    for (int c = 0; c < 8; c++) acc[c] = fmaf(qv[8 * i + c], kk[i][c], acc[c]);
                const float sc =
                    (((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]))) * scale;
                if (t0 + lane < te) {
                    pr[t0 + lane] = sc;
                    mx = fmaxf(mx, sc);
                }
            }
        }
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        if (lane == 0) wm[wave] = mx;
        __syncthreads();
        mx = wm[ATT_SPLIT * hs];
#pragma unroll
        for (int k = 1; k < ATT_SPLIT; k++) mx = fmaxf(mx, wm[ATT_SPLIT * hs + k]);
        float sum = 0.f;
        if (live)
            for (int t = tb + lane; t < te; t += 64) {
                const float ex = exact ? expf(pr[t] - mx) : tlg_fast_expf(pr[t] - mx);
                pr[t] = ex;
                sum += ex;
            }
        for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
        if (lane == 0) ws[wave] = sum;
        __syncthreads();
        float tot = ws[ATT_SPLIT * hs];
#pragma unroll
        for (int k = 1; k < ATT_SPLIT; k++) tot += ws[ATT_SPLIT * hs + k];
        const float inv = tot > 0.f ? 1.0f / tot : 0.f;
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
        if (live) {
            for (int t0 = tb; t0 < te; t0 += 8 * VU) {
                if (t0 > tb || round > 0) {
#pragma unroll
                    for (int u = 0; u < VU; u++) vv[u].load(vrow(min(t0 + 8 * u + sidx, cnt - 1)) + d0);
                }
#pragma unroll
                for (int u = 0; u < VU; u++) {
                    const int t = t0 + 8 * u + sidx;
                    const float pp = t < te ? pr[min(t, cnt - 1)] * inv : 0.f;
                    a.x = fmaf(pp, vv[u][0], a.x);
                    a.y = fmaf(pp, vv[u][1], a.y);
                    a.z = fmaf(pp, vv[u][2], a.z);
                    a.w = fmaf(pp, vv[u][3], a.w);
                }
            }
        }
#pragma unroll
        for (int o = 8; o < 64; o <<= 1) {
            a.x += __shfl_xor(a.x, o);
            a.y += __shfl_xor(a.y, o);
            a.z += __shfl_xor(a.z, o);
            a.w += __shfl_xor(a.w, o);
        }
        if (lane < 8) wacc[wave * 8 + lane] = a;
        __syncthreads();
        if (spl == 0 && lane < 8 && live) {
            f32x4 r = wacc[(ATT_SPLIT * hs) * 8 + lane];
#pragma unroll
            for (int k = 1; k < ATT_SPLIT; k++) r += wacc[(ATT_SPLIT * hs + k) * 8 + lane];
            *reinterpret_cast<f32x4 *>(ctx + (size_t)j * D + (size_t)(kvh * grp + g) * DEC_HD + d0) = r;
        }
    }
}

// One workgroup (4 ATT_SPLIT waves) per (row j, KV head).  Scores sit in dynamic LDS
// (4 * W floats, W <= DEC_MAXW).
template <int F16>
__global__ __launch_bounds__(64 * ATT_WAVES)
void k_dec_attn(const float *__restrict__ q, const void *__restrict__ Kc, const void *__restrict__ Vc,
                const int *__restrict__ pos, int H, int KV, int W, int wlim, int exact, float *__restrict__ ctx)
{
    extern __shared__ float sp[];
    typedef typename KvT<F16>::T E;
    // kn / vn are not read with NEW = 0 (no new rows); real addresses keep the inliner happy
    __shared__ __attribute__((aligned(16))) E none[8];
    __shared__ float wm[ATT_WAVES], ws[ATT_WAVES];
    __shared__ f32x4 wacc[ATT_WAVES * 8];
    attn_wg<F16, 0>(q, q, q, pos, q, q, 1, const_cast<void *>(Kc), const_cast<void *>(Vc), 0, H, KV, W, wlim, exact,
                    ctx, sp, none, none, wm, ws, wacc);
}

template <int F16>
__global__ __launch_bounds__(64 * ATT_WAVES)
void k_dec_rope_attn(const float *__restrict__ q, const float *__restrict__ kin, const float *__restrict__ vin,
                     const int *__restrict__ pos, const float *__restrict__ cs, const float *__restrict__ sn,
                     int maxpos, void *__restrict__ Kc, void *__restrict__ Vc, int m, int H, int KV, int W, int wlim,
                     int exact, float *__restrict__ ctx)
{
    extern __shared__ float sp[];
    typedef typename KvT<F16>::T E;
    __shared__ __attribute__((aligned(16))) E kn[DEC_MAXM * DEC_HD];
    __shared__ __attribute__((aligned(16))) E vn[DEC_MAXM * DEC_HD];
    __shared__ float wm[ATT_WAVES], ws[ATT_WAVES];
    __shared__ f32x4 wacc[ATT_WAVES * 8];
    attn_wg<F16, 1>(q, kin, vin, pos, cs, sn, maxpos, Kc, Vc, m, H, KV, W, wlim, exact, ctx, sp, kn, vn, wm, ws, wacc);
}

// Greedy next token of the last row (argmax_v: the first maximum), then
// advance the state by the chunk's rows; the token becomes the next chunk.
__global__ __launch_bounds__(1024) void k_dec_argmax(const float *__restrict__ logits, int V, int m,
                                                     int *__restrict__ state, int *__restrict__ tok)
{
    __shared__ float bv[1024];
    __shared__ int bi[1024];
    const float *row = logits + (size_t)(m - 1) * V;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    for (int i = threadIdx.x; i < V; i += 1024) {
        const float x = row[i];
        if (x > best) { best = x; bidx = i; }
    }
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = bidx;
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) {
            const float x = bv[threadIdx.x + o];
            const int xi = bi[threadIdx.x + o];
            if (x > bv[threadIdx.x] || (x == bv[threadIdx.x] && xi < bi[threadIdx.x])) {
                bv[threadIdx.x] = x;
                bi[threadIdx.x] = xi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int nx = bi[0] == 0x7fffffff ? 0 : bi[0];
        state[0] += m;
        state[1] = 1;
        state[2] = nx;
        tok[0] = nx;
    }
}

// qknorm_apply (tinylm.c:597-605) on the m new rows' q heads (H per row) and
// k heads (KV per row), hd = 32: half a wave per head, the sum of squares on
// the VALU (DPP row shifts, then row 0's (2's) lane 15 into row 1 (3)), then
// v * s * gain with s = 1 / sqrt(ss / hd + 1e-5).
template <int CTRL, int ROWMASK> __device__ __forceinline__ float dec_dpp(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROWMASK, 0xf, false));
}
__global__ __launch_bounds__(256) void k_dec_qknorm(float *__restrict__ q, float *__restrict__ k,
                                                    const float *__restrict__ qn, const float *__restrict__ kn,
                                                    int m, int H, int KV)
{
    const int head = blockIdx.x * 8 + (threadIdx.x >> 5), i = threadIdx.x & 31;
    const int nq = m * H, n = nq + m * KV;
    const bool live = head < n;
    const int hh = live ? head : n - 1;            // whole waves reach the DPP sum
    float *v;
    const float *g;
    if (hh < nq) { v = q + (size_t)(hh / H) * H * DEC_HD + (size_t)(hh % H) * DEC_HD; g = qn; }
    else {
        const int r = hh - nq;
        v = k + (size_t)(r / KV) * KV * DEC_HD + (size_t)(r % KV) * DEC_HD;
        g = kn;
    }
    const float x = v[i];
    float ss = x * x;
    ss += dec_dpp<0x111, 0xf>(ss);
    ss += dec_dpp<0x112, 0xf>(ss);
    ss += dec_dpp<0x114, 0xf>(ss);
    ss += dec_dpp<0x118, 0xf>(ss);
    ss += dec_dpp<0x142, 0xa>(ss);                   // lane 31 / 63: the half-wave's sum
    ss = __shfl(ss, (threadIdx.x & 32) | 31);
    const float sc = 1.0f / sqrtf(ss / (float)DEC_HD + 1e-5f);
    if (live) v[i] = x * sc * g[i];
}

// The decode MoE router's top-1 (moe_rt_body, tinylm.c:3332-3341): per row
// softmax of the E logits with expf and the first maximum of the normalised
// probabilities (strictly greater, ties to the lowest expert); gate = that
// probability.  One lane per row.
__global__ __launch_bounds__(64) void k_dec_moe_route(const float *__restrict__ rt, int m, int E,
                                                      int *__restrict__ assign, float *__restrict__ gate)
{
    const int j = threadIdx.x;
    if (j >= m) return;
    const float *r = rt + (size_t)j * E;
    float mx = -1e30f;
    for (int e = 0; e < E; e++) mx = r[e] > mx ? r[e] : mx;
    float s = 0.f;
    for (int e = 0; e < E; e++) s += expf(r[e] - mx);
    const float inv = 1.0f / s;
    int best = 0;
    float pb = expf(r[0] - mx) * inv;
    for (int e = 1; e < E; e++) {
        const float p = expf(r[e] - mx) * inv;
        if (p > pb) { pb = p; best = e; }
    }
    assign[j] = best;
    gate[j] = pb;
}

// mtp_argmax's middle (tinylm.c:3933): hh = fn + silu(ht) with fn the final
// RMSNorm of x (rmsnorm_fwd :540-548, gain nf) and silu(z) = z / (1 + e^-z).
__global__ __launch_bounds__(256) void k_dec_mtp_mix(float *__restrict__ hh, const float *__restrict__ x,
                                                     const float *__restrict__ nf, const float *__restrict__ ht,
                                                     int D)
{
    __shared__ float red[4];
    float ss = 0.f;
    for (int i = threadIdx.x; i < D; i += 256) ss = fmaf(x[i], x[i], ss);
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float t = (red[0] + red[1]) + (red[2] + red[3]);
    const float sc = 1.0f / sqrtf(t / (float)D + 1e-5f);
    for (int i = threadIdx.x; i < D; i += 256) {
        const float z = ht[i];
        hh[i] = x[i] * sc * nf[i] + z / (1.0f + expf(-z));
    }
}

// argmax_v (tinylm.c:3844: the first maximum) of each of m rows of [m][V].
__global__ __launch_bounds__(1024) void k_argmax_rows(const float *__restrict__ logits, int V, int *__restrict__ out)
{
    __shared__ float bv[1024];
    __shared__ int bi[1024];
    const float *row = logits + (size_t)blockIdx.x * V;
    float best = -INFINITY;
    int bidx = 0x7fffffff;
    for (int i = threadIdx.x; i < V; i += 1024) {
        const float x = row[i];
        if (x > best) { best = x; bidx = i; }
    }
    bv[threadIdx.x] = best;
    bi[threadIdx.x] = bidx;
    __syncthreads();
    for (int o = 512; o > 0; o >>= 1) {
        if ((int)threadIdx.x < o) {
            const float x = bv[threadIdx.x + o];
            const int xi = bi[threadIdx.x + o];
            if (x > bv[threadIdx.x] || (x == bv[threadIdx.x] && xi < bi[threadIdx.x])) {
                bv[threadIdx.x] = x;
                bi[threadIdx.x] = xi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = bi[0] == 0x7fffffff ? 0 : bi[0];
}

// ============================================================== entries ==
extern "C" int tlg_dev_dec_qknorm(float *q, float *k, const float *qn, const float *kn, int m, int H, int KV, int hd,
                                  void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (!q || !k || !qn || !kn || m <= 0 || H <= 0 || KV <= 0 || hd != DEC_HD)
        return tlg_fail(TLG_EINVAL, "dec_qknorm: m=%d H=%d KV=%d hd=%d (hd must be %d)", m, H, KV, hd, DEC_HD);
    const int n = m * (H + KV);
    hipLaunchKernelGGL(k_dec_qknorm, dim3((n + 7) / 8), dim3(256), 0, (hipStream_t)stream, q, k, qn, kn, m, H, KV);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

extern "C" int tlg_dev_dec_moe_route(const float *rt, int m, int E, int *assign, float *gate, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (!rt || !assign || !gate || m <= 0 || m > 64 || E < 1 || E > 64)
        return tlg_fail(TLG_EINVAL, "dec_moe_route: m=%d E=%d", m, E);
    hipLaunchKernelGGL(k_dec_moe_route, dim3(1), dim3(64), 0, (hipStream_t)stream, rt, m, E, assign, gate);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

extern "C" int tlg_dev_dec_mtp_mix(float *hh, const float *x, const float *nf, const float *ht, int D, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (!hh || !x || !nf || !ht || D <= 0) return tlg_fail(TLG_EINVAL, "dec_mtp_mix: D=%d", D);
    hipLaunchKernelGGL(k_dec_mtp_mix, dim3(1), dim3(256), 0, (hipStream_t)stream, hh, x, nf, ht, D);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

extern "C" int tlg_dev_argmax_rows(const float *logits, int V, int m, int *out, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (!logits || !out || V <= 0 || m <= 0) return tlg_fail(TLG_EINVAL, "argmax_rows: V=%d m=%d", V, m);
    hipLaunchKernelGGL(k_argmax_rows, dim3(m), dim3(1024), 0, (hipStream_t)stream, logits, V, out);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

// dst[c][r] = src[r][c] through a 32 x 33 LDS tile (conflict-free both ways):
// 32 x 8 threads, each moving 4 elements in and 4 out.
__global__ __launch_bounds__(256) void k_transpose(float *__restrict__ dst, const float *__restrict__ src, int rows,
                                                   int cols)
{
    __shared__ float t[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32, tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = r0 + ty + 8 * i, c = c0 + tx;
        if (r < rows && c < cols) t[ty + 8 * i][tx] = src[(size_t)r * cols + c];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = c0 + ty + 8 * i, r = r0 + tx;
        if (r < rows && c < cols) dst[(size_t)c * rows + r] = t[tx][ty + 8 * i];
    }
}

extern "C" int tlg_dev_transpose(float *dst, const float *src, int rows, int cols, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (!dst || !src || rows <= 0 || cols <= 0 || (cols + 31) / 32 > 0x7fffffff || (rows + 31) / 32 > 65535)
        return tlg_fail(TLG_EINVAL, "transpose: rows=%d cols=%d", rows, cols);
    const char *d0 = (const char *)dst, *s0 = (const char *)src;
    const size_t bytes = (size_t)rows * cols * sizeof(float);
    if (d0 < s0 + bytes && s0 < d0 + bytes) return tlg_fail(TLG_EINVAL, "transpose: dst and src overlap");
    hipLaunchKernelGGL(k_transpose, dim3((cols + 31) / 32, (rows + 31) / 32), dim3(256), 0, (hipStream_t)stream, dst,
                       src, rows, cols);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

extern "C" int tlg_dev_dec_embed(float *x, int *pos, const float *emb, const int *tok, const int *state, int start,
                                 int m, int D, int V, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (m <= 0 || D <= 0 || D % 4 || V <= 0 || !al16(x) || !al16(emb))
        return tlg_fail(TLG_EINVAL, "dec_embed: m=%d D=%d V=%d", m, D, V);
    const int work = m * (D / 4);
    hipLaunchKernelGGL(k_dec_embed, dim3((work + 255) / 256), dim3(256), 0, (hipStream_t)stream, emb, tok, state,
                       start, m, D, V, x, pos);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

extern "C" int tlg_dev_kv_store(const float *k, const float *v, const int *pos, int m, int KD, int W, int f16,
                                void *Kc, void *Vc, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (m <= 0 || KD <= 0 || W <= 0 || m > W) return tlg_fail(TLG_EINVAL, "kv_store: m=%d KD=%d W=%d", m, KD, W);
    hipLaunchKernelGGL(k_kv_store, dim3((m * KD + 255) / 256), dim3(256), 0, (hipStream_t)stream, k, v, pos, m, KD,
                       W, f16 ? 1 : 0, Kc, Vc);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

extern "C" int tlg_dev_dec_attn(const float *q, const void *Kc, const void *Vc, const int *pos, float *ctx, int m,
                                int H, int KV, int hd, int W, int win, int f16, int exact_exp, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (m <= 0 || H <= 0 || KV <= 0 || H % KV || hd != DEC_HD || W <= 0 || W > DEC_MAXW || !al16(q) || !al16(ctx) ||
        !al16(Kc) || !al16(Vc))
        return tlg_fail(TLG_EINVAL, "dec_attn: m=%d H=%d KV=%d hd=%d W=%d (head_dim 32, W <= %d)", m, H, KV, hd, W,
                        DEC_MAXW);
    const int wlim = (win > 0 && win < W) ? win : W;
    if (f16)
        hipLaunchKernelGGL(k_dec_attn<1>, dim3(m * KV), dim3(64 * ATT_WAVES), 16 * W, (hipStream_t)stream, q, Kc, Vc, pos, H, KV, W,
                           wlim, exact_exp ? 1 : 0, ctx);
    else
        hipLaunchKernelGGL(k_dec_attn<0>, dim3(m * KV), dim3(64 * ATT_WAVES), 16 * W, (hipStream_t)stream, q, Kc, Vc, pos, H, KV, W,
                           wlim, exact_exp ? 1 : 0, ctx);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

extern "C" int tlg_dev_dec_argmax(const float *logits, int V, int m, int *state, int *tok, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (V <= 0 || m <= 0) return tlg_fail(TLG_EINVAL, "dec_argmax: V=%d m=%d", V, m);
    hipLaunchKernelGGL(k_dec_argmax, dim3(1), dim3(1024), 0, (hipStream_t)stream, logits, V, m, state, tok);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

extern "C" int tlg_dev_dec_rope_attn(const float *q, const float *k, const float *v, const int *pos, const float *cs,
                                     const float *sn, int maxpos, void *Kc, void *Vc, float *ctx, int m, int H, int KV,
                                     int hd, int W, int win, int f16, int exact_exp, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (m <= 0 || m > DEC_MAXM || m > W || H <= 0 || KV <= 0 || H % KV || hd != DEC_HD || W <= 0 ||
        W > DEC_MAXW || maxpos <= 0 || !al16(q) || !al16(Kc) || !al16(Vc) || !al16(ctx) || !q || !k || !v || !pos ||
        !cs || !sn || !ctx)
        return tlg_fail(TLG_EINVAL, "dec_rope_attn: m=%d H=%d KV=%d hd=%d W=%d (m <= %d, head_dim 32, W <= %d)", m,
                        H, KV, hd, W, DEC_MAXM, DEC_MAXW);
    const int wlim = (win > 0 && win < W) ? win : W;
    if (f16)
        hipLaunchKernelGGL(k_dec_rope_attn<1>, dim3(m * KV), dim3(64 * ATT_WAVES), 16 * W, (hipStream_t)stream, q, k, v, pos,
                           cs, sn, maxpos, Kc, Vc, m, H, KV, W, wlim, exact_exp ? 1 : 0, ctx);
    else
        hipLaunchKernelGGL(k_dec_rope_attn<0>, dim3(m * KV), dim3(64 * ATT_WAVES), 16 * W, (hipStream_t)stream, q, k, v, pos,
                           cs, sn, maxpos, Kc, Vc, m, H, KV, W, wlim, exact_exp ? 1 : 0, ctx);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}
