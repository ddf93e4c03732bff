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

// The reference's fast_expf: clamp, split x log2(e) into integer and
// fraction, 2^f by its degree-5 Horner polynomial, 2^k into the exponent.
__device__ __forceinline__ float dec_fast_expf(float x)
{
    x = x < -87.0f ? -87.0f : (x > 88.0f ? 88.0f : x);
    const float t = x * 1.44269504088896f;
    const float k = floorf(t), f = t - k;
    const float p = 1.0f + f * (0.6931471805f + f * (0.2402265069f + f * (0.0555041087f +
                                                                        f * (0.0096181291f + f * 0.0013333558f))));
    return p * __uint_as_float((unsigned int)(((int)k + 127) << 23));
}

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

template <int F16>
__device__ __forceinline__ float kv_elem(const void *base, size_t i)
{
    if (F16) return (float)reinterpret_cast<const _Float16 *>(base)[i];
    return reinterpret_cast<const float *>(base)[i];
}

// One workgroup per (row j, KV head); wave w takes the heads kvh * grp + w,
// + 4, ...  For its head a wave scores every visible key (lanes over keys,
// the 32-dim dot in eight fma lanes then pairwise sums as kv_dot's F16C path
// does), takes the max and the exponentials (fast_expf or expf) and their
// sum, normalises, and accumulates sum_t p_t V[t] (lanes over dims, two key
// halves combined at the end).  Scores sit in dynamic LDS (4 * W floats,
// W <= DEC_MAXW).
#define DEC_MAXW 4096
#define DEC_HD 32
template <int F16>
__global__ __launch_bounds__(256) void k_dec_attn(const float *__restrict__ q, const void *__restrict__ Kc,
                                                  const void *__restrict__ Vc, const int *__restrict__ pos, int H,
                                                  int KV, int W, int wlim, int exact, float *__restrict__ ctx)
{
    extern __shared__ float sp[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = blockIdx.x / KV, kvh = blockIdx.x % KV, grp = H / KV;
    const int D = H * DEC_HD, KD = KV * DEC_HD;
    const float scale = 1.0f / sqrtf((float)DEC_HD);
    const int p = pos[j], lo = p >= wlim ? p - wlim + 1 : 0, cnt = p - lo + 1;
    float *pr = sp + (size_t)wave * W;
    for (int g = wave; g < grp; g += 4) {
        const int h = kvh * grp + g;
        const f32x4 *q4 = reinterpret_cast<const f32x4 *>(q + (size_t)j * D + (size_t)h * DEC_HD);
        float qv[DEC_HD];
#pragma unroll
        for (int c = 0; c < DEC_HD / 4; c++) {
            const f32x4 t = q4[c];
            qv[4 * c] = t.x; qv[4 * c + 1] = t.y; qv[4 * c + 2] = t.z; qv[4 * c + 3] = t.w;
        }
        float mx = -1e30f;
        for (int t = lane; t < cnt; t += 64) {
            const size_t row = (size_t)((lo + t) % W) * KD + (size_t)kvh * DEC_HD;
            float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < DEC_HD; i += 8)
#pragma unroll
                for (int c = 0; c < 8; c++) acc[c] = fmaf(qv[i + c], kv_elem<F16>(Kc, row + i + c), acc[c]);
            const float s = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
            pr[t] = s * scale;
            mx = fmaxf(mx, pr[t]);
        }
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        float sum = 0.f;
        for (int t = lane; t < cnt; t += 64) {
            const float e = exact ? expf(pr[t] - mx) : dec_fast_expf(pr[t] - mx);
            pr[t] = e;
            sum += e;
        }
        for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
        const float inv = sum > 0.f ? 1.0f / sum : 0.f;
        for (int t = lane; t < cnt; t += 64) pr[t] *= inv;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // lanes 0-31: even keys, 32-63: odd keys; dim d = lane % 32
        const int d = lane & 31;
        float a = 0.f;
        for (int t = lane >> 5; t < cnt; t += 2)
            a = fmaf(pr[t], kv_elem<F16>(Vc, (size_t)((lo + t) % W) * KD + (size_t)kvh * DEC_HD + d), a);
        a += __shfl_xor(a, 32);
        if (lane < 32) ctx[(size_t)j * D + (size_t)h * DEC_HD + d] = a;
        __builtin_amdgcn_wave_barrier();
    }
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

// ============================================================== entries ==
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
    if (m <= 0 || H <= 0 || KV <= 0 || H % KV || hd != DEC_HD || W <= 0 || W > DEC_MAXW || !al16(q))
        return tlg_fail(TLG_EINVAL, "dec_attn: m=%d H=%d KV=%d hd=%d W=%d (head_dim 32, W <= %d)", m, H, KV, hd, W,
                        DEC_MAXW);
    const int wlim = (win > 0 && win < W) ? win : W;
    if (f16)
        hipLaunchKernelGGL(k_dec_attn<1>, dim3(m * KV), dim3(256), 16 * W, (hipStream_t)stream, q, Kc, Vc, pos, H, KV, W,
                           wlim, exact_exp ? 1 : 0, ctx);
    else
        hipLaunchKernelGGL(k_dec_attn<0>, dim3(m * KV), dim3(256), 16 * W, (hipStream_t)stream, q, Kc, Vc, pos, H, KV, W,
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
