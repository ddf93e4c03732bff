// tlg_moe.hip -- the top-1 mixture-of-experts FFN of tinylm.c on gfx950:
// routing, the per-expert row index, and the expert GEMMs as expert-batched
// grouped launches over rows grouped by expert.
//
// Reference: moe_forward tinylm.c:857-891, moe_backward :895-947, moe_route
// :814-827 (K = 1, no router bias), MOE_AUX :849.
//
// Data layout in HBM.  Token-order buffers are the caller's (fnorm, fin, out,
// dout, d_fnorm: N x D; rprobs N x E; assign, gate: N).  The library keeps
// one scratch arena with the expert-grouped ("sorted") rows: row i of g, u,
// a, y, dy holds token idx[i]; expert e owns sorted rows [eoff[e],
// eoff[e+1]) in ascending token order, the order in which the reference
// gathers them (:876).  pos[n] is token n's sorted row.  The gathered
// input rows Xg = fnorm[idx] are never stored: the expert GEMMs read fnorm
// through idx.
//
// Kernels (one pass each over the data they touch):
//   k_moe_route     router logits as the reference's own FMA chain over D
//                   (so the argmax sees the reference's logits bit for bit),
//                   softmax, strict-greater argmax (ties -> lowest expert)
//   k_moe_index_blk stable counting sort of the tokens by expert: the
//                   router workgroups leave per-block expert counts and
//                   in-block ranks, every index workgroup sums the counts
//                   of the blocks before its own (no atomics)
//   k_moe_index     the same sort in one workgroup, from the assignments
//                   alone (the recomputing backward)
//   expert GEMMs    tlg_expert_launch (grouped MFMA tiles, every expert in
//                   one launch; the rows per expert stay on the device),
//                   with the MoE's elementwise steps fused in:
//                     W1 | W3   one paired-column launch, rows gathered from
//                               fnorm, a = silu(g) u in the epilogue
//                     W2 (fwd)  out[n] = fin[n] + gate[n] y in the epilogue
//                     da        the SwiGLU backward in the epilogue
//                     dW1, dW3  fnorm rows gathered along the reduction
//   k_moe_dgate     d_gate[n] = dout[n] . y[pos[n]],  dy = gate dout
//   k_moe_router_bwd  softmax backward with the load-balance term, then
//                   d_fnorm = dX[pos] + d_rt wr^T   (the router mm_bt, :944)
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
// With bcnt, the workgroup also leaves its expert counts in bcnt[blockIdx.x]
// [E] and each token's rank among its block's tokens of the same expert in
// rank[n] (k_moe_index_blk's inputs).
__global__ __launch_bounds__(256) void k_moe_route(const float *__restrict__ X, const float *__restrict__ Wr,
                                                   int N, int D, int E, int dch, float *__restrict__ rprobs,
                                                   int *__restrict__ assign, float *__restrict__ gate,
                                                   int *__restrict__ rank, int *__restrict__ bcnt)
{
    __shared__ int sel_s[MOE_TOK];
    extern __shared__ float lds_route[];
    float *xs = lds_route;                          // [MOE_TOK][dch + 1]
    float *wsm = xs + MOE_TOK * (dch + 1);          // [dch][E]
    float *lg = wsm + dch * E;                      // [MOE_TOK][E]
    const int n0 = blockIdx.x * MOE_TOK, tid = threadIdx.x;
    for (int p = tid; p < MOE_TOK * E; p += 256) lg[p] = 0.f;
    for (int d0 = 0; d0 < D; d0 += dch) {
        const int dn = min(dch, D - d0);        // a multiple of 4 (D and dch are)
        __syncthreads();
        // staging: RB loads per thread in flight before any is stored
        constexpr int RB = 4;
        const int nq = MOE_TOK * (dn / 4);
        for (int q0 = tid; q0 < nq; q0 += 256 * RB) {
            float4 v[RB];
#pragma unroll
            for (int k = 0; k < RB; k++) {
                const int q = q0 + k * 256, t = q / (dn / 4), c = q - t * (dn / 4);
                v[k] = (q < nq && n0 + t < N)
                           ? *reinterpret_cast<const float4 *>(X + (size_t)(n0 + t) * D + d0 + 4 * c)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int k = 0; k < RB; k++) {
                const int q = q0 + k * 256, t = q / (dn / 4), c = q - t * (dn / 4);
                if (q < nq) {
                    float *x = xs + t * (dch + 1) + 4 * c;
                    x[0] = v[k].x; x[1] = v[k].y; x[2] = v[k].z; x[3] = v[k].w;
                }
            }
        }
        const int nw = dn * E;
        for (int p0 = tid; p0 < nw; p0 += 256 * RB) {
            float v[RB];
#pragma unroll
            for (int k = 0; k < RB; k++) {
                const int p = p0 + k * 256;
                v[k] = p < nw ? Wr[(size_t)d0 * E + p] : 0.f;
            }
#pragma unroll
            for (int k = 0; k < RB; k++)
                if (p0 + k * 256 < nw) wsm[p0 + k * 256] = v[k];
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
    if (t < MOE_TOK) {
        int sel = -1;
        if (n < N) {
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
            sel = best < 0 ? 0 : best;
            assign[n] = sel;
            gate[n] = pr[sel];
        }
        sel_s[t] = sel;
    }
    if (!bcnt) return;
    __syncthreads();
    if (t < MOE_TOK && n < N) {
        const int a = sel_s[t];
        int r = 0;
        for (int j = 0; j < t; j++) r += sel_s[j] == a;
        rank[n] = r;
    }
    for (int e = t; e < E; e += 256) {
        int c = 0;
        for (int j = 0; j < MOE_TOK; j++) c += sel_s[j] == e;
        bcnt[(size_t)blockIdx.x * E + e] = c;
    }
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
// Token n = (8 r + k) 1024 + 64 w + lane sits in round r, chunk k, wave w.
// A round's assignments load at once (8 per thread); a wave ranks each
// lane among the lanes of its chunk routed to the same expert with one
// ballot per expert and keeps the per-(chunk, wave) counts in LDS; wave e
// then scans expert e's counts in token order (two slots per lane and a
// shuffle scan), carrying the running count across rounds.  So tokens keep
// ascending order inside each expert, with no atomics.  A token whose
// expert is out of range is left out (pos = -1) and, when `out` is given,
// gets out[n] = fin[n] (moe_forward's residual alone, :870).
#define MOE_IDX_CH 8
__global__ __launch_bounds__(1024) void k_moe_index(const int *__restrict__ assign, int N, int E,
                                                    int *__restrict__ idx, int *__restrict__ pos,
                                                    int *__restrict__ eoff, const float *__restrict__ fin,
                                                    float *__restrict__ out, int D)
{
    __shared__ int wc[MOE_IDX_CH * 16][TLG_MOE_MAXE];    // (chunk, wave) slot x expert
    __shared__ int run[TLG_MOE_MAXE];
    __shared__ int off[TLG_MOE_MAXE + 1];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int per_round = MOE_IDX_CH * 1024;
    const int rounds = (N + per_round - 1) / per_round;
    if (tid < TLG_MOE_MAXE) run[tid] = 0;
    int av[MOE_IDX_CH], rel[MOE_IDX_CH];
    for (int rd = 0; rd < rounds; rd++) {
        const int n0 = rd * per_round + tid;
#pragma unroll
        for (int k = 0; k < MOE_IDX_CH; k++) {
            const int n = n0 + k * 1024;
            av[k] = n < N ? assign[n] : -1;
        }
#pragma unroll
        for (int k = 0; k < MOE_IDX_CH; k++) {
            rel[k] = 0;
            for (int e = 0; e < E; e++) {
                const unsigned long long m = __ballot(av[k] == e);
                if (av[k] == e) rel[k] = __popcll(m & ((1ull << lane) - 1ull));
                if (lane == 0) wc[k * 16 + w][e] = __popcll(m);
            }
        }
        __syncthreads();
        // exclusive scan of expert e's 128 slot counts, plus the carry
        for (int e = w; e < E; e += 16) {
            const int c0 = wc[2 * lane][e], c1 = wc[2 * lane + 1][e];
            int inc = c0 + c1;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int t = __shfl_up(inc, o);
                if (lane >= o) inc += t;
            }
            const int ex = inc - (c0 + c1) + run[e];
            wc[2 * lane][e] = ex;
            wc[2 * lane + 1][e] = ex + c0;
            const int tot = __shfl(inc, 63);
            if (lane == 63) run[e] += tot;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < MOE_IDX_CH; k++) {
            const int a = av[k];
            rel[k] = (a >= 0 && a < E) ? rel[k] + wc[k * 16 + w][a] : -1;
            const int n = n0 + k * 1024;
            // several rounds: park the in-expert rank until the offsets exist
            if (rounds > 1 && n < N) pos[n] = rel[k];
        }
        __syncthreads();
    }
    if (w == 0) {
        // exclusive scan of the expert totals (E <= 64: one per lane)
        const int c = lane < E ? run[lane] : 0;
        int inc = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(inc, o);
            if (lane >= o) inc += t;
        }
        if (lane < E) off[lane] = inc - c;
        if (lane == 63) off[E] = inc;
    }
    __syncthreads();
    if (tid <= E) eoff[tid] = off[tid];
    for (int j = 0; j * 1024 < N; j++) {
        const int n = j * 1024 + tid;
        if (n >= N) break;
        int a, r;
        if (rounds == 1) {
            a = av[0]; r = rel[0];
#pragma unroll
            for (int k = 1; k < MOE_IDX_CH; k++)
                if (j == k) { a = av[k]; r = rel[k]; }
        } else {
            a = assign[n];
            r = pos[n];
        }
        const bool ok = a >= 0 && a < E;
        const int p = ok ? off[a] + r : -1;
        pos[n] = p;
        if (ok) idx[p] = n;
        else if (out)
            for (int d = 0; d < D; d += 4)
                *reinterpret_cast<float4 *>(out + (size_t)n * D + d) =
                    *reinterpret_cast<const float4 *>(fin + (size_t)n * D + d);
    }
}

// The same sort from the router's per-block counts (bcnt [nblk][E], blocks of
// MOE_TOK tokens) and in-block ranks (rank[n]): workgroup j places tokens
// 256 j .. 256 j + 255 (router blocks b0 = 16 j .. b0 + 15).  Wave w sums
// experts w, w + 4, ..: over the blocks before b0 (pre) and over all blocks
// (tot), lanes striding the blocks, then a shuffle reduction (integer sums:
// exact in any order).  Token n of in-workgroup block bb goes to
//   eoff[a] + pre[a] + sum_{bb' < bb} bcnt[b0 + bb'][a] + rank[n],
// which keeps ascending token order inside each expert, as k_moe_index does
// (same idx, pos and eoff).  Every workgroup finds eoff; workgroup 0 writes it.
#define MOE_IDX_TPB 256
static_assert(MOE_IDX_TPB % MOE_TOK == 0, "whole router blocks per index workgroup");
__global__ __launch_bounds__(MOE_IDX_TPB) void k_moe_index_blk(const int *__restrict__ assign,
                                                             const int *__restrict__ bcnt, int N, int E,
                                                             int *__restrict__ idx, int *__restrict__ pos,
                                                             int *__restrict__ eoff, const float *__restrict__ fin,
                                                             float *__restrict__ out, int D)
{
    constexpr int BPW = MOE_IDX_TPB / MOE_TOK;          // router blocks per workgroup
    __shared__ int pre[TLG_MOE_MAXE], tot[TLG_MOE_MAXE], off[TLG_MOE_MAXE + 1];
    __shared__ int loc[BPW][TLG_MOE_MAXE];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nblk = (N + MOE_TOK - 1) / MOE_TOK, b0 = blockIdx.x * BPW;
    for (int e = w; e < E; e += MOE_IDX_TPB / 64) {
        int sp = 0, st = 0;
        for (int b = lane; b < nblk; b += 64) {
            const int c = bcnt[(size_t)b * E + e];
            st += c;
            if (b < b0) sp += c;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            sp += __shfl_xor(sp, o);
            st += __shfl_xor(st, o);
        }
        if (lane == 0) { pre[e] = sp; tot[e] = st; }
    }
    for (int p = tid; p < BPW * E; p += MOE_IDX_TPB) {
        const int bb = p / E, e = p % E;
        loc[bb][e] = b0 + bb < nblk ? bcnt[(size_t)(b0 + bb) * E + e] : 0;
    }
    __syncthreads();
    if (w == 0) {
        // exclusive scan of the expert totals (E <= 64: one per lane)
        const int c = lane < E ? tot[lane] : 0;
        int inc = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(inc, o);
            if (lane >= o) inc += t;
        }
        if (lane < E) off[lane] = inc - c;
        if (lane == 63) off[E] = inc;
    }
    __syncthreads();
    if (blockIdx.x == 0 && tid <= E) eoff[tid] = off[tid];
    const int n = blockIdx.x * MOE_IDX_TPB + tid;
    if (n >= N) return;
    const int a = assign[n], bb = tid / MOE_TOK;
    if (a < 0 || a >= E) {          // not produced by k_moe_route; left out as k_moe_index does
        pos[n] = -1;
        if (out)
            for (int d = 0; d < D; d += 4)
                *reinterpret_cast<float4 *>(out + (size_t)n * D + d) =
                    *reinterpret_cast<const float4 *>(fin + (size_t)n * D + d);
        return;
    }
    int p = off[a] + pre[a] + pos[n];
    for (int j = 0; j < bb; j++) p += loc[j][a];
    pos[n] = p;
    idx[p] = n;
}

// ------------------------------------------------------------ backward --
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

// Router backward and d_fnorm (:928-944), MOE_TOK tokens per workgroup.
// First, per token (:933-943): dp_e = 0.01 E (cnt_e / N) / N, plus d_gate on
// the chosen expert; d_rt = p (dp - p.dp) -- kept in LDS and written out.
// Then d_fnorm[n][d] = dX[pos[n]][d] + sum_e d_rt[n][e] wr[d][e]: the expert
// scatter (:928-930) after the memset (:900), then the router mm_bt (:944).
// With wpart, the workgroup's share of dWr = fnorm^T d_rt (:945) goes to
// wpart[blockIdx.x][d * E + e] (its tokens in order), for a column sum.
__global__ __launch_bounds__(256) void k_moe_router_bwd(const float *__restrict__ rprobs, const int *__restrict__ pos,
                                                        const int *__restrict__ assign, const float *__restrict__ dgate,
                                                        const int *__restrict__ eoff, const float *__restrict__ dX,
                                                        const float *__restrict__ wr, int N, int D, int E,
                                                        float *__restrict__ drt, float *__restrict__ dfn,
                                                        const float *__restrict__ fnorm, float *__restrict__ wpart)
{
    __shared__ float sd[MOE_TOK][TLG_MOE_MAXE];
    __shared__ int sp[MOE_TOK];
    const int n0 = blockIdx.x * MOE_TOK, tid = threadIdx.x;
    if (tid < MOE_TOK) sp[tid] = n0 + tid < N ? pos[n0 + tid] : -1;
    if (tid < MOE_TOK && n0 + tid < N) {
        const int n = n0 + tid;
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
            const float v = pr[e] * (dp - dot);
            sd[tid][e] = v;
            dr[e] = v;
        }
    }
    __syncthreads();
    // one column d per thread, the block's token rows loaded together
    for (int d = tid; d < D; d += 256) {
        float x[MOE_TOK], f[MOE_TOK];
#pragma unroll
        for (int t = 0; t < MOE_TOK; t++) {
            x[t] = sp[t] >= 0 ? dX[(size_t)sp[t] * D + d] : 0.f;
            f[t] = wpart && n0 + t < N ? fnorm[(size_t)(n0 + t) * D + d] : 0.f;
        }
        const float *w = wr + (size_t)d * E;
#pragma unroll
        for (int t = 0; t < MOE_TOK; t++) {
            if (n0 + t >= N) break;
            float s = 0.f;
            for (int e = 0; e < E; e++) s = fmaf(sd[t][e], w[e], s);
            dfn[(size_t)(n0 + t) * D + d] = x[t] + s;
        }
        if (wpart) {
            float *wp = wpart + ((size_t)blockIdx.x * D + d) * E;
            for (int e = 0; e < E; e++) {
                float s = 0.f;
#pragma unroll
                for (int t = 0; t < MOE_TOK; t++) s = fmaf(f[t], n0 + t < N ? sd[t][e] : 0.f, s);
                wp[e] = s;
            }
        }
    }
}

// -------------------------------------------------------------- scratch --
// One arena, grown on demand and kept until tlg_shutdown (like the
// reference's me_ensure, :840-848).  Growing it synchronizes the device, so
// the first call at a new size cannot be captured into a graph; calls on
// different streams must not overlap (they share the arena).
struct MoeScratch {
    int *idx, *pos, *eoff;
    float *dgate, *drt, *y, *dy, *g, *u, *a;
    float *wpart;            // dWr partials, one row of D x E per router workgroup
    int *bcnt;               // expert counts per router workgroup [nblk][E]
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
    const size_t nblk = (n + MOE_TOK - 1) / MOE_TOK;
    const size_t sizes[12] = {n * 4, n * 4, (size_t)(TLG_MOE_MAXE + 1) * 4, n * 4, n * E * 4,
                              n * D * 4, n * D * 4, n * F * 4, n * F * 4, n * F * 4, nblk * D * E * 4,
                              nblk * E * 4};
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
    s->y = (float *)(b + offs[5]);
    s->dy = (float *)(b + offs[6]);
    s->g = (float *)(b + offs[7]);
    s->u = (float *)(b + offs[8]);
    s->a = (float *)(b + offs[9]);
    s->wpart = (float *)(b + offs[10]);
    s->bcnt = (int *)(b + offs[11]);
    return TLG_OK;
}

// ------------------------------------------------------------ launches --
static inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

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
static int moe_index(const int *assign, int N, int E, const MoeScratch &s, const float *fin, float *out, int D,
                     hipStream_t st)
{
    hipLaunchKernelGGL(k_moe_index, dim3(1), dim3(1024), 0, st, assign, N, E, s.idx, s.pos, s.eoff, fin, out, D);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

// The W1 | W3 GEMM pair as one expert launch of paired-column tiles, X rows
// gathered from fnorm by the sorted-row index (:876-878), the SwiGLU in the
// epilogue (:880-883): a = silu(Xg W1_e) (Xg W3_e).  g and u are kept too
// when the caller passes them (the backward needs them, :923-925).
static int moe_w13(const float *fnorm, int N, int D, int F, int E, const float *w1, const float *w3,
                   const MoeScratch &s, float *g, float *u, hipStream_t st)
{
    TlgExpertCall c;
    memset(&c, 0, sizeof c);
    c.op = 0; c.C = s.a; c.K = D; c.N = F; c.nseg = 1;
    c.A[0] = fnorm; c.B[0] = w1; c.es = (long long)D * F;
    c.amap = s.idx; c.B2 = w3; c.epi = TLG_EPI_SWIGLU; c.X1 = g; c.X2 = u;
    return tlg_expert_launch(&c, 1, s.eoff, E, N, st);
}

// Kept forward state (tlg_dev_moe_grouped_fwd_keep): the index and the
// expert rows the backward would otherwise recompute, in one caller buffer:
// idx, pos (N ints each), eoff (E + 1 ints), then g, u, a (N x F) and y
// (N x D), each 256-byte aligned.
static size_t keep_layout(int N, int D, int F, int E, size_t *offs)
{
    const size_t n = (size_t)N;
    const size_t sizes[7] = {n * 4, n * 4, (size_t)(E + 1) * 4, n * F * 4, n * F * 4, n * F * 4, n * D * 4};
    size_t total = 0;
    for (int k = 0; k < 7; k++) {
        if (offs) offs[k] = total;
        total += (sizes[k] + 255) & ~(size_t)255;
    }
    return total;
}

extern "C" size_t tlg_moe_keep_bytes(int N, int D, int F, int E)
{
    if (N < 0 || D <= 0 || F <= 0 || E < 1 || E > TLG_MOE_MAXE) return 0;
    return keep_layout(N, D, F, E, nullptr);
}

static void keep_view(void *keep, int N, int D, int F, int E, MoeScratch *s)
{
    size_t o[7];
    keep_layout(N, D, F, E, o);
    char *b = (char *)keep;
    s->idx = (int *)(b + o[0]);
    s->pos = (int *)(b + o[1]);
    s->eoff = (int *)(b + o[2]);
    s->g = (float *)(b + o[3]);
    s->u = (float *)(b + o[4]);
    s->a = (float *)(b + o[5]);
    s->y = (float *)(b + o[6]);
}

// keep: store the index, g, u, a and y in s (a kept view) as well
static int moe_fwd(const float *fnorm, const float *fin, float *out, int N, int D, int F, int E, const float *wr,
                   const float *w1, const float *w3, const float *w2, int *assign, float *gate, float *rprobs,
                   const MoeScratch &s, bool keep, hipStream_t st)
{
    int rc;
    const int dch = route_dch(D, E);
    // the router leaves per-block counts and in-block ranks (in pos) for the
    // many-workgroup index
    hipLaunchKernelGGL(k_moe_route, dim3((N + MOE_TOK - 1) / MOE_TOK), dim3(256), route_lds(dch, E), st, fnorm, wr,
                       N, D, E, dch, rprobs, assign, gate, s.pos, s.bcnt);
    TLG_HIP(hipGetLastError());
    // the index also sets out = fin for tokens without an expert
    hipLaunchKernelGGL(k_moe_index_blk, dim3((N + MOE_IDX_TPB - 1) / MOE_IDX_TPB), dim3(MOE_IDX_TPB), 0, st, assign,
                       s.bcnt, N, E, s.idx, s.pos, s.eoff, fin, out, D);
    TLG_HIP(hipGetLastError());
    if ((rc = moe_w13(fnorm, N, D, F, E, w1, w3, s, keep ? s.g : nullptr, keep ? s.u : nullptr, st))) return rc;
    // y = a W2_e with the combine in the epilogue: out[n] = fin[n] + gate[n] y
    TlgExpertCall c;
    memset(&c, 0, sizeof c);
    c.op = 0; c.C = out; c.K = F; c.N = D; c.nseg = 1;
    c.A[0] = s.a; c.B[0] = w2; c.es = (long long)F * D;
    c.epi = TLG_EPI_COMBINE; c.omap = s.idx; c.fin = fin; c.gate = gate;
    if (keep) c.X1 = s.y;
    return tlg_expert_launch(&c, 1, s.eoff, E, N, st);
}

int tlg_moe_fwd_launch(const float *fnorm, const float *fin, float *out, int N, int D, int F, int E,
                       const float *wr, const float *w1, const float *w3, const float *w2, int *assign,
                       float *gate, float *rprobs, void *keep, size_t keep_bytes, hipStream_t st)
{
    int rc = check_shape(N, D, F, E);
    if (rc) return rc;
    if (N == 0) return TLG_OK;
    if (!MOE_PTRS_OK(fnorm, fin, out, w1, w3, w2) || !wr || !assign || !gate || !rprobs)
        return tlg_fail(TLG_EINVAL, "MoE forward: NULL or misaligned (16-byte) pointer");
    if (keep && (!al16(keep) || keep_bytes < keep_layout(N, D, F, E, nullptr)))
        return tlg_fail(TLG_EINVAL, "MoE forward: kept state needs %zu bytes, 16-byte aligned",
                        keep_layout(N, D, F, E, nullptr));
    if ((rc = tlg_ensure_init())) return rc;
    if ((rc = tlg_group_flush_launch(st))) return rc;
    MoeScratch s;
    if ((rc = moe_scratch(N, D, F, E, &s))) return rc;
    if (keep) keep_view(keep, N, D, F, E, &s);
    return moe_fwd(fnorm, fin, out, N, D, F, E, wr, w1, w3, w2, assign, gate, rprobs, s, keep != nullptr, st);
}

// kept: s's index, g, u, a and y come from a kept forward (no recompute);
// g and u are overwritten (dg, du) as in the recomputing backward
static int moe_bwd(const float *fnorm, const float *dout, float *d_fnorm, const int *assign, const float *gate,
                   const float *rprobs, int N, int D, int F, int E, const float *wr, const float *w1, const float *w3,
                   const float *w2, float *gwr, float *gw1, float *gw3, float *gw2, const MoeScratch &s, bool kept,
                   hipStream_t st)
{
    int rc;
    if (!kept) {
        if ((rc = moe_index(assign, N, E, s, nullptr, nullptr, D, st))) return rc;
        // recompute the forward of every expert (:910-914): g, u, a, then y
        if ((rc = moe_w13(fnorm, N, D, F, E, w1, w3, s, s.g, s.u, st))) return rc;
        TlgExpertCall c;
        memset(&c, 0, sizeof c);
        c.op = 0; c.C = s.y; c.K = F; c.N = D; c.nseg = 1;
        c.A[0] = s.a; c.B[0] = w2; c.es = (long long)F * D;
        if ((rc = tlg_expert_launch(&c, 1, s.eoff, E, N, st))) return rc;
    }
    hipLaunchKernelGGL(k_moe_dgate, dim3((N + 3) / 4), dim3(256), 0, st, dout, s.y, s.idx, s.eoff, E, D, gate,
                       s.dgate, s.dy);
    TLG_HIP(hipGetLastError());
    // dW2_e += a^T dy ;  da = dy W2_e^T with the SwiGLU backward in its
    // epilogue: g <- dg, u <- du  (:921-925)
    TlgExpertCall c[3];
    memset(c, 0, sizeof c);
    c[0].op = 2; c[0].beta = 1; c[0].C = gw2; c[0].K = F; c[0].N = D; c[0].nseg = 1;
    c[0].A[0] = s.a; c[0].B[0] = s.dy; c[0].es = (long long)F * D;
    c[1].op = 1; c[1].beta = 0; c[1].C = nullptr; c[1].K = F; c[1].N = D; c[1].nseg = 1;
    c[1].A[0] = s.dy; c[1].B[0] = w2; c[1].es = (long long)F * D;
    c[1].epi = TLG_EPI_SWIGLU_BWD; c[1].X1 = s.g; c[1].X2 = s.u;
    // dW2's slice reduction runs as the last items of the next launch
    if ((rc = tlg_expert_launch(c, 2, s.eoff, E, N, st, TLG_ECARRY_OUT))) return rc;
    // dW1_e += Xg^T dg ; dW3_e += Xg^T du (Xg rows gathered from fnorm) ;
    // dX = dg W1_e^T + du W3_e^T  (:926-927)
    memset(c, 0, sizeof c);
    c[0].op = 2; c[0].beta = 1; c[0].C = gw1; c[0].K = D; c[0].N = F; c[0].nseg = 1;
    c[0].A[0] = fnorm; c[0].amap = s.idx; c[0].B[0] = s.g; c[0].es = (long long)D * F;
    c[1] = c[0];
    c[1].C = gw3; c[1].B[0] = s.u;
    c[2].op = 1; c[2].beta = 0; c[2].C = s.y; c[2].K = D; c[2].N = F; c[2].nseg = 2;
    c[2].A[0] = s.g; c[2].B[0] = w1; c[2].A[1] = s.u; c[2].B[1] = w3; c[2].Nseg[1] = F;
    c[2].es = (long long)D * F;
    // (its own slice reductions are held too: they run with dWr's column sum,
    // in one launch at the flush)
    if ((rc = tlg_expert_launch(c, 3, s.eoff, E, N, st, TLG_ECARRY_INOUT))) return rc;
    // router: softmax backward, d_fnorm, dWr  (:932-945).  dWr's per-block
    // partials are summed by a column-sum item: at once for the reference-
    // shaped entry, in the next grouped launch for the kept-state one (as a
    // split GEMM's reduction; the same sum either way).  An unaligned gwr
    // takes the mm_atb launch instead.
    const int nblk = (N + MOE_TOK - 1) / MOE_TOK;
    const bool cs = al16(gwr);
    hipLaunchKernelGGL(k_moe_router_bwd, dim3(nblk), dim3(256), 0, st, rprobs, s.pos, assign, s.dgate, s.eoff, s.y,
                       wr, N, D, E, s.drt, d_fnorm, fnorm, cs ? s.wpart : nullptr);
    TLG_HIP(hipGetLastError());
    if (!cs) return tlg_gemm_launch(TLG_TN, fnorm, s.drt, gwr, D, E, N, D, E, E, 1, st);
    if ((rc = tlg_defer_colsum(s.wpart, gwr, nblk, D * E, 1, st))) return rc;
    return kept ? TLG_OK : tlg_group_flush_launch(st);
}

int tlg_moe_bwd_launch(const float *fnorm, const float *dout, float *d_fnorm, const int *assign,
                       const float *gate, const float *rprobs, int N, int D, int F, int E, const float *wr,
                       const float *w1, const float *w3, const float *w2, float *gwr, float *gw1, float *gw3,
                       float *gw2, void *kept, size_t kept_bytes, hipStream_t st)
{
    int rc = check_shape(N, D, F, E);
    if (rc) return rc;
    if (N == 0) return TLG_OK;
    if (!MOE_PTRS_OK(fnorm, dout, d_fnorm, w1, w3, w2, gw1, gw3, gw2) || !wr || !gwr || !assign || !gate ||
        !rprobs)
        return tlg_fail(TLG_EINVAL, "MoE backward: NULL or misaligned (16-byte) pointer");
    if (kept && (!al16(kept) || kept_bytes < keep_layout(N, D, F, E, nullptr)))
        return tlg_fail(TLG_EINVAL, "MoE backward: kept state needs %zu bytes, 16-byte aligned",
                        keep_layout(N, D, F, E, nullptr));
    if ((rc = tlg_ensure_init())) return rc;
    if ((rc = tlg_group_flush_launch(st))) return rc;
    MoeScratch s;
    if ((rc = moe_scratch(N, D, F, E, &s))) return rc;
    if (kept) keep_view(kept, N, D, F, E, &s);
    return moe_bwd(fnorm, dout, d_fnorm, assign, gate, rprobs, N, D, F, E, wr, w1, w3, w2, gwr, gw1, gw3, gw2, s,
                   kept != nullptr, st);
}
