// tlg_gemv.hip -- the M <= 8 forms of mm and mm_bt (KV-cache decode) on gfx950.
//
// At M <= 8 rows a GEMM is a matrix-vector product: every weight is used M
// times, so a launch is one pass over the weight matrix and its speed is set
// by how much of that matrix is in flight at once.  The decode matrices are
// small (0.15-3.1 MB) next to what HBM has in flight at full rate (about
// 8 TB/s x 1.5 us = 12 MB), so a launch should request its whole matrix in
// its first round of loads: every lane issues all of its weight loads (16-byte
// vectors, each wave covering 256 contiguous bytes of a row) before it uses
// any, and the matrix is cut into a few hundred workgroups of 4-16 KB so all
// 256 CUs take part.
//
//   mm     Y[m][j] = sum_k X[m][k] W[k][j]       W rows run along the output
//          index j.  An item owns a 64-column block and a slice of KS rows:
//          16 lanes read one row's 256 bytes, a wave 4 rows at a time.  The
//          item's partial column sums meet in LDS in a fixed order.  When the
//          rows are split over S items, the S-1 "producer" items store their
//          partial block as tagged 64-bit words (value | 1 << 32) and the
//          item of the last slice, the "reducer", adds the S partials in
//          slice order and writes C, then clears the words it read.
//   mm_bt  dX[m][k] += sum_n dY[m][n] W[k][n]    W rows run along the
//          reduction.  An item owns 8 output rows, 2 per wave: 32 lanes read
//          one row in 512-byte steps, each dot product ends in a fixed-order
//          cross-lane sum over the 32 lanes (DPP).  No split is needed.
//
// Reducers wait: every producer item has a lower workgroup id than every
// reducer item, and the dispatcher starts the workgroups of a launch in id
// order, so a reducer only ever waits for items that have already started
// and never wait themselves.  The wait is bounded (10 ms of the real-time
// counter); past it the reducer writes NaN and sets an error word, so a fault
// shows as a wrong result, never as a hang.  Partial words are written and
// read with agent-scope accesses (they reach the device-coherent level, not
// only one XCD's L2).  The workspace is a ring of regions, one per launch in
// turn, so launches on different streams do not share words unless more than
// GV_RING of them overlap.
//
// Reference: mm tinylm.c:438-449 (serial at M <= 4 through tl_for, :444-446),
// mm_bt :480-489; the decode GEMV sites of forward_chunk :3748-3824 and the
// head :3035.  Several GEMVs that the reference issues back to back (q, k, v
// on the same input; w1, w3) run as one launch: a problem table in the
// kernel arguments.  Results match the reference to fp32 rounding: each
// output is a fixed-order sum (lane, then row group, then slice), the same in
// every launch.
#include "tlg_internal.h"
#include "../../include/tldecode.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned long long u64;
typedef unsigned int u32;

#define GV_T 256                      // threads per workgroup (4 waves)
#define GV_MAXPROB 8
#define GV_MAXSEG 3
#define GV_NT_ROWS 8                  // mm_bt: output rows per item (2 per wave)
#define GV_RING 16                    // workspace regions, used by launches in turn
#define GV_REGION_WORDS ((size_t)256 << 10)   // 64-bit partial words per region (2 MiB)
#define GV_SPIN 1000000ull            // 10 ms of the 100 MHz real-time counter
#define GV_TAG (1ull << 32)

// Every global access goes through global-address-space pointers: flat
// accesses would also count against lgkmcnt, so the LDS barriers would wait
// for the weight loads in flight.
#define GAS __attribute__((address_space(1)))

struct GvSeg { const float *A, *B; int R, lda, ldb; };
// Activation prologues (decode: the glue before a GEMV, applied as the rows
// are read): GV_PRO_RMS uses x * s * gain with s = 1 / sqrt(sum(x^2) / R +
// 1e-5) of the whole row (rmsnorm_fwd, tinylm.c:540-548); GV_PRO_SWIGLU uses
// silu(a) * a2 with silu(z) = z / (1 + e^-z) (:786, :1005-1006).
enum { GV_PRO_NONE = 0, GV_PRO_RMS = 1, GV_PRO_SWIGLU = 2 };
struct GvProb {
    float *C;
    int kind;                    // TLG_NN or TLG_NT
    int M, No, ldc, beta, nseg;
    const float *gain, *A2;      // RMS gain [R]; SwiGLU second operand (layout of A)
    GvSeg seg[GV_MAXSEG];
    // decomposition (host): nb column (NN) or row (NT) blocks; NN rows split
    // into S slices of KS rows; with S > 1 the partial words start at `part`
    int nb, S, KS;
    long long part;
    int direct, reducers;        // items that never wait; reducer items (nb when S > 1)
    int full;                    // NN over all K rows per item (32-column blocks, no split)
    const int *bsel;             // optional: every segment's B is offset by bsel[0] * bstride
    long long bstride;
    const float *cgate;          // optional: results scaled by cgate[0] before the store
};
struct GvArgs {
    int nprob;
    u64 *part;                   // this launch's region of partial words
    u32 *err;                    // set to 1 by a reducer whose wait timed out
    GvProb p[GV_MAXPROB];
};

template <int VEC> struct GvV;
template <> struct GvV<4> { typedef f32x4 T; };
template <> struct GvV<1> { typedef float T; };

template <int VEC> __device__ __forceinline__ typename GvV<VEC>::T gv_ld(const float *p)
{
    return *(const GAS typename GvV<VEC>::T *)p;
}
__device__ __forceinline__ float gv_ld1(const float *p) { return *(const GAS float *)p; }
__device__ __forceinline__ float gv_el(const f32x4 &v, int i) { return v[i]; }
__device__ __forceinline__ float gv_el(const float &v, int) { return v; }
__device__ __forceinline__ void gv_set(f32x4 &v, int i, float x) { v[i] = x; }
__device__ __forceinline__ void gv_set(float &v, int, float x) { v = x; }

__device__ __forceinline__ u64 gv_ld_agent(const u64 *p)
{
    return __hip_atomic_load((GAS u64 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void gv_st_agent(u64 *p, u64 v)
{
    __hip_atomic_store((GAS u64 *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float gv_silu_mul(float a, float b) { return a / (1.0f + expf(-a)) * b; }

// The weight of segment g as the problem sees it (a device-selected expert
// slice when bsel is set) and the output scale (1, or the row's gate).
template <class P_, class G_> __device__ __forceinline__ const float *gv_B(const P_ &P, const G_ &g)
{
    return P.bsel ? g.B + (long long)*(const GAS int *)P.bsel * P.bstride : g.B;
}
template <class P_> __device__ __forceinline__ float gv_cgate(const P_ &P)
{
    return P.cgate ? *(const GAS float *)P.cgate : 1.0f;
}

// Sums over each 32-lane half of a wave on the VALU (DPP), in a fixed order:
// row_shr 1, 2, 4, 8 within the 16-lane rows, then row_bcast:15 adds row 0's
// (row 2's) lane 15 into row 1 (row 3).  Lane 31 ends with the sum of lanes
// 0-31, lane 63 with that of lanes 32-63.
template <int CTRL, int ROWMASK> __device__ __forceinline__ float gv_dpp(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROWMASK, 0xf, false));
}
__device__ __forceinline__ float gv_half_sum(float x)
{
    x += gv_dpp<0x111, 0xf>(x);
    x += gv_dpp<0x112, 0xf>(x);
    x += gv_dpp<0x114, 0xf>(x);
    x += gv_dpp<0x118, 0xf>(x);
    x += gv_dpp<0x142, 0xa>(x);
    return x;
}

#define GV_FULL_ACT 8192               // full-K mm: activation floats staged in LDS (K x MB)
#define GV_FULL_K 1024                // full-K mm: at most this many rows (32 loads per lane)

template <int MB, int CB> struct __attribute__((aligned(16))) GvSmem {
    union {
        struct {                     // split mm
            float red[16][MB][CB];   // per (wave, lane row) partial blocks
            float own[MB * CB];      // this item's slice of the block
            float grp[16][GV_T];     // reducer: per-group slice sums
        } s;
        struct {                     // full-K mm
            float act[GV_FULL_ACT];  // activation rows, [k][MB]
            float red[32][MB][32];   // per (wave, lane row) partial blocks
        } f;
    };
    float rs[8];                     // RMS scale per row
    int timeout;
};

// RMS prologue: s_m = 1 / sqrt(sum_r A[m][r]^2 / R + 1e-5) for m < M, one
// wave per row (rows w and w + 4), into sh.rs; read after a barrier.  The
// scale multiplies the finished dot products (sum_r x g w scaled by s equals
// sum_r (x s g) w up to rounding), so the weight loads never wait for it.
template <int MB, int CB>
__device__ __forceinline__ void gv_rms_stats(const float *A, int lda, int R, int M, GvSmem<MB, CB> &sh)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int mm = 0; mm < 2; mm++) {
        const int m = w + 4 * mm;
        if (mm * 4 < MB && m < M) {
            float ss = 0.f;
            for (int r0 = 0; r0 < R; r0 += 1024) {
                f32x4 x[4];
#pragma unroll
                for (int i = 0; i < 4; i++) x[i] = gv_ld<4>(A + (size_t)m * lda + min(r0 + 256 * i + 4 * lane, R - 4));
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const bool ok = r0 + 256 * i + 4 * lane < R;
                    const f32x4 y = ok ? x[i] : f32x4{0.f, 0.f, 0.f, 0.f};
                    ss = fmaf(y.x, y.x, ss); ss = fmaf(y.y, y.y, ss);
                    ss = fmaf(y.z, y.z, ss); ss = fmaf(y.w, y.w, ss);
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
            if (lane == 0) sh.rs[m] = 1.0f / sqrtf(ss / (float)R + 1e-5f);
        }
    }
}

// The reducer's sum over slices [s_lo, s_hi) of output o: the words of up
// to 16 slices are loaded at once, then checked and added in slice order;
// slice s_own (the reducer's own) comes from own_v.  Repeats until every word
// carries the tag or the wait runs past GV_SPIN (then timeout = 1), and
// clears the words it read.
__device__ __forceinline__ float gv_slices(u64 *pw, int nout, int o, int s_lo, int s_hi, int s_own, float own_v,
                                           u64 t0, int &timeout)
{
    float v;
    for (;;) {
        bool ok = true;
        v = 0.f;
        for (int q0 = s_lo; q0 < s_hi; q0 += 16) {
            u64 x[16];
#pragma unroll
            for (int i = 0; i < 16; i++) x[i] = gv_ld_agent(pw + (size_t)min(q0 + i, s_hi - 1) * nout + o);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int q = q0 + i;
                if (q < s_hi) {
                    if (q == s_own) v += own_v;
                    else {
                        ok = ok && (x[i] >> 32) == 1ull;
                        v += __uint_as_float((u32)x[i]);
                    }
                }
            }
        }
        if (ok) break;
        if (wall_clock64() - t0 > GV_SPIN) { timeout = 1; break; }
    }
    for (int q = s_lo; q < s_hi; q++)
        if (q != s_own) gv_st_agent(pw + (size_t)q * nout + o, 0ull);
    return v;
}

// ------------------------------------------------------------------ mm --
// Item (s, cb) of an NN problem: rows [s KS, min(R, s KS + KS)) of column
// block cb.  Lane (r = lane / 16, c = lane % 16) of wave w reads row
// kb + 16 u + 4 w + r, columns cb CB + VEC c .. + VEC - 1, for u < U.
template <int MB, int VEC, int U, int PRO>
__device__ __forceinline__ void gv_nn(const GvArgs &g, const GvProb &P, int s, int cb, GvSmem<MB, 16 * VEC> &sh)
{
    constexpr int CB = 16 * VEC;
    typedef typename GvV<VEC>::T V;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane >> 4, c = lane & 15;
    const int M = P.M;
    const GvSeg &G = P.seg[0];
    const int j = cb * CB + c * VEC;
    const int jc = j < P.No ? j : 0;                  // in-bounds address for edge lanes
    const int k_lo = s * P.KS, k_hi = min(G.R, k_lo + P.KS);
    const float *Bb = gv_B(P, G);
    const float cg = gv_cgate(P);
    float acc[MB][VEC];
#pragma unroll
    for (int m = 0; m < MB; m++)
#pragma unroll
        for (int v = 0; v < VEC; v++) acc[m][v] = 0.f;
    // a batch: U rows per lane, every load first (clamped addresses), the
    // rows past the slice zeroed when used
    auto load = [&](V (&wv)[U], float (&av)[U][MB], int kb) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int k = min(kb + 16 * u + 4 * w + r, k_hi - 1);
            wv[u] = gv_ld<VEC>(Bb + (size_t)k * G.ldb + jc);
#pragma unroll
            for (int m = 0; m < MB; m++) {
                const size_t ai = (size_t)min(m, M - 1) * G.lda + k;
                float a = gv_ld1(G.A + ai);
                if (PRO == GV_PRO_SWIGLU) a = gv_silu_mul(a, gv_ld1(P.A2 + ai));
                if (PRO == GV_PRO_RMS) a *= gv_ld1(P.gain + k);
                av[u][m] = a;
            }
        }
    };
    auto fma_batch = [&](const V (&wv)[U], const float (&av)[U][MB], int kb) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const bool ok = kb + 16 * u + 4 * w + r < k_hi;
#pragma unroll
            for (int m = 0; m < MB; m++) {
                const float a = ok ? av[u][m] : 0.f;
#pragma unroll
                for (int v = 0; v < VEC; v++) acc[m][v] = fmaf(a, gv_el(wv[u], v), acc[m][v]);
            }
        }
    };
    V wv[U];
    float av[U][MB];
    load(wv, av, k_lo);
    // the RMS statistics' loads queue behind the first batch, in flight together
    if (PRO == GV_PRO_RMS) gv_rms_stats<MB, CB>(G.A, G.lda, G.R, M, sh);
    if (k_hi - k_lo <= 16 * U) {
        fma_batch(wv, av, k_lo);
    } else {
        // longer slices: the next batch in flight while this one is used (the
        // batch after the last re-reads the last rows, unused)
        for (int kb = k_lo; kb < k_hi; kb += 16 * U) {
            V nw[U];
            float na[U][MB];
            load(nw, na, min(kb + 16 * U, k_hi - 1));
            fma_batch(wv, av, kb);
#pragma unroll
            for (int u = 0; u < U; u++) {
                wv[u] = nw[u];
#pragma unroll
                for (int m = 0; m < MB; m++) av[u][m] = na[u][m];
            }
        }
    }
    // the 16 row groups of the item (4 lane rows x 4 waves), in fixed order
#pragma unroll
    for (int m = 0; m < MB; m++) {
        V x;
#pragma unroll
        for (int v = 0; v < VEC; v++) gv_set(x, v, acc[m][v]);
        *reinterpret_cast<V *>(&sh.s.red[w * 4 + r][m][c * VEC]) = x;
    }
    __syncthreads();
    const int nout = M * CB;
    const bool split = P.S > 1, reducer = split && s == P.S - 1;
    u64 *pw = g.part + P.part + (size_t)cb * P.S * nout;      // this block's S slices of nout words
    for (int o = tid; o < nout; o += GV_T) {
        const int m = o / CB, cc = o - m * CB;
        float v = sh.s.red[0][m][cc];
#pragma unroll
        for (int q = 1; q < 16; q++) v += sh.s.red[q][m][cc];
        if (!split) {
            const int jj = cb * CB + cc;
            if (jj < P.No) {
                if (PRO == GV_PRO_RMS) v *= sh.rs[m];
                v *= cg;
                float *out = P.C + (size_t)m * P.ldc + jj;
                *out = P.beta ? *out + v : v;
            }
        } else if (!reducer) {
            gv_st_agent(pw + (size_t)s * nout + o, GV_TAG | (u64)__float_as_uint(v));
        } else {
            sh.s.own[o] = v;
        }
    }
    if (!reducer) return;
    // the reducer: slices in order -- in G groups of consecutive slices per
    // output when the outputs do not fill the workgroup, then the groups in
    // order
    if (tid == 0) sh.timeout = 0;
    __syncthreads();
    const int S = P.S;
    const u64 t0 = wall_clock64();
    if (nout >= GV_T) {
        for (int o = tid; o < nout; o += GV_T)
            sh.s.own[o] = gv_slices(pw, nout, o, 0, S, S - 1, sh.s.own[o], t0, sh.timeout);
    } else {
        const int G = GV_T / nout, grp = tid / nout, o = tid - grp * nout;
        if (grp < G) sh.s.grp[grp][o] = gv_slices(pw, nout, o, grp * S / G, (grp + 1) * S / G, S - 1, sh.s.own[o], t0,
                                                sh.timeout);
    }
    __syncthreads();
    const bool bad = sh.timeout != 0;
    for (int o = tid; o < nout; o += GV_T) {
        const int m = o / CB, cc = o - m * CB, jj = cb * CB + cc;
        float v;
        if (nout >= GV_T) v = sh.s.own[o];
        else {
            const int G = GV_T / nout;
            v = sh.s.grp[0][o];
            for (int q = 1; q < G; q++) v += sh.s.grp[q][o];
        }
        if (jj < P.No) {
            if (PRO == GV_PRO_RMS) v *= sh.rs[m];
            v *= cg;
            float *out = P.C + (size_t)m * P.ldc + jj;
            *out = bad ? __builtin_nanf("") : (P.beta ? *out + v : v);
        }
    }
    if (bad && tid == 0) __hip_atomic_store((GAS u32 *)g.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------ mm, full K --
// Item cb of a full-K NN problem owns columns [32 cb, 32 cb + 32) over all K
// rows, so no other workgroup takes part in its sums.  Lane (rr = lane / 8,
// c = lane % 8) of wave w reads rows 32 u + 8 w + rr, columns 32 cb + 4 c ..
// + 3: 8 lanes cover one row's 128-byte line, and every load of the item
// (16 UB per lane, K <= 512 UB) is issued before any is used.  The
// activation rows are staged in LDS as [k][MB] through the prologue while the
// weight loads are in flight; the 32 row groups of a column then meet in LDS
// in a fixed order.
template <int MB, int UB, int PRO>
__device__ __forceinline__ void gv_nn_full(const GvProb &P, int cb, GvSmem<MB, 64> &sh)
{
    constexpr int UF = 16 * UB;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int rr = lane >> 3, c = lane & 7;
    const int M = P.M;
    const GvSeg &G = P.seg[0];
    const int K = G.R;
    const int j = cb * 32 + 4 * c;
    const float *Bp = gv_B(P, G) + (j < P.No ? j : 0);
    const float cg = gv_cgate(P);
    f32x4 wv[UF];
#pragma unroll
    for (int u = 0; u < UF; u++) wv[u] = gv_ld<4>(Bp + (size_t)min(32 * u + 8 * w + rr, K - 1) * G.ldb);
    if (PRO == GV_PRO_RMS) gv_rms_stats<MB, 64>(G.A, G.lda, K, M, sh);
    // the activation, [m][k] in memory -> act[k][m] in LDS: thread t takes
    // columns 4 t .. 4 t + 3 of every row (K <= 1024), all loads first
    {
        constexpr int AU = (1024 / 4 + GV_T - 1) / GV_T;
        f32x4 xa[AU][MB], xb[AU][MB];
        const int K4 = K >> 2;
#pragma unroll
        for (int i = 0; i < AU; i++) {
            const int k4 = min(tid + GV_T * i, K4 - 1);
#pragma unroll
            for (int m = 0; m < MB; m++) {
                const size_t ai = (size_t)min(m, M - 1) * G.lda + 4 * k4;
                xa[i][m] = gv_ld<4>(G.A + ai);
                if (PRO == GV_PRO_SWIGLU) xb[i][m] = gv_ld<4>(P.A2 + ai);
                if (PRO == GV_PRO_RMS && m == 0) xb[i][0] = gv_ld<4>(P.gain + 4 * k4);
            }
        }
#pragma unroll
        for (int i = 0; i < AU; i++) {
            const int k4 = tid + GV_T * i;
            if (k4 < K4) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    float a[MB];
#pragma unroll
                    for (int m = 0; m < MB; m++) {
                        a[m] = xa[i][m][q];
                        if (PRO == GV_PRO_SWIGLU) a[m] = gv_silu_mul(a[m], xb[i][m][q]);
                        if (PRO == GV_PRO_RMS) a[m] *= xb[i][0][q];
                    }
                    float *dst = &sh.f.act[(4 * k4 + q) * MB];
                    if (MB >= 4) {
#pragma unroll
                        for (int m4 = 0; m4 < MB; m4 += 4)
                            *reinterpret_cast<f32x4 *>(dst + m4) = f32x4{a[m4], a[m4 + 1], a[m4 + 2], a[m4 + 3]};
                    } else {
#pragma unroll
                        for (int m = 0; m < MB; m++) dst[m] = a[m];
                    }
                }
            }
        }
    }
    __syncthreads();
    float acc[MB][4];
#pragma unroll
    for (int m = 0; m < MB; m++)
#pragma unroll
        for (int v = 0; v < 4; v++) acc[m][v] = 0.f;
#pragma unroll
    for (int u = 0; u < UF; u++) {
        const int k = 32 * u + 8 * w + rr;
        const bool ok = k < K;
        const float *ak = &sh.f.act[min(k, K - 1) * MB];
        float a[MB];
        if (MB >= 4) {
#pragma unroll
            for (int m4 = 0; m4 < MB; m4 += 4) {
                const f32x4 t = *reinterpret_cast<const f32x4 *>(ak + m4);
                a[m4] = t.x; a[m4 + 1] = t.y; a[m4 + 2] = t.z; a[m4 + 3] = t.w;
            }
        } else {
#pragma unroll
            for (int m = 0; m < MB; m++) a[m] = ak[m];
        }
#pragma unroll
        for (int m = 0; m < MB; m++) {
            const float x = ok ? a[m] : 0.f;
#pragma unroll
            for (int v = 0; v < 4; v++) acc[m][v] = fmaf(x, wv[u][v], acc[m][v]);
        }
    }
#pragma unroll
    for (int m = 0; m < MB; m++)
        *reinterpret_cast<f32x4 *>(&sh.f.red[w * 8 + rr][m][4 * c]) = f32x4{acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
    __syncthreads();
    // the 32 row groups: NG groups of consecutive ones per output, then the
    // groups in order (the partial sums reuse the activation's LDS)
    constexpr int NO = 32 * MB, NG = GV_T / NO;
    {
        const int o = tid % NO, g = tid / NO, m = o / 32, cc = o % 32;
        float v = sh.f.red[g * (32 / NG)][m][cc];
#pragma unroll
        for (int q = 1; q < 32 / NG; q++) v += sh.f.red[g * (32 / NG) + q][m][cc];
        sh.f.act[g * NO + o] = v;
    }
    __syncthreads();
    if (tid < NO) {
        const int m = tid / 32, cc = tid % 32, jj = cb * 32 + cc;
        float v = sh.f.act[tid];
#pragma unroll
        for (int g = 1; g < NG; g++) v += sh.f.act[g * NO + tid];
        if (m < M && jj < P.No) {
            if (PRO == GV_PRO_RMS) v *= sh.rs[m];
            v *= cg;
            float *out = P.C + (size_t)m * P.ldc + jj;
            *out = P.beta ? *out + v : v;
        }
    }
}

// --------------------------------------------------------------- mm_bt --
// Item b of an NT problem: output rows o = 8 b + 2 w + lane / 32.  The 32
// lanes of a half-wave read the row's reduction index in steps of 32 VEC
// floats (U steps per batch, all loads of a batch first), then a DPP sum
// over the 32 lanes gives the M dot products.
template <int MB, int VEC, int U, int PRO>
__device__ __forceinline__ void gv_nt(const GvProb &P, int b, GvSmem<MB, 16 * VEC> &sh)
{
    typedef typename GvV<VEC>::T V;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l = lane & 31;
    const int o = b * GV_NT_ROWS + 2 * w + (lane >> 5);
    const int oc = min(o, P.No - 1);
    const int M = P.M;
    const float cg = gv_cgate(P);
    float acc[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) acc[m] = 0.f;
    auto load = [&](V (&wv)[U], V (&av)[U][MB], const GvSeg &G, const float *Brow, int r0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int rr = min(r0 + (32 * u + l) * VEC, G.R - VEC);
            wv[u] = gv_ld<VEC>(Brow + rr);
#pragma unroll
            for (int m = 0; m < MB; m++) {
                const size_t ai = (size_t)min(m, M - 1) * G.lda + rr;
                V a = gv_ld<VEC>(G.A + ai);
                if (PRO == GV_PRO_SWIGLU) {
                    const V a2 = gv_ld<VEC>(P.A2 + ai);
#pragma unroll
                    for (int v = 0; v < VEC; v++) gv_set(a, v, gv_silu_mul(gv_el(a, v), gv_el(a2, v)));
                }
                if (PRO == GV_PRO_RMS) {
                    const V gn = gv_ld<VEC>(P.gain + rr);
#pragma unroll
                    for (int v = 0; v < VEC; v++) gv_set(a, v, gv_el(a, v) * gv_el(gn, v));
                }
                av[u][m] = a;
            }
        }
    };
    auto fma_batch = [&](const V (&wv)[U], const V (&av)[U][MB], const GvSeg &G, int r0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const bool ok = r0 + (32 * u + l) * VEC < G.R;
#pragma unroll
            for (int m = 0; m < MB; m++)
#pragma unroll
                for (int v = 0; v < VEC; v++)
                    acc[m] = fmaf(ok ? gv_el(av[u][m], v) : 0.f, gv_el(wv[u], v), acc[m]);
        }
    };
    for (int sg = 0; sg < P.nseg; sg++) {
        const GvSeg &G = P.seg[sg];
        const float *Brow = gv_B(P, G) + (size_t)oc * G.ldb;
        V wv[U];
        V av[U][MB];
        load(wv, av, G, Brow, 0);
        if (PRO == GV_PRO_RMS && sg == 0) gv_rms_stats<MB, 16 * VEC>(G.A, G.lda, G.R, M, sh);
        if (G.R <= 32 * VEC * U) {
            fma_batch(wv, av, G, 0);
        } else {
            for (int r0 = 0; r0 < G.R; r0 += 32 * VEC * U) {
                V nw[U];
                V na[U][MB];
                load(nw, na, G, Brow, min(r0 + 32 * VEC * U, G.R - VEC));
                fma_batch(wv, av, G, r0);
#pragma unroll
                for (int u = 0; u < U; u++) {
                    wv[u] = nw[u];
#pragma unroll
                    for (int m = 0; m < MB; m++) av[u][m] = na[u][m];
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MB; m++) acc[m] = gv_half_sum(acc[m]);
    if (PRO == GV_PRO_RMS) __syncthreads();           // sh.rs
    if (l == 31 && o < P.No) {
#pragma unroll
        for (int m = 0; m < MB; m++)
            if (m < M) {
                float v = acc[m];
                if (PRO == GV_PRO_RMS) v *= sh.rs[m];
                v *= cg;
                float *out = P.C + (size_t)m * P.ldc + o;
                *out = P.beta ? *out + v : v;
            }
    }
}

// Workgroup b: the items that never wait first (every problem's direct
// items in problem order), then the reducers.
template <int MB, int VEC, int U, int PRO>
__global__ __launch_bounds__(GV_T) void k_gemv(GvArgs g)
{
    __shared__ GvSmem<MB, 16 * VEC> sh;
    int b = blockIdx.x, p = 0;
    while (p < g.nprob && b >= g.p[p].direct) { b -= g.p[p].direct; p++; }
    if (p < g.nprob) {
        const GvProb &P = g.p[p];
        if (P.kind == TLG_NN && P.full) {
            if constexpr (VEC == 4) gv_nn_full<MB, (U >= 2 ? 2 : 1), PRO>(P, b, sh);
        } else if (P.kind == TLG_NN) gv_nn<MB, VEC, U, PRO>(g, P, b / P.nb, b % P.nb, sh);
        else gv_nt<MB, VEC, U, PRO>(P, b, sh);
        return;
    }
    p = 0;
    while (p < g.nprob && b >= g.p[p].reducers) { b -= g.p[p].reducers; p++; }
    if (p >= g.nprob) return;
    const GvProb &P = g.p[p];
    gv_nn<MB, VEC, U, PRO>(g, P, P.S - 1, b, sh);
}

// ------------------------------------------------- mm_bt over one matrix --
// The common decode launch: every problem of it is an mm_bt over the same
// activation rows, and the problems' weights follow each other in memory (q |
// k | v and w1 | w3 of the decode layout), so the launch is one matrix B
// [nrows][K] whose row r gives output r - rs_s of segment s (rs_0 = 0, rs_1 =
// r1, rs_2 = r2).  The arguments are plain scalars in the order the kernel
// needs them, and the first 14 dwords (B, A, K, nrows, M | beta << 8, C0-C2,
// r1 | r2 << 16: all that the 16 user SGPRs hold besides the argument-block
// pointer) reach SGPRs before the first instruction (kernarg preload,
// -amdgpu-kernarg-preload-count), so the weight loads issue at once and a
// launch at M = 1 without a prologue or the MoE operands (SEL) reads nothing
// from its argument block; a table of problems in
// the argument block (k_gemv) puts a chain of dependent scalar loads in front
// of them, ~1.2 us of a ~3.7 us launch (probe on the box: a 33-launch decode
// GEMV set 124.7 us through k_gemv, 78.2 us through this form, 78.1 us for a
// kernel that only streams the same bytes).
//
// Item b: rows 8 b + 2 w + lane / 32; the 32 lanes of a half-wave read the row
// in steps of 128 floats, KU float4 per lane per batch, every load of a batch
// first.  The activation rows come from global memory (hot in L2: every
// workgroup reads them) into registers, so no LDS and no barrier; the RMS
// prologue's sum of squares comes from the same registers (each half-wave
// reads the whole row), reduced like the dot products.  Each output is a
// fixed-order sum: lane partials (4 floats at a time, batch after batch),
// then the DPP half-wave sum of gv_half_sum.
struct GvRowsTail {               // what the kernel needs only after its weight loads are issued
    int lda, ldc0, ldc1, ldc2;   // row strides (M > 1 only)
    const float *gain, *A2;      // RMS gain [K]; SwiGLU second operand (layout of A)
    const int *bsel;             // SEL: B is offset by bsel[0] * bstride
    long long bstride;
    const float *cgate;          // SEL: results scaled by cgate[0]
};

template <int MB, int KU, int PRO, int SEL>
__global__ __launch_bounds__(GV_T) void k_gemv_rows(const float *B, const float *A, int K, int nrows, int mbeta,
                                                    float *C0, float *C1, float *C2, int r12, GvRowsTail t)
{
    const int M = mbeta & 0xff, beta = mbeta >> 8, r1 = r12 & 0xffff, r2 = r12 >> 16;
    const int lane = threadIdx.x & 63, l = lane & 31;
    const int row = blockIdx.x * GV_NT_ROWS + (threadIdx.x >> 5);
    const int rowc = min(row, nrows - 1);
    const float *Bm = SEL ? B + (long long)*(const GAS int *)t.bsel * t.bstride : B;
    const float *Brow = Bm + (size_t)rowc * K;
    // activation row m (row 0 alone at MB = 1, so its stride is never read)
    auto arow = [&](int m) { return MB == 1 ? (size_t)0 : (size_t)min(m, M - 1) * t.lda; };
    constexpr int STEP = 128 * KU;
    float acc[MB], ss[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) acc[m] = ss[m] = 0.f;
    auto load_w = [&](f32x4 (&wv)[KU], int k0) {
#pragma unroll
        for (int u = 0; u < KU; u++) wv[u] = gv_ld<4>(Brow + min(k0 + 4 * (32 * u + l), K - 4));
    };
    auto use = [&](const f32x4 (&wv)[KU], int k0) {
        f32x4 av[MB][KU], gv[KU];
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const int k = min(k0 + 4 * (32 * u + l), K - 4);
#pragma unroll
            for (int m = 0; m < MB; m++) av[m][u] = gv_ld<4>(A + arow(m) + k);
            if (PRO == GV_PRO_RMS) gv[u] = gv_ld<4>(t.gain + k);
            if (PRO == GV_PRO_SWIGLU) {
#pragma unroll
                for (int m = 0; m < MB; m++) {
                    const f32x4 a2 = gv_ld<4>(t.A2 + arow(m) + k);
#pragma unroll
                    for (int v = 0; v < 4; v++) av[m][u][v] = gv_silu_mul(av[m][u][v], a2[v]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < KU; u++) {
            const bool ok = k0 + 4 * (32 * u + l) < K;
#pragma unroll
            for (int m = 0; m < MB; m++) {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    float a = ok ? av[m][u][v] : 0.f;
                    if (PRO == GV_PRO_RMS) {
                        ss[m] = fmaf(a, a, ss[m]);
                        a *= gv[u][v];
                    }
                    acc[m] = fmaf(a, wv[u][v], acc[m]);
                }
            }
        }
    };
    f32x4 wv[KU];
    load_w(wv, 0);
    if (K <= STEP) {
        use(wv, 0);
    } else {
        for (int k0 = 0; k0 < K; k0 += STEP) {          // the next batch in flight while this one is used
            f32x4 nw[KU];
            load_w(nw, min(k0 + STEP, K - 4));
            use(wv, k0);
#pragma unroll
            for (int u = 0; u < KU; u++) wv[u] = nw[u];
        }
    }
#pragma unroll
    for (int m = 0; m < MB; m++) {
        acc[m] = gv_half_sum(acc[m]);
        if (PRO == GV_PRO_RMS) ss[m] = gv_half_sum(ss[m]);
    }
    if (l == 31 && row < nrows) {
        const int s = (row >= r1) + (row >= r2);
        float *C = s == 0 ? C0 : s == 1 ? C1 : C2;
        const int col = row - (s == 0 ? 0 : s == 1 ? r1 : r2);
        const float cg = SEL && t.cgate ? *(const GAS float *)t.cgate : 1.0f;
#pragma unroll
        for (int m = 0; m < MB; m++)
            if (m < M) {
                float v = acc[m];
                if (PRO == GV_PRO_RMS) v *= 1.0f / sqrtf(ss[m] / (float)K + 1e-5f);
                v *= cg;
                float *out = C + col;
                if (MB > 1) out += (size_t)m * (s == 0 ? t.ldc0 : s == 1 ? t.ldc1 : t.ldc2);
                *out = beta ? *out + v : v;
            }
    }
}

// -------------------------------------------------- mm over one matrix --
// The reference layout's decode launch (W [in][out], the drop-in's mm at
// M <= 8): up to 3 problems over the same activation rows whose weights
// follow each other in memory (wq | wk | wv, w1 | w3 of map_weights), with
// the same scalar-argument design as k_gemv_rows (B, A, K, N0 | N1 << 16, N2,
// M | beta << 8, C0-C2 preloaded).  Workgroup b owns CB = 4
// CL columns of one segment over all K rows: CL lanes cover a row's 16 CL
// bytes, the RG = 256 / CL row groups of the workgroup take rows 4 (g + RG
// u4) + i (i < 4), so a lane reads 4 consecutive rows per step -- 4 weight
// float4 and, at M = 1, one activation float4 straight from global memory.
// At M > 1 the activation rows are staged in LDS ([k][MB]) behind one
// barrier.  Partial sums: per lane over its rows in order, then the RG row
// groups in LDS in a fixed order (NG groups of RG / NG, then the groups).
#define GV_COLS_K 1024                 // rows per launch at most (one batch of loads)

struct GvColsTail {
    int lda, ldc0, ldc1, ldc2;       // row strides (M > 1 only)
};

template <int MB, int CL, int U4, int TPB>
__global__ __launch_bounds__(TPB) void k_gemv_cols(const float *B, const float *A, int K, int N01, int N2, int mbeta,
                                                   float *C0, float *C1, float *C2, GvColsTail t)
{
    const int N0 = N01 & 0xffff, N1 = N01 >> 16, M = mbeta & 0xff, beta = (mbeta >> 8) & 1, pair = mbeta >> 16;
    constexpr int RG = TPB / CL, CB = 4 * CL, UF = 4 * U4;
    __shared__ __attribute__((aligned(16))) float act[MB > 1 ? GV_COLS_K * MB : 4];
    __shared__ __attribute__((aligned(16))) float red[RG][MB][CB];
    const int tid = threadIdx.x, c = tid % CL, g = tid / CL;
    // the workgroup's segment: blocks [0, nb0) of N0 columns, then N1, then N2
    const int nb0 = (N0 + CB - 1) / CB, nb1 = (N1 + CB - 1) / CB;
    int b = blockIdx.x, N = N0, seg = 0;
    if (pair) {
        // blocks 2p and 2p + 1 (the two halves of each 128-byte line) on
        // workgroups 16 (p / 8) + p % 8 and that + 8: the same XCD
        const int x = b & 7, i = b >> 3;
        b = (((i >> 1) << 3) + x) * 2 + (i & 1);
        if (b >= nb0 + nb1 + (N2 + CB - 1) / CB) return;
    }
    const float *Bs = B;
    if (b >= nb0) {
        b -= nb0; N = N1; seg = 1; Bs = B + (size_t)K * N0;
        if (b >= nb1) { b -= nb1; N = N2; seg = 2; Bs += (size_t)K * N1; }
    }
    const int j = b * CB + 4 * c;
    const float *Bc = Bs + min(j, N - 4);
    f32x4 wv[UF];
#pragma unroll
    for (int u = 0; u < UF; u++) wv[u] = gv_ld<4>(Bc + (size_t)min(4 * (g + RG * (u >> 2)) + (u & 3), K - 1) * N);
    __builtin_amdgcn_sched_barrier(0);                  // every weight load in flight before any is used
    float acc[MB][4];
#pragma unroll
    for (int m = 0; m < MB; m++)
#pragma unroll
        for (int v = 0; v < 4; v++) acc[m][v] = 0.f;
    if constexpr (MB == 1) {
        f32x4 xv[U4];
#pragma unroll
        for (int u4 = 0; u4 < U4; u4++) xv[u4] = gv_ld<4>(A + min(4 * (g + RG * u4), K - 4));
#pragma unroll
        for (int u = 0; u < UF; u++) {
            const float x = 4 * (g + RG * (u >> 2)) < K ? xv[u >> 2][u & 3] : 0.f;
#pragma unroll
            for (int v = 0; v < 4; v++) acc[0][v] = fmaf(x, wv[u][v], acc[0][v]);
        }
    } else {
        // activation rows [m][k] -> act[k][m]: thread t takes floats 4 t .. 4 t + 3 of every row
        for (int k4 = tid; 4 * k4 < K; k4 += TPB) {
            f32x4 xa[MB];
#pragma unroll
            for (int m = 0; m < MB; m++) xa[m] = gv_ld<4>(A + (size_t)min(m, M - 1) * t.lda + 4 * k4);
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int m4 = 0; m4 < MB; m4 += 4) {
                    f32x4 y;
#pragma unroll
                    for (int i = 0; i < 4; i++) y[i] = m4 + i < MB ? xa[min(m4 + i, MB - 1)][q] : 0.f;
                    if (MB >= 4) *reinterpret_cast<f32x4 *>(&act[(4 * k4 + q) * MB + m4]) = y;
                    else
#pragma unroll
                        for (int i = 0; i < MB; i++) act[(4 * k4 + q) * MB + i] = y[i];
                }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < UF; u++) {
            const int k = 4 * (g + RG * (u >> 2)) + (u & 3);
            const bool ok = k < K;
            const float *ak = &act[min(k, K - 1) * MB];
#pragma unroll
            for (int m = 0; m < MB; m++) {
                const float x = ok ? ak[m] : 0.f;
#pragma unroll
                for (int v = 0; v < 4; v++) acc[m][v] = fmaf(x, wv[u][v], acc[m][v]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MB; m++)
        *reinterpret_cast<f32x4 *>(&red[g][m][4 * c]) = f32x4{acc[m][0], acc[m][1], acc[m][2], acc[m][3]};
    __syncthreads();
    // the RG row groups: NG groups of RG / NG consecutive ones per output,
    // then the NG group sums in order
    constexpr int NO = CB * MB, NG = TPB / NO >= 1 ? TPB / NO : 1;
    float v = 0.f;
    const int o = tid % NO, grp = tid / NO, m = o / CB, cc = o % CB;
    if (grp < NG) {
        v = red[grp * (RG / NG)][m][cc];
#pragma unroll
        for (int q = 1; q < RG / NG; q++) v += red[grp * (RG / NG) + q][m][cc];
    }
    __syncthreads();
    if (grp < NG) (&red[0][0][0])[grp * NO + o] = v;
    __syncthreads();
    if (tid < NO) {
        float r = (&red[0][0][0])[tid];
#pragma unroll
        for (int q = 1; q < NG; q++) r += (&red[0][0][0])[q * NO + tid];
        const int jj = b * CB + cc;
        if (m < M && jj < N) {
            float *C = seg == 0 ? C0 : seg == 1 ? C1 : C2;
            float *out = C + jj;
            if (MB > 1) out += (size_t)m * (seg == 0 ? t.ldc0 : seg == 1 ? t.ldc1 : t.ldc2);
            *out = beta ? *out + r : r;
        }
    }
}

// ---------------------------------------------------------------- host --
bool tlg_gemv_fits(TlgKind kind, int Mo) { return kind != TLG_TN && Mo >= 1 && Mo <= 8; }

static int rows_bucket(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

static u64 *g_part;                 // GV_RING regions of GV_REGION_WORDS
static u32 *g_err;
static unsigned g_ring;
static char g_last_name[48] = "k_gemv";
// A dry run (tlg_gemv_describe) picks the kernel without allocating or
// launching and writes its name to g_name instead of g_last_name.
static bool g_dry = false;
static char *g_name = g_last_name;

int tlg_gemv_init(void)
{
    if (g_part) return TLG_OK;
    void *p = nullptr;
    const size_t bytes = GV_RING * GV_REGION_WORDS * sizeof(u64) + 256;
    if (hipMalloc(&p, bytes) != hipSuccess) return tlg_fail(TLG_ENOMEM, "GEMV workspace of %zu bytes", bytes);
    TLG_HIP(hipMemset(p, 0, bytes));
    TLG_HIP(hipDeviceSynchronize());
    g_part = (u64 *)p;
    g_err = (u32 *)((char *)p + GV_RING * GV_REGION_WORDS * sizeof(u64));
    g_ring = 0;
    return TLG_OK;
}

void tlg_gemv_release(void)
{
    if (g_part) (void)hipFree(g_part);
    g_part = nullptr;
    g_err = nullptr;
}

extern "C" int tlg_gemv_status(void)
{
    if (!g_err) return 0;
    u32 v = 0;
    if (hipMemcpy(&v, g_err, sizeof v, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    return (int)v;
}

// Rows per NN item: the launch's NN bytes over a target item count, in
// multiples of 16 rows (TLG_GEMV_ITEMS, TLG_GEMV_KS override for sweeps).
static int env_int(const char *name, int dflt)
{
    const char *e = getenv(name);
    return e && *e ? atoi(e) : dflt;
}

template <int MB, int VEC, int PRO>
static void launch_u(const GvArgs &a, int grid, int U, hipStream_t st)
{
    switch (U) {
    case 1: hipLaunchKernelGGL((k_gemv<MB, VEC, 1, PRO>), dim3(grid), dim3(GV_T), 0, st, a); break;
    case 2: hipLaunchKernelGGL((k_gemv<MB, VEC, 2, PRO>), dim3(grid), dim3(GV_T), 0, st, a); break;
    case 3: hipLaunchKernelGGL((k_gemv<MB, VEC, 3, PRO>), dim3(grid), dim3(GV_T), 0, st, a); break;
    default: hipLaunchKernelGGL((k_gemv<MB, VEC, 4, PRO>), dim3(grid), dim3(GV_T), 0, st, a); break;
    }
}
template <int MB>
static void launch_mb(const GvArgs &a, int grid, int vec, int U, int pro, hipStream_t st)
{
    if (vec == 1) { hipLaunchKernelGGL((k_gemv<MB, 1, 4, GV_PRO_NONE>), dim3(grid), dim3(GV_T), 0, st, a); return; }
    switch (pro) {
    case GV_PRO_RMS: launch_u<MB, 4, GV_PRO_RMS>(a, grid, U, st); break;
    case GV_PRO_SWIGLU: launch_u<MB, 4, GV_PRO_SWIGLU>(a, grid, U, st); break;
    default: launch_u<MB, 4, GV_PRO_NONE>(a, grid, U, st); break;
    }
}

static bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// k_gemv_rows: float4 batches per lane (KU) for a row of K floats at MB
// activation rows, within a register budget of 16 activation float4 per lane.
static int rows_ku(int K, int mb)
{
    const int cap = mb <= 2 ? 8 : mb == 4 ? 4 : 2;
    const int need = (K + 127) / 128;
    const int ku = need <= 1 ? 1 : need <= 2 ? 2 : need <= 3 ? 3 : need <= 4 ? 4 : 8;
    return min(ku, cap);
}

struct GvRowsArgs {
    const float *B, *A;
    int K, nrows, mbeta;
    float *C0, *C1, *C2;
    int r12;
    GvRowsTail t;
};

template <int MB, int KU, int SEL>
static void launch_rows_sel(int pro, int grid, const GvRowsArgs &r, hipStream_t st)
{
#define GV_ROWS_ARGS r.B, r.A, r.K, r.nrows, r.mbeta, r.C0, r.C1, r.C2, r.r12, r.t
    switch (pro) {
    case GV_PRO_RMS:
        hipLaunchKernelGGL((k_gemv_rows<MB, KU, GV_PRO_RMS, SEL>), dim3(grid), dim3(GV_T), 0, st, GV_ROWS_ARGS);
        break;
    case GV_PRO_SWIGLU:
        hipLaunchKernelGGL((k_gemv_rows<MB, KU, GV_PRO_SWIGLU, SEL>), dim3(grid), dim3(GV_T), 0, st, GV_ROWS_ARGS);
        break;
    default:
        hipLaunchKernelGGL((k_gemv_rows<MB, KU, GV_PRO_NONE, SEL>), dim3(grid), dim3(GV_T), 0, st, GV_ROWS_ARGS);
        break;
    }
#undef GV_ROWS_ARGS
}
template <int MB, int KU>
static void launch_rows_ku(int sel, int pro, int grid, const GvRowsArgs &r, hipStream_t st)
{
    if constexpr (MB == 1) {
        if (sel) { launch_rows_sel<MB, KU, 1>(pro, grid, r, st); return; }
    }
    launch_rows_sel<MB, KU, 0>(pro, grid, r, st);
}
template <int MB>
static void launch_rows_mb(int ku, int sel, int pro, int grid, const GvRowsArgs &r, hipStream_t st)
{
    switch (ku) {
    case 1: launch_rows_ku<MB, 1>(sel, pro, grid, r, st); break;
    case 2: launch_rows_ku<MB, 2>(sel, pro, grid, r, st); break;
    case 3:
        if constexpr (MB <= 4) launch_rows_ku<MB, 3>(sel, pro, grid, r, st);
        break;
    case 4:
        if constexpr (MB <= 4) launch_rows_ku<MB, 4>(sel, pro, grid, r, st);
        break;
    default:
        if constexpr (MB <= 2) launch_rows_ku<MB, 8>(sel, pro, grid, r, st);
        break;
    }
}

// The launch as one matrix (k_gemv_rows) when every problem is an mm_bt over
// the same activation rows (same prologue operands, beta, weight selection
// and gate), 16-byte aligned rows of a multiple of 4 floats, and each
// problem's weight rows directly follow the previous problem's.  Weight
// selection and gate (the MoE decode rows) only at M = 1.  Returns 1 when
// launched, 0 when the launch needs the general kernel.
static int launch_rows(const GvArgs &a, int pro, hipStream_t st)
{
    if (a.nprob < 1 || a.nprob > 3 || env_int("TLG_GEMV_ROWS", 1) == 0) return 0;
    const GvProb &P0 = a.p[0];
    const GvSeg &g0 = P0.seg[0];
    const int K = g0.R;
    if (P0.kind != TLG_NT || P0.nseg != 1 || K % 4 || g0.lda % 4 || g0.ldb != K || !al16(g0.A) || !al16(g0.B))
        return 0;
    if (pro == GV_PRO_RMS && !al16(P0.gain)) return 0;
    if (pro == GV_PRO_SWIGLU && !al16(P0.A2)) return 0;
    const int sel = P0.bsel || P0.cgate;
    if (sel && (P0.M != 1 || !P0.bsel || P0.bstride % 4)) return 0;
    const float *next = g0.B + (size_t)P0.No * K;
    for (int i = 1; i < a.nprob; i++) {
        const GvProb &P = a.p[i];
        const GvSeg &g = P.seg[0];
        if (P.kind != TLG_NT || P.nseg != 1 || g.R != K || g.lda != g0.lda || g.ldb != K || g.A != g0.A ||
            g.B != next || P.M != P0.M || P.beta != P0.beta || P.gain != P0.gain || P.A2 != P0.A2 ||
            P.bsel != P0.bsel || P.bstride != P0.bstride || P.cgate != P0.cgate)
            return 0;
        next += (size_t)P.No * K;
    }
    GvRowsArgs r;
    memset(&r, 0, sizeof r);
    float *C[3] = {P0.C, P0.C, P0.C};
    int ldc[3] = {P0.ldc, P0.ldc, P0.ldc}, rs[3] = {0, 0, 0}, n = 0;
    for (int i = 0; i < a.nprob; i++) {
        rs[i] = n;
        C[i] = a.p[i].C;
        ldc[i] = a.p[i].ldc;
        n += a.p[i].No;
    }
    if (n >= 0xffff) return 0;                       // r1, r2 in 16 bits each
    r.B = g0.B; r.A = g0.A; r.K = K; r.nrows = n; r.mbeta = P0.M | (P0.beta ? 1 : 0) << 8;
    r.C0 = C[0]; r.C1 = C[1]; r.C2 = C[2];
    // segments past the last start at nrows, so no row selects them
    r.r12 = (a.nprob > 1 ? rs[1] : n) | (a.nprob > 2 ? rs[2] : n) << 16;
    r.t.lda = g0.lda;
    r.t.ldc0 = ldc[0]; r.t.ldc1 = ldc[1]; r.t.ldc2 = ldc[2];
    r.t.gain = P0.gain; r.t.A2 = P0.A2; r.t.bsel = P0.bsel; r.t.bstride = P0.bstride; r.t.cgate = P0.cgate;
    const int mb = rows_bucket(P0.M), ku = rows_ku(K, mb);
    const int grid = (n + GV_NT_ROWS - 1) / GV_NT_ROWS;
    if (!g_dry) switch (mb) {
    case 1: launch_rows_mb<1>(ku, sel, pro, grid, r, st); break;
    case 2: launch_rows_mb<2>(ku, sel, pro, grid, r, st); break;
    case 4: launch_rows_mb<4>(ku, sel, pro, grid, r, st); break;
    default: launch_rows_mb<8>(ku, sel, pro, grid, r, st); break;
    }
    snprintf(g_name, sizeof g_last_name, "k_gemv_rows<%d, %d, %d, %d>", mb, ku, pro, sel);
    return 1;
}

template <int MB, int CL, int TPB>
static void launch_cols_cl(int u4, int grid, int pair, const float *B, const float *A, int K, const int *N, int M,
                           int beta, float *const *C, const GvColsTail &t, hipStream_t st)
{
#define GV_COLS(U4)                                                                                      \
    hipLaunchKernelGGL((k_gemv_cols<MB, CL, U4, TPB>), dim3(grid), dim3(TPB), 0, st, B, A, K,              \
                       N[0] | N[1] << 16, N[2], M | (beta ? 1 : 0) << 8 | pair << 16, C[0], C[1], C[2], t)
    switch (u4) {
    case 1: GV_COLS(1); break;
    case 2: GV_COLS(2); break;
    case 3: GV_COLS(3); break;
    case 4: GV_COLS(4); break;
    default:
        if constexpr (TPB / CL == 32) GV_COLS(8);
        break;
    }
#undef GV_COLS
}

// The launch as one matrix in the reference layout (k_gemv_cols): every
// problem an mm over the same activation rows with no prologue, weight
// selection or gate, dense rows (ldb = N) of a multiple of 4 floats, K <=
// GV_COLS_K, and each problem's weight matrix directly after the previous
// one.  Returns 1 when launched, 0 when the launch needs the general kernel.
static int launch_cols(const GvArgs &a, int pro, hipStream_t st)
{
    if (a.nprob < 1 || a.nprob > 3 || pro != GV_PRO_NONE || env_int("TLG_GEMV_ROWS", 1) == 0) return 0;
    const GvProb &P0 = a.p[0];
    const GvSeg &g0 = P0.seg[0];
    const int K = g0.R;
    if (K % 4 || K > GV_COLS_K || g0.lda % 4 || !al16(g0.A) || !al16(g0.B)) return 0;
    const float *next = g0.B;
    int N[3] = {0, 0, 0}, ldc[3] = {0, 0, 0}, nb = 0;
    float *C[3] = {P0.C, P0.C, P0.C};
    const int cle = env_int("TLG_GEMV_CL", 4), CL = cle == 8 ? 8 : cle == 2 ? 2 : 4, CB = 4 * CL;
    for (int i = 0; i < a.nprob; i++) {
        const GvProb &P = a.p[i];
        const GvSeg &g = P.seg[0];
        if (P.kind != TLG_NN || P.nseg != 1 || g.R != K || g.A != g0.A || g.lda != g0.lda || g.B != next ||
            g.ldb != P.No || P.No % 4 || P.M != P0.M || P.beta != P0.beta || P.bsel || P.cgate)
            return 0;
        next += (size_t)K * P.No;
        N[i] = P.No; C[i] = P.C; ldc[i] = P.ldc;
        nb += (P.No + CB - 1) / CB;
    }
    if (N[0] >= 0x10000 || N[1] >= 0x8000) return 0;    // N0, N1 in 16 bits each
    GvColsTail t = {g0.lda, ldc[0], ldc[1], ldc[2]};
    const int tpb = env_int("TLG_GEMV_TPB", 256) == 128 ? 128 : 256;
    const int RG = tpb / CL, need = (K + 4 * RG - 1) / (4 * RG);
    if (need > 4 && (need > 8 || RG != 32)) return 0;    // instances: U4 <= 4, and 8 at 32 row groups
    const int u4 = need <= 1 ? 1 : need <= 2 ? 2 : need <= 3 ? 3 : need <= 4 ? 4 : 8;
    const int mb = rows_bucket(P0.M);
    const int pair = CL < 8 && env_int("TLG_GEMV_PAIR", 1) ? 1 : 0;
    const int grid = pair ? (nb + 15) / 16 * 16 : nb;
#define GV_COLS_MB(MB)                                                                                     \
    (tpb == 128 ? (CL == 8   ? launch_cols_cl<MB, 8, 128>(u4, grid, pair, g0.B, g0.A, K, N, P0.M, P0.beta, C, t, st)  \
                   : CL == 4 ? launch_cols_cl<MB, 4, 128>(u4, grid, pair, g0.B, g0.A, K, N, P0.M, P0.beta, C, t, st)  \
                             : launch_cols_cl<MB, 2, 128>(u4, grid, pair, g0.B, g0.A, K, N, P0.M, P0.beta, C, t, st)) \
                : (CL == 8   ? launch_cols_cl<MB, 8, 256>(u4, grid, pair, g0.B, g0.A, K, N, P0.M, P0.beta, C, t, st)  \
                   : CL == 4 ? launch_cols_cl<MB, 4, 256>(u4, grid, pair, g0.B, g0.A, K, N, P0.M, P0.beta, C, t, st)  \
                             : launch_cols_cl<MB, 2, 256>(u4, grid, pair, g0.B, g0.A, K, N, P0.M, P0.beta, C, t, st)))
    if (!g_dry) switch (mb) {
    case 1: GV_COLS_MB(1); break;
    case 2: GV_COLS_MB(2); break;
    case 4: GV_COLS_MB(4); break;
    default: GV_COLS_MB(8); break;
    }
#undef GV_COLS_MB
    snprintf(g_name, sizeof g_last_name, "k_gemv_cols<%d, %d, %d, %d>", mb, CL, u4, tpb);
    return 1;
}

// Decompose the problems, pick the instance and launch.  pro is the launch's
// prologue (every problem shares it).
static int launch(GvArgs &a, int pro, hipStream_t st)
{
    if (!g_dry) {
        int rc = tlg_gemv_init();
        if (rc) return rc;
    }
    if (launch_rows(a, pro, st) || launch_cols(a, pro, st)) {
        if (!g_dry) TLG_HIP(hipGetLastError());
        return TLG_OK;
    }
    int mb = 1, vec = 4;
    for (int i = 0; i < a.nprob; i++) {
        GvProb &P = a.p[i];
        mb = max(mb, rows_bucket(P.M));
        bool v4 = true;
        for (int s = 0; s < P.nseg; s++) {
            const GvSeg &g = P.seg[s];
            if (P.kind == TLG_NN) v4 = v4 && P.No % 4 == 0 && g.ldb % 4 == 0 && al16(g.B);
            else v4 = v4 && g.R % 4 == 0 && g.lda % 4 == 0 && g.ldb % 4 == 0 && al16(g.A) && al16(g.B);
        }
        if (P.bsel) v4 = v4 && P.bstride % 4 == 0;
        if (pro == GV_PRO_SWIGLU) v4 = v4 && al16(P.A2);
        if (pro == GV_PRO_RMS) v4 = v4 && al16(P.gain);
        if (pro != GV_PRO_NONE) v4 = v4 && P.seg[0].R % 4 == 0 && P.seg[0].lda % 4 == 0 && al16(P.seg[0].A);
        if (!v4) vec = 1;
    }
    if (vec == 1 && pro != GV_PRO_NONE)
        return tlg_fail(TLG_EINVAL, "dec_gemv: prologue operands need 16-byte aligned rows of 4k floats");
    const int CB = 16 * vec;
    // full-K items where the activation fits LDS (TLG_GEMV_SPLIT=1 forces
    // the split form, for sweeps)
    const int force_split = env_int("TLG_GEMV_SPLIT", 0);
    for (int i = 0; i < a.nprob; i++) {
        GvProb &P = a.p[i];
        const GvSeg &g = P.seg[0];
        P.full = P.kind == TLG_NN && vec == 4 && !force_split && g.R % 4 == 0 && g.lda % 4 == 0 && al16(g.A) &&
                 g.R <= GV_FULL_K && (long long)g.R * mb <= GV_FULL_ACT;
    }
    // rows per split NN item: the split problems' bytes over a target item
    // count, in multiples of 16 rows (TLG_GEMV_ITEMS, TLG_GEMV_KS override)
    double nn_bytes = 0;
    int nt_items = 0, maxr_nt = 0, maxr_nn = 0;
    bool any_split = false;
    for (int i = 0; i < a.nprob; i++) {
        GvProb &P = a.p[i];
        if (P.kind == TLG_NN && !P.full) {
            nn_bytes += 4.0 * P.seg[0].R * ((P.No + CB - 1) / CB) * CB;
            maxr_nn = max(maxr_nn, P.seg[0].R);
            any_split = true;
        } else if (P.kind == TLG_NT) {
            nt_items += (P.No + GV_NT_ROWS - 1) / GV_NT_ROWS;
            for (int s = 0; s < P.nseg; s++) maxr_nt = max(maxr_nt, P.seg[s].R);
        }
    }
    const int target = max(64, env_int("TLG_GEMV_ITEMS", 512) - nt_items);
    int KS = env_int("TLG_GEMV_KS", 0);
    if (KS <= 0) {
        const double rows = nn_bytes / target / (4.0 * CB);
        KS = 16 * max(1, (int)(rows / 16 + 0.5));
    }
    // at most 64 / M slices per column block: the reducer then reads at most
    // 16 words per output and thread
    const int smax = max(4, 64 / mb);
    if (maxr_nn > (long long)smax * KS) KS = (maxr_nn + smax - 1) / smax;
    KS = (KS + 15) / 16 * 16;
    for (;;) {
        size_t words = 0;
        for (int i = 0; i < a.nprob; i++) {
            GvProb &P = a.p[i];
            if (P.kind != TLG_NN || P.full) continue;
            P.nb = (P.No + CB - 1) / CB;
            P.KS = KS;
            P.S = (P.seg[0].R + KS - 1) / KS;
            if (P.S > 1) words += (size_t)P.nb * P.S * P.M * CB;
        }
        if (words <= GV_REGION_WORDS) break;
        KS *= 2;
    }
    long long off = 0;
    int grid = 0;
    for (int i = 0; i < a.nprob; i++) {
        GvProb &P = a.p[i];
        if (P.full) {
            P.nb = (P.No + 31) / 32;
            P.S = 1; P.KS = P.seg[0].R; P.part = 0;
            P.direct = P.nb;
            P.reducers = 0;
        } else if (P.kind == TLG_NN) {
            P.part = off;
            if (P.S > 1) off += (long long)P.nb * P.S * P.M * CB;
            P.reducers = P.S > 1 ? P.nb : 0;
            P.direct = P.nb * P.S - P.reducers;
        } else {
            P.nb = (P.No + GV_NT_ROWS - 1) / GV_NT_ROWS;
            P.S = 1; P.KS = 0; P.part = 0;
            P.direct = P.nb; P.reducers = 0;
        }
        grid += P.direct + P.reducers;
    }
    if (grid == 0) return TLG_OK;
    if (!g_dry) {
        a.part = g_part + (size_t)(g_ring++ % GV_RING) * GV_REGION_WORDS;
        a.err = g_err;
    }
    // batch depth of the split mm and mm_bt paths (full-K items use their own)
    int U = 4;
    if (vec == 4) {
        int maxr_full = 0;
        for (int i = 0; i < a.nprob; i++) if (a.p[i].full) maxr_full = max(maxr_full, a.p[i].seg[0].R);
        const int u_nn = any_split ? min(4, KS / 16) : 0;
        const int u_nt = maxr_nt ? min(4, (maxr_nt + 127) / 128) : 0;
        const int u_full = maxr_full > 512 ? 2 : maxr_full ? 1 : 0;     // full-K batches: min(U, 2)
        U = max(1, max(u_full, max(u_nn, u_nt)));
    }
    snprintf(g_name, sizeof g_last_name, "k_gemv<%d, %d, %d, %d>", mb, vec, vec == 1 ? 4 : U, vec == 1 ? 0 : pro);
    if (g_dry) return TLG_OK;
    switch (mb) {
    case 1: launch_mb<1>(a, grid, vec, U, pro, st); break;
    case 2: launch_mb<2>(a, grid, vec, U, pro, st); break;
    case 4: launch_mb<4>(a, grid, vec, U, pro, st); break;
    default: launch_mb<8>(a, grid, vec, U, pro, st); break;
    }
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

// The instance name of the last launch, as rocprofv3 prints it.
const char *tlg_gemv_kernel_name(int M)
{
    (void)M;
    return g_last_name;
}

// The instance a single device call (the drop-in's mm / mm_bt at M <= 8,
// operands as tlg_gemv_launch receives them from the C ABI: 16-byte aligned,
// dense rows) would launch, without launching it.
void tlg_gemv_describe(TlgKind kind, int Mo, int No, int R, char *buf, int len)
{
    GvArgs a;
    memset(&a, 0, sizeof a);
    GvProb &P = a.p[0];
    float *const any = (float *)(uintptr_t)256;       // aligned stand-in, never dereferenced
    P.C = any; P.kind = kind; P.M = Mo; P.No = No; P.ldc = No; P.beta = kind == TLG_NT; P.nseg = 1;
    P.seg[0] = GvSeg{any, any, R, R, kind == TLG_NN ? No : R};
    a.nprob = 1;
    char name[48];
    g_dry = true;
    g_name = name;
    snprintf(name, sizeof name, "k_gemv");
    (void)launch(a, GV_PRO_NONE, 0);
    g_dry = false;
    g_name = g_last_name;
    snprintf(buf, (size_t)len, "%s", name);
}

int tlg_gemv_launch(TlgKind kind, const float *A, const float *B, float *C, int Mo, int No, int R, int lda,
                    int ldb, int ldc, int beta, hipStream_t st)
{
    GvArgs a;
    memset(&a, 0, sizeof a);
    GvProb &P = a.p[0];
    P.C = C; P.kind = kind; P.M = Mo; P.No = No; P.ldc = ldc; P.beta = beta; P.nseg = 1;
    P.seg[0] = GvSeg{A, B, R, lda, ldb};
    a.nprob = 1;
    return launch(a, GV_PRO_NONE, st);
}

// A grouped launch whose calls are all mm / mm_bt at M <= 8 (decode runs).
int tlg_gemv_group_launch(const TlgGemmCall *calls, int n, hipStream_t st)
{
    if (n > GV_MAXPROB) return tlg_fail(TLG_EINVAL, "GEMV group: at most %d calls", GV_MAXPROB);
    GvArgs a;
    memset(&a, 0, sizeof a);
    for (int i = 0; i < n; i++) {
        const TlgGemmCall &c = calls[i];
        GvProb &P = a.p[i];
        P.C = c.C;
        P.M = c.M;
        P.nseg = c.nseg;
        if (c.op == 0) {
            P.kind = TLG_NN; P.No = c.N; P.ldc = c.N; P.beta = 0;
            P.seg[0] = GvSeg{c.A[0], c.B[0], c.K, c.K, c.N};
        } else {
            P.kind = TLG_NT; P.No = c.K; P.ldc = c.K; P.beta = c.beta ? 1 : 0;
            for (int s = 0; s < c.nseg; s++) {
                const int Ns = s ? c.Nseg[s] : c.N;
                P.seg[s] = GvSeg{c.A[s], c.B[s], Ns, Ns, Ns};
            }
        }
        for (int s = 0; s < P.nseg; s++)
            if (!P.seg[s].A || !P.seg[s].B || P.seg[s].R <= 0)
                return tlg_fail(TLG_EINVAL, "GEMV group: call %d: empty or NULL operand", i);
        if (!P.C || P.No <= 0) return tlg_fail(TLG_EINVAL, "GEMV group: call %d: empty output", i);
    }
    a.nprob = n;
    return launch(a, GV_PRO_NONE, st);
}

// A decode run with the glue folded in (include/tldecode.h): the calls'
// prologues (RMSNorm, SwiGLU) apply as the activation rows are read, and
// beta = 1 adds the result into C (mm's residual add).  Calls with different
// prologues go to separate launches, one per prologue, in call order.
extern "C" int tlg_dev_dec_gemv(const TlgDecGemv *calls, int n, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (!calls || n <= 0 || n > GV_MAXPROB) return tlg_fail(TLG_EINVAL, "dec_gemv: 1 to %d calls", GV_MAXPROB);
    hipStream_t st = (hipStream_t)stream;
    for (int i = 0; i < n; i++) {
        const TlgDecGemv &c = calls[i];
        const int R = c.op == 0 ? c.K : c.N;
        if ((c.op != 0 && c.op != 1) || c.M < 1 || c.M > 8 || c.K <= 0 || c.N <= 0 || !c.A || !c.B || !c.C ||
            c.pro < GV_PRO_NONE || c.pro > GV_PRO_SWIGLU || (c.pro == GV_PRO_RMS && !c.gain) ||
            (c.pro == GV_PRO_SWIGLU && !c.A2) || (c.pro != GV_PRO_NONE && (R % 4 || !al16(c.A))))
            return tlg_fail(TLG_EINVAL, "dec_gemv: call %d: op=%d M=%d K=%d N=%d pro=%d", i, c.op, c.M, c.K, c.N,
                            c.pro);
    }
    rc = tlg_group_flush_launch(st);             // pending split reductions land first
    if (rc) return rc;
    for (int pro = GV_PRO_NONE; pro <= GV_PRO_SWIGLU; pro++) {
        GvArgs a;
        memset(&a, 0, sizeof a);
        for (int i = 0; i < n; i++) {
            const TlgDecGemv &c = calls[i];
            if (c.pro != pro) continue;
            GvProb &P = a.p[a.nprob++];
            P.C = c.C;
            P.M = c.M;
            P.nseg = 1;
            P.beta = c.beta ? 1 : 0;
            P.gain = c.gain;
            P.A2 = c.A2;
            P.bsel = c.bsel;
            P.bstride = c.bsel ? c.bstride : 0;
            P.cgate = c.cgate;
            if (c.op == 0) {
                P.kind = TLG_NN; P.No = c.N; P.ldc = c.N;
                P.seg[0] = GvSeg{c.A, c.B, c.K, c.K, c.N};
            } else {
                P.kind = TLG_NT; P.No = c.K; P.ldc = c.K;
                P.seg[0] = GvSeg{c.A, c.B, c.N, c.N, c.N};
            }
        }
        if (a.nprob) {
            rc = launch(a, pro, st);
            if (rc) return rc;
        }
    }
    return TLG_OK;
}
