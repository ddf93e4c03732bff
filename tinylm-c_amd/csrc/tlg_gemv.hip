// tlg_gemv.hip -- the M <= 8 forms of mm and mm_bt (KV-cache decode) on gfx950.
//
// At M <= 8 rows a GEMM is a matrix-vector product: every weight is used M
// times, so the work is one pass over the weight matrix and its speed is set
// by how many bytes per cycle the CUs pull from HBM.  MFMA tiles would waste
// 24/32 of every block and stage weights through LDS for nothing; these
// kernels stream the weights once, straight from global memory into FMAs.
// The M activation rows are staged in LDS (4096 floats at a time), and each
// workgroup spreads its reduction over many row slots so that every lane has
// several weight loads in flight: a few microseconds of memory latency, not
// a chain of dependent loads, bounds a launch.
//
//   mm     Y[m][j] = sum_k X[m][k] W[k][j]       W rows are contiguous along
//          the output index j: a workgroup owns 8 or 16 columns, as many
//          lanes read one contiguous row segment, and the workgroup's 64 or
//          32 row slots walk down W together.  The partial sums of a column
//          meet in fixed order (shuffles, then LDS).
//   mm_bt  dX[m][k] += sum_n dY[m][n] W[k][n]    W rows are contiguous along
//          the reduction index n: a wave owns 2 W rows, its lanes stride n
//          (coalesced), and each of the 2*M dot products ends in a butterfly
//          reduction over the 64 lanes.
//
// Reference: mm tinylm.c:438-449 (serial at M <= 4 through tl_for, :444-446),
// mm_bt :480-489; the decode GEMV sites of forward_chunk :3748-3824 and the
// head :3035.  Several GEMVs that the reference issues back to back (q, k, v
// on the same input; w1, w3) run as one launch: a problem table in the
// kernel arguments, workgroups dealt to problems in order.
#include "tlg_internal.h"
#include "../../include/tldecode.h"
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define GV_WAVES 8              // waves per workgroup (512 threads)
#define GV_NT_ROWS 2            // mm_bt: W rows per wave
#define GV_ACHUNK 4096          // floats of the activation rows staged in LDS at a time
#define NN_U 16                 // mm: weight rows per lane per batch of loads
#define NT_U 8                  // mm_bt: reduction steps per lane per batch of loads
#define GV_MAXPROB 8
#define GV_MAXSEG 3

// mm: output columns per workgroup.  Narrower column blocks give more
// workgroups (more loads in flight across the chip) at the cost of shorter
// row segments; measured on MI355X, 8 is best at M <= 2 and 16 above.
__host__ __device__ constexpr int nn_cols(int mb) { return mb <= 2 ? 8 : 16; }

struct GvSeg { const float *A, *B; int R, lda, ldb; };
// Activation prologues (decode: the glue before a GEMV, applied while the
// rows are staged): GV_PRO_RMS stages x * s * gain with s = 1 / sqrt(sum(x^2)
// / R + 1e-5) of the whole row (rmsnorm_fwd, tinylm.c:540-548); GV_PRO_SWIGLU
// stages silu(a) * a2 with silu(z) = z / (1 + e^-z) (:786, :1005-1006).
enum { GV_PRO_NONE = 0, GV_PRO_RMS = 1, GV_PRO_SWIGLU = 2 };
struct GvProb {
    float *C;
    int kind;                    // TLG_NN or TLG_NT
    int M, No, ldc, beta, nseg;
    int blocks;
    int pro;                     // GV_PRO_* (single-segment problems only)
    const float *gain, *A2;      // RMS gain [R]; SwiGLU second operand (layout of A)
    GvSeg seg[GV_MAXSEG];
};
struct GvArgs {
    int nprob;
    GvProb p[GV_MAXPROB];
};

// Stage activation rows A[m][r0 .. r0+kc) (m < M) into LDS as As[m*kc + r-r0],
// through the problem's prologue: SwiGLU completes here; RMSNorm stages the
// raw rows and its gain (Gs) in the same pass -- one global round trip --
// and rms_finish applies the scales.
__device__ __forceinline__ void stage_rows(float *As, float *Gs, const GvProb &P, const GvSeg &g, int r0, int kc)
{
    for (int e = threadIdx.x; e < P.M * kc; e += blockDim.x) {
        const int m = e / kc, r = e - m * kc;
        const size_t i = (size_t)m * g.lda + r0 + r;
        float a = g.A[i];
        if (P.pro == GV_PRO_SWIGLU) a = a / (1.0f + expf(-a)) * P.A2[i];
        else if (P.pro == GV_PRO_RMS && m == 0) Gs[r] = P.gain[r0 + r];
        As[e] = a;
    }
}

// RMSNorm of the staged rows (the whole row is in LDS: M * R <= GV_ACHUNK):
// s_m = 1 / sqrt(sum_k x^2 / R + 1e-5), one wave per row (M <= GV_WAVES),
// then x * s_m * gain in place.
__device__ __forceinline__ void rms_finish(float *As, const float *Gs, float *rsc, int M, int R)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (w < M) {
        float ms = 0.f;
        for (int k = lane; k < R; k += 64) ms = fmaf(As[w * R + k], As[w * R + k], ms);
        for (int o = 32; o > 0; o >>= 1) ms += __shfl_xor(ms, o);
        if (lane == 0) rsc[w] = 1.0f / sqrtf(ms / (float)R + 1e-5f);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < M * R; e += blockDim.x) {
        const int m = e / R, r = e - m * R;
        As[e] = As[e] * rsc[m] * Gs[r];
    }
}

// mm form.  Workgroup `blk` owns output columns [COLS blk, COLS blk + COLS).
// Lane (c = lane % COLS, sub = lane / COLS) of wave w reads column c of W
// rows k = q, q + SLOTS, q + 2 SLOTS, ... with q = (64 / COLS) w + sub: COLS
// lanes cover 4 COLS contiguous bytes of a row, and the workgroup's SLOTS row
// slots move through W together.  The partial sums of a column meet in fixed
// order (shuffles within a wave, then LDS across waves).
template <int MB, int COLS>
__device__ __forceinline__ void gemv_nn(const GvProb &P, int blk, float *As, float *red, float *rsc, float *Gs)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    constexpr int SUBS = 64 / COLS, SLOTS = GV_WAVES * SUBS;
    const int c = lane % COLS, q = w * SUBS + lane / COLS;
    const int j = blk * COLS + c;
    const int jc = j < P.No ? j : P.No - 1;      // in-bounds address for edge lanes
    float acc[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) acc[m] = 0.f;
    for (int s = 0; s < P.nseg; s++) {
        const GvSeg &g = P.seg[s];
        const float *__restrict__ Bp = g.B + jc;
        const int kc = GV_ACHUNK / P.M;
        for (int r0 = 0; r0 < g.R; r0 += kc) {
            const int kn = min(kc, g.R - r0);
            // rows k = q + SLOTS u of this chunk, in batches of NN_U: every load
            // of a batch is issued before any is used (rows past the chunk
            // read a clamped address and are zeroed), and the next batch is
            // in flight while the current one is consumed
            float b[NN_U], nb[NN_U];
            auto load = [&](float (&v)[NN_U], int k) {
#pragma unroll
                for (int u = 0; u < NN_U; u++) {
                    const int kk = k + SLOTS * u;
                    const float x = Bp[(size_t)(r0 + min(kk, kn - 1)) * g.ldb];
                    v[u] = kk < kn ? x : 0.f;
                }
            };
            load(b, q);
            __syncthreads();                     // previous chunk fully read
            stage_rows(As, Gs, P, g, r0, kn);
            __syncthreads();
            if (P.pro == GV_PRO_RMS) {
                rms_finish(As, Gs, rsc, P.M, kn);
                __syncthreads();
            }
            for (int k = q; k < kn; k += SLOTS * NN_U) {
                if (k + SLOTS * NN_U < kn) load(nb, k + SLOTS * NN_U);
#pragma unroll
                for (int m = 0; m < MB; m++)
                    if (m < P.M)
#pragma unroll
                        for (int u = 0; u < NN_U; u++)
                            acc[m] = fmaf(As[m * kn + min(k + SLOTS * u, kn - 1)], b[u], acc[m]);
#pragma unroll
                for (int u = 0; u < NN_U; u++) b[u] = nb[u];
            }
        }
    }
    // the 4 row slots of a wave, then the 8 waves, in fixed order
#pragma unroll
    for (int m = 0; m < MB; m++) {
#pragma unroll
        for (int o = COLS; o < 64; o <<= 1) acc[m] += __shfl_xor(acc[m], o);
    }
    if (lane < COLS)
#pragma unroll
        for (int m = 0; m < MB; m++) red[(w * MB + m) * COLS + lane] = acc[m];
    __syncthreads();
    const int t = threadIdx.x;
    if (t < COLS * MB) {
        const int m = t / COLS, cc = t % COLS, jj = blk * COLS + cc;
        if (m < P.M && jj < P.No) {
            float v = red[m * COLS + cc];
#pragma unroll
            for (int ww = 1; ww < GV_WAVES; ww++) v += red[(ww * MB + m) * COLS + cc];
            float *o = P.C + (size_t)m * P.ldc + jj;
            *o = P.beta ? *o + v : v;
        }
    }
}

// mm_bt form.  Wave w of workgroup `blk` owns W rows k0, k0 + 1; its lanes
// stride the reduction index n (coalesced), and each of the 2*M dot
// products ends in a butterfly reduction over the 64 lanes.
template <int MB>
__device__ __forceinline__ void gemv_nt(const GvProb &P, int blk, float *As, float *rsc, float *Gs)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int k0 = (blk * GV_WAVES + w) * GV_NT_ROWS;
    float acc[GV_NT_ROWS][MB];
#pragma unroll
    for (int r = 0; r < GV_NT_ROWS; r++)
#pragma unroll
        for (int m = 0; m < MB; m++) acc[r][m] = 0.f;
    for (int s = 0; s < P.nseg; s++) {
        const GvSeg &g = P.seg[s];
        const float *brow[GV_NT_ROWS];
#pragma unroll
        for (int r = 0; r < GV_NT_ROWS; r++) brow[r] = g.B + (size_t)min(k0 + r, P.No - 1) * g.ldb;
        const int kc = GV_ACHUNK / P.M;
        for (int r0 = 0; r0 < g.R; r0 += kc) {
            const int kn = min(kc, g.R - r0);
            // n = lane + 64 u in batches of NT_U, issued ahead as in gemv_nn
            float b[GV_NT_ROWS][NT_U], nb[GV_NT_ROWS][NT_U];
            auto load = [&](float (&v)[GV_NT_ROWS][NT_U], int n) {
#pragma unroll
                for (int r = 0; r < GV_NT_ROWS; r++)
#pragma unroll
                    for (int u = 0; u < NT_U; u++) {
                        const int nn = n + 64 * u;
                        const float x = brow[r][r0 + min(nn, kn - 1)];
                        v[r][u] = nn < kn ? x : 0.f;
                    }
            };
            load(b, lane);
            __syncthreads();
            stage_rows(As, Gs, P, g, r0, kn);
            __syncthreads();
            if (P.pro == GV_PRO_RMS) {
                rms_finish(As, Gs, rsc, P.M, kn);
                __syncthreads();
            }
            for (int n = lane; n < kn; n += 64 * NT_U) {
                if (n + 64 * NT_U < kn) load(nb, n + 64 * NT_U);
#pragma unroll
                for (int m = 0; m < MB; m++)
                    if (m < P.M)
#pragma unroll
                        for (int u = 0; u < NT_U; u++) {
                            const float a = As[m * kn + min(n + 64 * u, kn - 1)];
#pragma unroll
                            for (int r = 0; r < GV_NT_ROWS; r++) acc[r][m] = fmaf(a, b[r][u], acc[r][m]);
                        }
#pragma unroll
                for (int r = 0; r < GV_NT_ROWS; r++)
#pragma unroll
                    for (int u = 0; u < NT_U; u++) b[r][u] = nb[r][u];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < GV_NT_ROWS; r++)
#pragma unroll
        for (int m = 0; m < MB; m++) {
            float v = acc[r][m];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
            acc[r][m] = v;
        }
    if (lane < GV_NT_ROWS * MB) {
        // lane (r, m) writes output (m, k0 + r); select its value without
        // indexing the register array by a lane-dependent index
        const int r = lane / MB, m = lane % MB;
        float v = 0.f;
#pragma unroll
        for (int rr = 0; rr < GV_NT_ROWS; rr++)
#pragma unroll
            for (int mm = 0; mm < MB; mm++)
                if (rr == r && mm == m) v = acc[rr][mm];
        const int k = k0 + r;
        if (k < P.No && m < P.M) {
            float *o = P.C + (size_t)m * P.ldc + k;
            *o = P.beta ? *o + v : v;
        }
    }
}

template <int MB, int COLS>
__global__ __launch_bounds__(64 * GV_WAVES) void k_gemv(GvArgs g)
{
    __shared__ float As[GV_ACHUNK];
    __shared__ float red[GV_WAVES * MB * COLS];
    __shared__ float rsc[GV_WAVES];
    __shared__ float Gs[GV_ACHUNK];
    // consecutive column blocks share cache lines (a block reads COLS floats
    // of each row, a line holds 32): dealt to one XCD they meet in its L2
    // instead of being fetched from HBM once per XCD
    int b = xcd_remap(blockIdx.x, gridDim.x), p = 0;
    while (p < g.nprob && b >= g.p[p].blocks) { b -= g.p[p].blocks; p++; }
    if (p >= g.nprob) return;
    const GvProb &P = g.p[p];
    if (P.kind == TLG_NN) gemv_nn<MB, COLS>(P, b, As, red, rsc, Gs);
    else gemv_nt<MB>(P, b, As, rsc, Gs);
}

// ---------------------------------------------------------------- host --
bool tlg_gemv_fits(TlgKind kind, int Mo) { return kind != TLG_TN && Mo >= 1 && Mo <= 8; }

static int rows_bucket(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

static void set_blocks(GvProb &P, int cols)
{
    const int per = P.kind == TLG_NN ? cols : GV_WAVES * GV_NT_ROWS;
    P.blocks = (P.No + per - 1) / per;
}

// Columns per workgroup of the mm form for a launch: nn_cols(), unless
// TLG_GEMV_COLS (4, 8 or 16) pins it for sweeps.
static int launch_cols(int mb)
{
    static int forced = -1;
    if (forced < 0) {
        const char *e = getenv("TLG_GEMV_COLS");
        const int v = e ? atoi(e) : 0;
        forced = (v == 4 || v == 8 || v == 16) ? v : 0;
    }
    return forced ? forced : nn_cols(mb);
}

template <int MB>
static void launch_mb(const GvArgs &a, int grid, int cols, hipStream_t st)
{
    switch (cols) {
    case 4: hipLaunchKernelGGL((k_gemv<MB, 4>), dim3(grid), dim3(64 * GV_WAVES), 0, st, a); break;
    case 8: hipLaunchKernelGGL((k_gemv<MB, 8>), dim3(grid), dim3(64 * GV_WAVES), 0, st, a); break;
    default: hipLaunchKernelGGL((k_gemv<MB, 16>), dim3(grid), dim3(64 * GV_WAVES), 0, st, a); break;
    }
}

static int launch(GvArgs &a, int mb, hipStream_t st)
{
    const int cols = launch_cols(mb);
    int grid = 0;
    for (int i = 0; i < a.nprob; i++) {
        set_blocks(a.p[i], cols);
        grid += a.p[i].blocks;
    }
    if (grid == 0) return TLG_OK;
    switch (mb) {
    case 1: launch_mb<1>(a, grid, cols, st); break;
    case 2: launch_mb<2>(a, grid, cols, st); break;
    case 4: launch_mb<4>(a, grid, cols, st); break;
    default: launch_mb<8>(a, grid, cols, st); break;
    }
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

const char *tlg_gemv_kernel_name(int M)
{
    // as rocprofv3 names the instance the launch uses
    static char names[4][3][24];
    const int mb = rows_bucket(M), cols = launch_cols(mb);
    const int mi = mb == 1 ? 0 : mb == 2 ? 1 : mb == 4 ? 2 : 3, ci = cols == 4 ? 0 : cols == 8 ? 1 : 2;
    char *n = names[mi][ci];
    if (!n[0]) snprintf(n, sizeof names[0][0], "k_gemv<%d, %d>", mb, cols);
    return n;
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
    return launch(a, rows_bucket(Mo), st);
}

// A grouped launch whose calls are all mm / mm_bt at M <= 8 (decode runs).
int tlg_gemv_group_launch(const TlgGemmCall *calls, int n, hipStream_t st)
{
    if (n > GV_MAXPROB) return tlg_fail(TLG_EINVAL, "GEMV group: at most %d calls", GV_MAXPROB);
    GvArgs a;
    memset(&a, 0, sizeof a);
    int mmax = 1;
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
        if (P.M > mmax) mmax = P.M;
    }
    a.nprob = n;
    return launch(a, rows_bucket(mmax), st);
}

// A decode run with the glue folded in (include/tldecode.h): the calls'
// prologues (RMSNorm, SwiGLU) apply while the activation rows are staged,
// and beta = 1 adds the result into C (mm's residual add).
extern "C" int tlg_dev_dec_gemv(const TlgDecGemv *calls, int n, void *stream)
{
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (!calls || n <= 0 || n > GV_MAXPROB) return tlg_fail(TLG_EINVAL, "dec_gemv: 1 to %d calls", GV_MAXPROB);
    hipStream_t st = (hipStream_t)stream;
    rc = tlg_group_flush_launch(st);             // pending split reductions land first
    if (rc) return rc;
    GvArgs a;
    memset(&a, 0, sizeof a);
    int mmax = 1;
    for (int i = 0; i < n; i++) {
        const TlgDecGemv &c = calls[i];
        GvProb &P = a.p[i];
        if ((c.op != 0 && c.op != 1) || c.M < 1 || c.M > 8 || c.K <= 0 || c.N <= 0 || !c.A || !c.B || !c.C ||
            c.pro < GV_PRO_NONE || c.pro > GV_PRO_SWIGLU || (c.pro == GV_PRO_RMS && !c.gain) ||
            (c.pro == GV_PRO_SWIGLU && !c.A2) || (c.pro == GV_PRO_RMS && c.M * (c.op == 0 ? c.K : c.N) > GV_ACHUNK))
            return tlg_fail(TLG_EINVAL, "dec_gemv: call %d: op=%d M=%d K=%d N=%d pro=%d", i, c.op, c.M, c.K, c.N,
                            c.pro);
        P.C = c.C;
        P.M = c.M;
        P.nseg = 1;
        P.beta = c.beta ? 1 : 0;
        P.pro = c.pro;
        P.gain = c.gain;
        P.A2 = c.A2;
        if (c.op == 0) {
            P.kind = TLG_NN; P.No = c.N; P.ldc = c.N;
            P.seg[0] = GvSeg{c.A, c.B, c.K, c.K, c.N};
        } else {
            P.kind = TLG_NT; P.No = c.K; P.ldc = c.K;
            P.seg[0] = GvSeg{c.A, c.B, c.N, c.N, c.N};
        }
        if (c.M > mmax) mmax = c.M;
    }
    a.nprob = n;
    return launch(a, rows_bucket(mmax), st);
}
