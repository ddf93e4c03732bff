// tlg_gemm.hip -- fp32 MFMA GEMM kernels for gfx950 behind mm / mm_bt / mm_atb.
//
// One tile routine serves the three reference primitives (tinylm.c:438-537):
//
//   mm      Y  = X  W      C(i,j) = sum_r X[i][r]  W[r][j]     NN
//   mm_bt   dX += dY W^T   C(i,j) = sum_r dY[i][r] W[j][r]     NT
//   mm_atb  dW += X^T dY   C(i,j) = sum_r X[r][i]  dY[r][j]    TN
//
// Each operand is either contiguous along the reduction index r ("RC") or
// along its output index ("OC").  A workgroup of 4 wave64s owns a BM x BN
// tile of C; each wave owns a (BM/WGM) x (BN/WGN) sub-tile built from 32x32
// v_mfma_f32_32x32x2_f32 blocks.  Operand tiles of BK reduction steps are
// staged global -> registers -> LDS: loads run two stages ahead of the MFMAs
// (two register stages), LDS is double buffered, one barrier per stage.
//
// LDS layouts (both give conflict-free fragment reads):
//   RC operand: [outer][BK+4]  -- a lane reads BK/2 consecutive r of one row
//                                 with ds_read_b128; the +4 pad rotates rows
//                                 across banks.
//   OC operand: [BK][outer+4]  -- 32 lanes read 32 consecutive outer indices
//                                 of one r row (ds_read_b32).
//
// Reduction order inside a tile: MFMA lanes 0-31 supply r in the first half
// of each BK step and lanes 32-63 the second half, so a lane's BK/2 values
// are contiguous in an RC tile.  Any fixed bijection of r is a valid MFMA
// k-order; the result differs from the reference's sequential chain only by
// fp32 rounding (parity bar: max|err| / mean|ref| <= 1e-4).
//
// Split reduction: when output tiles are too few to fill 256 CUs (mm_atb's
// dW is small, its reduction long), the r range is split over `splits`
// workgroups.  Each writes its partial sum as a plain Mo x No matrix into a
// workspace; a later kernel adds the partials to C in split order
// (deterministic) and applies beta.  Nothing crosses workgroups inside a
// kernel, so no device-scope fence is needed: on gfx950 such a fence writes
// back and invalidates the XCD's L2, which costs every co-resident workgroup
// its cached operands.
//
// Grouped launches (tlg_dev_gemm_group): one kernel runs a list of problems
// of any of the three kinds -- the GEMMs a caller issues back to back with
// no other work in between -- plus the deferred split reductions of the
// previous grouped launch.  The kernel boundary between the two launches is
// what makes the partials visible, so a split costs no extra launch.
#include "tlg_internal.h"
#include <stdio.h>
#include <string.h>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { RC = 0, OC = 1 };

// Workgroup id -> logical work item, so that consecutive logical items land
// on the same XCD (the dispatcher deals workgroups round-robin over the 8
// XCDs and each XCD has its own L2).  A bijection on [0, nb).
__device__ __forceinline__ int xcd_remap(int b, int nb)
{
    const int per = nb >> 3, rem = nb & 7;
    const int x = b & 7, slot = b >> 3;
    const int base = (x < rem) ? x * (per + 1) : rem * (per + 1) + (x - rem) * per;
    return base + slot;
}

// Stage one operand tile into registers.  OUTER = tile extent along the
// operand's output index, rows/cols beyond `oext` or r beyond `rend` read 0.
template <int LAY, int OUTER, int BK, bool VEC>
struct TileLoader {
    static constexpr int NCH = OUTER * BK / 4;        // float4 chunks per tile
    static constexpr int PER = NCH / 256;             // chunks per thread
    static_assert(NCH % 256 == 0, "tile must split evenly over 256 threads");
    f32x4 v[PER];
    unsigned ok;                                      // bit q: chunk q in range

    // The float4 path issues every load unconditionally from a clamped, in-
    // bounds address and zeroes out-of-range chunks at store time: branch-free
    // loads let the compiler count outstanding loads exactly, so waiting for
    // one stage does not wait for the stages prefetched after it.
    __device__ __forceinline__ void load(const float *__restrict__ P, int ld, int o0, int oext,
                                         int r0, int rend, int tid)
    {
        ok = 0;
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int e = tid + 256 * q;
            int o, r;
            if (LAY == RC) { o = e / (BK / 4); r = (e % (BK / 4)) * 4; }
            else           { r = e / (OUTER / 4); o = (e % (OUTER / 4)) * 4; }
            const int go = o0 + o, gr = r0 + r;
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if (VEC) {
                ok |= (go < oext && gr < rend) ? (1u << q) : 0u;
                // RC: rows clamp to oext-1, r to rend-4; OC: columns clamp to
                // oext-4, rows to rend-1 (rend, oext are multiples of 4 here)
                const int gc = (LAY == RC) ? min(go, oext - 1) : min(go, oext - 4);
                const int rc = (LAY == RC) ? min(gr, rend - 4) : min(gr, rend - 1);
                const float *p = (LAY == RC) ? P + (size_t)gc * ld + rc : P + (size_t)rc * ld + gc;
                x = *reinterpret_cast<const f32x4 *>(p);
            } else {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int oo = (LAY == RC) ? go : go + c;
                    const int rr = (LAY == RC) ? gr + c : gr;
                    if (oo < oext && rr < rend)
                        x[c] = (LAY == RC) ? P[(size_t)oo * ld + rr] : P[(size_t)rr * ld + oo];
                }
            }
            v[q] = x;
        }
    }

    __device__ __forceinline__ void store(float *__restrict__ L, int tid) const
    {
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int e = tid + 256 * q;
            int o, r;
            if (LAY == RC) { o = e / (BK / 4); r = (e % (BK / 4)) * 4; }
            else           { r = e / (OUTER / 4); o = (e % (OUTER / 4)) * 4; }
            const int off = (LAY == RC) ? o * (BK + 4) + r : r * (OUTER + 4) + o;
            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
            *reinterpret_cast<f32x4 *>(L + off) = (!VEC || ((ok >> q) & 1u)) ? v[q] : z;
        }
    }
};

template <int LAY, int OUTER, int BK>
struct LdsSize {
    static constexpr int value = (LAY == RC) ? OUTER * (BK + 4) : BK * (OUTER + 4);
};

// Fragment of one 32-wide MFMA block: the BK/2 r-values lane (o, h) feeds.
template <int LAY, int OUTER, int BK>
__device__ __forceinline__ void read_frag(const float *__restrict__ L, int o_base, int lane,
                                          float (&f)[BK / 2])
{
    const int o = o_base + (lane & 31), h = lane >> 5;
    if (LAY == RC) {
        const float *p = L + o * (BK + 4) + h * (BK / 2);
#pragma unroll
        for (int s = 0; s < BK / 2; s += 4) {
            const f32x4 x = *reinterpret_cast<const f32x4 *>(p + s);
            f[s] = x[0]; f[s + 1] = x[1]; f[s + 2] = x[2]; f[s + 3] = x[3];
        }
    } else {
#pragma unroll
        for (int s = 0; s < BK / 2; s++) f[s] = L[(h * (BK / 2) + s) * (OUTER + 4) + o];
    }
}

// Tile geometry shared by the kernels.
template <int BM, int BN, int BK, int WGM>
struct Tile {
    static constexpr int WGN = 4 / WGM;
    static constexpr int WM = BM / WGM, WN = BN / WGN, FM = WM / 32, FN = WN / 32;
    static_assert(WGM * WGN == 4 && FM >= 1 && FN >= 1, "4 waves, 32x32 blocks");
    template <int LA, int LB>
    static constexpr int lds() { return 2 * (LdsSize<LA, BM, BK>::value + LdsSize<LB, BN, BK>::value); }
    static constexpr int lds_max()
    {
        constexpr int a = lds<RC, OC>(), b = lds<RC, RC>(), c = lds<OC, OC>();
        return a > b ? (a > c ? a : c) : (b > c ? b : c);
    }
};

// acc += A(i0.., r) B(r, j0..) over r in [rbeg, rend).  A tile's loads run
// two stages ahead: register set S&1 holds stage S while stage S-2 computes
// from LDS; LDS buffer S&1 holds stage S from the store after stage S-1.
template <int BM, int BN, int BK, int WGM, int LA, int LB, bool VEC>
__device__ __forceinline__ void tile_accumulate(float *__restrict__ smem, const float *__restrict__ A,
                                                const float *__restrict__ B, int lda, int ldb,
                                                int i0, int j0, int Mo, int No, int rbeg, int rend,
                                                f32x16 (&acc)[Tile<BM, BN, BK, WGM>::FM][Tile<BM, BN, BK, WGM>::FN])
{
    using T = Tile<BM, BN, BK, WGM>;
    constexpr int SA = LdsSize<LA, BM, BK>::value, SB = LdsSize<LB, BN, BK>::value;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / T::WGN, wn = wave % T::WGN;
    const int nsteps = (rend - rbeg + BK - 1) / BK;
    if (nsteps <= 0) return;

    TileLoader<LA, BM, BK, VEC> la0, la1;
    TileLoader<LB, BN, BK, VEC> lb0, lb1;
    la0.load(A, lda, i0, Mo, rbeg, rend, tid);
    lb0.load(B, ldb, j0, No, rbeg, rend, tid);
    if (nsteps > 1) {
        la1.load(A, lda, i0, Mo, rbeg + BK, rend, tid);
        lb1.load(B, ldb, j0, No, rbeg + BK, rend, tid);
    }
    la0.store(smem, tid);
    lb0.store(smem + SA, tid);
    __syncthreads();

    auto compute = [&](const float *As, const float *Bs) {
        float fa[T::FM][BK / 2], fb[T::FN][BK / 2];
#pragma unroll
        for (int a = 0; a < T::FM; a++) read_frag<LA, BM, BK>(As, wm * T::WM + a * 32, lane, fa[a]);
#pragma unroll
        for (int b = 0; b < T::FN; b++) read_frag<LB, BN, BK>(Bs, wn * T::WN + b * 32, lane, fb[b]);
#pragma unroll
        for (int s = 0; s < BK / 2; s++)
#pragma unroll
            for (int a = 0; a < T::FM; a++)
#pragma unroll
                for (int b = 0; b < T::FN; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[a][s], fb[b][s], acc[a][b], 0, 0, 0);
    };

    // Stage st lives in LDS buffer st&1.  Its half-iteration prefetches stage
    // st+2 into the register set stage st came from, computes, then moves
    // stage st+1 from the other register set into the other LDS buffer.
    int st = 0;
    for (; st + 1 < nsteps; st += 2) {
        if (st + 2 < nsteps) {
            la0.load(A, lda, i0, Mo, rbeg + (st + 2) * BK, rend, tid);
            lb0.load(B, ldb, j0, No, rbeg + (st + 2) * BK, rend, tid);
        }
        compute(smem, smem + SA);
        la1.store(smem + SA + SB, tid);
        lb1.store(smem + 2 * SA + SB, tid);
        __syncthreads();
        if (st + 3 < nsteps) {
            la1.load(A, lda, i0, Mo, rbeg + (st + 3) * BK, rend, tid);
            lb1.load(B, ldb, j0, No, rbeg + (st + 3) * BK, rend, tid);
        }
        compute(smem + SA + SB, smem + 2 * SA + SB);
        if (st + 2 < nsteps) {
            la0.store(smem, tid);
            lb0.store(smem + SA, tid);
        }
        __syncthreads();
    }
    if (st < nsteps) {              // odd stage count: the last stage is in buffer 0
        compute(smem, smem + SA);
        __syncthreads();
    }
}

// C (beta ? += : =) acc for the valid part of the tile.  32x32 MFMA result
// layout: lane l, register v holds row 8*(v/4) + 4*(l/32) + v%4, column l%32.
template <int BM, int BN, int BK, int WGM>
__device__ __forceinline__ void tile_store(const f32x16 (&acc)[Tile<BM, BN, BK, WGM>::FM][Tile<BM, BN, BK, WGM>::FN],
                                           float *__restrict__ C, int ldc, int beta, int Mo, int No,
                                           int i0, int j0)
{
    using T = Tile<BM, BN, BK, WGM>;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / T::WGN, wn = wave % T::WGN;
    const int h = lane >> 5, col = lane & 31;
#pragma unroll
    for (int a = 0; a < T::FM; a++)
#pragma unroll
        for (int b = 0; b < T::FN; b++) {
            const int j = j0 + wn * T::WN + b * 32 + col;
            if (j >= No) continue;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int i = i0 + wm * T::WM + a * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (i < Mo) {
                    float *p = C + (size_t)i * ldc + j;
                    *p = beta ? (*p + acc[a][b][v]) : acc[a][b][v];
                }
            }
        }
}

template <int FM, int FN>
__device__ __forceinline__ void zero_acc(f32x16 (&acc)[FM][FN])
{
#pragma unroll
    for (int a = 0; a < FM; a++)
#pragma unroll
        for (int b = 0; b < FN; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.f;
}

// ------------------------------------------------------- single problem --
struct GemmArgs {
    const float *A;
    const float *B;
    float *C;
    int Mo, No, R;
    int lda, ldb, ldc;
    int beta;
    int tiles_n;     // tiles along No
    int tiles;       // tiles_m * tiles_n
    int splits;      // workgroups per tile along r
    int rps;         // r per split (multiple of BK)
    float *ws;       // splits x Mo x No partials (splits > 1)
};

template <int BM, int BN, int BK, int WGM, int LA, int LB, bool VEC>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs g)
{
    using T = Tile<BM, BN, BK, WGM>;
    __shared__ __attribute__((aligned(16))) float smem[T::template lds<LA, LB>()];
    const int item = xcd_remap(blockIdx.x, gridDim.x);
    const int z = item / g.tiles, tile = item % g.tiles;
    const int i0 = (tile / g.tiles_n) * BM, j0 = (tile % g.tiles_n) * BN;
    const int rbeg = z * g.rps;
    const int rend = min(g.R, rbeg + g.rps);
    f32x16 acc[T::FM][T::FN];
    zero_acc(acc);
    tile_accumulate<BM, BN, BK, WGM, LA, LB, VEC>(smem, g.A, g.B, g.lda, g.ldb, i0, j0, g.Mo, g.No,
                                                  rbeg, rend, acc);
    // a split writes its partial (beta 0) into workspace slice z
    if (g.splits > 1)
        tile_store<BM, BN, BK, WGM>(acc, g.ws + (size_t)z * g.Mo * g.No, g.No, 0, g.Mo, g.No, i0, j0);
    else
        tile_store<BM, BN, BK, WGM>(acc, g.C, g.ldc, g.beta, g.Mo, g.No, i0, j0);
}

// C (beta ? += : =) sum_{z < splits} ws[z], in z order; Mo x No elements.
__device__ __forceinline__ void reduce_range(const float *__restrict__ ws, float *__restrict__ C,
                                             int No, int ldc, int splits, int beta,
                                             size_t e0, size_t e1, size_t n)
{
    for (size_t e = e0 + threadIdx.x; e < e1; e += blockDim.x) {
        float s = ws[e];
        for (int z = 1; z < splits; z++) s += ws[(size_t)z * n + e];
        const size_t i = e / (size_t)No, j = e % (size_t)No;
        float *p = C + i * (size_t)ldc + j;
        *p = beta ? (*p + s) : s;
    }
}

__global__ void k_split_reduce(const float *__restrict__ ws, float *__restrict__ C, int Mo, int No,
                               int ldc, int splits, int beta)
{
    const size_t n = (size_t)Mo * No;
    const size_t per = 256;
    for (size_t e0 = (size_t)blockIdx.x * per; e0 < n; e0 += (size_t)gridDim.x * per)
        reduce_range(ws, C, No, ldc, splits, beta, e0, e0 + per < n ? e0 + per : n, n);
}

// ------------------------------------------------------ grouped problems --
enum { PK_NN = 0, PK_NT = 1, PK_TN = 2, PK_RED = 3 };
#define TLG_MAXSEG 3
#define TLG_MAXPROB 16
#define TLG_RED_CHUNK (256 * 4)

struct Seg { const float *A, *B; int R, lda, ldb; };
struct Prob {
    float *C;
    const float *ws;      // PK_RED: partials; split GEMM: its partial slice base
    int Mo, No, ldc, beta;
    int kind, nseg;
    int tiles_n, tiles, splits, rps;
    int item0;            // first work item of this problem
    Seg seg[TLG_MAXSEG];
};
struct GroupArgs {
    int nprob;
    Prob p[TLG_MAXPROB];
};

template <int BM, int BN, int BK, int WGM, int LA, int LB>
__device__ __forceinline__ void group_tile(float *smem, const Prob &P, int local)
{
    using T = Tile<BM, BN, BK, WGM>;
    const int z = local / P.tiles, tile = local % P.tiles;
    const int i0 = (tile / P.tiles_n) * BM, j0 = (tile % P.tiles_n) * BN;
    f32x16 acc[T::FM][T::FN];
    zero_acc(acc);
    if (P.splits > 1) {
        const Seg &s = P.seg[0];
        const int rbeg = z * P.rps, rend = min(s.R, rbeg + P.rps);
        tile_accumulate<BM, BN, BK, WGM, LA, LB, true>(smem, s.A, s.B, s.lda, s.ldb, i0, j0, P.Mo, P.No,
                                                       rbeg, rend, acc);
        tile_store<BM, BN, BK, WGM>(acc, (float *)P.ws + (size_t)z * P.Mo * P.No, P.No, 0, P.Mo, P.No, i0, j0);
        return;
    }
    for (int k = 0; k < P.nseg; k++) {
        const Seg &s = P.seg[k];
        tile_accumulate<BM, BN, BK, WGM, LA, LB, true>(smem, s.A, s.B, s.lda, s.ldb, i0, j0, P.Mo, P.No,
                                                       0, s.R, acc);
        if (k + 1 < P.nseg) __syncthreads();      // LDS reuse by the next segment
    }
    tile_store<BM, BN, BK, WGM>(acc, P.C, P.ldc, P.beta, P.Mo, P.No, i0, j0);
}

template <int BM, int BN, int BK, int WGM>
__global__ __launch_bounds__(256) void k_group(GroupArgs g)
{
    using T = Tile<BM, BN, BK, WGM>;
    __shared__ __attribute__((aligned(16))) float smem[T::lds_max()];
    const int item = xcd_remap(blockIdx.x, gridDim.x);
    int p = 0;
    while (p + 1 < g.nprob && item >= g.p[p + 1].item0) p++;
    const Prob &P = g.p[p];
    const int local = item - P.item0;
    switch (P.kind) {
    case PK_NN: group_tile<BM, BN, BK, WGM, RC, OC>(smem, P, local); break;
    case PK_NT: group_tile<BM, BN, BK, WGM, RC, RC>(smem, P, local); break;
    case PK_TN: group_tile<BM, BN, BK, WGM, OC, OC>(smem, P, local); break;
    default: {
        const size_t n = (size_t)P.Mo * P.No;
        const size_t e0 = (size_t)local * TLG_RED_CHUNK;
        const size_t e1 = e0 + TLG_RED_CHUNK < n ? e0 + TLG_RED_CHUNK : n;
        reduce_range(P.ws, P.C, P.No, P.ldc, P.splits, P.beta, e0, e1, n);
    }
    }
}

__global__ void k_zero(float *__restrict__ p, size_t n)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) p[i] = 0.f;
}

int tlg_zero_launch(float *dst, size_t n, hipStream_t st)
{
    if (n == 0) return TLG_OK;
    if (!dst) return tlg_fail(TLG_EINVAL, "tlg_dev_zero: NULL destination");
    size_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(k_zero, dim3((unsigned)blocks), dim3(256), 0, st, dst, n);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

// ---------------------------------------------------------------- launch --
// Tile shapes: BM x BN output per workgroup, BK reduction steps per stage,
// WGM waves along M (4 / WGM along N).
struct TileCfg { int bm, bn, bk, wgm; };
static const TileCfg kCfgs[] = {
    {128, 128, 16, 2},   // 0: wave tile 64x64
    {128, 64, 32, 2},    // 1: 64x32
    {64, 128, 32, 2},    // 2: 32x64
    {64, 64, 32, 2},     // 3: 32x32
    {32, 128, 32, 1},    // 4: 32x32, waves side by side along N
    {128, 32, 32, 4},    // 5: 32x32, waves stacked along M
};
static const int kNumCfgs = (int)(sizeof(kCfgs) / sizeof(kCfgs[0]));

template <int BM, int BN, int BK, int WGM, int LA, int LB>
static void launch_t(const GemmArgs &a, int grid, bool vec, hipStream_t st)
{
    if (vec) hipLaunchKernelGGL((k_gemm<BM, BN, BK, WGM, LA, LB, true>), dim3(grid), dim3(256), 0, st, a);
    else     hipLaunchKernelGGL((k_gemm<BM, BN, BK, WGM, LA, LB, false>), dim3(grid), dim3(256), 0, st, a);
}

template <int LA, int LB>
static void launch_kind(int ci, const GemmArgs &a, int grid, bool vec, hipStream_t st)
{
    switch (ci) {
    case 0: launch_t<128, 128, 16, 2, LA, LB>(a, grid, vec, st); break;
    case 1: launch_t<128, 64, 32, 2, LA, LB>(a, grid, vec, st); break;
    case 2: launch_t<64, 128, 32, 2, LA, LB>(a, grid, vec, st); break;
    case 3: launch_t<64, 64, 32, 2, LA, LB>(a, grid, vec, st); break;
    case 4: launch_t<32, 128, 32, 1, LA, LB>(a, grid, vec, st); break;
    default: launch_t<128, 32, 32, 4, LA, LB>(a, grid, vec, st); break;
    }
}

static inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }
static inline int cdiv(int a, int b) { return (a + b - 1) / b; }

struct GemmPlan { int ci; int tiles_n, tiles, splits, rps; };

// Forced choice for tuning sweeps (tlg_tune_force); -1 = automatic.
static int g_force_cfg = -1, g_force_splits = 0;

static GemmPlan make_plan(int ci, int Mo, int No, int R, int splits, size_t ws_floats)
{
    const TileCfg &c = kCfgs[ci];
    GemmPlan p;
    p.ci = ci;
    p.tiles_n = cdiv(No, c.bn);
    p.tiles = cdiv(Mo, c.bm) * p.tiles_n;
    if (splits < 1) splits = 1;
    int rps = cdiv(cdiv(R, splits), c.bk) * c.bk;
    splits = cdiv(R, rps);
    if (splits > 1 && (size_t)splits * Mo * No > ws_floats) {
        splits = 1;
        rps = cdiv(R, c.bk) * c.bk;
    }
    p.splits = splits;
    p.rps = rps;
    return p;
}

// Automatic choice: the largest tile that still yields about one wave of
// workgroups over the 256 CUs; when even 64x64 tiles are too few (small
// outputs with long reductions, i.e. mm_atb's dW), split the reduction so
// every split keeps >= 256 reduction steps.
static GemmPlan plan_gemm(int Mo, int No, int R)
{
    if (g_force_cfg >= 0 && g_force_cfg < kNumCfgs)
        return make_plan(g_force_cfg, Mo, No, R, g_force_splits, g_tlg.ws_floats);
    static const int order[] = {0, 1, 2, 3};
    for (int k = 0; k < 4; k++) {
        const TileCfg &c = kCfgs[order[k]];
        const int tiles = cdiv(Mo, c.bm) * cdiv(No, c.bn);
        if (tiles >= 240) return make_plan(order[k], Mo, No, R, 1, g_tlg.ws_floats);
    }
    const int tiles = cdiv(Mo, 64) * cdiv(No, 64);
    int splits = cdiv(256, tiles);
    const int maxs = R / 256 > 1 ? R / 256 : 1;
    if (splits > maxs) splits = maxs;
    return make_plan(3, Mo, No, R, splits, g_tlg.ws_floats);
}

// Name of the kernel instance a device-pointer call with aligned operands
// launches, as rocprofv3 prints it, and its split count.
int tlg_describe(TlgKind kind, int Mo, int No, int R, char *buf, int len, int *splits)
{
    if (tlg_ensure_init()) return TLG_ESTATE;
    if (Mo <= 0 || No <= 0 || R <= 0) {
        snprintf(buf, (size_t)len, "%s", R == 0 ? "k_zero" : "none");
        if (splits) *splits = 0;
        return TLG_OK;
    }
    const GemmPlan p = plan_gemm(Mo, No, R);
    const TileCfg &c = kCfgs[p.ci];
    const int la = (kind == TLG_TN) ? OC : RC;
    const int lb = (kind == TLG_NT) ? RC : OC;
    const bool vec = (la == RC ? (R % 4 == 0) : (Mo % 4 == 0)) && (lb == RC ? (R % 4 == 0) : (No % 4 == 0));
    snprintf(buf, (size_t)len, "k_gemm<%d, %d, %d, %d, %d, %d, %s>", c.bm, c.bn, c.bk, c.wgm,
             la, lb, vec ? "true" : "false");
    if (splits) *splits = p.splits;
    return TLG_OK;
}

extern "C" int tlg_tune_force(int cfg, int splits)
{
    if (cfg >= kNumCfgs) return tlg_fail(TLG_EINVAL, "tlg_tune_force: config %d of %d", cfg, kNumCfgs);
    g_force_cfg = cfg;
    g_force_splits = splits;
    return TLG_OK;
}

static int launch_reduce(const float *ws, float *C, int Mo, int No, int ldc, int splits, int beta,
                         hipStream_t st)
{
    const size_t n = (size_t)Mo * No;
    size_t blocks = (n + 255) / 256;
    if (blocks > 2048) blocks = 2048;
    hipLaunchKernelGGL(k_split_reduce, dim3((unsigned)blocks), dim3(256), 0, st, ws, C, Mo, No, ldc,
                       splits, beta);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

int tlg_gemm_launch(TlgKind kind, const float *A, const float *B, float *C,
                    int Mo, int No, int R, int lda, int ldb, int ldc, int beta,
                    hipStream_t st)
{
    if (Mo < 0 || No < 0 || R < 0) return tlg_fail(TLG_EINVAL, "negative GEMM dimension");
    if (Mo == 0 || No == 0) return TLG_OK;
    if (!C) return tlg_fail(TLG_EINVAL, "NULL output pointer");
    if (R == 0) {
        // Empty reduction: mm clears its rows (tinylm.c:461), the accumulating
        // forms add nothing.
        if (beta) return TLG_OK;
        if (ldc != No) return tlg_fail(TLG_EINVAL, "strided empty-reduction clear");
        return tlg_zero_launch(C, (size_t)Mo * No, st);
    }
    if (!A || !B) return tlg_fail(TLG_EINVAL, "NULL input pointer");
    int rc = tlg_ensure_init();
    if (rc) return rc;
    // a single-problem launch must not overtake partials a grouped launch
    // left for its successor
    rc = tlg_group_flush_launch(st);
    if (rc) return rc;

    const int la = (kind == TLG_TN) ? OC : RC;
    const int lb = (kind == TLG_NT) ? RC : OC;
    // float4 staging needs 16-byte aligned operands whose contiguous extent
    // and leading dimension are multiples of 4.
    const bool vec = al16(A) && al16(B) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                     (la == RC ? (R % 4 == 0) : (Mo % 4 == 0)) &&
                     (lb == RC ? (R % 4 == 0) : (No % 4 == 0));
    const GemmPlan pl = plan_gemm(Mo, No, R);

    GemmArgs a;
    a.A = A; a.B = B; a.C = C;
    a.Mo = Mo; a.No = No; a.R = R;
    a.lda = lda; a.ldb = ldb; a.ldc = ldc;
    a.beta = beta;
    a.tiles_n = pl.tiles_n; a.tiles = pl.tiles;
    a.splits = pl.splits; a.rps = pl.rps;
    a.ws = g_tlg.ws;
    const int grid = pl.tiles * pl.splits;
    if (la == RC && lb == OC)      launch_kind<RC, OC>(pl.ci, a, grid, vec, st);
    else if (la == RC && lb == RC) launch_kind<RC, RC>(pl.ci, a, grid, vec, st);
    else                           launch_kind<OC, OC>(pl.ci, a, grid, vec, st);
    TLG_HIP(hipGetLastError());
    if (pl.splits > 1) return launch_reduce(g_tlg.ws, C, Mo, No, ldc, pl.splits, beta, st);
    return TLG_OK;
}

// ------------------------------------------------------- grouped launch --
// Host side of k_group.  Split partials of a grouped launch live in one half
// of the workspace and are reduced by the next grouped launch (or a flush);
// the halves alternate so a launch never overwrites partials still pending.
static Prob g_pending[TLG_MAXPROB];
static int g_npending = 0;
static int g_ws_half = 0;

typedef void (*GroupLauncher)(const GroupArgs &, int, hipStream_t);
template <int BM, int BN, int BK, int WGM>
static void launch_group_t(const GroupArgs &a, int grid, hipStream_t st)
{
    hipLaunchKernelGGL((k_group<BM, BN, BK, WGM>), dim3(grid), dim3(256), 0, st, a);
}

static int add_reductions(GroupArgs &a, int &items)
{
    for (int k = 0; k < g_npending; k++) {
        Prob r = g_pending[k];
        r.kind = PK_RED;
        r.item0 = items;
        items += (int)(((size_t)r.Mo * r.No + TLG_RED_CHUNK - 1) / TLG_RED_CHUNK);
        a.p[a.nprob++] = r;
    }
    g_npending = 0;
    return TLG_OK;
}

int tlg_group_flush_launch(hipStream_t st)
{
    if (g_npending == 0) return TLG_OK;
    GroupArgs a;
    a.nprob = 0;
    int items = 0;
    add_reductions(a, items);
    launch_group_t<64, 64, 32, 2>(a, items, st);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

// [lo, hi) byte range touched by a row-major operand of `rows` x `cols`
// with leading dimension ld.
static void span(const void *p, int rows, int cols, int ld, const char **lo, const char **hi)
{
    *lo = (const char *)p;
    *hi = *lo + ((size_t)(rows - 1) * ld + cols) * sizeof(float);
}
static bool overlap(const char *a0, const char *a1, const char *b0, const char *b1)
{
    return a0 < b1 && b0 < a1;
}

int tlg_group_launch(const TlgGemmCall *calls, int n, hipStream_t st)
{
    if (n <= 0) return TLG_OK;
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (n > TLG_MAXPROB / 2) return tlg_fail(TLG_EINVAL, "tlg_dev_gemm_group: at most %d calls", TLG_MAXPROB / 2);

    // Pending reductions write their C; a call that touches such a range must
    // see them first, so they go in a launch of their own.
    for (int k = 0; k < g_npending && g_npending; k++) {
        const Prob &r = g_pending[k];
        const char *c0, *c1;
        span(r.C, r.Mo, r.No, r.ldc, &c0, &c1);
        for (int i = 0; i < n; i++) {
            const TlgGemmCall &c = calls[i];
            const int op = c.op;
            const int Mo = op == 2 ? c.K : c.M, No = op == 1 ? c.K : c.N;
            const char *o0, *o1;
            span(c.C, Mo, No, No, &o0, &o1);
            bool hit = overlap(c0, c1, o0, o1);
            for (int s = 0; s < c.nseg && !hit; s++) {
                const int Ns = s ? c.Nseg[s] : c.N;
                const char *x0, *x1, *y0, *y1;
                if (op == 0)      { span(c.A[s], c.M, c.K, c.K, &x0, &x1); span(c.B[s], c.K, Ns, Ns, &y0, &y1); }
                else if (op == 1) { span(c.A[s], c.M, Ns, Ns, &x0, &x1); span(c.B[s], c.K, Ns, Ns, &y0, &y1); }
                else              { span(c.A[s], c.M, c.K, c.K, &x0, &x1); span(c.B[s], c.M, Ns, Ns, &y0, &y1); }
                hit = overlap(c0, c1, x0, x1) || overlap(c0, c1, y0, y1);
            }
            if (hit) { rc = tlg_group_flush_launch(st); if (rc) return rc; break; }
        }
    }

    GroupArgs a;
    a.nprob = 0;
    int items = 0;
    add_reductions(a, items);
    float *ws = g_tlg.ws + (size_t)g_ws_half * (g_tlg.ws_floats / 2);
    size_t ws_used = 0;
    const size_t ws_cap = g_tlg.ws_floats / 2;
    // reduction length the non-split problems of this group run per tile:
    // split problems aim for about the same per-item work
    int rmax = 0;
    for (int i = 0; i < n; i++) {
        const TlgGemmCall &c = calls[i];
        if (c.op == 2) continue;
        int r = 0;
        for (int s = 0; s < c.nseg; s++) r += (c.op == 0) ? c.K : (s ? c.Nseg[s] : c.N);
        if (r > rmax) rmax = r;
    }
    const int rtarget = rmax > 384 ? rmax : 384;

    for (int i = 0; i < n; i++) {
        const TlgGemmCall &c = calls[i];
        if (c.op < 0 || c.op > 2 || c.nseg < 1 || c.nseg > TLG_MAXSEG || (c.nseg > 1 && c.op != 1))
            return tlg_fail(TLG_EINVAL, "tlg_dev_gemm_group: call %d: bad op/nseg", i);
        if (c.M < 0 || c.K < 0 || c.N < 0) return tlg_fail(TLG_EINVAL, "negative dimension");
        Prob P;
        memset(&P, 0, sizeof P);
        P.kind = c.op == 0 ? PK_NN : (c.op == 1 ? PK_NT : PK_TN);
        P.C = c.C;
        P.beta = c.op == 0 ? 0 : (c.beta ? 1 : 0);
        P.nseg = c.nseg;
        int R = 0;
        bool vec = true;
        for (int s = 0; s < c.nseg; s++) {
            const int Ns = s ? c.Nseg[s] : c.N;
            Seg &g = P.seg[s];
            g.A = c.A[s]; g.B = c.B[s];
            switch (c.op) {
            case 0: P.Mo = c.M; P.No = c.N; g.R = c.K; g.lda = c.K; g.ldb = c.N; break;
            case 1: P.Mo = c.M; P.No = c.K; g.R = Ns; g.lda = Ns; g.ldb = Ns; break;
            default: P.Mo = c.K; P.No = c.N; g.R = c.M; g.lda = c.K; g.ldb = c.N; break;
            }
            R += g.R;
            const int la = (P.kind == PK_TN) ? OC : RC, lb = (P.kind == PK_NT) ? RC : OC;
            vec = vec && al16(g.A) && al16(g.B) && g.lda % 4 == 0 && g.ldb % 4 == 0 &&
                  (la == RC ? g.R % 4 == 0 : P.Mo % 4 == 0) && (lb == RC ? g.R % 4 == 0 : P.No % 4 == 0);
        }
        P.ldc = P.No;
        if (!vec || !c.C || R == 0 || P.Mo == 0 || P.No == 0)
            return tlg_fail(TLG_EINVAL, "tlg_dev_gemm_group: call %d needs aligned, non-empty operands", i);
        P.tiles_n = cdiv(P.No, 64);
        P.tiles = cdiv(P.Mo, 64) * P.tiles_n;
        P.splits = 1;
        P.rps = R;
        if (P.kind == PK_TN && R > rtarget + rtarget / 2) {
            int sp = cdiv(R, rtarget);
            if (sp > 32) sp = 32;
            int rps = cdiv(cdiv(R, sp), 32) * 32;
            sp = cdiv(R, rps);
            if (sp > 1 && ws_used + (size_t)sp * P.Mo * P.No <= ws_cap) {
                P.splits = sp;
                P.rps = rps;
                P.ws = ws + ws_used;
                ws_used += (size_t)sp * P.Mo * P.No;
            }
        }
        P.item0 = items;
        items += P.tiles * P.splits;
        a.p[a.nprob++] = P;
        if (P.splits > 1) g_pending[g_npending++] = P;
    }
    launch_group_t<64, 64, 32, 2>(a, items, st);
    TLG_HIP(hipGetLastError());
    if (g_npending) g_ws_half ^= 1;
    return TLG_OK;
}

// ------------------------------------------------------ seeded fill ------
// splitmix64 of (seed, pair index) -> two 53-bit uniforms -> Box-Muller pair.
__device__ __forceinline__ unsigned long long splitmix64(unsigned long long x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__global__ void k_fill_normal(float *__restrict__ p, size_t n, unsigned long long seed, float scale)
{
    const size_t pairs = (n + 1) / 2;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < pairs; i += stride) {
        const unsigned long long h1 = splitmix64(seed ^ (2 * i));
        const unsigned long long h2 = splitmix64(h1 ^ (2 * i + 1));
        double u1 = (double)(h1 >> 11) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(h2 >> 11) * (1.0 / 9007199254740992.0);
        if (u1 < 1e-300) u1 = 1e-300;
        const double r = sqrt(-2.0 * log(u1));
        const double t = 6.283185307179586 * u2;
        p[2 * i] = scale * (float)(r * cos(t));
        if (2 * i + 1 < n) p[2 * i + 1] = scale * (float)(r * sin(t));
    }
}

int tlg_fill_normal_launch(float *dst, size_t n, unsigned long long seed, float scale, hipStream_t st)
{
    if (n == 0) return TLG_OK;
    if (!dst) return tlg_fail(TLG_EINVAL, "tlg_dev_fill_normal: NULL destination");
    size_t blocks = ((n + 1) / 2 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(k_fill_normal, dim3((unsigned)blocks), dim3(256), 0, st, dst, n, seed, scale);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

// ------------------------------------------------------ measurement probes --
// Plain streaming copy (the calibration kernel for HBM byte counters and the
// achievable-bandwidth probe): dst[i] = src[i], float4 per thread.
__global__ void k_copy(const f32x4 *__restrict__ src, f32x4 *__restrict__ dst, size_t n4)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride)
        dst[i] = __builtin_nontemporal_load(src + i);
}

int tlg_copy_launch(float *dst, const float *src, size_t n, hipStream_t st)
{
    if (n % 4 || ((uintptr_t)dst & 15) || ((uintptr_t)src & 15))
        return tlg_fail(TLG_EINVAL, "tlg_dev_copy: needs 16-byte aligned buffers and n %% 4 == 0");
    const size_t n4 = n / 4;
    size_t blocks = (n4 + 255) / 256;
    if (blocks > 256 * 16) blocks = 256 * 16;
    if (blocks == 0) return TLG_OK;
    hipLaunchKernelGGL(k_copy, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const f32x4 *)src, (f32x4 *)dst, n4);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

// Achievable fp32 MFMA rate: every wave runs `iters` x 4 independent
// v_mfma_f32_32x32x2_f32 chains on register operands, then stores one value
// per lane so the work is not eliminated.
__global__ __launch_bounds__(256) void k_mfma_peak(float *__restrict__ out, int iters, float seed)
{
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    const float a = seed + threadIdx.x * 1e-7f, b = seed - threadIdx.x * 1e-7f;
    for (int i = 0; i < iters; i++) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(b, a, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x2f32(a, a, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x2f32(b, b, c3, 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < 16; v++) s += c0[v] + c1[v] + c2[v] + c3[v];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

int tlg_mfma_peak_launch(float *out, int blocks, int iters, hipStream_t st)
{
    if (blocks <= 0 || iters <= 0) return tlg_fail(TLG_EINVAL, "tlg_dev_mfma_peak: bad size");
    hipLaunchKernelGGL(k_mfma_peak, dim3(blocks), dim3(256), 0, st, out, iters, 0.5f);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}
