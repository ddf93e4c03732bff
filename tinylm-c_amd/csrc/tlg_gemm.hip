// tlg_gemm.hip -- fp32 MFMA GEMM kernels for gfx950 behind mm / mm_bt / mm_atb.
//
// One kernel template serves the three reference primitives (tinylm.c:438-537):
//
//   mm      Y  = X  W      C(i,j) = sum_r X[i][r]  W[r][j]     NN
//   mm_bt   dX += dY W^T   C(i,j) = sum_r dY[i][r] W[j][r]     NT
//   mm_atb  dW += X^T dY   C(i,j) = sum_r X[r][i]  dY[r][j]    TN
//
// Each operand is either contiguous along the reduction index r ("RC") or
// along its output index ("OC").  A workgroup of 4 wave64s owns a BM x BN
// tile of C; each wave owns a (BM/2) x (BN/2) quadrant built from 32x32
// v_mfma_f32_32x32x2_f32 blocks.  Operand tiles of BK reduction steps are
// staged global -> registers -> LDS, double buffered, one barrier per step.
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
// workgroups.  Each writes its partial to a workspace, bumps the tile's
// arrival counter, and the last arrival sums the partials in split order
// (deterministic) and applies beta.  The counter is reset by that block, so
// it is zero again for the next launch on the stream.
#include "tlg_internal.h"

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { RC = 0, OC = 1 };

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
    float *ws;       // splits * tiles * BM * BN partials (splits > 1)
    unsigned int *cnt;
};

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

    __device__ __forceinline__ void load(const float *__restrict__ P, int ld, int o0, int oext,
                                         int r0, int rend, int tid)
    {
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int e = tid + 256 * q;
            int o, r;
            if (LAY == RC) { o = e / (BK / 4); r = (e % (BK / 4)) * 4; }
            else           { r = e / (OUTER / 4); o = (e % (OUTER / 4)) * 4; }
            const int go = o0 + o, gr = r0 + r;
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if (VEC) {
                if (go < oext && gr < rend) {
                    const float *p = (LAY == RC) ? P + (size_t)go * ld + gr : P + (size_t)gr * ld + go;
                    x = *reinterpret_cast<const f32x4 *>(p);
                }
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
            *reinterpret_cast<f32x4 *>(L + off) = v[q];
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

template <int BM, int BN, int BK, int LA, int LB, bool VEC>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs g)
{
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 32, FN = WN / 32;
    constexpr int SA = LdsSize<LA, BM, BK>::value, SB = LdsSize<LB, BN, BK>::value;
    __shared__ __attribute__((aligned(16))) float smem[2 * (SA + SB)];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    const int item = xcd_remap(blockIdx.x, gridDim.x);
    const int z = item / g.tiles, tile = item % g.tiles;
    const int tm = tile / g.tiles_n, tn = tile % g.tiles_n;
    const int i0 = tm * BM, j0 = tn * BN;
    const int rbeg = z * g.rps;
    const int rend = min(g.R, rbeg + g.rps);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; a++)
#pragma unroll
        for (int b = 0; b < FN; b++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[a][b][v] = 0.f;

    TileLoader<LA, BM, BK, VEC> la;
    TileLoader<LB, BN, BK, VEC> lb;
    const int nsteps = (rend - rbeg + BK - 1) / BK;

    if (nsteps > 0) {
        la.load(g.A, g.lda, i0, g.Mo, rbeg, rend, tid);
        lb.load(g.B, g.ldb, j0, g.No, rbeg, rend, tid);
        la.store(smem, tid);
        lb.store(smem + SA, tid);
        __syncthreads();
    }
    for (int st = 0; st < nsteps; st++) {
        const int buf = st & 1;
        const float *As = smem + buf * (SA + SB);
        const float *Bs = As + SA;
        const bool more = st + 1 < nsteps;
        if (more) {
            const int r = rbeg + (st + 1) * BK;
            la.load(g.A, g.lda, i0, g.Mo, r, rend, tid);
            lb.load(g.B, g.ldb, j0, g.No, r, rend, tid);
        }
        float fa[FM][BK / 2], fb[FN][BK / 2];
#pragma unroll
        for (int a = 0; a < FM; a++) read_frag<LA, BM, BK>(As, wm * WM + a * 32, lane, fa[a]);
#pragma unroll
        for (int b = 0; b < FN; b++) read_frag<LB, BN, BK>(Bs, wn * WN + b * 32, lane, fb[b]);
#pragma unroll
        for (int s = 0; s < BK / 2; s++)
#pragma unroll
            for (int a = 0; a < FM; a++)
#pragma unroll
                for (int b = 0; b < FN; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[a][s], fb[b][s], acc[a][b], 0, 0, 0);
        if (more) {
            float *Ns = smem + (buf ^ 1) * (SA + SB);
            la.store(Ns, tid);
            lb.store(Ns + SA, tid);
        }
        __syncthreads();
    }

    if (g.splits > 1) {
        // Partials in fragment order: element (a, b, v) of lane `lane` in wave
        // `wave` sits at ((((wave*FM + a)*FN + b)*16 + v)*64 + lane).
        constexpr int TILE = BM * BN;
        float *wt = g.ws + (size_t)tile * g.splits * TILE;
#pragma unroll
        for (int a = 0; a < FM; a++)
#pragma unroll
            for (int b = 0; b < FN; b++)
#pragma unroll
                for (int v = 0; v < 16; v++)
                    wt[(size_t)z * TILE + ((((wave * FM + a) * FN + b) * 16 + v) * 64 + lane)] = acc[a][b][v];
        __threadfence();
        __syncthreads();
        if (tid == 0) s_last = (atomicAdd(&g.cnt[tile], 1u) == (unsigned)(g.splits - 1));
        __syncthreads();
        if (!s_last) return;
        __threadfence();
#pragma unroll
        for (int a = 0; a < FM; a++)
#pragma unroll
            for (int b = 0; b < FN; b++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const size_t f = ((((wave * FM + a) * FN + b) * 16 + v) * 64 + lane);
                    float s = 0.f;
                    for (int q = 0; q < g.splits; q++) s += (q == z) ? acc[a][b][v] : __builtin_nontemporal_load(wt + (size_t)q * TILE + f);
                    acc[a][b][v] = s;
                }
        if (tid == 0) g.cnt[tile] = 0u;
    }

    // Epilogue.  32x32 MFMA result layout: lane l, register v holds
    // row 8*(v/4) + 4*(l/32) + v%4, column l%32 of the block.
    const int h = lane >> 5, col = lane & 31;
#pragma unroll
    for (int a = 0; a < FM; a++)
#pragma unroll
        for (int b = 0; b < FN; b++) {
            const int j = j0 + wn * WN + b * 32 + col;
            if (j >= g.No) continue;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int i = i0 + wm * WM + a * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (i < g.Mo) {
                    float *p = g.C + (size_t)i * g.ldc + j;
                    *p = g.beta ? (*p + acc[a][b][v]) : acc[a][b][v];
                }
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
struct TileCfg { int bm, bn, bk; };
static const TileCfg kCfg128 = {128, 128, 16};
static const TileCfg kCfg64 = {64, 64, 32};

template <int BM, int BN, int BK, int LA, int LB>
static void launch_t(const GemmArgs &a, int grid, bool vec, hipStream_t st)
{
    if (vec) hipLaunchKernelGGL((k_gemm<BM, BN, BK, LA, LB, true>), dim3(grid), dim3(256), 0, st, a);
    else     hipLaunchKernelGGL((k_gemm<BM, BN, BK, LA, LB, false>), dim3(grid), dim3(256), 0, st, a);
}

template <int LA, int LB>
static void launch_kind(const TileCfg &c, const GemmArgs &a, int grid, bool vec, hipStream_t st)
{
    if (c.bm == 128) launch_t<128, 128, 16, LA, LB>(a, grid, vec, st);
    else             launch_t<64, 64, 32, LA, LB>(a, grid, vec, st);
}

static inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }
static inline int cdiv(int a, int b) { return (a + b - 1) / b; }

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

    const int la = (kind == TLG_TN) ? OC : RC;
    const int lb = (kind == TLG_NT) ? RC : OC;
    // float4 staging needs 16-byte aligned operands whose contiguous extent
    // and leading dimension are multiples of 4.
    const bool vec = al16(A) && al16(B) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                     (la == RC ? (R % 4 == 0) : (Mo % 4 == 0)) &&
                     (lb == RC ? (R % 4 == 0) : (No % 4 == 0));

    // Tile choice: 128x128 when that alone gives ~a wave of work over the
    // 256 CUs, else 64x64 plus a split reduction up to ~256 work items with at
    // least 128 reduction steps each.
    const int t128 = cdiv(Mo, 128) * cdiv(No, 128);
    const TileCfg &c = (t128 >= 192) ? kCfg128 : kCfg64;
    const int tiles_m = cdiv(Mo, c.bm), tiles_n = cdiv(No, c.bn), tiles = tiles_m * tiles_n;
    int splits = 1;
    if (tiles < 256) {
        splits = cdiv(256, tiles);
        const int maxs = R / 128 > 1 ? R / 128 : 1;
        if (splits > maxs) splits = maxs;
    }
    int rps = cdiv(cdiv(R, splits), c.bk) * c.bk;
    splits = cdiv(R, rps);
    if (splits > 1) {
        const size_t need = (size_t)splits * tiles * c.bm * c.bn;
        if (need > g_tlg.ws_floats || (size_t)tiles > g_tlg.cnt_n) {
            splits = 1;
            rps = cdiv(R, c.bk) * c.bk;
        }
    }

    GemmArgs a;
    a.A = A; a.B = B; a.C = C;
    a.Mo = Mo; a.No = No; a.R = R;
    a.lda = lda; a.ldb = ldb; a.ldc = ldc;
    a.beta = beta;
    a.tiles_n = tiles_n; a.tiles = tiles;
    a.splits = splits; a.rps = rps;
    a.ws = g_tlg.ws; a.cnt = g_tlg.cnt;
    const int grid = tiles * splits;
    if (la == RC && lb == OC)      launch_kind<RC, OC>(c, a, grid, vec, st);
    else if (la == RC && lb == RC) launch_kind<RC, RC>(c, a, grid, vec, st);
    else                           launch_kind<OC, OC>(c, a, grid, vec, st);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}
