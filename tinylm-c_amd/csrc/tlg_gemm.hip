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
// workgroups.  Each writes its partial sum as a plain Mo x No matrix into a
// workspace; a second kernel then adds the partials to C in split order
// (deterministic) and applies beta.  Nothing crosses workgroups inside a
// kernel, so no device-scope fence is needed: on gfx950 such a fence writes
// back and invalidates the XCD's L2, which costs every co-resident workgroup
// its cached operands.
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
    float *ws;       // splits x Mo x No partials (splits > 1)
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

template <int BM, int BN, int BK, int WGM, int LA, int LB, bool VEC>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs g)
{
    constexpr int WGN = 4 / WGM;
    constexpr int WM = BM / WGM, WN = BN / WGN, FM = WM / 32, FN = WN / 32;
    static_assert(WGM * WGN == 4 && FM >= 1 && FN >= 1, "4 waves, 32x32 blocks");
    constexpr int SA = LdsSize<LA, BM, BK>::value, SB = LdsSize<LB, BN, BK>::value;
    __shared__ __attribute__((aligned(16))) float smem[2 * (SA + SB)];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;

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

    // Epilogue.  32x32 MFMA result layout: lane l, register v holds row
    // 8*(v/4) + 4*(l/32) + v%4, column l%32 of the block.  A split writes its
    // partial (beta 0) into workspace slice z, a Mo x No row-major matrix.
    float *C = g.C;
    int ldc = g.ldc, beta = g.beta;
    if (g.splits > 1) {
        C = g.ws + (size_t)z * g.Mo * g.No;
        ldc = g.No;
        beta = 0;
    }
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
                    float *p = C + (size_t)i * ldc + j;
                    *p = beta ? (*p + acc[a][b][v]) : acc[a][b][v];
                }
            }
        }
}

// C (beta ? += : =) sum_{z < splits} ws[z], in z order; Mo x No elements.
__global__ void k_split_reduce(const float *__restrict__ ws, float *__restrict__ C, int Mo, int No,
                               int ldc, int splits, int beta)
{
    const size_t n = (size_t)Mo * No;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += stride) {
        float s = ws[e];
        for (int z = 1; z < splits; z++) s += ws[(size_t)z * n + e];
        const size_t i = e / (size_t)No, j = e % (size_t)No;
        float *p = C + i * (size_t)ldc + j;
        *p = beta ? (*p + s) : s;
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

static GemmPlan make_plan(int ci, int Mo, int No, int R, int splits)
{
    const TileCfg &c = kCfgs[ci];
    GemmPlan p;
    p.ci = ci;
    p.tiles_n = cdiv(No, c.bn);
    p.tiles = cdiv(Mo, c.bm) * p.tiles_n;
    if (splits < 1) splits = 1;
    int rps = cdiv(cdiv(R, splits), c.bk) * c.bk;
    splits = cdiv(R, rps);
    if (splits > 1 && (size_t)splits * Mo * No > g_tlg.ws_floats) {
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
        return make_plan(g_force_cfg, Mo, No, R, g_force_splits);
    static const int order[] = {0, 1, 2, 3};
    for (int k = 0; k < 4; k++) {
        const TileCfg &c = kCfgs[order[k]];
        const int tiles = cdiv(Mo, c.bm) * cdiv(No, c.bn);
        if (tiles >= 240) return make_plan(order[k], Mo, No, R, 1);
    }
    const int tiles = cdiv(Mo, 64) * cdiv(No, 64);
    int splits = cdiv(256, tiles);
    const int maxs = R / 256 > 1 ? R / 256 : 1;
    if (splits > maxs) splits = maxs;
    return make_plan(3, Mo, No, R, splits);
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
    if (pl.splits > 1) {
        const size_t n = (size_t)Mo * No;
        size_t blocks = (n + 255) / 256;
        if (blocks > 2048) blocks = 2048;
        hipLaunchKernelGGL(k_split_reduce, dim3((unsigned)blocks), dim3(256), 0, st,
                           (const float *)g_tlg.ws, C, Mo, No, ldc, pl.splits, beta);
        TLG_HIP(hipGetLastError());
    }
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
