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
#include <mutex>
#include <stdio.h>
#include <string.h>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { RC = 0, OC = 1 };

// Stage one operand tile into registers.  OUTER = tile extent along the
// operand's output index, rows/cols beyond `oext` or r beyond `rend` read 0.
//
// Two forms serve the expert GEMMs of the MoE layer (float4 path only):
//   G   gathered rows: the operand's memory row of tile row x is rs[q], read
//       from a row map -- once per tile for an RC operand (rows(): the rows
//       are output rows), once per stage for an OC operand (prep(): the rows
//       are reduction steps; prep runs a full prefetch round ahead of the
//       load that uses it, so waiting for the map never waits for the
//       operand loads issued after it).
//   PB  paired columns (OC only): tile columns [0, OUTER/2) come from P and
//       [OUTER/2, OUTER) from P2, both at columns o0 + [0, OUTER/2).
// Sixteen zero bytes in global memory: with ZP a chunk outside the operand
// is loaded from here instead of being zeroed after its load, so nothing
// between a stage's loads and its LDS store waits on the loaded values.
__device__ __attribute__((aligned(16))) float g_zero_chunk[4] = {0.f, 0.f, 0.f, 0.f};

template <int LAY, int OUTER, int BK, bool VEC, int NT, bool G = false, bool PB = false, bool ZP = false>
struct TileLoader {
    static constexpr int NCH = OUTER * BK / 4;        // float4 chunks per tile
    static constexpr int PER = NCH / NT;              // chunks per thread
    static constexpr int HALF = OUTER / 2;
    static_assert(NCH % NT == 0, "tile must split evenly over the workgroup's threads");
    static_assert(!PB || (LAY == OC && HALF % 4 == 0), "paired columns: OC tiles");
    static_assert(!(G || PB) || VEC, "gathered / paired tiles load float4");
    f32x4 v[PER];
    unsigned ok;                                      // bit q: chunk q in range
    int rs[G ? PER : 1];                              // gathered memory rows

    __device__ __forceinline__ void rows(const int *__restrict__ map, int o0, int oext, int tid)
    {
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int e = tid + NT * q;
            rs[q] = map[min(o0 + e / (BK / 4), oext - 1)];
        }
    }
    __device__ __forceinline__ void prep(const int *__restrict__ map, int r0, int rend, int tid)
    {
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int e = tid + NT * q;
            rs[q] = map[min(r0 + e / (OUTER / 4), rend - 1)];
        }
    }

    // The float4 path issues every load unconditionally from a clamped, in-
    // bounds address and zeroes out-of-range chunks at store time: branch-free
    // loads let the compiler count outstanding loads exactly, so waiting for
    // one stage does not wait for the stages prefetched after it.
    __device__ __forceinline__ void load(const float *__restrict__ P, int ld, int o0, int oext,
                                         int r0, int rend, int tid, const float *__restrict__ P2 = nullptr)
    {
        ok = 0;
#pragma unroll
        for (int q = 0; q < PER; q++) {
            const int e = tid + NT * q;
            int o, r;
            if (LAY == RC) { o = e / (BK / 4); r = (e % (BK / 4)) * 4; }
            else           { r = e / (OUTER / 4); o = (e % (OUTER / 4)) * 4; }
            const float *Pq = P;
            if (PB && o >= HALF) { o -= HALF; Pq = P2; }
            const int go = o0 + o, gr = r0 + r;
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
            if (VEC) {
                const bool in = go < oext && gr < rend;
                if (!ZP) ok |= in ? (1u << q) : 0u;
                // RC: rows clamp to oext-1, r to rend-4; OC: columns clamp to
                // oext-4, rows to rend-1 (rend, oext are multiples of 4 here)
                const int gc = (LAY == RC) ? min(go, oext - 1) : min(go, oext - 4);
                const int rc = (LAY == RC) ? min(gr, rend - 4) : min(gr, rend - 1);
                const size_t row = G ? (size_t)rs[q] : (size_t)((LAY == RC) ? gc : rc);
                const float *p = (LAY == RC) ? Pq + row * ld + rc : Pq + row * ld + gc;
                if (ZP) p = in ? p : g_zero_chunk;
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
            const int e = tid + NT * q;
            int o, r;
            if (LAY == RC) { o = e / (BK / 4); r = (e % (BK / 4)) * 4; }
            else           { r = e / (OUTER / 4); o = (e % (OUTER / 4)) * 4; }
            const int off = (LAY == RC) ? o * (BK + 4) + r : r * (OUTER + 4) + o;
            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
            *reinterpret_cast<f32x4 *>(L + off) = (!VEC || ZP || ((ok >> q) & 1u)) ? v[q] : z;
        }
    }
};

template <int LAY, int OUTER, int BK>
struct LdsSize {
    static constexpr int value = (LAY == RC) ? OUTER * (BK + 4) : BK * (OUTER + 4);
};

// Fragment of one 32-wide MFMA block: the RW/2 r-values lane (o, h) feeds,
// from the RW reduction steps [r_base, r_base + RW) of a BK-step stage.
template <int LAY, int OUTER, int BK, int RW>
__device__ __forceinline__ void read_frag(const float *__restrict__ L, int o_base, int r_base, int lane,
                                          float (&f)[RW / 2])
{
    const int o = o_base + (lane & 31), h = lane >> 5;
    if (LAY == RC) {
        const float *p = L + o * (BK + 4) + r_base + h * (RW / 2);
#pragma unroll
        for (int s = 0; s < RW / 2; s += 4) {
            const f32x4 x = *reinterpret_cast<const f32x4 *>(p + s);
            f[s] = x[0]; f[s + 1] = x[1]; f[s + 2] = x[2]; f[s + 3] = x[3];
        }
    } else {
#pragma unroll
        for (int s = 0; s < RW / 2; s++) f[s] = L[(r_base + h * (RW / 2) + s) * (OUTER + 4) + o];
    }
}

// Tile geometry.  The 4 waves of a workgroup form a WGM x WGN grid over the
// BM x BN tile and WK groups along the reduction: with WK > 1 every wave
// computes its (BM/WGM) x (BN/WGN) sub-tile over RW = BK/WK of each stage's
// reduction steps, and the WK partial sub-tiles are summed through LDS in
// fixed order at the end.  WK > 1 gives small tiles several independent MFMA
// accumulator chains per wave instead of one dependent chain.
template <int BM_, int BN_, int BK_, int WGM_, int WK_, int NR_ = 2, int NCH_ = 0, int NW_ = 4>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WK = WK_, NR = NR_;
    // instruction order of a stage (sched_step): 0 = the compiler's; Sched<>
    // below selects the others
    static constexpr int SCH = 0;
    static constexpr int NW = NW_, THREADS = 64 * NW_;      // waves / threads per workgroup
    static constexpr int WGN = NW / (WGM * WK);
    static constexpr int WM = BM / WGM, WN = BN / WGN, FM = WM / 32, FN = WN / 32;
    static constexpr int RW = BK / WK;
    // accumulator chains per 32x32 block (the reduction steps of a block
    // alternate between its NCH chains, summed in fixed order at the store);
    // measured on MI355X: one chain is as fast and keeps occupancy higher
    static constexpr int NCH = NCH_ ? NCH_ : 1;
    static_assert(WGM * WGN * WK == NW && FM >= 1 && FN >= 1, "NW waves, 32x32 blocks");
    static_assert(RW >= 8 && RW % 8 == 0, "a wave takes a multiple of 8 reduction steps per stage");
    static constexpr int TILE = BM * BN;
    template <int LA, int LB>
    static constexpr int stage_lds() { return 2 * (LdsSize<LA, BM, BK>::value + LdsSize<LB, BN, BK>::value); }
    static constexpr int red_lds() { return WK > 1 ? WK * TILE : 0; }
    static constexpr int mx(int a, int b) { return a > b ? a : b; }
    template <int LA, int LB>
    static constexpr int lds() { return mx(stage_lds<LA, LB>(), red_lds()); }
    static constexpr int lds_max() { return mx(mx(lds<RC, OC>(), lds<RC, RC>()), lds<OC, OC>()); }
    __device__ static int wave() { return threadIdx.x >> 6; }
    __device__ static int wk() { return wave() / (WGM * WGN); }
    __device__ static int wm() { return (wave() % (WGM * WGN)) / WGN; }
    __device__ static int wn() { return (wave() % (WGM * WGN)) % WGN; }
};

// Instruction order inside one stage's scheduling region (between two
// barriers).  Left to itself the scheduler interleaves each fragment read
// with the MFMA pair that consumes it, to save registers, so at one wave
// per SIMD every MFMA pair waits out a full LDS round trip; the explicit
// orders issue all of a stage's fragment reads first (the MFMAs then wait
// only for the oldest ones), optionally behind the prefetch loads.
template <class T>
__device__ __forceinline__ void sched_step()
{
    constexpr int VMEM_RD = 0x020, DS_RD = 0x100, DS_WR = 0x200, MFMA = 0x008;
    if constexpr ((T::SCH & 3) == 1) {
        __builtin_amdgcn_sched_group_barrier(DS_RD, 64, 0);
        __builtin_amdgcn_sched_group_barrier(MFMA, 64, 0);
        __builtin_amdgcn_sched_group_barrier(DS_WR, 32, 0);
    } else if constexpr ((T::SCH & 3) == 2) {
        __builtin_amdgcn_sched_group_barrier(VMEM_RD, 32, 0);
        __builtin_amdgcn_sched_group_barrier(DS_RD, 64, 0);
        __builtin_amdgcn_sched_group_barrier(MFMA, 64, 0);
        __builtin_amdgcn_sched_group_barrier(DS_WR, 32, 0);
    }
}

// A tile shape with an explicit instruction order per stage: 1 = every
// fragment read of the stage issued before its first MFMA; 2 = the prefetch
// loads first, then the fragment reads, then the MFMAs.  + 4: the tile's
// outputs leave with nontemporal (streaming) stores.
template <class T, int S>
struct Sched : T {
    static constexpr int SCH = S;
};

// acc += A(i0.., r) B(r, j0..) over r in [rbeg, rend).  A tile's loads run
// NR stages ahead through NR register sets; LDS is double buffered.
// GA: A's rows go through the row map `amap` (RC A: amap[i0 + x] for tile
// row x; OC A: amap[r]).  PB: B is the column pair (B, B2) of TileLoader.
template <class T, int LA, int LB, bool VEC, bool GA = false, bool PB = false>
__device__ __forceinline__ void tile_accumulate(float *__restrict__ smem, const float *__restrict__ A,
                                                const float *__restrict__ B, int lda, int ldb,
                                                int i0, int j0, int Mo, int No, int rbeg, int rend,
                                                f32x16 (&acc)[T::FM][T::FN][T::NCH],
                                                const int *__restrict__ amap = nullptr,
                                                const float *__restrict__ B2 = nullptr)
{
    constexpr int BM = T::BM, BN = T::BN, BK = T::BK, RW = T::RW;
    constexpr int SA = LdsSize<LA, BM, BK>::value, SB = LdsSize<LB, BN, BK>::value;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wm = T::wm(), wn = T::wn(), rb = T::wk() * RW;
    const int nsteps = (rend - rbeg + BK - 1) / BK;
    if (nsteps <= 0) return;

    // Every prefetch is issued unconditionally: a stage past the end re-reads
    // the last stage's (in-bounds) addresses and is never stored.  Loads under
    // a branch would leave the compiler unsure how many are outstanding where
    // the paths meet, and it would then wait for all of them, the prefetch
    // included, before every LDS store.
    auto stage_r = [&](int st) { return rbeg + min(st, nsteps - 1) * BK; };
    constexpr bool ZP = T::SCH > 0;
    TileLoader<LA, BM, BK, VEC, T::THREADS, GA, false, ZP> la0, la1, la2;
    TileLoader<LB, BN, BK, VEC, T::THREADS, false, PB, ZP> lb0, lb1, lb2;
    if constexpr (GA && LA == RC) {
        la0.rows(amap, i0, Mo, tid);
        la1.rows(amap, i0, Mo, tid);
        if constexpr (T::NR > 2) la2.rows(amap, i0, Mo, tid);
    }
    if constexpr (GA && LA == OC) {
        la0.prep(amap, rbeg, rend, tid);
        la1.prep(amap, stage_r(1), rend, tid);
        if constexpr (T::NR > 2) la2.prep(amap, stage_r(2), rend, tid);
    }
    // an OC gather re-arms each register set's row map for the stage it
    // loads next, NR stages on
    auto reprep = [&](auto &l, int st) {
        if constexpr (GA && LA == OC) l.prep(amap, stage_r(st), rend, tid);
    };
    la0.load(A, lda, i0, Mo, rbeg, rend, tid);
    reprep(la0, T::NR);
    lb0.load(B, ldb, j0, No, rbeg, rend, tid, B2);
    la1.load(A, lda, i0, Mo, stage_r(1), rend, tid);
    reprep(la1, 1 + T::NR);
    lb1.load(B, ldb, j0, No, stage_r(1), rend, tid, B2);
    if constexpr (T::NR > 2) {
        la2.load(A, lda, i0, Mo, stage_r(2), rend, tid);
        reprep(la2, 2 + T::NR);
        lb2.load(B, ldb, j0, No, stage_r(2), rend, tid, B2);
    }
    la0.store(smem, tid);
    lb0.store(smem + SA, tid);
    __syncthreads();

    auto compute = [&](const float *As, const float *Bs) {
        float fa[T::FM][RW / 2], fb[T::FN][RW / 2];
#pragma unroll
        for (int a = 0; a < T::FM; a++) read_frag<LA, BM, BK, RW>(As, wm * T::WM + a * 32, rb, lane, fa[a]);
#pragma unroll
        for (int b = 0; b < T::FN; b++) read_frag<LB, BN, BK, RW>(Bs, wn * T::WN + b * 32, rb, lane, fb[b]);
#pragma unroll
        for (int s = 0; s < RW / 2; s++)
#pragma unroll
            for (int a = 0; a < T::FM; a++)
#pragma unroll
                for (int b = 0; b < T::FN; b++)
                    acc[a][b][s % T::NCH] =
                        __builtin_amdgcn_mfma_f32_32x32x2f32(fa[a][s], fb[b][s], acc[a][b][s % T::NCH], 0, 0, 0);
    };

    // Stage st lives in LDS buffer st&1 and, before that, in register set
    // st % NR.  Step st prefetches stage st+NR into the set stage st came
    // from, computes stage st, then moves stage st+1 from its register set
    // into the other LDS buffer.  NR = 3 keeps loads three stages ahead.
    //
    // Two loop forms, chosen by measurement on MI355X (m3 GEMM set 1.544 ->
    // 1.51 ms, nano 0.130 -> 0.120 ms, m8 unchanged):
    // * WK > 1 (the waves split each stage): whole rounds of NR steps with no
    //   branch inside, the store of stage st+1 unconditional (past the last
    //   stage it stores the clamped re-read, which nothing reads; the final
    //   barrier orders it before the caller reuses the LDS), and a scheduling
    //   fence that keeps a step's loads ahead of its fragment reads and MFMAs
    //   (left alone the scheduler issues them after the MFMAs, their registers
    //   doubling as fragment registers).  A guarded step or store would give
    //   the loop header a predecessor with the other register set's loads
    //   outstanding, and the compiler then waits for every load in flight --
    //   the prefetch one step old included -- before each round's first
    //   fragment read.
    // * WK = 1: the guarded form, whose interleaving measured 1-4 % faster on
    //   these tiles despite that wait; the fence, or a fence before the store
    //   as well, cost up to 10 %.
    auto step = [&](int st, auto &lac, auto &lbc, auto &lan, auto &lbn) {
        lac.load(A, lda, i0, Mo, stage_r(st + T::NR), rend, tid);
        reprep(lac, st + 2 * T::NR);
        lbc.load(B, ldb, j0, No, stage_r(st + T::NR), rend, tid, B2);
        if constexpr (T::WK > 1 && T::SCH == 0) __builtin_amdgcn_sched_barrier(0);
        float *cur = smem + (st & 1) * (SA + SB);
        compute(cur, cur + SA);
        if (T::WK > 1 || T::SCH > 0 || st + 1 < nsteps) {
            float *nxt = smem + ((st + 1) & 1) * (SA + SB);
            lan.store(nxt, tid);
            lbn.store(nxt + SA, tid);
        }
        sched_step<T>();
        __syncthreads();
    };
    if constexpr (T::WK > 1 || T::SCH > 0) {
        int st = 0;
        if constexpr (T::NR == 2) {
            for (; st + 1 < nsteps; st += 2) {
                step(st, la0, lb0, la1, lb1);
                step(st + 1, la1, lb1, la0, lb0);
            }
            if (st < nsteps) step(st, la0, lb0, la1, lb1);
        } else {
            for (; st + 2 < nsteps; st += 3) {
                step(st, la0, lb0, la1, lb1);
                step(st + 1, la1, lb1, la2, lb2);
                step(st + 2, la2, lb2, la0, lb0);
            }
            if (st < nsteps) step(st, la0, lb0, la1, lb1);
            if (st + 1 < nsteps) step(st + 1, la1, lb1, la2, lb2);
        }
    } else if constexpr (T::NR == 2) {
        for (int st = 0; st < nsteps; st += 2) {
            step(st, la0, lb0, la1, lb1);
            if (st + 1 < nsteps) step(st + 1, la1, lb1, la0, lb0);
        }
    } else {
        for (int st = 0; st < nsteps; st += 3) {
            step(st, la0, lb0, la1, lb1);
            if (st + 1 < nsteps) step(st + 1, la1, lb1, la2, lb2);
            if (st + 2 < nsteps) step(st + 2, la2, lb2, la0, lb0);
        }
    }
}

// put(i, j, v) for every element (i, j) of the tile's valid part (i < Mo,
// j < No), v its sum.  32x32 MFMA result layout: lane l, register v holds
// row 8*(v/4) + 4*(l/32) + v%4, column l%32.  With WK > 1 the wave groups'
// partial tiles go through `red` (LDS, WK*BM*BN floats, free once
// tile_accumulate has returned) and are summed in wave-group order, so the
// result does not depend on timing.  STASH: every element's value (valid
// or not) is also left in red[f], f its fragment-order index (below), for a
// row-wise epilogue after the next barrier; red must hold TILE floats.
template <class T, bool STASH = false, class Put>
__device__ __forceinline__ void tile_epi(const f32x16 (&accs)[T::FM][T::FN][T::NCH], int Mo, int No, int i0,
                                         int j0, float *__restrict__ red, Put put)
{
    const int lane = threadIdx.x & 63;
    f32x16 acc[T::FM][T::FN];
#pragma unroll
    for (int a = 0; a < T::FM; a++)
#pragma unroll
        for (int b = 0; b < T::FN; b++) {
            acc[a][b] = accs[a][b][0];
#pragma unroll
            for (int c = 1; c < T::NCH; c++) acc[a][b] += accs[a][b][c];
        }
    if constexpr (T::WK == 1) {
        const int wm = T::wm(), wn = T::wn();
        const int h = lane >> 5, col = lane & 31;
        if constexpr (STASH) {
            const int g = T::wave() % (T::WGM * T::WGN);
#pragma unroll
            for (int a = 0; a < T::FM; a++)
#pragma unroll
                for (int b = 0; b < T::FN; b++)
#pragma unroll
                    for (int v = 0; v < 16; v++)
                        red[(((g * T::FM + a) * T::FN + b) * 16 + v) * 64 + lane] = acc[a][b][v];
        }
#pragma unroll
        for (int a = 0; a < T::FM; a++)
#pragma unroll
            for (int b = 0; b < T::FN; b++) {
                const int j = j0 + wn * T::WN + b * 32 + col;
                if (j >= No) continue;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int i = i0 + wm * T::WM + a * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                    if (i < Mo) put(i, j, acc[a][b][v]);
                }
            }
    } else {
        // fragment-order index of (wave-in-group g, a, b, v, lane)
        const int g = T::wave() % (T::WGM * T::WGN);
        float *mine = red + T::wk() * T::TILE;
#pragma unroll
        for (int a = 0; a < T::FM; a++)
#pragma unroll
            for (int b = 0; b < T::FN; b++)
#pragma unroll
                for (int v = 0; v < 16; v++)
                    mine[(((g * T::FM + a) * T::FN + b) * 16 + v) * 64 + lane] = acc[a][b][v];
        __syncthreads();
#pragma unroll 4
        for (int f = threadIdx.x; f < T::TILE; f += T::THREADS) {
            float s = red[f];
#pragma unroll
            for (int k = 1; k < T::WK; k++) s += red[k * T::TILE + f];
            const int l = f & 63, v = (f >> 6) & 15, ab = f >> 10;
            const int b = ab % T::FN, a = (ab / T::FN) % T::FM, gg = ab / (T::FN * T::FM);
            const int i = i0 + (gg / T::WGN) * T::WM + a * 32 + 8 * (v >> 2) + 4 * (l >> 5) + (v & 3);
            const int j = j0 + (gg % T::WGN) * T::WN + b * 32 + (l & 31);
            if (i < Mo && j < No) put(i, j, s);
            if constexpr (STASH) red[f] = s;     // only this thread reads slot f of slice 0
        }
        __syncthreads();            // `red` aliases the stage buffers of the next tile
    }
}

// One output element of a tile: a streaming store for the Sched<T, 4 + ..>
// shapes (it goes past the L2, so the kernel's end does not wait to write
// back lines the next launch reads through another XCD's L2 anyway).
template <class T>
__device__ __forceinline__ void st_out(float *p, float v)
{
    if constexpr ((T::SCH & 4) != 0) __builtin_nontemporal_store(v, p);
    else *p = v;
}

// C (beta ? += : =) acc for the valid part of the tile.
template <class T>
__device__ __forceinline__ void tile_store(const f32x16 (&accs)[T::FM][T::FN][T::NCH], float *__restrict__ C,
                                           int ldc, int beta, int Mo, int No, int i0, int j0,
                                           float *__restrict__ red)
{
    tile_epi<T>(accs, Mo, No, i0, j0, red, [&](int i, int j, float v) {
        float *p = C + (size_t)i * ldc + j;
        st_out<T>(p, beta ? (*p + v) : v);
    });
}

// C = acc (beta 0) and, for every 32-column block of each valid row, the dot
// product of the block with the same block of O:  out[i][j / 32] =
// sum_{c < 32} C[i][32 (j / 32) + c] O[i][32 (j / 32) + c] (O with C's row
// stride, out [Mo][No / 32]).  This is the attention backward's per-row term
// D = dO . O of each 32-wide head (tinylm.c:750-768) formed where dO is made
// (the O-projection backward's dX tile), in the dQ item's order: two 16-term
// fma chains, then their sum.  Needs No % 32 == 0 and TILE <= the LDS the
// tile's stages use (every shape but the 128 x 128 ones; the host checks).
template <class T>
__device__ __forceinline__ void tile_store_dot(const f32x16 (&accs)[T::FM][T::FN][T::NCH], float *__restrict__ C,
                                               int ldc, int Mo, int No, int i0, int j0, const float *__restrict__ O,
                                               float *__restrict__ out, float *__restrict__ red)
{
    if constexpr (T::TILE <= T::lds_max()) {
        tile_epi<T, true>(accs, Mo, No, i0, j0, red,
                          [&](int i, int j, float v) { st_out<T>(C + (size_t)i * ldc + j, v); });
        __syncthreads();
        // eight lanes per (row, block), lane q holding float4 q of the block
        // (a wave's O loads: eight 128-byte row segments); each half's chain
        // passes through its four lanes in order, lane q continuing the sum
        // lane q - 1 ended with.  Every count here is a multiple of 64, so
        // whole waves take part in the shuffles.
        constexpr int NB = T::BN / 32;
        static_assert(T::BM * NB * 8 % 64 == 0, "whole waves");
        const int q = threadIdx.x & 7;
        for (int p8 = threadIdx.x; p8 < T::BM * NB * 8; p8 += T::THREADS) {
            const int p = p8 >> 3, row = p / NB, cb = p % NB;
            const int i = i0 + row, jb = j0 + cb * 32;
            // fragment-order index of (row, column 0 of block cb)
            const int rr = row % T::WM, a = rr / 32, r32 = rr % 32;
            const int v = 4 * (r32 >> 3) + (r32 & 3), hb = (r32 >> 2) & 1;
            const int b = ((cb * 32) % T::WN) / 32;
            const int g = (row / T::WM) * T::WGN + (cb * 32) / T::WN;
            const f32x4 x = *reinterpret_cast<const f32x4 *>(
                red + ((((g * T::FM + a) * T::FN + b) * 16 + v) * 64 + hb * 32) + 4 * q);
            const int ic = min(i, Mo - 1), jc = min(jb, No - 32);
            const f32x4 y = *reinterpret_cast<const f32x4 *>(O + (size_t)ic * ldc + jc + 4 * q);
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
            if (q == 7 && i < Mo && jb < No) out[(size_t)i * (No / 32) + jb / 32] = h0 + d;
        }
        __syncthreads();
    }
}

// 1 / (1 + e^-z) with the hardware exp2 and reciprocal (within a few ulp of
// the reference's expf and division; e^-z = inf gives 0, as there).
__device__ __forceinline__ float hw_sigmoid(float z)
{
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z * -1.44269504088896341f));
}

// LDS of an expert-launch workgroup: the tile's stages or partials, and the
// SwiGLU epilogue's staged tile beside the partials.
template <class T>
__host__ __device__ constexpr int expert_lds()
{
    return T::mx(T::lds_max(), (T::WK > 1 ? T::WK * T::TILE : 0) + T::BM * (T::BN + 1));
}

// SwiGLU epilogue of a paired-column tile (TileLoader PB): tile columns
// [0, BN/2) hold g = X W1 and [BN/2, BN) hold u = X W3 for the output
// columns jh + [0, BN/2).  The summed tile goes through LDS (after the WK
// partials, which it must not overlap) so one thread sees both halves; then
// a = silu(g) u  (tinylm.c:786, :882) for i < Mo, j < No, and g, u too where
// Cg / Cu are given.
template <class T>
__device__ __forceinline__ void tile_swiglu(const f32x16 (&accs)[T::FM][T::FN][T::NCH], float *__restrict__ Ca,
                                            float *__restrict__ Cg, float *__restrict__ Cu, int ldc, int Mo,
                                            int No, int i0, int jh, float *__restrict__ red)
{
    constexpr int H = T::BN / 2, LD = T::BN + 1;
    constexpr int OFF = T::WK > 1 ? T::WK * T::TILE : 0;
    static_assert(OFF + T::BM * LD <= expert_lds<T>(), "paired tile fits beside the partials");
    float *L = red + OFF;
    tile_epi<T>(accs, T::BM, T::BN, 0, 0, red, [&](int i, int j, float v) { L[i * LD + j] = v; });
    __syncthreads();
    for (int f = threadIdx.x; f < T::BM * H; f += T::THREADS) {
        const int x = f / H, c = f % H;
        const int i = i0 + x, j = jh + c;
        if (i >= Mo || j >= No) continue;
        const float g = L[x * LD + c], u = L[x * LD + c + H];
        const size_t o = (size_t)i * ldc + j;
        st_out<T>(Ca + o, g * hw_sigmoid(g) * u);
        if (Cg) st_out<T>(Cg + o, g);
        if (Cu) st_out<T>(Cu + o, u);
    }
    __syncthreads();
}

template <int FM, int FN, int NCH>
__device__ __forceinline__ void zero_acc(f32x16 (&acc)[FM][FN][NCH])
{
#pragma unroll
    for (int a = 0; a < FM; a++)
#pragma unroll
        for (int b = 0; b < FN; b++)
#pragma unroll
            for (int c = 0; c < NCH; c++)
#pragma unroll
                for (int v = 0; v < 16; v++) acc[a][b][c][v] = 0.f;
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

template <class T, int LA, int LB, bool VEC>
__global__ __launch_bounds__(T::THREADS) void k_gemm(GemmArgs g)
{
    __shared__ __attribute__((aligned(16))) float smem[T::template lds<LA, LB>()];
    const int item = xcd_remap(blockIdx.x, gridDim.x);
    const int z = item / g.tiles, tile = item % g.tiles;
    const int i0 = (tile / g.tiles_n) * T::BM, j0 = (tile % g.tiles_n) * T::BN;
    const int rbeg = z * g.rps;
    const int rend = min(g.R, rbeg + g.rps);
    f32x16 acc[T::FM][T::FN][T::NCH];
    zero_acc(acc);
    tile_accumulate<T, LA, LB, VEC>(smem, g.A, g.B, g.lda, g.ldb, i0, j0, g.Mo, g.No, rbeg, rend, acc);
    // a split writes its partial (beta 0) into workspace slice z
    if (g.splits > 1)
        tile_store<T>(acc, g.ws + (size_t)z * g.Mo * g.No, g.No, 0, g.Mo, g.No, i0, j0, smem);
    else
        tile_store<T>(acc, g.C, g.ldc, g.beta, g.Mo, g.No, i0, j0, smem);
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
enum { PK_NN = 0, PK_NT = 1, PK_TN = 2, PK_RED = 3, PK_ZERO = 4, PK_COLSUM = 5 };
#define TLG_ZERO_CHUNK 4096          // floats a clear's work item sets to 0
#define TLG_MAXSEG 3
#define TLG_MAXPROB 16                // group_item pins 16 counts
#define TLG_RED_CHUNK 256
#define TLG_ERED_CHUNK 2048            // elements per work item of an expert reduction

struct Seg { const float *A, *B; int R, lda, ldb; };
// The fields every work item reads lie in the first 160 bytes (C to items,
// then the segments), so a workgroup fetches them in a few scalar loads
// issued together.
struct Prob {
    float *C;
    const float *ws;      // PK_RED: partials; split GEMM: its partial slice base
    int Mo, No, ldc, beta;
    int kind, nseg;
    int tiles_n, tiles, splits, rps;
    int items;            // work items: tiles * splits, or reduction chunks
    Seg seg[TLG_MAXSEG];
    // Expert-batched problem (nexp > 0): the rows of a top-1 MoE layer are
    // grouped by expert, expert e owning rows [eoff[e], eoff[e+1]) of every
    // row operand.  NN / NT: the output rows are expert rows and the weight
    // operand B of expert e is B + e*es.  TN: the reduction runs over expert
    // rows in slices of rps, and the output of expert e is C + e*es.  `unit`
    // is the row extent of one item (BM for NN / NT, rps for TN).
    const int *eoff;
    long long es;
    int nexp, unit;
    // Fused forms of the MoE expert GEMMs (tinylm.c:876-888, :911-927):
    //   amap  A rows gathered through it (the sorted row -> token index)
    //   B2    NN: second weight of a column pair (W3 beside W1), SwiGLU
    //         epilogue; tiles_n then counts BN/2-column tiles
    //   epi   TLG_EPI_*: plain store, SwiGLU (C = a, X1 = g, X2 = u when
    //         given), SwiGLU backward (da from the tile, g / u in X1 / X2
    //         replaced by dg / du; C unused), or the top-1 combine (C = out,
    //         out[omap[i]] = fin[..] + gate[..] * tile row i; X1 = the rows
    //         themselves, sorted order, when given); on a dense NT problem
    //         ROWDOT: C stored, and X1 [Mo][No/32] the dot of each row's
    //         32-column blocks with those of `fin` (tile_store_dot)
    const int *amap, *omap;
    const float *B2;
    float *X1, *X2;
    const float *fin, *gate;
    int epi;
};
// items / devcount: filled from p[] by group_seal() before every launch (0
// past nprob), so the search for a workgroup's problem reads one contiguous
// block of counts instead of one problem struct after another.
struct GroupArgs {
    int nprob;
    int rows1;            // expert launches: > 0 = one expert owning rows [0, rows1)
    int items[TLG_MAXPROB];
    unsigned devcount;    // bit p: problem p's count is known only on the device (experts)
    Prob p[TLG_MAXPROB];
};

// Real work items of an expert-batched problem, from the device-resident
// row offsets: sum over experts of ceil(rows_e / unit) row units, times the
// column tiles (NN / NT) or the output tiles (TN).
__device__ __forceinline__ int expert_items(const Prob &P, const int *eo)
{
    int units = 0;
    for (int e = 0; e < P.nexp; e++) {
        const int c = eo[e + 1] - eo[e];
        units += c > 0 ? (c + P.unit - 1) / P.unit : 0;
    }
    return units * (P.kind == PK_TN ? P.tiles : P.tiles_n);
}

// Item -> (expert e, row unit t of that expert, first partial slot of e).
// Returns false when the item is past the experts' real work.
__device__ __forceinline__ bool expert_of(const Prob &P, const int *eo, int t, int *e_out, int *t_out,
                                          int *base, int *rows, int *slot0)
{
    int slot = 0;
    for (int e = 0; e < P.nexp; e++) {
        const int b = eo[e], c = eo[e + 1] - b;
        const int n = c > 0 ? (c + P.unit - 1) / P.unit : 0;
        if (t < n) { *e_out = e; *t_out = t; *base = b; *rows = c; *slot0 = slot; return true; }
        t -= n;
        slot += n;
    }
    return false;
}

// Accumulation of one expert tile, with its gather / pair form chosen at run
// time (uniform per problem): PB only for NN problems.
template <class T, int LA, int LB>
__device__ __forceinline__ void expert_acc(float *smem, const Prob &P, const Seg &s, const float *A,
                                           const float *B, const int *amap, int i0, int j0, int Mo, int No,
                                           int rbeg, int rend, f32x16 (&acc)[T::FM][T::FN][T::NCH])
{
    if constexpr (LA == RC && LB == OC) {
        if (P.B2) {
            const float *B2 = P.B2 + (B - s.B);
            if (amap)
                tile_accumulate<T, LA, LB, true, true, true>(smem, A, B, s.lda, s.ldb, i0, j0, Mo, No, rbeg,
                                                             rend, acc, amap, B2);
            else
                tile_accumulate<T, LA, LB, true, false, true>(smem, A, B, s.lda, s.ldb, i0, j0, Mo, No, rbeg,
                                                              rend, acc, nullptr, B2);
            return;
        }
    }
    if (amap)
        tile_accumulate<T, LA, LB, true, true>(smem, A, B, s.lda, s.ldb, i0, j0, Mo, No, rbeg, rend, acc, amap);
    else
        tile_accumulate<T, LA, LB, true>(smem, A, B, s.lda, s.ldb, i0, j0, Mo, No, rbeg, rend, acc);
}

template <class T, int LA, int LB>
__device__ __forceinline__ void expert_tile(float *smem, const Prob &P, int local, const int *eo)
{
    f32x16 acc[T::FM][T::FN][T::NCH];
    int e, t, base, rows, slot0;
    if (P.kind != PK_TN) {
        if (!expert_of(P, eo, local / P.tiles_n, &e, &t, &base, &rows, &slot0)) return;
        // a paired tile covers BN/2 output columns
        const int i0 = t * T::BM, j0 = (local % P.tiles_n) * (P.B2 ? T::BN / 2 : T::BN);
        // combine: the tile rows' tokens and gates, staged before the
        // accumulation so the epilogue waits on one load level, not three
        __shared__ int s_tok[(LA == RC && LB == OC) ? T::BM : 1];
        __shared__ float s_gate[(LA == RC && LB == OC) ? T::BM : 1];
        if constexpr (LA == RC && LB == OC) {
            if (P.epi == TLG_EPI_COMBINE && (int)threadIdx.x < T::BM) {
                const int x = threadIdx.x, n = P.omap[base + min(i0 + x, rows - 1)];
                s_tok[x] = n;
                s_gate[x] = P.gate[n];
            }
        }
        zero_acc(acc);
        for (int k = 0; k < P.nseg; k++) {
            const Seg &s = P.seg[k];
            // gathered: rows of A through amap[base + x]; else A's expert rows
            const float *A = P.amap ? s.A : s.A + (size_t)base * s.lda;
            const int *amap = P.amap ? P.amap + base : nullptr;
            expert_acc<T, LA, LB>(smem, P, s, A, s.B + (size_t)e * P.es, amap, i0, j0, rows, P.No, 0, s.R,
                                  acc);
        }
        const size_t cb = (size_t)base * P.ldc;
        switch (P.epi) {
        case TLG_EPI_SWIGLU:
            tile_swiglu<T>(acc, P.C + cb, P.X1 ? P.X1 + cb : nullptr, P.X2 ? P.X2 + cb : nullptr, P.ldc, rows,
                           P.No, i0, j0, smem);
            break;
        case TLG_EPI_SWIGLU_BWD: {
            // In place: g <- da u silu'(g), u <- da silu(g)  (tinylm.c:923-925)
            float *G = P.X1 + cb, *U = P.X2 + cb;
            const int ld = P.ldc;
            tile_epi<T>(acc, rows, P.No, i0, j0, smem, [&](int i, int j, float d) {
                const size_t o = (size_t)i * ld + j;
                const float z = G[o], uv = U[o];
                const float sg = hw_sigmoid(z);
                const float si = z * sg;
                const float ds = sg + z * sg * (1.0f - sg);
                st_out<T>(G + o, d * uv * ds);
                st_out<T>(U + o, d * si);
            });
            break;
        }
        case TLG_EPI_COMBINE: {
            // out[n] = fin[n] + gate[n] y  for token n of sorted row i (:870, :886-888)
            if constexpr (LA == RC && LB == OC) {
                __syncthreads();          // the staged tokens, also when the reduction was empty
                const int ld = P.ldc;
                float *C = P.C;
                const float *fin = P.fin;
                float *Y = P.X1 ? P.X1 + cb : nullptr;      // the expert rows too, when kept
                tile_epi<T>(acc, rows, P.No, i0, j0, smem, [&](int i, int j, float y) {
                    const int x = i - i0;
                    const size_t o = (size_t)s_tok[x] * ld + j;
                    st_out<T>(C + o, fmaf(s_gate[x], y, fin[o]));
                    if (Y) st_out<T>(Y + (size_t)i * ld + j, y);
                });
            }
            break;
        }
        default:
            tile_store<T>(acc, P.C + cb, P.ldc, P.beta, rows, P.No, i0, j0, smem);
        }
    } else {
        if (!expert_of(P, eo, local / P.tiles, &e, &t, &base, &rows, &slot0)) return;
        const int tile = local % P.tiles;
        const int i0 = (tile / P.tiles_n) * T::BM, j0 = (tile % P.tiles_n) * T::BN;
        const int rbeg = base + t * P.unit, rend = min(base + rows, rbeg + P.unit);
        const Seg &s = P.seg[0];
        zero_acc(acc);
        // A's reduction rows are sorted rows; gathered ones map through amap
        expert_acc<T, LA, LB>(smem, P, s, s.A, s.B, P.amap, i0, j0, P.Mo, P.No, rbeg, rend, acc);
        tile_store<T>(acc, (float *)P.ws + (size_t)(slot0 + t) * P.Mo * P.No, P.No, 0, P.Mo, P.No, i0, j0,
                      smem);
    }
}

// Reduction of an expert TN problem: C_e (beta ? += : =) the sum of expert
// e's partial slots, in slot order.
__device__ __forceinline__ void expert_reduce(const Prob &P, int local, const int *eo)
{
    const size_t n = (size_t)P.Mo * P.No;
    const int chunks = (int)((n + TLG_ERED_CHUNK - 1) / TLG_ERED_CHUNK);
    const int e = local / chunks;
    int slot0 = 0;
    for (int k = 0; k < e; k++) {
        const int c = eo[k + 1] - eo[k];
        slot0 += c > 0 ? (c + P.unit - 1) / P.unit : 0;
    }
    const int c = eo[e + 1] - eo[e];
    const int ns = c > 0 ? (c + P.unit - 1) / P.unit : 0;
    const size_t e0 = (size_t)(local % chunks) * TLG_ERED_CHUNK;
    const size_t e1 = e0 + TLG_ERED_CHUNK < n ? e0 + TLG_ERED_CHUNK : n;
    float *C = P.C + (size_t)e * P.es;
    if (ns == 0) {
        if (!P.beta)
            for (size_t i = e0 + threadIdx.x; i < e1; i += blockDim.x) C[i] = 0.f;
        return;
    }
    reduce_range(P.ws + (size_t)slot0 * n, C, P.No, P.No, ns, P.beta, e0, e1, n);
}

template <class T, int LA, int LB, bool EXP>
__device__ __forceinline__ void group_tile(float *smem, const Prob &P, int local, const int *eo)
{
    if constexpr (EXP) {
        if (P.nexp) { expert_tile<T, LA, LB>(smem, P, local, eo); return; }
    }
    const int z = local / P.tiles, tile = local % P.tiles;
    const int i0 = (tile / P.tiles_n) * T::BM, j0 = (tile % P.tiles_n) * T::BN;
    f32x16 acc[T::FM][T::FN][T::NCH];
    zero_acc(acc);
    if (P.splits > 1) {
        const Seg &s = P.seg[0];
        const int rbeg = z * P.rps, rend = min(s.R, rbeg + P.rps);
        tile_accumulate<T, LA, LB, true>(smem, s.A, s.B, s.lda, s.ldb, i0, j0, P.Mo, P.No, rbeg, rend, acc);
        tile_store<T>(acc, (float *)P.ws + (size_t)z * P.Mo * P.No, P.No, 0, P.Mo, P.No, i0, j0, smem);
        return;
    }
    for (int k = 0; k < P.nseg; k++) {
        const Seg &s = P.seg[k];
        tile_accumulate<T, LA, LB, true>(smem, s.A, s.B, s.lda, s.ldb, i0, j0, P.Mo, P.No, 0, s.R, acc);
    }
    if (LA == RC && LB == OC && P.fin) {
        // mm with its residual add: C = R + acc (R in `fin`, C's layout)
        float *C = P.C;
        const float *Rr = P.fin;
        const int ld = P.ldc;
        tile_epi<T>(acc, P.Mo, P.No, i0, j0, smem, [&](int i, int j, float v) {
            const size_t o = (size_t)i * ld + j;
            st_out<T>(C + o, Rr[o] + v);
        });
        return;
    }
    if constexpr (LA == RC && LB == RC) {
        if (P.epi == TLG_EPI_ROWDOT) {
            tile_store_dot<T>(acc, P.C, P.ldc, P.Mo, P.No, i0, j0, P.fin, P.X1, smem);
            return;
        }
    }
    tile_store<T>(acc, P.C, P.ldc, P.beta, P.Mo, P.No, i0, j0, smem);
}

// Work-item mapping of a grouped launch.  The dispatcher deals workgroup b
// to XCD b % 8; XCD x takes an equal contiguous slice of EVERY problem's
// items (so each XCD's L2 sees neighbouring tiles of a problem, and every
// XCD gets the same mix of long and short items), problem by problem in
// list order (the host lists problems longest item first).  Workgroups past
// their XCD's share exit at once.
static_assert(TLG_MAXPROB == 16, "group_item pins exactly 16 item counts");
__device__ __forceinline__ int group_item(const GroupArgs &g, int b, int *local, const int *eo)
{
    const int x = b & 7;
    int slot = b >> 3;
    int cnt[TLG_MAXPROB];
#pragma unroll
    for (int p = 0; p < TLG_MAXPROB; p++) cnt[p] = g.items[p];
    const unsigned dev = g.devcount;
    // every count in flight at once: one round trip, then scalar arithmetic
    // (counts past nprob are 0, so nprob itself is not needed)
    asm volatile("" ::"s"(dev), "s"(cnt[0]), "s"(cnt[1]), "s"(cnt[2]), "s"(cnt[3]), "s"(cnt[4]), "s"(cnt[5]),
                 "s"(cnt[6]), "s"(cnt[7]), "s"(cnt[8]), "s"(cnt[9]), "s"(cnt[10]), "s"(cnt[11]), "s"(cnt[12]),
                 "s"(cnt[13]), "s"(cnt[14]), "s"(cnt[15]));
#pragma unroll
    for (int p = 0; p < TLG_MAXPROB; p++) {
        // expert-batched GEMMs: the real item count, known only on the device
        const int n = (dev >> p & 1u) ? expert_items(g.p[p], eo) : cnt[p];
        const int lo = (x * n) >> 3, hi = ((x + 1) * n) >> 3;
        if (slot < hi - lo) { *local = lo + slot; return p; }
        slot -= hi - lo;
    }
    return -1;
}

// `eo`: the expert row offsets of an expert-batched launch, staged in LDS
// (nullptr for dense launches, which have no expert problems).
// PK_COLSUM: C[0, No) (beta ? += : =) the sum of the `splits` partial rows
// ws[z][0, No) (a row-block reduction queued by tlg_defer_colsum).  Item
// `local` covers float4 columns [4 local, 4 local + 4), one wave per
// column at a time: lane l adds rows l, l + 64, ... in order, then a fixed
// butterfly, so the sum does not depend on timing.
#define TLG_COLSUM_CH 4
__device__ __forceinline__ void colsum(const Prob &P, int local)
{
    const int lane = threadIdx.x & 63, nw = blockDim.x >> 6, w = threadIdx.x >> 6;
    const int c4 = P.No >> 2, cend = min(TLG_COLSUM_CH * (local + 1), c4);
    for (int c = TLG_COLSUM_CH * local + w; c < cend; c += nw) {
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
        for (int z = lane; z < P.splits; z += 64) s += reinterpret_cast<const f32x4 *>(P.ws + (size_t)z * P.No)[c];
        for (int o = 32; o > 0; o >>= 1) {
            s.x += __shfl_xor(s.x, o);
            s.y += __shfl_xor(s.y, o);
            s.z += __shfl_xor(s.z, o);
            s.w += __shfl_xor(s.w, o);
        }
        if (lane == 0) {
            f32x4 *out = reinterpret_cast<f32x4 *>(P.C) + c;
            *out = P.beta ? *out + s : s;
        }
    }
}

template <class T, bool EXP>
__device__ __forceinline__ void group_body(const GroupArgs &g, float *smem, const int *eo)
{
    int local = 0;
    const int p = group_item(g, blockIdx.x, &local, eo);
    if (p < 0) return;
    const Prob &P = g.p[p];
    // The fields a tile reads first, fetched together: one round trip to the
    // argument block before the tile's first loads, not one per field.
    asm volatile("" ::"s"(P.kind), "s"(P.nseg), "s"(P.Mo), "s"(P.No), "s"(P.tiles), "s"(P.tiles_n),
                 "s"(P.splits), "s"(P.rps), "s"(P.seg[0].A), "s"(P.seg[0].B), "s"(P.seg[0].R), "s"(P.seg[0].lda),
                 "s"(P.seg[0].ldb));
    switch (P.kind) {
    case PK_NN: group_tile<T, RC, OC, EXP>(smem, P, local, eo); break;
    case PK_NT: group_tile<T, RC, RC, EXP>(smem, P, local, eo); break;
    case PK_TN: group_tile<T, OC, OC, EXP>(smem, P, local, eo); break;
    case PK_COLSUM: colsum(P, local); break;
    case PK_ZERO: {
        const size_t n = (size_t)P.Mo * P.No, e0 = (size_t)local * TLG_ZERO_CHUNK;
        const size_t e1 = e0 + TLG_ZERO_CHUNK < n ? e0 + TLG_ZERO_CHUNK : n;
        for (size_t e = e0 + threadIdx.x; e < e1; e += blockDim.x) P.C[e] = 0.f;
        break;
    }
    default: {
        if constexpr (EXP) {
            if (P.nexp) { expert_reduce(P, local, eo); break; }
        }
        const size_t n = (size_t)P.Mo * P.No;
        const size_t e0 = (size_t)local * TLG_RED_CHUNK;
        const size_t e1 = e0 + TLG_RED_CHUNK < n ? e0 + TLG_RED_CHUNK : n;
        reduce_range(P.ws, P.C, P.No, P.ldc, P.splits, P.beta, e0, e1, n);
    }
    }
}

template <class T>
__global__ __launch_bounds__(T::THREADS) void k_group(GroupArgs g)
{
    __shared__ __attribute__((aligned(16))) float smem[T::lds_max()];
    group_body<T, false>(g, smem, nullptr);
}

// The same code for the expert-batched launches of the MoE layer, under its
// own name so profiles separate MoE launches from the dense grouped GEMMs.
// Every problem of such a launch shares one row-offset array; it is staged in
// LDS once, so finding a work item's expert costs no dependent global loads.
// The fused variants (gathered rows, paired columns, epilogues) are separate
// inlined code paths; left alone the compiler gives their accumulators
// disjoint AGPRs and the kernel drops to 3 waves per SIMD, so it is held to
// the dense kernels' 4 (no spills at that bound).
#define TLG_MAX_EXPERTS 64
template <class T>
__global__ __launch_bounds__(T::THREADS) __attribute__((amdgpu_waves_per_eu(4))) void k_expert_group(GroupArgs g)
{
    __shared__ __attribute__((aligned(16))) float smem[expert_lds<T>()];
    __shared__ int eo[TLG_MAX_EXPERTS + 1];
    const int E = g.p[0].nexp;
    if (g.rows1 > 0) {
        if (threadIdx.x < 2) eo[threadIdx.x] = threadIdx.x ? g.rows1 : 0;
    } else {
        for (int i = threadIdx.x; i <= E; i += blockDim.x) eo[i] = g.p[0].eoff[i];
    }
    __syncthreads();
    group_body<T, true>(g, smem, eo);
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
// WGM x WGN waves over the tile, WK wave groups along the reduction.
struct TileCfg { int bm, bn, bk, wgm, wk, nw; };   // nw 0 = 4 waves
static const TileCfg kCfgs[] = {
    {128, 128, 16, 2, 1},   // 0: wave tile 64x64, 4 accumulator chains
    {128, 64, 32, 2, 1},    // 1: 64x32
    {64, 128, 32, 2, 1},    // 2: 32x64
    {64, 64, 32, 2, 1},     // 3: 32x32, one chain per wave
    {64, 64, 32, 1, 4},     // 4: 64x64 per wave over a quarter of each stage
    {64, 64, 64, 1, 4},     // 5: same, 64-step stages
    {64, 128, 32, 1, 2},    // 6: 64x64 per wave, half of each stage
    {128, 64, 32, 2, 2},    // 7: 64x64 per wave, half of each stage
    {64, 64, 64, 2, 1},     // 8: 32x32 per wave, 64-step stages
    {64, 64, 32, 2, 1},     // 9-12: 64x64 tiles (prefetch / chain variants)
    {64, 64, 32, 2, 1},
    {64, 64, 32, 2, 1},
    {64, 64, 32, 2, 1},
    {32, 64, 32, 1, 2},     // 13: 32x32 per wave, half of each stage
    {64, 32, 32, 2, 2},     // 14: 32x32 per wave, half of each stage
    {32, 32, 32, 1, 4},     // 15: 32x32 per wave, a quarter of each stage
    {64, 64, 32, 2, 1, 2},  // 16: 2 waves, 32x64 per wave
    {64, 64, 32, 1, 1, 2},  // 17: 2 waves, 64x32 per wave
    {64, 64, 16, 2, 1},     // 18: 32x32 per wave, 16-step stages
    {64, 64, 16, 2, 1},     // 19: same, loads three stages ahead
    {64, 64, 32, 2, 2, 8},  // 20: 8 waves, 32x32 per wave, half of each stage
    {64, 32, 64, 2, 2},     // 21: 32x32 per wave, half of each 64-step stage
    {64, 64, 64, 2, 4, 16}, // 22: 16 waves, 32x32 per wave, a quarter of each 64-step stage
    {64, 64, 64, 2, 2, 8},  // 23: 8 waves, 32x32 per wave, half of each 64-step stage
    {64, 64, 32, 2, 1},     // 24-25: 3 with a stage's fragment reads first (Sched 1, 2)
    {64, 64, 32, 2, 1},
    {64, 32, 32, 2, 2},     // 26: 14, Sched 1
    {64, 64, 32, 2, 2, 8},  // 27: 20, Sched 1
    {64, 64, 64, 2, 4, 16}, // 28: 22, Sched 1
    {32, 64, 32, 1, 2},     // 29: 13, Sched 1
    {32, 32, 32, 1, 4},     // 30: 15, Sched 1
    {128, 128, 16, 2, 1},   // 31: 0, Sched 1
    {128, 64, 32, 2, 1},    // 32: 1, Sched 1
    {64, 64, 64, 2, 1},     // 33: 8, Sched 1
    {64, 64, 32, 2, 1},     // 34: 11 (loads three stages ahead), Sched 1
    {64, 32, 64, 2, 2},     // 35: 21, Sched 1
    {64, 64, 64, 2, 2, 8},  // 36: 23, Sched 1
    {64, 64, 16, 2, 1},     // 37: 18, Sched 1
    {64, 64, 32, 2, 1},     // 38: 3, Sched 1 + streaming stores
    {64, 64, 16, 2, 1},     // 39: 18, Sched 1 + streaming stores
    {64, 32, 32, 2, 2},     // 40: 14, Sched 1 + streaming stores
    {64, 64, 64, 2, 4, 16}, // 41: 22, Sched 1 + streaming stores
    {64, 64, 32, 2, 2, 8}, // 42: 20, Sched 1 + streaming stores
    {32, 64, 32, 1, 2},    // 43: 13, Sched 1 + streaming stores
    {32, 32, 32, 1, 4},    // 44: 15, Sched 1 + streaming stores
    {128, 128, 16, 2, 1},  // 45: 0, Sched 1 + streaming stores
    {128, 64, 32, 2, 1},   // 46: 1, Sched 1 + streaming stores
    {64, 64, 64, 2, 1},    // 47: 8, Sched 1 + streaming stores
    {64, 64, 32, 2, 1},    // 48: 11, Sched 1 + streaming stores
    {64, 32, 64, 2, 2},    // 49: 21, Sched 1 + streaming stores
    {64, 64, 64, 2, 2, 8}, // 50: 23, Sched 1 + streaming stores
};
static const int kNumCfgs = (int)(sizeof(kCfgs) / sizeof(kCfgs[0]));
using T0 = Tile<128, 128, 16, 2, 1>;
using T1 = Tile<128, 64, 32, 2, 1>;
using T2 = Tile<64, 128, 32, 2, 1>;
using T3 = Tile<64, 64, 32, 2, 1>;
using T4 = Tile<64, 64, 32, 1, 4>;
using T5 = Tile<64, 64, 64, 1, 4>;
using T6 = Tile<64, 128, 32, 1, 2>;
using T7 = Tile<128, 64, 32, 2, 2>;
using T8 = Tile<64, 64, 64, 2, 1>;
// grouped-launch variants for sweeps: prefetch depth NR, chains per block
using T9 = Tile<64, 64, 32, 2, 1, 2, 2>;
using T10 = Tile<64, 64, 32, 2, 1, 2, 1>;
using T11 = Tile<64, 64, 32, 2, 1, 3, 1>;
using T12 = Tile<64, 64, 32, 2, 1, 3, 4>;
using T13 = Tile<32, 64, 32, 1, 2>;
using T14 = Tile<64, 32, 32, 2, 2>;
using T15 = Tile<32, 32, 32, 1, 4>;
using T16 = Tile<64, 64, 32, 2, 1, 2, 0, 2>;
using T17 = Tile<64, 64, 32, 1, 1, 2, 0, 2>;
using T18 = Tile<64, 64, 16, 2, 1, 2, 0, 4>;
using T19 = Tile<64, 64, 16, 2, 1, 3, 0, 4>;
using T20 = Tile<64, 64, 32, 2, 2, 2, 0, 8>;
using T21 = Tile<64, 32, 64, 2, 2, 2, 0, 4>;
using T22 = Tile<64, 64, 64, 2, 4, 2, 0, 16>;
using T23 = Tile<64, 64, 64, 2, 2, 2, 0, 8>;
using T24 = Sched<T3, 1>;
using T25 = Sched<T3, 2>;
using T26 = Sched<T14, 1>;
using T27 = Sched<T20, 1>;
using T28 = Sched<T22, 1>;
using T29 = Sched<T13, 1>;
using T30 = Sched<T15, 1>;
using T31 = Sched<T0, 1>;
using T32 = Sched<T1, 1>;
using T33 = Sched<T8, 1>;
using T34 = Sched<T11, 1>;
using T35 = Sched<T21, 1>;
using T36 = Sched<T23, 1>;
using T37 = Sched<T18, 1>;
using T38 = Sched<T3, 5>;
using T39 = Sched<T18, 5>;
using T40 = Sched<T14, 5>;
using T41 = Sched<T22, 5>;
using T42 = Sched<T20, 5>;
using T43 = Sched<T13, 5>;
using T44 = Sched<T15, 5>;
using T45 = Sched<T0, 5>;
using T46 = Sched<T1, 5>;
using T47 = Sched<T8, 5>;
using T48 = Sched<T11, 5>;
using T49 = Sched<T21, 5>;
using T50 = Sched<T23, 5>;

template <class T, int LA, int LB>
static void launch_t(const GemmArgs &a, int grid, bool vec, hipStream_t st)
{
    if (vec) hipLaunchKernelGGL((k_gemm<T, LA, LB, true>), dim3(grid), dim3(256), 0, st, a);
    else     hipLaunchKernelGGL((k_gemm<T, LA, LB, false>), dim3(grid), dim3(256), 0, st, a);
}

// Single-call launches of the automatic plan's shapes (0-3) in the Sched<.., 5>
// form (a stage's fragment reads before its MFMAs, streaming stores) unless
// TLG_GEMM_SCHED=0.
static int g_gemm_sched = -1;
static bool gemm_sched(void)
{
    if (g_gemm_sched < 0) {
        const char *e = getenv("TLG_GEMM_SCHED");
        g_gemm_sched = (e && *e) ? (atoi(e) != 0) : 1;
    }
    return g_gemm_sched != 0;
}

template <int LA, int LB>
static void launch_kind(int ci, const GemmArgs &a, int grid, bool vec, hipStream_t st)
{
    if (ci <= 3 && gemm_sched()) {
        switch (ci) {
        case 0: launch_t<Sched<T0, 5>, LA, LB>(a, grid, vec, st); return;
        case 1: launch_t<Sched<T1, 5>, LA, LB>(a, grid, vec, st); return;
        case 2: launch_t<Sched<T2, 5>, LA, LB>(a, grid, vec, st); return;
        default: launch_t<Sched<T3, 5>, LA, LB>(a, grid, vec, st); return;
        }
    }
    switch (ci) {
    case 0: launch_t<T0, LA, LB>(a, grid, vec, st); break;
    case 1: launch_t<T1, LA, LB>(a, grid, vec, st); break;
    case 2: launch_t<T2, LA, LB>(a, grid, vec, st); break;
    case 3: launch_t<T3, LA, LB>(a, grid, vec, st); break;
    case 4: launch_t<T4, LA, LB>(a, grid, vec, st); break;
    case 5: launch_t<T5, LA, LB>(a, grid, vec, st); break;
    case 6: launch_t<T6, LA, LB>(a, grid, vec, st); break;
    case 7: launch_t<T7, LA, LB>(a, grid, vec, st); break;
    case 13: launch_t<T13, LA, LB>(a, grid, vec, st); break;
    case 14: launch_t<T14, LA, LB>(a, grid, vec, st); break;
    case 15: launch_t<T15, LA, LB>(a, grid, vec, st); break;
    default: launch_t<T8, LA, LB>(a, grid, vec, st); break;
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
static GemmPlan plan_gemm(int Mo, int No, int R, size_t ws_floats)
{
    if (g_force_cfg >= 0 && g_force_cfg < kNumCfgs)
        return make_plan(g_force_cfg, Mo, No, R, g_force_splits, ws_floats);
    static const int order[] = {0, 1, 2, 3};
    for (int k = 0; k < 4; k++) {
        const TileCfg &c = kCfgs[order[k]];
        const int tiles = cdiv(Mo, c.bm) * cdiv(No, c.bn);
        if (tiles >= 240) return make_plan(order[k], Mo, No, R, 1, ws_floats);
    }
    const int tiles = cdiv(Mo, 64) * cdiv(No, 64);
    int splits = cdiv(256, tiles);
    const int maxs = R / 256 > 1 ? R / 256 : 1;
    if (splits > maxs) splits = maxs;
    return make_plan(3, Mo, No, R, splits, ws_floats);
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
    if (tlg_gemv_fits(kind, Mo)) {
        tlg_gemv_describe(kind, Mo, No, R, buf, len);
        if (splits) *splits = 1;
        return TLG_OK;
    }
    const GemmPlan p = plan_gemm(Mo, No, R, g_tlg.ws_floats);
    const TileCfg &c = kCfgs[p.ci];
    const int la = (kind == TLG_TN) ? OC : RC;
    const int lb = (kind == TLG_NT) ? RC : OC;
    const bool vec = (la == RC ? (R % 4 == 0) : (Mo % 4 == 0)) && (lb == RC ? (R % 4 == 0) : (No % 4 == 0));
    if (p.ci <= 3 && gemm_sched())
        snprintf(buf, (size_t)len, "k_gemm<Sched<Tile<%d, %d, %d, %d, %d, 2, 0, 4>, 5>, %d, %d, %s>", c.bm, c.bn,
                 c.bk, c.wgm, c.wk, la, lb, vec ? "true" : "false");
    else
        snprintf(buf, (size_t)len, "k_gemm<Tile<%d, %d, %d, %d, %d, 2, 0, 4>, %d, %d, %s>", c.bm, c.bn, c.bk,
                 c.wgm, c.wk, la, lb, vec ? "true" : "false");
    if (splits) *splits = p.splits;
    return TLG_OK;
}

extern "C" int tlg_tune_force(int cfg, int splits)
{
    // single-call launches instantiate configs 0-15 (16+ are grouped-only shapes)
    if (cfg >= 16) return tlg_fail(TLG_EINVAL, "tlg_tune_force: config %d of 16", cfg);
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

// One GEMM on `st` whose split partials (if any) go to ws[0, ws_floats).
// Allocates nothing: the caller owns ws (the library's workspace, or the
// no-allocation scratch below).  max_splits caps the reduction split.
static int gemm_launch_ws(TlgKind kind, const float *A, const float *B, float *C, int Mo, int No, int R,
                          int lda, int ldb, int ldc, int beta, float *ws, size_t ws_floats, hipStream_t st)
{
    if (tlg_gemv_fits(kind, Mo)) return tlg_gemv_launch(kind, A, B, C, Mo, No, R, lda, ldb, ldc, beta, st);

    const int la = (kind == TLG_TN) ? OC : RC;
    const int lb = (kind == TLG_NT) ? RC : OC;
    // float4 staging needs 16-byte aligned operands whose contiguous extent
    // and leading dimension are multiples of 4.
    const bool vec = al16(A) && al16(B) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                     (la == RC ? (R % 4 == 0) : (Mo % 4 == 0)) &&
                     (lb == RC ? (R % 4 == 0) : (No % 4 == 0));
    // the split count the library workspace would give, reduced to what ws holds
    GemmPlan pl = plan_gemm(Mo, No, R, TLG_WS_FLOATS);
    if (pl.splits > 1 && (size_t)pl.splits * Mo * No > ws_floats)
        pl = make_plan(pl.ci, Mo, No, R, (int)(ws_floats / ((size_t)Mo * No)), ws_floats);

    GemmArgs a;
    a.A = A; a.B = B; a.C = C;
    a.Mo = Mo; a.No = No; a.R = R;
    a.lda = lda; a.ldb = ldb; a.ldc = ldc;
    a.beta = beta;
    a.tiles_n = pl.tiles_n; a.tiles = pl.tiles;
    a.splits = pl.splits; a.rps = pl.rps;
    a.ws = ws;
    const int grid = pl.tiles * pl.splits;
    if (la == RC && lb == OC)      launch_kind<RC, OC>(pl.ci, a, grid, vec, st);
    else if (la == RC && lb == RC) launch_kind<RC, RC>(pl.ci, a, grid, vec, st);
    else                           launch_kind<OC, OC>(pl.ci, a, grid, vec, st);
    TLG_HIP(hipGetLastError());
    if (pl.splits > 1) return launch_reduce(ws, C, Mo, No, ldc, pl.splits, beta, st);
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
    return gemm_launch_ws(kind, A, B, C, Mo, No, R, lda, ldb, ldc, beta, g_tlg.ws, g_tlg.ws_floats, st);
}

// --------------------------------------------- mm_atb without allocation --
// Callers that must not allocate device memory (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc) get mm_atb with
// its split partials in this fixed array instead of the library workspace.
// Each GPU the library runs on holds its own copy until the process ends.
// Host code never passes `scratch` itself to a kernel (on the host the name
// is only a stand-in); it uses the device address hipGetSymbolAddress gives
// for the current device, looked up once per device.
#define TLG_SCRATCH_FLOATS ((size_t)4 << 20)          // 16 MiB
static __device__ __align__(256) float scratch[TLG_SCRATCH_FLOATS];

#define TLG_MAX_DEVICES 64
static float *g_scratch_dev[TLG_MAX_DEVICES];
static std::mutex g_scratch_mu;

static int scratch_for_current_device(float **out)
{
    int dev = -1;
    TLG_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= TLG_MAX_DEVICES) return tlg_fail(TLG_EINVAL, "no-alloc scratch: device %d", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        TLG_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return tlg_fail(TLG_EHIP, "no-alloc scratch: no device address on device %d", dev);
        g_scratch_dev[dev] = (float *)p;
    }
    *out = g_scratch_dev[dev];
    return TLG_OK;
}

extern "C" int tlg_dev_sgemm_tn_acc_noalloc(float *dW, const float *X, const float *dY, int M, int K, int N,
                                            void *stream)
{
    if (M < 0 || K < 0 || N < 0) return tlg_fail(TLG_EINVAL, "negative dimension");
    if ((size_t)K * N > TLG_SCRATCH_FLOATS / 2)
        return tlg_fail(TLG_EINVAL,
                        "tlg_dev_sgemm_tn_acc_noalloc: dW of %d x %d floats exceeds the no-allocation limit of "
                        "%zu floats (half the %zu-float scratch)",
                        K, N, TLG_SCRATCH_FLOATS / 2, TLG_SCRATCH_FLOATS);
    if (K == 0 || N == 0 || M == 0) return TLG_OK;         // mm_atb adds nothing
    if (!dW || !X || !dY) return tlg_fail(TLG_EINVAL, "NULL pointer");
    hipStream_t st = (hipStream_t)stream;
    float *ws = nullptr;
    int rc = scratch_for_current_device(&ws);
    if (rc) return rc;
    // partials a grouped launch left for its successor must land first
    if (g_tlg.initialised) {
        rc = tlg_group_flush_launch(st);
        if (rc) return rc;
    }
    return gemm_launch_ws(TLG_TN, X, dY, dW, K, N, M, K, N, N, 1, ws, TLG_SCRATCH_FLOATS, st);
}

// ------------------------------------------------------- grouped launch --
// Host side of k_group.  Split partials of a grouped launch live in one half
// of the workspace and are reduced by the next grouped launch (or a flush);
// the halves alternate so a launch never overwrites partials still pending.
static Prob g_pending[TLG_MAXPROB];
static int g_npending = 0;
static hipStream_t g_pending_st = nullptr;     // the stream their partials were written on
#include <stdlib.h>
static int g_ws_half = 0;
static int flush_foreign(hipStream_t st);

// Tile shape of a grouped launch (all problems of a group share it): the
// first candidate that still gives every CU `g_min_waves` workgroups, else
// the last.  Measured on MI355X over the m3 training step (graph replay):
// 64x64 tiles where a launch has >= 3 x 256 of them, else 64x32 tiles whose
// two wave pairs split each stage's reduction (more, smaller work items and
// 5 waves per SIMD instead of 4), with dW splits of about 512 reduction
// steps: 1.548 ms/step, against 1.637 for 64x64 tiles and 384-step splits
// (m8: 6.95 against 7.91 ms).  TLG_GROUP_CANDS, TLG_GROUP_MINWAVES and
// TLG_GROUP_RTARGET (or tlg_tune_group_policy) override the policy,
// tlg_tune_group pins one shape.
static int g_group_cfg = -1;
static int g_group_rt = 0;               // split target pinned for the next launches (tlg_tune_group_split)
static double g_min_waves = 3.0;
static int g_cand[4] = {24, 26, -1, -1};  // 64x64, then 64x32 (2 x 2 waves), both in the Sched<.., 1> order
static int g_rtarget = 512;
static int g_erps = 1024;                // expert TN slice (TLG_EXPERT_RPS)
static int g_expert_cfg = -1;            // expert tile shape pinned (TLG_EXPERT_CFG: 3, 14, 15, 18, 22)
static int g_expert_sched = -1;          // expert tiles: 0 the compiler's order, 1 Sched<.., 1>, 2 Sched<.., 5>
                                         // (that order with streaming stores), -1 automatic: 2 for launches of
                                         // dense rows (the training step's fused SwiGLU: 2.003 -> 1.995 ms), 1 for
                                         // MoE launches (streaming measured 0.232 -> 0.237 ms per kept pair: the
                                         // next launch reads their g, u, a, y right away) (TLG_EXPERT_SCHED)
static int g_expert_bk16 = 1;            // 64x64 expert tiles with 16-step stages (TLG_EXPERT_BK16=0: 32-step)
static int g_expert_w16 = 0;             // 16-wave 64x64 tiles for launches short of 64x64 items (TLG_EXPERT_W16=1;
                                         // measured slower: kept MoE pair 0.2345 -> 0.2489 ms)
static int g_group_last = 3;          // shape of the most recent grouped launch
static const char *g_group_last_name = nullptr;   // set when that launch was a GEMV group

static void group_env(void)
{
    static int done = 0;
    if (done) return;
    done = 1;
    const char *e = getenv("TLG_GROUP_MINWAVES");
    if (e && atof(e) > 0) g_min_waves = atof(e);
    e = getenv("TLG_GROUP_CFG");
    if (e && *e) g_group_cfg = atoi(e);
    e = getenv("TLG_GROUP_CANDS");            // e.g. "3,13,15"
    if (e && *e) {
        int k = 0;
        for (const char *q = e; *q && k < 3; ) {
            g_cand[k++] = atoi(q);
            while (*q && *q != ',') q++;
            if (*q == ',') q++;
        }
        g_cand[k] = -1;
    }
    e = getenv("TLG_EXPERT_RPS");
    if (e && atoi(e) >= 64) g_erps = atoi(e);
    e = getenv("TLG_EXPERT_CFG");
    if (e && (atoi(e) == 3 || atoi(e) == 14 || atoi(e) == 15 || atoi(e) == 18 || atoi(e) == 22))
        g_expert_cfg = atoi(e);
    if ((e = getenv("TLG_EXPERT_SCHED")) && atoi(e) >= -1 && atoi(e) <= 2) g_expert_sched = atoi(e);
    if ((e = getenv("TLG_EXPERT_W16"))) g_expert_w16 = atoi(e) != 0;
    if ((e = getenv("TLG_EXPERT_BK16"))) g_expert_bk16 = atoi(e) != 0;
    e = getenv("TLG_GROUP_RTARGET");
    if (e && atoi(e) >= 64) g_rtarget = atoi(e);
}

// The item-count header of a launch's arguments (GroupArgs.items, devcount).
static const GroupArgs &group_seal(const GroupArgs &a)
{
    static GroupArgs b;
    b = a;
    b.devcount = 0;
    for (int p = 0; p < TLG_MAXPROB; p++) {
        b.items[p] = p < a.nprob ? a.p[p].items : 0;
        if (p < a.nprob && a.p[p].nexp && a.p[p].kind != PK_RED) b.devcount |= 1u << p;
    }
    return b;
}

template <class T>
static void lgroup(const GroupArgs &a, int grid, hipStream_t st)
{
    hipLaunchKernelGGL((k_group<T>), dim3(grid), dim3(T::THREADS), 0, st, group_seal(a));
}

static void launch_group(int ci, const GroupArgs &a, int grid, hipStream_t st)
{
    switch (ci) {
    case 0: lgroup<T0>(a, grid, st); break;
    case 1: lgroup<T1>(a, grid, st); break;
    case 4: lgroup<T4>(a, grid, st); break;
    case 8: lgroup<T8>(a, grid, st); break;
    case 9: lgroup<T9>(a, grid, st); break;
    case 10: lgroup<T10>(a, grid, st); break;
    case 11: lgroup<T11>(a, grid, st); break;
    case 12: lgroup<T12>(a, grid, st); break;
    case 13: lgroup<T13>(a, grid, st); break;
    case 14: lgroup<T14>(a, grid, st); break;
    case 15: lgroup<T15>(a, grid, st); break;
    case 16: lgroup<T16>(a, grid, st); break;
    case 17: lgroup<T17>(a, grid, st); break;
    case 18: lgroup<T18>(a, grid, st); break;
    case 19: lgroup<T19>(a, grid, st); break;
    case 20: lgroup<T20>(a, grid, st); break;
    case 21: lgroup<T21>(a, grid, st); break;
    case 22: lgroup<T22>(a, grid, st); break;
    case 23: lgroup<T23>(a, grid, st); break;
    case 24: lgroup<T24>(a, grid, st); break;
    case 25: lgroup<T25>(a, grid, st); break;
    case 26: lgroup<T26>(a, grid, st); break;
    case 27: lgroup<T27>(a, grid, st); break;
    case 28: lgroup<T28>(a, grid, st); break;
    case 29: lgroup<T29>(a, grid, st); break;
    case 30: lgroup<T30>(a, grid, st); break;
    case 31: lgroup<T31>(a, grid, st); break;
    case 32: lgroup<T32>(a, grid, st); break;
    case 33: lgroup<T33>(a, grid, st); break;
    case 34: lgroup<T34>(a, grid, st); break;
    case 35: lgroup<T35>(a, grid, st); break;
    case 36: lgroup<T36>(a, grid, st); break;
    case 37: lgroup<T37>(a, grid, st); break;
    case 38: lgroup<T38>(a, grid, st); break;
    case 39: lgroup<T39>(a, grid, st); break;
    case 40: lgroup<T40>(a, grid, st); break;
    case 41: lgroup<T41>(a, grid, st); break;
    case 42: lgroup<T42>(a, grid, st); break;
    case 43: lgroup<T43>(a, grid, st); break;
    case 44: lgroup<T44>(a, grid, st); break;
    case 45: lgroup<T45>(a, grid, st); break;
    case 46: lgroup<T46>(a, grid, st); break;
    case 47: lgroup<T47>(a, grid, st); break;
    case 48: lgroup<T48>(a, grid, st); break;
    case 49: lgroup<T49>(a, grid, st); break;
    case 50: lgroup<T50>(a, grid, st); break;
    default: lgroup<T3>(a, grid, st); break;
    }
    g_group_last = ci;
    g_group_last_name = nullptr;
}

extern "C" int tlg_tune_group_policy(const int *cands, int ncands, double min_waves, int rtarget)
{
    group_env();
    if (ncands < 0 || ncands > 3 || (ncands > 0 && !cands) || min_waves < 0 || (rtarget && rtarget < 64))
        return tlg_fail(TLG_EINVAL, "tlg_tune_group_policy: bad arguments");
    for (int k = 0; k < ncands; k++)
        if (cands[k] < 0 || cands[k] >= kNumCfgs || cands[k] == 2 || (cands[k] >= 5 && cands[k] <= 7))
            return tlg_fail(TLG_EINVAL, "tlg_tune_group_policy: config %d", cands[k]);
    if (ncands > 0) {
        for (int k = 0; k < ncands; k++) g_cand[k] = cands[k];
        g_cand[ncands] = -1;
    }
    if (min_waves > 0) g_min_waves = min_waves;
    if (rtarget) g_rtarget = rtarget;
    return TLG_OK;
}

extern "C" int tlg_tune_expert(int cfg, int sched)
{
    group_env();
    if ((cfg != -1 && cfg != 3 && cfg != 14 && cfg != 15 && cfg != 18 && cfg != 22) || sched < -1 || sched > 2)
        return tlg_fail(TLG_EINVAL, "tlg_tune_expert: config %d, order %d", cfg, sched);
    g_expert_cfg = cfg;
    g_expert_sched = sched;
    return TLG_OK;
}

extern "C" int tlg_tune_group(int cfg)
{
    if (cfg != -1 && cfg != 0 && cfg != 1 && cfg != 3 && cfg != 4 && (cfg < 8 || cfg >= kNumCfgs))
        return tlg_fail(TLG_EINVAL, "tlg_tune_group: config %d", cfg);
    g_group_cfg = cfg;
    return TLG_OK;
}

extern "C" int tlg_tune_group_split(int rtarget)
{
    if (rtarget != 0 && rtarget < 64)
        return tlg_fail(TLG_EINVAL, "tlg_tune_group_split: target %d (0 or >= 64)", rtarget);
    g_group_rt = rtarget;
    return TLG_OK;
}

const char *tlg_group_kernel_name(void)
{
    if (g_group_last_name) return g_group_last_name;
    switch (g_group_last) {
    case 0: return "k_group<Tile<128, 128, 16, 2, 1, 2, 0, 4> >";
    case 1: return "k_group<Tile<128, 64, 32, 2, 1, 2, 0, 4> >";
    case 4: return "k_group<Tile<64, 64, 32, 1, 4, 2, 0, 4> >";
    case 8: return "k_group<Tile<64, 64, 64, 2, 1, 2, 0, 4> >";
    case 9: return "k_group<Tile<64, 64, 32, 2, 1, 2, 2, 4> >";
    case 10: return "k_group<Tile<64, 64, 32, 2, 1, 2, 1, 4> >";
    case 11: return "k_group<Tile<64, 64, 32, 2, 1, 3, 1, 4> >";
    case 12: return "k_group<Tile<64, 64, 32, 2, 1, 3, 4, 4> >";
    case 13: return "k_group<Tile<32, 64, 32, 1, 2, 2, 0, 4> >";
    case 14: return "k_group<Tile<64, 32, 32, 2, 2, 2, 0, 4> >";
    case 15: return "k_group<Tile<32, 32, 32, 1, 4, 2, 0, 4> >";
    case 16: return "k_group<Tile<64, 64, 32, 2, 1, 2, 0, 2> >";
    case 17: return "k_group<Tile<64, 64, 32, 1, 1, 2, 0, 2> >";
    case 18: return "k_group<Tile<64, 64, 16, 2, 1, 2, 0, 4> >";
    case 19: return "k_group<Tile<64, 64, 16, 2, 1, 3, 0, 4> >";
    case 20: return "k_group<Tile<64, 64, 32, 2, 2, 2, 0, 8> >";
    case 21: return "k_group<Tile<64, 32, 64, 2, 2, 2, 0, 4> >";
    case 22: return "k_group<Tile<64, 64, 64, 2, 4, 2, 0, 16> >";
    case 23: return "k_group<Tile<64, 64, 64, 2, 2, 2, 0, 8> >";
    case 24: return "k_group<Sched<Tile<64, 64, 32, 2, 1, 2, 0, 4>, 1> >";
    case 25: return "k_group<Sched<Tile<64, 64, 32, 2, 1, 2, 0, 4>, 2> >";
    case 26: return "k_group<Sched<Tile<64, 32, 32, 2, 2, 2, 0, 4>, 1> >";
    case 27: return "k_group<Sched<Tile<64, 64, 32, 2, 2, 2, 0, 8>, 1> >";
    case 28: return "k_group<Sched<Tile<64, 64, 64, 2, 4, 2, 0, 16>, 1> >";
    case 29: return "k_group<Sched<Tile<32, 64, 32, 1, 2, 2, 0, 4>, 1> >";
    case 30: return "k_group<Sched<Tile<32, 32, 32, 1, 4, 2, 0, 4>, 1> >";
    case 31: return "k_group<Sched<Tile<128, 128, 16, 2, 1, 2, 0, 4>, 1> >";
    case 32: return "k_group<Sched<Tile<128, 64, 32, 2, 1, 2, 0, 4>, 1> >";
    case 33: return "k_group<Sched<Tile<64, 64, 64, 2, 1, 2, 0, 4>, 1> >";
    case 34: return "k_group<Sched<Tile<64, 64, 32, 2, 1, 3, 1, 4>, 1> >";
    case 35: return "k_group<Sched<Tile<64, 32, 64, 2, 2, 2, 0, 4>, 1> >";
    case 36: return "k_group<Sched<Tile<64, 64, 64, 2, 2, 2, 0, 8>, 1> >";
    case 37: return "k_group<Sched<Tile<64, 64, 16, 2, 1, 2, 0, 4>, 1> >";
    case 38: return "k_group<Sched<Tile<64, 64, 32, 2, 1, 2, 0, 4>, 5> >";
    case 39: return "k_group<Sched<Tile<64, 64, 16, 2, 1, 2, 0, 4>, 5> >";
    case 40: return "k_group<Sched<Tile<64, 32, 32, 2, 2, 2, 0, 4>, 5> >";
    case 41: return "k_group<Sched<Tile<64, 64, 64, 2, 4, 2, 0, 16>, 5> >";
    case 42: return "k_group<Sched<Tile<64, 64, 32, 2, 2, 2, 0, 8>, 5> >";
    case 43: return "k_group<Sched<Tile<32, 64, 32, 1, 2, 2, 0, 4>, 5> >";
    case 44: return "k_group<Sched<Tile<32, 32, 32, 1, 4, 2, 0, 4>, 5> >";
    case 45: return "k_group<Sched<Tile<128, 128, 16, 2, 1, 2, 0, 4>, 5> >";
    case 46: return "k_group<Sched<Tile<128, 64, 32, 2, 1, 2, 0, 4>, 5> >";
    case 47: return "k_group<Sched<Tile<64, 64, 64, 2, 1, 2, 0, 4>, 5> >";
    case 48: return "k_group<Sched<Tile<64, 64, 32, 2, 1, 3, 1, 4>, 5> >";
    case 49: return "k_group<Sched<Tile<64, 32, 64, 2, 2, 2, 0, 4>, 5> >";
    case 50: return "k_group<Sched<Tile<64, 64, 64, 2, 2, 2, 0, 8>, 5> >";
    default: return "k_group<Tile<64, 64, 32, 2, 1, 2, 0, 4> >";
    }
}

// Grid for the XCD-sliced mapping of group_item: 8 x the largest per-XCD
// share.
static int group_grid(const GroupArgs &a)
{
    int most = 0;
    for (int x = 0; x < 8; x++) {
        int t = 0;
        for (int p = 0; p < a.nprob; p++) {
            const int n = a.p[p].items;
            t += ((x + 1) * n >> 3) - (x * n >> 3);
        }
        if (t > most) most = t;
    }
    return 8 * most;
}

static int add_reductions(GroupArgs &a)
{
    for (int k = 0; k < g_npending; k++) {
        Prob r = g_pending[k];
        if (r.kind == PK_COLSUM) {
            r.items = cdiv(r.No / 4, TLG_COLSUM_CH);
        } else {
            r.kind = PK_RED;
            r.items = (int)(((size_t)r.Mo * r.No + TLG_RED_CHUNK - 1) / TLG_RED_CHUNK);
        }
        a.p[a.nprob++] = r;
    }
    g_npending = 0;
    return TLG_OK;
}

int tlg_group_pending(void);     // (below: the queued reductions and the held expert ones)

// Queue C[0, No) (beta ? += : =) sum over z of part[z][0, No) (z < splits,
// No % 4 == 0, 16-byte aligned rows) to ride along in the next grouped or
// expert launch (or tlg_dev_gemm_flush) on the stream.  A reduction still
// queued on the same partials, or a full queue, is flushed first, so `part`
// may be rewritten by the caller's next kernel only after this call.
int tlg_defer_colsum(const float *part, float *C, int splits, int No, int beta, hipStream_t st)
{
    int rc = TLG_OK;
    bool busy = g_npending >= TLG_MAXPROB / 2 - 1;
    for (int k = 0; k < g_npending && !busy; k++) busy = g_pending[k].ws == part;
    if (busy) {
        rc = tlg_group_flush_launch(st);
        if (rc) return rc;
    }
    rc = flush_foreign(st);
    if (rc) return rc;
    g_pending_st = st;
    Prob &r = g_pending[g_npending++];
    memset(&r, 0, sizeof r);
    r.kind = PK_COLSUM;
    r.C = C;
    r.ws = part;
    r.Mo = 1;
    r.No = No;
    r.ldc = No;
    r.beta = beta ? 1 : 0;
    r.splits = splits;
    return TLG_OK;
}

static int group_flush_dense(hipStream_t st)
{
    if (g_npending == 0) return TLG_OK;
    GroupArgs a;
    a.nprob = 0;
    a.rows1 = 0;
    add_reductions(a);
    launch_group(3, a, group_grid(a), st);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

static int ecarry_flush(hipStream_t st);

static int ecarry_flush_with_pending(hipStream_t st, bool *done);

int tlg_group_flush_launch(hipStream_t st)
{
    int rc = flush_foreign(st);
    if (rc) return rc;
    bool done = false;
    if ((rc = ecarry_flush_with_pending(st, &done)) || done) return rc;
    rc = ecarry_flush(st);
    return rc ? rc : group_flush_dense(st);
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

// Split problem P's reduction so one item runs about `rtarget` steps; partials
// go to ws (bounded by ws_cap floats).
static void plan_split(Prob &P, int R, int rtarget, float *ws, size_t &ws_used, size_t ws_cap)
{
    P.splits = 1;
    P.rps = R;
    if (P.kind != PK_TN || R <= rtarget + rtarget / 2) return;
    int sp = cdiv(R, rtarget);
    if (sp > 32) sp = 32;
    const int rps = cdiv(cdiv(R, sp), 64) * 64;      // a multiple of every group BK
    sp = cdiv(R, rps);
    if (sp > 1 && ws_used + (size_t)sp * P.Mo * P.No <= ws_cap) {
        P.splits = sp;
        P.rps = rps;
        P.ws = ws + ws_used;
        ws_used += (size_t)sp * P.Mo * P.No;
    }
}

int tlg_group_launch(const TlgGemmCall *calls, int n, hipStream_t st)
{
    if (n <= 0) return TLG_OK;
    int rc = tlg_ensure_init();
    if (rc) return rc;
    group_env();
    if (n > TLG_MAXPROB / 2) return tlg_fail(TLG_EINVAL, "tlg_dev_gemm_group: at most %d calls", TLG_MAXPROB / 2);

    // Decode runs (every call mm / mm_bt at M <= 8, no residual) go to the
    // GEMV kernels.
    bool gemv = true;
    int mmax = 1;
    for (int i = 0; i < n && gemv; i++) {
        gemv = (calls[i].op == 0 || calls[i].op == 1) && !calls[i].R && !calls[i].dotOut && calls[i].M >= 1 &&
               calls[i].M <= 8 &&
               calls[i].K > 0 &&
               calls[i].N > 0 && calls[i].nseg >= 1 && calls[i].nseg <= TLG_MAXSEG &&
               (calls[i].nseg == 1 || calls[i].op == 1);
        if (calls[i].M > mmax) mmax = calls[i].M;
    }
    if (gemv) {
        rc = tlg_group_flush_launch(st);
        if (rc) return rc;
        rc = tlg_gemv_group_launch(calls, n, st);
        g_group_last_name = tlg_gemv_kernel_name(mmax);
        return rc;
    }

    if ((rc = flush_foreign(st))) return rc;
    if ((rc = ecarry_flush(st))) return rc;
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
            for (int s = 0; s < c.nseg && !hit && op != 3; s++) {
                const int Ns = s ? c.Nseg[s] : c.N;
                const char *x0, *x1, *y0, *y1;
                if (op == 0)      { span(c.A[s], c.M, c.K, c.K, &x0, &x1); span(c.B[s], c.K, Ns, Ns, &y0, &y1); }
                else if (op == 1) { span(c.A[s], c.M, Ns, Ns, &x0, &x1); span(c.B[s], c.K, Ns, Ns, &y0, &y1); }
                else              { span(c.A[s], c.M, c.K, c.K, &x0, &x1); span(c.B[s], c.M, Ns, Ns, &y0, &y1); }
                hit = overlap(c0, c1, x0, x1) || overlap(c0, c1, y0, y1);
            }
            if (!hit && op == 0 && c.R) {
                const char *r0, *r1;
                span(c.R, c.M, c.N, c.N, &r0, &r1);
                hit = overlap(c0, c1, r0, r1);
            }
            if (!hit && op == 1 && c.dotOut) {
                const char *r0, *r1, *d0, *d1;
                span(c.dotB, c.M, c.K, c.K, &r0, &r1);
                span(c.dotOut, c.M, c.K / 32, c.K / 32, &d0, &d1);
                hit = overlap(c0, c1, r0, r1) || overlap(c0, c1, d0, d1);
            }
            if (hit) { rc = tlg_group_flush_launch(st); if (rc) return rc; break; }
        }
    }

    // Problems as the kernel sees them (tiles and splits filled in below).
    Prob probs[TLG_MAXPROB / 2];
    int Rtot[TLG_MAXPROB / 2];
    int rmax = 0;
    bool rowdot = false;
    for (int i = 0; i < n; i++) {
        const TlgGemmCall &c = calls[i];
        if (c.op == 3) {
            // a clear of C[0, M*N) riding along with the GEMMs
            if (c.M <= 0 || c.N <= 0 || !c.C)
                return tlg_fail(TLG_EINVAL, "tlg_dev_gemm_group: call %d: empty clear", i);
            Prob &P = probs[i];
            memset(&P, 0, sizeof P);
            P.kind = PK_ZERO;
            P.C = c.C;
            P.Mo = c.M;
            P.No = c.N;
            P.ldc = c.N;
            P.items = (int)(((size_t)c.M * c.N + TLG_ZERO_CHUNK - 1) / TLG_ZERO_CHUNK);
            Rtot[i] = 0;
            continue;
        }
        if (c.op < 0 || c.op > 2 || c.nseg < 1 || c.nseg > TLG_MAXSEG || (c.nseg > 1 && c.op != 1))
            return tlg_fail(TLG_EINVAL, "tlg_dev_gemm_group: call %d: bad op/nseg", i);
        if (c.M < 0 || c.K < 0 || c.N < 0) return tlg_fail(TLG_EINVAL, "negative dimension");
        Prob &P = probs[i];
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
        if (c.dotOut || c.dotB) {
            if (c.op != 1 || c.beta || !c.dotOut || !c.dotB || !al16(c.dotB) || c.K % 32 || c.dotB == c.C)
                return tlg_fail(TLG_EINVAL, "tlg_dev_gemm_group: call %d: block dot only on mm_bt with beta 0, "
                                "K %% 32 == 0, an aligned dotB that is not C", i);
            P.epi = TLG_EPI_ROWDOT;
            P.fin = c.dotB;
            P.X1 = c.dotOut;
            rowdot = true;
        }
        if (c.R) {
            if (c.op != 0 || !al16(c.R) || c.R == c.C)
                return tlg_fail(TLG_EINVAL, "tlg_dev_gemm_group: call %d: residual only on mm, aligned, not C", i);
            P.fin = c.R;
        }
        Rtot[i] = R;
        if (c.op != 2 && R > rmax) rmax = R;
    }
    // split problems aim for about the per-item work of the unsplit ones
    // (or the pinned target)
    const int rtarget = g_group_rt > 0 ? g_group_rt : rmax > g_rtarget ? rmax : g_rtarget;

    // tile shape: pinned, or the largest with >= g_min_waves waves of items
    int ci = g_group_cfg;
    if (ci < 0) {
        int last = 24;
        ci = -1;
        for (int k = 0; k < 4 && g_cand[k] >= 0 && ci < 0; k++) {
            last = g_cand[k];
            const TileCfg &tc = kCfgs[g_cand[k]];
            double items = 0;
            for (int i = 0; i < n; i++) {
                if (probs[i].kind == PK_ZERO) continue;
                const double tiles = (double)cdiv(probs[i].Mo, tc.bm) * cdiv(probs[i].No, tc.bn);
                const double sp = (probs[i].kind == PK_TN && Rtot[i] > rtarget + rtarget / 2)
                                ? (double)cdiv(Rtot[i], rtarget) : 1.0;
                items += tiles * sp;
            }
            if (items >= g_min_waves * 256) ci = g_cand[k];
        }
        if (ci < 0) ci = last;                 // smallest candidate
    }
    // the block-dot epilogue stages a whole tile in the stage buffers: not on
    // the 128 x 128 shapes, whose tile is larger than their stages
    if (rowdot && ci >= 0 && ci < kNumCfgs && kCfgs[ci].bm * kCfgs[ci].bn > 64 * 128) ci = 38;
    // geometry of the chosen shape (the sweep variants 9-12 are 64x64 tiles)
    const TileCfg &tc = kCfgs[(ci >= 0 && ci < kNumCfgs) ? ci : 3];

    GroupArgs a;
    a.nprob = 0;
    a.rows1 = 0;
    add_reductions(a);
    float *ws = g_tlg.ws + (size_t)g_ws_half * (g_tlg.ws_floats / 2);
    size_t ws_used = 0;
    const size_t ws_cap = g_tlg.ws_floats / 2;
    int order[TLG_MAXPROB / 2];
    double cost[TLG_MAXPROB / 2];
    for (int i = 0; i < n; i++) {
        Prob &P = probs[i];
        order[i] = i;
        if (P.kind == PK_ZERO) { cost[i] = 0.0; continue; }
        P.tiles_n = cdiv(P.No, tc.bn);
        P.tiles = cdiv(P.Mo, tc.bm) * P.tiles_n;
        plan_split(P, Rtot[i], rtarget, ws, ws_used, ws_cap);
        P.items = P.tiles * P.splits;
        cost[i] = (double)P.rps;              // reduction steps per item
    }
    // longest item first (stable: ties keep call order)
    for (int i = 1; i < n; i++)
        for (int j = i; j > 0 && cost[order[j]] > cost[order[j - 1]]; j--) {
            const int t = order[j]; order[j] = order[j - 1]; order[j - 1] = t;
        }
    // the reduction items of the previous launch are short: they go last
    Prob red[TLG_MAXPROB];
    const int nred = a.nprob;
    for (int k = 0; k < nred; k++) red[k] = a.p[k];
    a.nprob = 0;
    for (int k = 0; k < n; k++) {
        const Prob &P = probs[order[k]];
        a.p[a.nprob++] = P;
        if (P.splits > 1) { g_pending[g_npending++] = P; g_pending_st = st; }
    }
    for (int k = 0; k < nred; k++) a.p[a.nprob++] = red[k];
    launch_group(ci, a, group_grid(a), st);
    TLG_HIP(hipGetLastError());
    if (g_npending) g_ws_half ^= 1;
    return TLG_OK;
}

// ----------------------------------------------- expert-batched launch --
// One launch runs `n` expert-batched GEMMs (every expert of each), then, if
// any is a TN problem, one more launch adds their partial slots into the
// outputs.  Rows per expert live on the device (eoff), so the host sizes the
// grid for the worst case: ceil(rows_e / u) summed over experts is at most
// rows / u + E units of u rows.
// Slice reductions an expert launch held back (carry TLG_ECARRY_OUT) for the
// next expert launch over the same row offsets (carry TLG_ECARRY_IN), which
// runs them as its last items and places its own partial slots after
// theirs: the kernel boundary between the two makes the partials visible,
// as for the grouped launches' deferred reductions.  Any other launch that
// uses the workspace launches them first.
static GroupArgs g_ecarry;              // nprob 0: nothing held
static size_t g_ecarry_used = 0;        // workspace floats their partials occupy
static const int *g_ecarry_eoff = nullptr;
static hipStream_t g_ecarry_st = nullptr;

// Queued work whose producer ran on another stream than `st` runs first on
// the producer's stream (ordered after the kernels that wrote its partials),
// so a launch on `st` never sums partials it is not ordered after.  Work
// queued on `st` itself keeps riding along.
static int flush_foreign(hipStream_t st)
{
    if (g_ecarry.nprob && g_ecarry_st != st) {
        const int rc = ecarry_flush(g_ecarry_st);
        if (rc) return rc;
    }
    if (g_npending && g_pending_st != st) {
        const int rc = group_flush_dense(g_pending_st);
        if (rc) return rc;
    }
    return TLG_OK;
}

static int ecarry_flush(hipStream_t st)
{
    if (!g_ecarry.nprob) return TLG_OK;
    hipLaunchKernelGGL((k_expert_group<T3>), dim3(group_grid(g_ecarry)), dim3(T3::THREADS), 0, st,
                       group_seal(g_ecarry));
    g_ecarry.nprob = 0;
    g_ecarry_used = 0;
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

// Held expert reductions and queued dense ones (column sums, split
// reductions) on one stream: one launch for both, the held expert
// reductions first (the expert kernel stages p[0]'s row offsets), then the
// queued ones, which it runs as the dense kernel does.  *done = false when
// there are not both kinds (or too many problems for one launch).
static int ecarry_flush_with_pending(hipStream_t st, bool *done)
{
    *done = false;
    if (!g_ecarry.nprob || !g_npending || g_ecarry.nprob + g_npending > TLG_MAXPROB) return TLG_OK;
    GroupArgs a = g_ecarry;
    add_reductions(a);
    hipLaunchKernelGGL((k_expert_group<T3>), dim3(group_grid(a)), dim3(T3::THREADS), 0, st, group_seal(a));
    g_ecarry.nprob = 0;
    g_ecarry_used = 0;
    TLG_HIP(hipGetLastError());
    *done = true;
    return TLG_OK;
}

int tlg_group_pending(void) { return g_npending + g_ecarry.nprob; }

// Every queued reduction (and an expert launch's held carry) launched now,
// each on the stream its partials were written on: what tlg_dev_free runs
// before it releases memory that queued work may read or write.
int tlg_group_flush_all(void)
{
    if (g_ecarry.nprob) {
        const int rc = tlg_group_flush_launch(g_ecarry_st);
        if (rc) return rc;
    }
    return g_npending ? tlg_group_flush_launch(g_pending_st) : TLG_OK;
}

// Queued work whose partials were written on `st` launched now, on `st`:
// what tlg_stream_destroy runs before the handle goes away.
int tlg_group_flush_stream(hipStream_t st)
{
    if ((g_ecarry.nprob && g_ecarry_st == st) || (g_npending && g_pending_st == st))
        return tlg_group_flush_launch(st);
    return TLG_OK;
}

// Shutdown: the queued reductions (and an expert launch's held carry) run
// on `st` while the workspace they read still exists; then the queue is
// empty and the workspace halves start over, so nothing queued before a
// tlg_shutdown can run against freed memory after a later tlg_init.
int tlg_group_drain(hipStream_t st)
{
    const int rc = tlg_group_flush_launch(st);
    g_npending = 0;
    g_ecarry.nprob = 0;
    g_ecarry_used = 0;
    g_ecarry_eoff = nullptr;
    g_ws_half = 0;
    return rc;
}

int tlg_expert_launch(const TlgExpertCall *calls, int n, const int *eoff, int E, int rows, hipStream_t st,
                      int carry)
{
    if (n <= 0) return TLG_OK;
    int rc = tlg_ensure_init();
    if (rc) return rc;
    if (n > TLG_MAXPROB / 2) return tlg_fail(TLG_EINVAL, "expert launch: at most %d calls", TLG_MAXPROB / 2);
    // eoff NULL: one expert owning every row (dense rows, known on the host)
    const bool dense = eoff == nullptr;
    if ((dense && E != 1) || E < 1 || E > TLG_MAX_EXPERTS || rows < 0)
        return tlg_fail(TLG_EINVAL, "expert launch: bad row offsets or %d experts", E);
    if (rows == 0) return TLG_OK;
    if ((rc = flush_foreign(st))) return rc;
    // held slice reductions join this launch only if it asks for them and
    // shares their row offsets
    const bool cin = (carry & TLG_ECARRY_IN) && g_ecarry.nprob && g_ecarry_eoff == eoff && !dense;
    if (!cin && (rc = ecarry_flush(st))) return rc;
    // Pending split reductions of grouped launches ride along when this
    // launch writes no partial slots (they reuse the whole workspace) and
    // touches none of their outputs; otherwise they are flushed first.
    bool ride = dense;
    for (int i = 0; i < n && ride; i++) {
        const TlgExpertCall &c = calls[i];
        if (c.op == 2 || c.amap || c.omap) { ride = false; break; }
        const int Nr = c.op == 0 ? c.N : c.K;          // output / epilogue row width
        const int Na = c.op == 0 ? c.K : c.N;          // A row width
        const char *r0[7], *r1[7];
        int m = 0;
        if (c.C) span(c.C, rows, Nr, Nr, &r0[m], &r1[m]), m++;
        if (c.X1) span(c.X1, rows, Nr, Nr, &r0[m], &r1[m]), m++;
        if (c.X2) span(c.X2, rows, Nr, Nr, &r0[m], &r1[m]), m++;
        if (c.fin) span(c.fin, rows, Nr, Nr, &r0[m], &r1[m]), m++;
        span(c.A[0], rows, Na, Na, &r0[m], &r1[m]), m++;
        span(c.B[0], c.K, c.N, c.N, &r0[m], &r1[m]), m++;
        if (c.B2) span(c.B2, c.K, c.N, c.N, &r0[m], &r1[m]), m++;
        for (int k = 0; k < g_npending && ride; k++) {
            const char *c0, *c1;
            span(g_pending[k].C, g_pending[k].Mo, g_pending[k].No, g_pending[k].ldc, &c0, &c1);
            for (int j = 0; j < m && ride; j++) ride = !overlap(c0, c1, r0[j], r1[j]);
        }
    }
    if (!ride) {
        rc = group_flush_dense(st);
        if (rc) return rc;
    }

    group_env();
    Prob probs[TLG_MAXPROB / 2];
    for (int i = 0; i < n; i++) {
        const TlgExpertCall &c = calls[i];
        if (c.op < 0 || c.op > 2 || c.nseg < 1 || c.nseg > 2 || (c.nseg > 1 && c.op != 1))
            return tlg_fail(TLG_EINVAL, "expert launch: call %d: bad op/nseg", i);
        Prob &P = probs[i];
        memset(&P, 0, sizeof P);
        P.kind = c.op == 0 ? PK_NN : (c.op == 1 ? PK_NT : PK_TN);
        P.C = c.C;
        P.beta = c.beta ? 1 : 0;
        P.nseg = c.nseg;
        P.eoff = eoff;
        P.nexp = E;
        P.es = c.es;
        P.amap = c.amap;
        P.omap = c.omap;
        P.B2 = c.B2;
        P.epi = c.epi;
        P.X1 = c.X1;
        P.X2 = c.X2;
        P.fin = c.fin;
        P.gate = c.gate;
        // fused forms: the pair only with the SwiGLU epilogue of an NN call;
        // SwiGLU backward on NT (da = dy W2^T); the combine on NN
        const bool epi_ok =
            (c.epi == TLG_EPI_STORE && !c.B2) ||
            (c.epi == TLG_EPI_SWIGLU && c.op == 0 && c.B2 && al16(c.B2) && c.nseg == 1 && !c.beta) ||
            (c.epi == TLG_EPI_SWIGLU_BWD && c.op == 1 && !c.B2 && c.X1 && c.X2) ||
            (c.epi == TLG_EPI_COMBINE && c.op == 0 && !c.B2 && c.omap && c.fin && c.gate && c.nseg == 1 &&
             !c.beta && !c.amap);
        if (!epi_ok || (c.amap && c.nseg != 1))
            return tlg_fail(TLG_EINVAL, "expert launch: call %d: bad epilogue %d / gather / pair", i, c.epi);
        bool vec = (c.C || c.epi == TLG_EPI_SWIGLU_BWD) && (c.es % 4 == 0);
        for (int s = 0; s < c.nseg; s++) {
            const int Ns = s ? c.Nseg[s] : c.N;
            Seg &g = P.seg[s];
            g.A = c.A[s]; g.B = c.B[s];
            switch (c.op) {
            case 0: P.No = c.N; g.R = c.K; g.lda = c.K; g.ldb = c.N; break;
            case 1: P.No = c.K; g.R = Ns; g.lda = Ns; g.ldb = Ns; break;
            default: P.Mo = c.K; P.No = c.N; g.R = rows; g.lda = c.K; g.ldb = c.N; break;
            }
            vec = vec && g.A && g.B && al16(g.A) && al16(g.B) && g.lda % 4 == 0 && g.ldb % 4 == 0 && g.R > 0;
        }
        P.ldc = P.No;
        if (!vec || P.No <= 0 || (c.op == 2 && P.Mo <= 0) || P.No % 4 || P.Mo % 4)
            return tlg_fail(TLG_EINVAL, "expert launch: call %d needs aligned operands, widths %% 4 == 0", i);
    }
    // reduction slices of the TN problems (g_erps rows, doubled until the
    // partials fit): short slices balance experts of very different sizes
    int rps = cdiv(g_erps, 64) * 64;
    const size_t used0 = cin ? g_ecarry_used : 0;     // the held partials come first
    auto need = [&](int u) {
        size_t t = used0;
        for (int i = 0; i < n; i++)
            if (probs[i].kind == PK_TN) t += (size_t)(rows / u + E) * probs[i].Mo * probs[i].No;
        return t;
    };
    while (need(rps) > g_tlg.ws_floats && rps < rows) rps *= 2;
    if (need(rps) > g_tlg.ws_floats)
        return tlg_fail(TLG_ENOMEM, "expert launch: %d experts' partials exceed the workspace", E);

    // tile shape: the largest of 64x64, 64x32 (2 x 2 waves) and 32x32 (a
    // quarter stage per wave) that gives about g_min_waves x 256 items, as
    // for dense grouped launches (measured at configs[4]: W2's N = 256
    // launches run 15 % faster on 32x32 tiles than on 64x32; the 8-wave
    // 64x64 tile was slower on every expert launch)
    auto items_for = [&](const TileCfg &c) {
        double t = 0;
        for (int i = 0; i < n; i++) {
            const Prob &P = probs[i];
            const double tn = cdiv(P.No, P.B2 ? c.bn / 2 : c.bn);
            t += P.kind == PK_TN ? cdiv(P.Mo, c.bm) * tn * (rows / rps + E) : (cdiv(rows, c.bm) + E) * tn;
        }
        return t;
    };
    const double enough = g_min_waves * 256;
    // (TLG_EXPERT_W16=1: launches with fewer 64x64 items than that but about
    // one per CU -- the N = 256 W2 launches -- run 64x64 tiles of 16 waves,
    // as the dense W2 forward does; slower on every configs[4] launch)
    const int ci = g_expert_cfg >= 0 ? g_expert_cfg
                 : items_for(kCfgs[3]) >= enough ? (g_expert_bk16 ? 18 : 3)
                 : (g_expert_w16 && items_for(kCfgs[22]) >= 240) ? 22
                 : items_for(kCfgs[14]) >= enough ? 14 : 15;
    const TileCfg &tc = kCfgs[ci];
    GroupArgs a, red, pend;
    a.nprob = red.nprob = pend.nprob = 0;
    a.rows1 = red.rows1 = pend.rows1 = dense ? rows : 0;
    if (ride) add_reductions(pend);
    size_t used = used0;
    int order[TLG_MAXPROB / 2];
    for (int i = 0; i < n; i++) {
        Prob &P = probs[i];
        P.tiles_n = cdiv(P.No, P.B2 ? tc.bn / 2 : tc.bn);
        if (P.kind == PK_TN) {
            P.tiles = cdiv(P.Mo, tc.bm) * P.tiles_n;
            P.unit = rps;
            P.rps = rps;
            P.items = P.tiles * (rows / rps + E);
            P.ws = g_tlg.ws + used;
            used += (size_t)(rows / rps + E) * P.Mo * P.No;
        } else {
            P.unit = tc.bm;
            P.items = (cdiv(rows, tc.bm) + E) * P.tiles_n;
        }
        order[i] = i;
    }
    // longest item first: TN items run rps rows, the others their full R
    auto cost = [&](const Prob &P) {
        int r = 0;
        for (int s = 0; s < P.nseg; s++) r += P.seg[s].R;
        return P.kind == PK_TN ? P.unit : r;
    };
    for (int i = 1; i < n; i++)
        for (int j = i; j > 0 && cost(probs[order[j]]) > cost(probs[order[j - 1]]); j--) {
            const int t = order[j]; order[j] = order[j - 1]; order[j - 1] = t;
        }
    for (int k = 0; k < n; k++) {
        const Prob &P = probs[order[k]];
        a.p[a.nprob++] = P;
        if (P.kind == PK_TN) {
            Prob r = P;
            r.kind = PK_RED;
            r.items = E * (int)(((size_t)P.Mo * P.No + TLG_ERED_CHUNK - 1) / TLG_ERED_CHUNK);
            red.p[red.nprob++] = r;
        }
    }
    // the grouped launches' reductions that ride along go last (short items),
    // with the held slice reductions of the previous expert launch
    for (int k = 0; k < pend.nprob; k++) a.p[a.nprob++] = pend.p[k];
    if (cin) {
        if (a.nprob + g_ecarry.nprob > TLG_MAXPROB) return tlg_fail(TLG_EINVAL, "expert launch: too many problems");
        for (int k = 0; k < g_ecarry.nprob; k++) a.p[a.nprob++] = g_ecarry.p[k];
        g_ecarry.nprob = 0;
        g_ecarry_used = 0;
    }
    // an XCD's share of the real items can exceed its share of the upper
    // bound by one per expert problem
    static_assert(sizeof(GroupArgs) <= 4096, "kernel arguments");
    const dim3 eg(group_grid(a) + 8 * n);
    // +100: the Sched<.., 1> order; +200: that order with streaming stores
    const int key = ci + 100 * (g_expert_sched >= 0 ? g_expert_sched : dense ? 2 : 1);
#define TLG_EXPERT_CASE(k, TT)                                                                                  \
    case k: hipLaunchKernelGGL((k_expert_group<TT>), eg, dim3(TT::THREADS), 0, st, group_seal(a)); break;
    switch (key) {
    TLG_EXPERT_CASE(3, T3) TLG_EXPERT_CASE(14, T14) TLG_EXPERT_CASE(15, T15) TLG_EXPERT_CASE(18, T18)
    TLG_EXPERT_CASE(22, T22)
    TLG_EXPERT_CASE(103, T24) TLG_EXPERT_CASE(114, T26) TLG_EXPERT_CASE(115, T30) TLG_EXPERT_CASE(118, T37)
    TLG_EXPERT_CASE(122, T28)
    TLG_EXPERT_CASE(203, T38) TLG_EXPERT_CASE(214, T40) TLG_EXPERT_CASE(215, T44) TLG_EXPERT_CASE(218, T39)
    TLG_EXPERT_CASE(222, T41)
    default: return tlg_fail(TLG_EINVAL, "expert launch: no kernel for tile form %d", key);
    }
#undef TLG_EXPERT_CASE
    TLG_HIP(hipGetLastError());
    if (red.nprob && (carry & TLG_ECARRY_OUT) && !dense && g_npending == 0) {
        g_ecarry = red;                  // the next expert launch runs them
        g_ecarry_used = used;
        g_ecarry_eoff = eoff;
        g_ecarry_st = st;
    } else if (red.nprob) {
        hipLaunchKernelGGL((k_expert_group<T3>), dim3(group_grid(red)), dim3(T3::THREADS), 0, st, group_seal(red));
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
// Streaming probes: each thread moves 8 float4 per round (all 8 loads in
// flight before any is used), rounds stride over the grid's chunks of 8 x 256
// float4; loads and stores are nontemporal (the data is not reused).
#define TLG_CP_U 8
__global__ __launch_bounds__(256) void k_copy(const f32x4 *__restrict__ src, f32x4 *__restrict__ dst, size_t n4)
{
    const size_t chunk = (size_t)TLG_CP_U * 256;
    for (size_t c = (size_t)blockIdx.x * chunk; c < n4; c += (size_t)gridDim.x * chunk) {
        f32x4 v[TLG_CP_U];
#pragma unroll
        for (int k = 0; k < TLG_CP_U; k++) {
            const size_t i = c + threadIdx.x + (size_t)k * 256;
            v[k] = __builtin_nontemporal_load(src + (i < n4 ? i : n4 - 1));
        }
#pragma unroll
        for (int k = 0; k < TLG_CP_U; k++) {
            const size_t i = c + threadIdx.x + (size_t)k * 256;
            if (i < n4) __builtin_nontemporal_store(v[k], dst + i);
        }
    }
}

// Read-only stream: the sum of src (kept so the loads are not removed) goes
// to sink[0] only if it equals a value no probe input produces.
__global__ __launch_bounds__(256) void k_read(const f32x4 *__restrict__ src, size_t n4, float *__restrict__ sink)
{
    const size_t chunk = (size_t)TLG_CP_U * 256;
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
    for (size_t c = (size_t)blockIdx.x * chunk; c < n4; c += (size_t)gridDim.x * chunk) {
        f32x4 v[TLG_CP_U];
#pragma unroll
        for (int k = 0; k < TLG_CP_U; k++) {
            const size_t i = c + threadIdx.x + (size_t)k * 256;
            v[k] = __builtin_nontemporal_load(src + (i < n4 ? i : n4 - 1));
        }
#pragma unroll
        for (int k = 0; k < TLG_CP_U; k++) a += v[k];
    }
    if (a.x + a.y + a.z + a.w == -1.2345e30f) sink[0] = 1.f;
}

static size_t stream_blocks(size_t n4)
{
    size_t blocks = (n4 + TLG_CP_U * 256 - 1) / (TLG_CP_U * 256);
    return blocks > 256 * 8 ? 256 * 8 : blocks;
}

int tlg_copy_launch(float *dst, const float *src, size_t n, hipStream_t st)
{
    if (n % 4 || ((uintptr_t)dst & 15) || ((uintptr_t)src & 15))
        return tlg_fail(TLG_EINVAL, "tlg_dev_copy: needs 16-byte aligned buffers and n %% 4 == 0");
    const size_t n4 = n / 4, blocks = stream_blocks(n4);
    if (blocks == 0) return TLG_OK;
    hipLaunchKernelGGL(k_copy, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const f32x4 *)src, (f32x4 *)dst, n4);
    TLG_HIP(hipGetLastError());
    return TLG_OK;
}

int tlg_read_launch(const float *src, size_t n, float *sink, hipStream_t st)
{
    if (n % 4 || ((uintptr_t)src & 15) || !sink)
        return tlg_fail(TLG_EINVAL, "tlg_dev_read: needs a 16-byte aligned buffer, n %% 4 == 0 and a sink");
    const size_t n4 = n / 4, blocks = stream_blocks(n4);
    if (blocks == 0) return TLG_OK;
    hipLaunchKernelGGL(k_read, dim3((unsigned)blocks), dim3(256), 0, st, (const f32x4 *)src, n4, sink);
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
