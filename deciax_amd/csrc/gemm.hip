// bf16 "NT" GEMM on gfx950 MFMA: C[m, n] = sum_k A[m, k] * B[n, k].
//
// A is activations [M, K] and B is a weight in PyTorch [out, in] layout, so
// both operands are K-contiguous and every MFMA operand is one 16-byte LDS
// read. Block tile BM x 256 x 64 over 4 waves (2 x 2), one wave per SIMD; each
// wave owns a BM/2 x 128 quadrant in 32x32x16 MFMA blocks with fp32
// accumulators (a single wave saturates the matrix core with this shape).
//
// Two data paths (256-row tiles, and 128-row tiles with K <= 8192, take the second):
//
// Register-staged. Per thread and K tile: 16-byte chunks arrive through buffer loads
// (the resource is based at the tile origin, so rows past M read as zero and
// 32-bit offsets cover every supported shape) into registers one K tile ahead,
// are written to the idle half of a double-buffered LDS tile, and are read back
// as MFMA fragments, themselves double-buffered in registers one k-step ahead.
// Each k-step is a scheduling region of its own in which the 16 MFMAs carry,
// interleaved at fixed slots, that k-step's share of the chunk loads (one per
// four MFMAs), the LDS writes of the next tile and the next fragment reads: the
// address unit never receives a burst large enough to stall instruction issue,
// which is what bounds this kernel when loads are issued in clumps. Loads run two
// tiles ahead of the MFMAs, which long-K shapes (activations streamed from HBM)
// need.
//
// Direct-to-LDS. Buffer loads write the LDS tile themselves (buffer_load ... lds),
// so there are no staging registers and no LDS writes. 256-row tiles keep A in a
// ring of three stages and B in a ring of two (the whole 160 KB): A's loads can then
// run a full iteration ahead, and every k-step carries the same 4 loads per wave,
// one per 4 MFMAs. 128-row tiles use two stages of both. The loads are what bounds
// this loop: without them it runs at 83 % of the clock's MFMA peak, with them at
// about 70 %, and it is neither their latency nor their rate at the address unit
// (both measured).
//
// LDS layout: row-major [rows][64] bf16, 16-byte chunk c of row r stored at
// chunk position c ^ ((r >> 1) & 7): a 32-lane fragment read touches 32 rows
// at one logical chunk, and the XOR spreads 16 consecutive rows over all 16
// chunk slots of a 256-byte bank line (conflict-free on gfx950's 64 banks).
//
// Epilogues: bf16 store (staged through LDS for 16-byte row stores), fp32
// store, and the gated activation for a gate|up weight packed in 64-row
// blocks (dx_pack_gate_up), which writes act = bf16(bf16(act(g)) * u) with
// g, u rounded to bf16 first — the rounding points of the reference's fused
// MLP epilogue (src/deciax/kernels/swiglu.py:100-101). The QKV epilogue
// (q | k | v packed weight) applies rotate-half RoPE to the q and k heads of the
// tile with the rounding of dx_rope (the RoPE-in-projection pattern of
// src/deciax/kernels/fused.py:93-99,120-122 on the formula of
// src/deciax/nn.py:35-44), and scatters v transposed into V^T, the layout the
// attention kernel stages (one column per token: vt_col[row]).
#include "common.h"
#include "kernels.h"
#include "rownorm.h"

namespace {

template <bool B>
struct Flag {
  static constexpr bool value = B;
};

template <int I>
struct Int {
  static constexpr int value = I;
};

constexpr int BK = 64;
// Column tile: 256, or 128 for the 64-row tiles that serve small M (plain epilogues only). Every output
// element runs the same MFMA chain in the same k order in either shape, so its value does not depend on
// the tile configuration, hence not on M.
template <int BM>
constexpr int tile_n() { return BM == 64 ? 128 : 256; }
constexpr int THREADS = 256;

enum { EPI_BF16 = 0, EPI_F32 = 1, EPI_GATED = 2, EPI_QKV = 3, EPI_NORM = 4 };

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2). Renumber so each XCD gets a contiguous run of logical tiles, then walk
// tiles in groups of group_m tile-rows so concurrently running tiles share A
// rows and B columns inside one L2.
DX_DEVICE void tile_coords(int pid, int nblocks, int num_m, int num_n, int group_m, int &tm, int &tn) {
  const int per = nblocks / 8, rem = nblocks % 8;
  const int xcd = pid % 8, idx = pid / 8;
  const int lpid = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  const int group_size = group_m * num_n;
  const int group = lpid / group_size;
  const int first_m = group * group_m;
  const int gm = min(num_m - first_m, group_m);
  const int in = lpid % group_size;
  tm = first_m + in % gm;
  tn = in / gm;
}

DX_DEVICE int swz(int row, int chunk) { return row * 64 + ((chunk ^ ((row >> 1) & 7)) << 3); }

typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes per lane from a buffer resource into LDS at lds + 16 * lane. The builtin is compiled in the
// device pass only: this clang drops a kernel's host-side symbols when the host pass sees it.
DX_DEVICE void lds_load16(__amdgpu_buffer_rsrc_t rsrc, uint16_t *lds, int voffset, int soffset) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void *)lds, 16, voffset, soffset, 0, 0);
#endif
}

DX_DEVICE __amdgpu_buffer_rsrc_t make_rsrc(const uint16_t *base, long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}

// After a workgroup's y tile has been stored (system-coherent), count its row block; the workgroup that
// completes the block's num_n column tiles applies the residual update to the block's rows, one wave
// per row (add_rmsnorm_row, the arithmetic of dx_add_rmsnorm), and resets the counter for the next
// call. No workgroup waits for another, so the grid needs no co-residency.
template <int BM>
DX_DEVICE void norm_epilogue(const uint16_t *Y, int M, int N, long ldy, int m0, int tm, int num_n,
                             const NormEpilogue &ne, int *flag) {
  // wave is wave-uniform, which the compiler is told: each row's coherent-load descriptor then stays in
  // scalar registers instead of costing a waterfall loop around every load
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's y stores have reached memory
  __syncthreads();  // ... every thread's; the staged tile in LDS is no longer read, so `flag` may reuse it
  if (tid == 0)
    *flag = __hip_atomic_fetch_add(ne.counters + tm, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == num_n - 1;
  __syncthreads();
  if (!*flag) return;
  const int rows = min(BM, M - m0);
  // Each wave takes RB rows at a time and requests all of their y and x before computing any, so a
  // wave keeps RB rows of memory latency in flight instead of one.
  constexpr int WAVES = THREADS / 64;
  auto run = [&](auto maxc, auto next) __attribute__((always_inline)) {
    constexpr int MC = decltype(maxc)::value;
    constexpr bool NX = decltype(next)::value;
    constexpr int RB = MC <= 8 ? 3 : 2;  // 2 RB MC 16-byte chunks of registers per lane
    const int nch = N / 8;
    for (int r0 = wave; r0 < rows; r0 += RB * WAVES) {
      Row<MC> yr[RB], xr[RB];
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const int r = r0 + b * WAVES;
        if (r < rows) {
          load_row_coherent(yr[b], Y + (long)(m0 + r) * ldy, nch, lane);
          load_row(xr[b], ne.x + (long)(m0 + r) * N, nch, lane);
        }
      }
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const int r = r0 + b * WAVES;
        if (r < rows) {
          const long row = m0 + r;
          add_rmsnorm_regs<MC, NX>(yr[b], xr[b], ne.post_w, ne.x + row * N, ne.next_w,
                                   NX ? ne.h + row * N : nullptr, N, ne.eps, lane);
        }
      }
    }
  };
  // up to 8 chunks of 8 columns per lane (N <= 4096, the 9B width) or 12 (N <= 6144, the 27B width)
  const bool wide = N > 64 * 8 * 8;
  if (ne.next_w) {
    if (wide) run(Int<12>(), Flag<true>());
    else run(Int<8>(), Flag<true>());
  } else {
    if (wide) run(Int<12>(), Flag<false>());
    else run(Int<8>(), Flag<false>());
  }
  if (tid == 0) __hip_atomic_store(ne.counters + tm, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// EB (256-row ring only): B's loads of the next tile all go before A's loads of the tile after it, so the
// per-iteration wait leaves A's 8 loads in flight (see the ring schedule below).
template <int BM, int EPI, bool DTL, bool EB = false>
__global__ void __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_nt_kernel(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B, void *__restrict__ C, int M, int N,
               int K, long lda, long ldb, long ldc, int act, int group_m, QkvEpilogue qe, NormEpilogue ne) {
  constexpr int BN = tile_n<BM>();
  constexpr int TM = BM / 64, TN = BN / 64;  // 32x32 blocks per wave along m, n
  // the narrow tiles have too few MFMAs per k-step for the fixed-slot schedules: the compiler schedules them
  constexpr bool SMALL = BM == 64;
  static_assert(!SMALL || EPI == EPI_BF16 || EPI == EPI_F32, "narrow tiles take the plain epilogues only");
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int AC = BM * BK / 8 / THREADS, BC = BN * BK / 8 / THREADS;  // 16-byte chunks per thread
  constexpr int NC = AC + BC;
  constexpr int RATIO = NC / AC;  // chunk j is an A chunk iff j % RATIO == 0
  static_assert((SMALL || NC % 4 == 0) && NC % AC == 0, "chunk schedule");
  constexpr int OUT_W = EPI == EPI_GATED ? BN / 2 : BN;
  constexpr int OUT_PITCH = OUT_W + 8;
  // 256-row direct-to-LDS tiles use a ring of 3 A and 2 B stages (5 x 32 KB = the whole 160 KB)
  constexpr bool RING = DTL && BM == 256;
  constexpr int OPERANDS = RING ? 5 * BM * BK : 2 * STAGE;
  constexpr int SMEM = (OPERANDS > BM * OUT_PITCH) ? OPERANDS : BM * OUT_PITCH;
  // q|k|v epilogue: each tile row's clamped RoPE position and V^T column (2 BM int32) sit in LDS above
  // the staged tile (row-major BM x OUT_PITCH, or transposed BN x (BM + 8) for a V^T tile)
  constexpr int ROW_INFO = BN * (BM + 8) > BM * OUT_PITCH ? BN * (BM + 8) : BM * OUT_PITCH;
  static_assert(EPI != EPI_QKV || ROW_INFO + 4 * BM <= SMEM, "q|k|v row info fits the LDS");
  __shared__ __attribute__((aligned(1024))) uint16_t smem[SMEM];

  const int num_m = (M + BM - 1) / BM, num_n = N / BN;
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, num_m, num_n, group_m, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A + (long)m0 * lda, (long)min(M - m0, BM) * lda * 2);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(B + (long)n0 * ldb, (long)BN * ldb * 2);
  // register path: chunk j of this thread (A iff j % RATIO == 0), its global offset and LDS slot
  int voff[DTL ? 1 : NC], dst[DTL ? 1 : NC];
#pragma unroll
  for (int j = 0; j < (DTL ? 0 : NC); ++j) {
    const bool isa = j % RATIO == 0;
    const int jj = isa ? j / RATIO : j - j / RATIO - 1;
    const int id = tid + THREADS * jj, row = id >> 3, c = id & 7;
    voff[j] = (int)((isa ? row * lda : row * ldb) * 2 + c * 16);
    dst[j] = (isa ? 0 : BM * BK) + swz(row, c);
  }
  u32x4 rg[DTL ? 1 : NC];
  auto gl = [&](int kt, int j0, int j1) {
#pragma unroll
    for (int j = j0; j < j1; ++j)
      rg[j] = __builtin_bit_cast(u32x4,
                                 __builtin_amdgcn_raw_buffer_load_b128(j % RATIO == 0 ? ra : rb, voff[j], kt * BK * 2, 0));
  };
  auto sw = [&](int stage, int j0, int j1) {
#pragma unroll
    for (int j = j0; j < j1; ++j) *reinterpret_cast<u32x4 *>(smem + stage * STAGE + dst[j]) = rg[j];
  };

  // direct-to-LDS path: instruction i of an operand fills LDS rows [8 i, 8 i + 8) (1 KB); lane l
  // takes row 8 i + l / 8, slot l % 8, i.e. global chunk (l % 8) ^ ((row >> 1) & 7). Wave w issues A
  // instructions [w AI, (w + 1) AI) and B instructions [w BI, (w + 1) BI).
  constexpr int AI = BM / 8 / 4, BI = BN / 8 / 4, NI = AI + BI;  // per wave
  int aoff[DTL ? AI : 1], boff[DTL ? BI : 1];
#pragma unroll
  for (int j = 0; j < (DTL ? AI : 0); ++j) {
    const int row = 8 * (wave * AI + j) + (lane >> 3), c = (lane & 7) ^ ((row >> 1) & 7);
    aoff[j] = (int)(row * lda * 2) + c * 16;
  }
#pragma unroll
  for (int j = 0; j < (DTL ? BI : 0); ++j) {
    const int row = 8 * (wave * BI + j) + (lane >> 3), c = (lane & 7) ^ ((row >> 1) & 7);
    boff[j] = (int)(row * ldb * 2) + c * 16;
  }
  // this wave's instructions [j0, j1) for tile kt into stage (A first, then B)
  auto dl = [&](int kt, int stage, int j0, int j1) {
    uint16_t *base = smem + stage * STAGE;
#pragma unroll
    for (int j = j0; j < j1; ++j) {
      if (j < AI) lds_load16(ra, base + (wave * AI + j) * 512, aoff[j], kt * BK * 2);
      else lds_load16(rb, base + BM * BK + (wave * BI + j - AI) * 512, boff[j - AI], kt * BK * 2);
    }
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int lrow = lane & 31, lhalf = lane >> 5;
  bf16x8 fa0[TM], fb0[TN], fa1[TM], fb1[TN];
  auto rd = [&](bf16x8 *fa, bf16x8 *fb, int stage, int ks) {
    const uint16_t *sa = smem + stage * STAGE;
    const uint16_t *sb = sa + BM * BK;
    const int c = ks * 2 + lhalf;
#pragma unroll
    for (int i = 0; i < TM; ++i)
      fa[i] = as_bf16x8(*reinterpret_cast<const u32x4 *>(sa + swz(wm * (BM / 2) + i * 32 + lrow, c)));
#pragma unroll
    for (int j = 0; j < TN; ++j)
      fb[j] = as_bf16x8(*reinterpret_cast<const u32x4 *>(sb + swz(wn * (BN / 2) + j * 32 + lrow, c)));
  };
  // B as the first MFMA operand: block (i, j) holds the transposed product, so lane (lrow, lhalf) has
  // register r at row i * 32 + lrow and column j * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3) of the wave's
  // quadrant, four consecutive columns per register group (8-byte staging writes, 16-byte fp32 stores)
  auto mm = [&](const bf16x8 *fa, const bf16x8 *fb) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = mfma32(fb[j], fa[i], acc[i][j]);
  };

  // One k-step region: NM MFMAs; nw LDS writes in the first slots, one load after every GS
  // MFMAs, the NR fragment reads from slot R0 on.
  constexpr int NR = TM + TN, NM = TM * TN;
  constexpr int NG = NC / 4;                           // chunk loads per k-step
  constexpr int GS = NM / NG;                          // MFMAs between two loads
  constexpr int W0 = (NC + 2) / 3, W1 = (NC + 1) / 3;  // writes per pre-barrier k-step
  constexpr int R0 = BM == 256 ? 6 : NM / 4;          // first fragment-read slot
  static_assert(SMALL || (GS >= 2 && W0 <= NM && R0 + NR <= NM), "region schedule");
#define DX_REGION(nw, ng)                                                                          \
  if constexpr (!SMALL) do {                                                                       \
    _Pragma("unroll") for (int t = 0; t < NM; ++t) {                                               \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                           \
      if (t < (nw)) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);                             \
      if (t % GS == GS - 1 && t / GS < (ng)) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);    \
      if (t >= R0 && t - R0 < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);               \
    }                                                                                              \
  } while (0)

  const int KT = K / BK;
  if constexpr (RING) {
    // A tile T goes to A stage T % 3, free once the barrier of iteration T - 3 has passed; its 8 loads
    // per wave go out in k-steps 0 / 1 / 2 of iteration T - 2 (2 / 2 / 4), a full iteration or more
    // before use. B tile T goes to B stage T % 2, free after the barrier of iteration T - 2; 4 loads
    // follow that barrier and 2 / 2 go in k-steps 0 / 1 of iteration T - 1. Every k-step thus
    // carries 4 loads per wave, one per 4 MFMAs (measured against the two-stage ring: +2-5% on the
    // 9B and 27B q|k|v, o and gate|up shapes, bit-identical results).
    // With EB, B's second 4 loads all go in k-step 0 and A's 8 in k-steps 1 / 2 (4 / 4). The counter
    // drains in issue order, so the wait that makes B of tile T + 1 visible then leaves all 8 A loads
    // in flight, instead of waiting for A's first 4 as well: B gets about a k-step more to land.
    static_assert(AI == 8 && BI == 8, "ring schedule: 8 A and 8 B instructions per wave");
    constexpr int RS = BM * BK;  // elements per stage (A or B)
    auto la = [&](int kt, int sa, int j0, int j1) __attribute__((always_inline)) {
#pragma unroll
      for (int j = j0; j < j1; ++j) lds_load16(ra, smem + sa * RS + (wave * AI + j) * 512, aoff[j], kt * BK * 2);
    };
    auto lb = [&](int kt, int sb, int j0, int j1) __attribute__((always_inline)) {
#pragma unroll
      for (int j = j0; j < j1; ++j)
        lds_load16(rb, smem + (3 + sb) * RS + (wave * BI + j) * 512, boff[j], kt * BK * 2);
    };
    auto rdr = [&](bf16x8 *fa, bf16x8 *fb, int sa, int sb, int ks) __attribute__((always_inline)) {
      const uint16_t *pa = smem + sa * RS;
      const uint16_t *pb = smem + (3 + sb) * RS;
      const int c = ks * 2 + lhalf;
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i] = as_bf16x8(*reinterpret_cast<const u32x4 *>(pa + swz(wm * (BM / 2) + i * 32 + lrow, c)));
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j] = as_bf16x8(*reinterpret_cast<const u32x4 *>(pb + swz(wn * (BN / 2) + j * 32 + lrow, c)));
    };
    constexpr int DR0 = 6;  // fragment reads in MFMA slots 6..13
    static_assert(DR0 + NR <= NM, "ring region schedule");
#define DX_RREGION()                                                                               \
  do {                                                                                             \
    _Pragma("unroll") for (int t = 0; t < NM; ++t) {                                               \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                           \
      if (t % 4 == 0) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                           \
      if (t >= DR0 && t - DR0 < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);             \
    }                                                                                              \
  } while (0)
    auto cl = [&](int t) { return min(t, KT - 1); };  // past the end: reload the last tile into a freed stage
    // tiles 0 and 1 of A, tile 0 of B and the loads of B tile 1 that precede iteration 0
    la(0, 0, 0, 8);
    lb(0, 0, 0, 8);
    la(cl(1), 1, 0, 8);
    lb(cl(1), 1, 0, 4);
    asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    __syncthreads();
    rdr(fa0, fb0, 0, 0, 0);
    // Iteration kt (q = kt % 6 at compile time, so every stage is an immediate).
    auto iteration = [&](const int kt, auto qc) __attribute__((always_inline)) {
      constexpr int q = decltype(qc)::value;
      constexpr int sa = q % 3, sb = q % 2, sa1 = (q + 1) % 3, sb1 = (q + 1) % 2, sa2 = (q + 2) % 3;
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (EB) {
        lb(cl(kt + 1), sb1, 4, 8);
      } else {
        lb(cl(kt + 1), sb1, 4, 6);
        la(cl(kt + 2), sa2, 0, 2);
      }
      rdr(fa1, fb1, sa, sb, 1);
      mm(fa0, fb0);
      DX_RREGION();
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (EB) {
        la(cl(kt + 2), sa2, 0, 4);
      } else {
        lb(cl(kt + 1), sb1, 6, 8);
        la(cl(kt + 2), sa2, 2, 4);
      }
      rdr(fa0, fb0, sa, sb, 2);
      mm(fa1, fb1);
      DX_RREGION();
      __builtin_amdgcn_sched_barrier(0);
      la(cl(kt + 2), sa2, 4, 8);
      rdr(fa1, fb1, sa, sb, 3);
      mm(fa0, fb0);
      DX_RREGION();
      __builtin_amdgcn_sched_barrier(0);
      // A and B of tile kt + 1 have landed (younger loads: this k-step's 4, or with EB the 8 of A's tile
      // kt + 2), and every wave is done with tile kt, whose stages the next loads refill
      if constexpr (EB) asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      lb(cl(kt + 2), sb, 0, 4);
      rdr(fa0, fb0, sa1, sb1, 0);
      mm(fa1, fb1);
      DX_RREGION();
      __builtin_amdgcn_sched_barrier(0);
    };
    int kt = 0;
    for (; kt + 5 < KT; kt += 6) {
      iteration(kt, Int<0>());
      iteration(kt + 1, Int<1>());
      iteration(kt + 2, Int<2>());
      iteration(kt + 3, Int<3>());
      iteration(kt + 4, Int<4>());
      iteration(kt + 5, Int<5>());
    }
    if (kt < KT) iteration(kt, Int<0>());
    if (kt + 1 < KT) iteration(kt + 1, Int<1>());
    if (kt + 2 < KT) iteration(kt + 2, Int<2>());
    if (kt + 3 < KT) iteration(kt + 3, Int<3>());
    if (kt + 4 < KT) iteration(kt + 4, Int<4>());
#undef DX_RREGION
  } else if constexpr (DTL) {
    // Two stages (128-row tiles): the NI loads of a tile go out half (P3) after the barrier that frees
    // their stage and half (P0) in the next k-step, at evenly spaced MFMA slots.
    constexpr int P3 = NI / 2, P0 = NI - NI / 2, P1 = NI - P3 - P0;
    constexpr int DR0 = R0;
    static_assert(P1 >= 0 && (SMALL || DR0 + NR <= NM), "load schedule");
#define DX_DREGION(nl)                                                                             \
  if constexpr (!SMALL) do {                                                                       \
    _Pragma("unroll") for (int t = 0; t < NM; ++t) {                                               \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                           \
      if ((t * (nl)) % NM < (nl)) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);               \
      if (t >= DR0 && t - DR0 < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);             \
    }                                                                                              \
  } while (0)
    // tile 0 into stage 0, the first P3 loads of tile 1 into stage 1
    dl(0, 0, 0, NI);
    dl(min(1, KT - 1), 1, 0, P3);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(P3) : "memory");
    __syncthreads();
    rd(fa0, fb0, 0, 0);
    // Tile kt sits in stage st. The rest of its successor is fetched in the first two k-steps; after the
    // barrier (every wave done with tile kt, tile kt + 1 landed) the first loads of tile kt + 2 go into
    // stage st (clamped past the end: the last tiles reload into a free stage, harmlessly).
    auto iteration = [&](const int kt, auto stc) {
      constexpr int st = decltype(stc)::value;
      __builtin_amdgcn_sched_barrier(0);
      dl(min(kt + 1, KT - 1), st ^ 1, P3, P3 + P0);
      rd(fa1, fb1, st, 1);
      mm(fa0, fb0);
      DX_DREGION(P0);
      __builtin_amdgcn_sched_barrier(0);
      dl(min(kt + 1, KT - 1), st ^ 1, P3 + P0, NI);
      rd(fa0, fb0, st, 2);
      mm(fa1, fb1);
      DX_DREGION(P1);
      __builtin_amdgcn_sched_barrier(0);
      rd(fa1, fb1, st, 3);
      mm(fa0, fb0);
      DX_DREGION(0);
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      dl(min(kt + 2, KT - 1), st, 0, P3);
      rd(fa0, fb0, st ^ 1, 0);
      mm(fa1, fb1);
      DX_DREGION(P3);
      __builtin_amdgcn_sched_barrier(0);
    };
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
      iteration(kt, Int<0>());
      iteration(kt + 1, Int<1>());
    }
    if (kt < KT) iteration(kt, Int<0>());
#undef DX_DREGION
  } else {
    gl(0, 0, NC);
    sw(0, 0, NC);
    gl(min(1, KT - 1), 0, NC);
    __syncthreads();
    rd(fa0, fb0, 0, 0);
    // One K tile; st (compile-time, hence the loop unrolled by two) is the stage holding tile kt. The
    // registers hold tile kt + 1, which goes to the other stage while the registers refill with tile
    // kt + 2 (clamped: the last tiles reload themselves). A constant stage keeps every LDS address a
    // loop-invariant register plus an immediate.
    auto iteration = [&](const int kt, auto stc) {
      constexpr int st = decltype(stc)::value;
      const int k2 = min(kt + 2, KT - 1);
      __builtin_amdgcn_sched_barrier(0);
      sw(st ^ 1, 0, W0);
      gl(k2, 0, NG);
      rd(fa1, fb1, st, 1);
      mm(fa0, fb0);
      DX_REGION(W0, NG);
      __builtin_amdgcn_sched_barrier(0);
      sw(st ^ 1, W0, W0 + W1);
      gl(k2, NG, 2 * NG);
      rd(fa0, fb0, st, 2);
      mm(fa1, fb1);
      DX_REGION(W1, NG);
      __builtin_amdgcn_sched_barrier(0);
      sw(st ^ 1, W0 + W1, NC);
      gl(k2, 2 * NG, 3 * NG);
      rd(fa1, fb1, st, 3);
      mm(fa0, fb0);
      DX_REGION(NC - W0 - W1, NG);
      __builtin_amdgcn_sched_barrier(0);
      // every wave's writes of tile kt + 1 and reads of tile kt are complete past this point
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      gl(k2, 3 * NG, NC);
      rd(fa0, fb0, st ^ 1, 0);
      mm(fa1, fb1);
      DX_REGION(0, NG);
      __builtin_amdgcn_sched_barrier(0);
    };
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
      iteration(kt, Int<0>());
      iteration(kt + 1, Int<1>());
    }
    if (kt < KT) iteration(kt, Int<0>());
  }
#undef DX_REGION
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __syncthreads();

  if constexpr (EPI == EPI_F32) {
    float *Cf = reinterpret_cast<float *>(C);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = m0 + wm * (BM / 2) + i * 32 + lrow;
      if (row < M) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int col = n0 + wn * (BN / 2) + j * 32 + q * 8 + lhalf * 4;
            const floatx4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            *reinterpret_cast<floatx4 *>(Cf + (long)row * ldc + col) = v;
          }
      }
    }
  } else {
    // Stage the bf16 tile through LDS, then store 16-byte row chunks. A QKV tile made only of v
    // columns is staged transposed ([col][row], pitch BM + 8): its stores walk V^T rows.
    const bool vt_tile = EPI == EPI_QKV && n0 >= qe.qk_cols;
    int *const row_pos = reinterpret_cast<int *>(smem + ROW_INFO), *const row_col = row_pos + BM;
    if (EPI == EPI_QKV && tid < BM) {
      // one global load per row, issued before the staging so its latency hides behind it
      const bool live = m0 + tid < M;
      row_pos[tid] = live ? min(max(qe.pos[m0 + tid], 0), qe.max_pos - 1) : 0;
      row_col[tid] = live ? qe.vt_col[m0 + tid] : 0;
    }
    if (vt_tile) {
      constexpr int TP = BM + 8;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * (BM / 2) + i * 32 + lrow;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int col = wn * (BN / 2) + j * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
            smem[col * TP + row] = f2bf(acc[i][j][r]);
          }
      }
    } else if constexpr (EPI == EPI_BF16 || EPI == EPI_QKV || EPI == EPI_NORM) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * (BM / 2) + i * 32 + lrow;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int col = wn * (BN / 2) + j * 32 + q * 8 + lhalf * 4;
            u32x2 w;
            w[0] = pack_bf2(acc[i][j][4 * q], acc[i][j][4 * q + 1]);
            w[1] = pack_bf2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
            *reinterpret_cast<u32x2 *>(smem + row * OUT_PITCH + col) = w;
          }
      }
    } else {
      // Wave columns [0, BN/4) are gate, [BN/4, BN/2) the matching up: blocks j and j + TN/2 of the same
      // lane. The activation is chosen once for the whole loop.
      auto gated = [&](auto silu_c) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int row = wm * (BM / 2) + i * 32 + lrow;
#pragma unroll
          for (int j = 0; j < TN / 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              // g and u are rounded to bf16 two values per conversion (pack_bf2 rounds like round_bf, and
              // lo_bf / hi_bf return the two halves exactly), act(g) one value per conversion (round_bf)
              const floatx16 &ga = acc[i][j], &ua = acc[i][j + TN / 2];
              const uint32_t g2[2] = {pack_bf2(ga[4 * q], ga[4 * q + 1]), pack_bf2(ga[4 * q + 2], ga[4 * q + 3])};
              const uint32_t u2[2] = {pack_bf2(ua[4 * q], ua[4 * q + 1]), pack_bf2(ua[4 * q + 2], ua[4 * q + 3])};
              float o[4];
#pragma unroll
              for (int h = 0; h < 2; ++h) {
                const float g0 = lo_bf(g2[h]), g1 = hi_bf(g2[h]);
                const float a0 = round_bf(decltype(silu_c)::value ? silu(g0) : gelu_tanh(g0));
                const float a1 = round_bf(decltype(silu_c)::value ? silu(g1) : gelu_tanh(g1));
                o[2 * h] = a0 * lo_bf(u2[h]);
                o[2 * h + 1] = a1 * hi_bf(u2[h]);
              }
              const int col = wn * (BN / 4) + j * 32 + q * 8 + lhalf * 4;
              u32x2 w;
              w[0] = pack_bf2(o[0], o[1]);
              w[1] = pack_bf2(o[2], o[3]);
              *reinterpret_cast<u32x2 *>(smem + row * OUT_PITCH + col) = w;
            }
        }
      };
      if (act == DX_ACT_SILU) gated(Flag<true>());
      else gated(Flag<false>());
    }
    __syncthreads();
    uint16_t *Cb = reinterpret_cast<uint16_t *>(C);
    if constexpr (EPI == EPI_QKV) {
      // q / k heads (head columns below qk_cols): thread t rotates the pairs (j0 .. j0 + 7, + half) of one
      // head in tile rows t / 16 + 16 i. The cos / sin rows of 8 such rows are all requested before the
      // first is used, so the table reads cost one round trip per 8 rows.
      const int d = qe.d, half = d / 2, per_head = d / 16;
      const int rem = tid % (BN / 16), j0 = (rem % per_head) * 8, c1 = (rem / per_head) * d + j0;
      if (!vt_tile && n0 + c1 < qe.qk_cols) {
        constexpr int RSTEP = THREADS / (BN / 16), NR = BM / RSTEP, BATCH = 8;
        static_assert(NR % BATCH == 0, "rotary row batches");
#pragma unroll
        for (int i0 = 0; i0 < NR; i0 += BATCH) {
          u32x4 cs[BATCH], sn[BATCH];
#pragma unroll
          for (int i = 0; i < BATCH; ++i) {
            const long p = row_pos[tid / (BN / 16) + RSTEP * (i0 + i)];
            cs[i] = *reinterpret_cast<const u32x4 *>(qe.cos + p * half + j0);
            sn[i] = *reinterpret_cast<const u32x4 *>(qe.sin + p * half + j0);
          }
#pragma unroll
          for (int i = 0; i < BATCH; ++i) {
            const int row = tid / (BN / 16) + RSTEP * (i0 + i);
            if (m0 + row >= M) continue;
            const u32x4 a = *reinterpret_cast<const u32x4 *>(smem + row * OUT_PITCH + c1);
            const u32x4 b = *reinterpret_cast<const u32x4 *>(smem + row * OUT_PITCH + c1 + half);
            u32x4 o1, o2;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              float r1[2], r2[2];
              const float av[2] = {lo_bf(a[j]), hi_bf(a[j])}, bv[2] = {lo_bf(b[j]), hi_bf(b[j])};
              const float cv[2] = {lo_bf(cs[i][j]), hi_bf(cs[i][j])}, sv[2] = {lo_bf(sn[i][j]), hi_bf(sn[i][j])};
#pragma unroll
              for (int e = 0; e < 2; ++e) {
                r1[e] = round_bf(av[e] * cv[e]) - round_bf(bv[e] * sv[e]);
                r2[e] = round_bf(bv[e] * cv[e]) + round_bf(av[e] * sv[e]);
              }
              o1[j] = pack_bf2(r1[0], r1[1]);
              o2[j] = pack_bf2(r2[0], r2[1]);
            }
            uint16_t *dst = Cb + (long)(m0 + row) * ldc + n0 + c1;
            *reinterpret_cast<u32x4 *>(dst) = o1;
            *reinterpret_cast<u32x4 *>(dst + half) = o2;
          }
        }
      }
      if (vt_tile) {
        // Thread c owns V^T row n0 + c - qk_cols and walks the tile's tokens: 8 tokens whose V^T columns
        // are consecutive and 8-aligned go out as one 16-byte store, others one by one. The walk
        // depends on the rows only, so every thread takes the same branches.
        constexpr int TP = BM + 8;
        const int valid = min(BM, M - m0);
        for (int c = tid; c < BN; c += THREADS) {
          uint16_t *vrow = qe.vt + (long)(n0 + c - qe.qk_cols) * qe.vt_ld;
          const uint16_t *src = smem + c * TP;
          for (int r = 0; r < valid;) {
            const int col = row_col[r];
            if ((col & 7) == 0 && r + 8 <= valid && row_col[r + 7] == col + 7) {
              *reinterpret_cast<u32x4 *>(vrow + col) = *reinterpret_cast<const u32x4 *>(src + r);
              r += 8;
            } else {
              vrow[col] = src[r];
              r += 1;
            }
          }
        }
      } else if (n0 + BN > qe.qk_cols) {
        // a tile holding both q|k and v columns: v one element at a time (tile column c is V^T row
        // n0 + c - qk_cols; the lanes of a store instruction write consecutive V^T columns)
        const int row = tid % BM;
        if (m0 + row < M) {
          const long col = row_col[row];
          for (int c = max(qe.qk_cols - n0, 0) + tid / BM; c < BN; c += THREADS / BM)
            qe.vt[(long)(n0 + c - qe.qk_cols) * qe.vt_ld + col] = smem[row * OUT_PITCH + c];
        }
      }
    } else if constexpr (EPI == EPI_NORM) {
      // System-coherent stores (sc0 sc1: they reach memory, not only this XCD's L2): the row block's last
      // workgroup reads the tile back within this kernel, possibly from another XCD.
      constexpr int CPR = OUT_W / 8;
      const __amdgpu_buffer_rsrc_t rc = make_rsrc(Cb + (long)m0 * ldc, (long)min(M - m0, BM) * ldc * 2);
      for (int idx = tid; idx < BM * CPR; idx += THREADS) {
        const int row = idx / CPR, c = idx % CPR;
        if (m0 + row < M)
          __builtin_amdgcn_raw_buffer_store_b128(*reinterpret_cast<const u32x4 *>(smem + row * OUT_PITCH + c * 8),
                                                 rc, (int)((row * ldc + n0 + c * 8) * 2), 0, 17);
      }
      norm_epilogue<BM>(Cb, M, N, ldc, m0, tm, num_n, ne, reinterpret_cast<int *>(smem));
    } else {
      const int out_n0 = EPI == EPI_GATED ? n0 / 2 : n0;
      constexpr int CPR = OUT_W / 8;  // 16-byte chunks per row
      for (int idx = tid; idx < BM * CPR; idx += THREADS) {
        const int row = idx / CPR, c = idx % CPR;
        if (m0 + row < M)
          *reinterpret_cast<u32x4 *>(Cb + (long)(m0 + row) * ldc + out_n0 + c * 8) =
              *reinterpret_cast<const u32x4 *>(smem + row * OUT_PITCH + c * 8);
      }
    }
  }
}

template <int BM, int EPI>
hipError_t launch(const uint16_t *A, const uint16_t *B, void *C, long M, long N, long K, long lda, long ldb,
                  long ldc, int act, const QkvEpilogue &qe, const NormEpilogue &ne, hipStream_t s) {
  const long num_m = (M + BM - 1) / BM, num_n = N / tile_n<BM>();
  const bool weight_cached = N * K * 2 <= (256L << 20);  // the weight fits the 256 MB Infinity Cache
  // 256-row tiles always take the direct-to-LDS ring: its A stages give long-K shapes the latency slack
  // (against the register-staged path: down K 14336 +3-8 % alone and -0.8 % step time in the 9B
  // forward, K 36864 +4.5 %, 1344- and 448-tile down shapes +2.5 % / +1 %). 128-row tiles (M <= 1024)
  // have two stages only, so long K keeps the register-staged path and its two tiles of slack there.
  auto kern = gemm_nt_kernel<BM, EPI, true>;
  if constexpr (BM != 256)
    if (K > 8192) kern = gemm_nt_kernel<BM, EPI, false>;
  // The early-B order of the ring gains where the weight fits the 256 MB Infinity Cache (9B forward: gate|up
  // +2.8%, down +1.9%, q|k|v +1.2%, step -1.7%) and loses where it does not (27B gate|up and down, 680 and
  // 340 MB: -3% each); bit-identical either way.
  if constexpr (BM == 256)
    if (weight_cached) kern = gemm_nt_kernel<BM, EPI, true, true>;
  // Tile rows walked together per XCD. Long K: an A row tile is megabytes, and groups of 8 re-read it
  // once per 4 column tiles. So 1 row when the weight fits the Infinity Cache, where the weight's
  // re-reads are cheap and the A tile's are not (9B down, K 14336: +1.3% against 2, +5% against 8), and
  // 2 when it does not (27B down, K 36864: 1 and 3 within 0.2% of 2). 4 for the plain bf16 / fp32
  // epilogues (o at 9B and 27B: +1.5-2%). 8 for the q|k|v epilogue, where 4 measured mixed (27B q|k|v
  // -4.7%) and 6 too (9B +0.7%, 27B -1.2%). The gated epilogue takes 6 when its weight is cached (9B
  // gate|up +1.1%) and 8 when not (27B gate|up: 6 is 10% slower).
  const int short_k = (EPI == EPI_BF16 || EPI == EPI_F32 || EPI == EPI_NORM) ? 4
                      : EPI == EPI_GATED && weight_cached                    ? 6
                                                                             : 8;
  const int group_m = K >= 8192 ? (weight_cached ? 1 : 2) : short_k;
  kern<<<dim3((unsigned)(num_m * num_n)), dim3(THREADS), 0, s>>>(A, B, C, (int)M, (int)N, (int)K, lda, ldb, ldc,
                                                                 act, group_m, qe, ne);
  return hipGetLastError();
}

template <int EPI>
hipError_t dispatch(const uint16_t *A, const uint16_t *B, void *C, long M, long N, long K, long lda, long ldb,
                    long ldc, int act, hipStream_t s, const QkvEpilogue &qe = QkvEpilogue{},
                    const NormEpilogue &ne = NormEpilogue{}) {
  // Small M: halve the row tile so more workgroups exist. For the plain epilogues, 64 x 128 tiles when the
  // 128 x 256 ones would leave three quarters of the CUs idle (under 64 tiles: o and down of one 9B
  // request of up to 512 tokens; its forward -12 to -16% at 128-512 tokens, unchanged from 768 on).
  if constexpr (EPI == EPI_BF16 || EPI == EPI_F32)
    if (M <= 1024 && (M + 127) / 128 * (N / tile_n<128>()) < 64)
      return launch<64, EPI>(A, B, C, M, N, K, lda, ldb, ldc, act, qe, ne, s);
  if (M <= 1024) return launch<128, EPI>(A, B, C, M, N, K, lda, ldb, ldc, act, qe, ne, s);
  return launch<256, EPI>(A, B, C, M, N, K, lda, ldb, ldc, act, qe, ne, s);
}

}  // namespace

hipError_t dx_gemm_bf16(const uint16_t *A, const uint16_t *B, uint16_t *C, long M, long N, long K, long lda,
                        long ldb, long ldc, hipStream_t s) {
  return dispatch<EPI_BF16>(A, B, C, M, N, K, lda, ldb, ldc, 0, s);
}

hipError_t dx_gemm_f32(const uint16_t *A, const uint16_t *B, float *C, long M, long N, long K, long lda, long ldb,
                       long ldc, hipStream_t s) {
  return dispatch<EPI_F32>(A, B, C, M, N, K, lda, ldb, ldc, 0, s);
}

hipError_t dx_gemm_gated(const uint16_t *A, const uint16_t *B, uint16_t *C, long M, long F, long K, long lda,
                         long ldc, int act, hipStream_t s) {
  return dispatch<EPI_GATED>(A, B, C, M, 2 * F, K, lda, K, ldc, act, s);
}

hipError_t dx_gemm_qkv(const uint16_t *A, const uint16_t *B, uint16_t *QK, long M, long N, long K, long lda, long ldb,
                       long ld_qk, const QkvEpilogue &qe, hipStream_t s) {
  return dispatch<EPI_QKV>(A, B, QK, M, N, K, lda, ldb, ld_qk, 0, s, qe);
}

hipError_t dx_gemm_norm(const uint16_t *A, const uint16_t *B, uint16_t *C, long M, long N, long K, long lda,
                        long ldb, const NormEpilogue &ne, hipStream_t s) {
  return dispatch<EPI_NORM>(A, B, C, M, N, K, lda, ldb, N, 0, s, QkvEpilogue{}, ne);
}

long dx_gemm_norm_row_blocks(long M) { return M <= 1024 ? (M + 127) / 128 : (M + 255) / 256; }
