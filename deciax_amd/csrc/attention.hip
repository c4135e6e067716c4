// Causal GQA prefill attention for gfx950: a bf16 MFMA path, an fp32 MFMA path (head_dim <= 128) and
// an fp32 VALU path (head_dim 256).
//
// Algorithm (the reference's blocked causal GQA attention,
// src/deciax/kernels/attention/blocked.py:9-32, in the online form of its TPU
// flash kernel, src/deciax/kernels/attention/pallas.py:52-135): each
// workgroup owns one sequence, one KV head and a tile of query rows for all
// G = Hq / Hkv query heads sharing that KV head, so K/V tiles are staged in LDS
// once per group instead of being repeated per head (blocked.py:12-13 repeats
// them). Key tiles entirely outside the causal / sliding window are never
// visited; only tiles that straddle a boundary evaluate the mask.
//
// bf16 path, per wave (32 query rows of one head):
//   S^T = K Q^T  with 32x32x16 MFMAs: A = K rows from LDS, B = Q^T held in
//        registers for the whole key loop. Lane l then owns query (l % 32) and
//        16 keys per 32-key block, so row statistics are lane-local plus one
//        exchange with lane l ^ 32.
//   K rows are fed in the order kperm() so that the 8 keys a lane owns in
//   each half of a 32-key block are consecutive; those 8 scores become, after
//   bf16 rounding, the lane's B operand of O^T = V^T P^T directly, and the A
//   operand is one 16-byte read of the V^T tile (V transposed, [D][64] in LDS).
//
// Softmax: with logit soft-capping (Gemma-2, cap <= 56) every capped score
// lies in (-cap, cap), so p = exp(t - cap/2) is computed with a fixed shift:
// no running max, no rescaling of the O accumulator, no cross-lane max.
// t - cap/2 = cap/2 - 2 cap / (1 + e^{2x}), x = scale * s / cap, hence in log2
// units c3 + c2 / (1 + exp2(c1 s)) with c1 = 2 log2(e) scale / cap,
// c2 = -2 cap log2(e), c3 = cap log2(e) / 2. The kernel multiplies q by c1 as it
// loads it (one bf16 rounding of c1 q), so the MFMA yields c1 s directly, and
// folds c2 into the reciprocal:
//   p = exp2(c3 + 1 / fma(exp2(c1 s), 1/c2, 1/c2)),
// three transcendentals and two ordinary VALU operations per score.
// p stays within [e^{-3cap/2}, e^{cap/2}] — normal fp32 and bf16 numbers for
// cap <= 56 — and softmax is invariant to the shift. Without soft-capping (or
// for larger caps) the kernel keeps the usual running max in log2 units.
// P is rounded to bf16 before P.V (the reference rounds the normalised
// weights to q.dtype, blocked.py:27); O is divided by the fp32 row sum.
#include "common.h"
#include "kernels.h"

namespace {

constexpr int THREADS = 256;        // fp32 path and the V^T transpose
constexpr int BKV = 64;     // V^T block alignment of dx_transpose_v
// bf16 path: waves per workgroup and LDS ring depth. The long form, 8 waves (two per SIMD, 32 query rows
// each) over a 4-stage ring (128 KB), runs one workgroup per CU. The short form, 4 waves over a 2-stage
// ring (64 KB), runs two workgroups per CU that fall out of step with each other, so one's prologue,
// epilogue and barrier waits overlap the other's key loop; it halves the query rows per staged K/V tile.
// Head_dim 128 takes the short form when a query row sees 2048 keys or fewer on average (window <= 2048,
// or causal sequences up to 4096): 27B heads, 8 x 2048 -4%, window 512 -12 to -15%, window 1024 -5 to
// -10%, 16 x 3400 -2%; on longer spans it measured +0.2 to +1.1% (4 x 16384). Head_dim 256 keeps the long
// form everywhere: the short one measured 6-11% slower on every shape but window 512 (within 1.5%).
// bf16 grid order switch (see attn_bf16_kernel). Whole units per XCD measured 3-9% faster at 3257-4096
// tokens (16 sequences, 9B and 27B heads), 2% slower at 8 x 3072 and 15% slower at 8 x 2048.
constexpr int SHORT_SEQ = 3072;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float NEG_BIG = -1e30f;  // the reference's MASK_FILL (reference.py:8)

enum { MODE_FIXED = 0, MODE_ONLINE = 1 };

DX_DEVICE bool visible(int qi, int key, int len, int window, int causal) {
  if (key >= len) return false;
  if (causal) return key <= qi && (window <= 0 || key > qi - window);
  return window <= 0 || abs(qi - key) <= window;
}

// K tile in LDS: [TK keys][D], 16-byte chunk c of row r at slot c ^ k_swz<D>(r) (see below).

// V^T tile in LDS: [D][T keys]; with 64-byte rows (T = 32) chunk c of row r sits at slot c ^ ((r >> 2) & 3),
// with 128-byte rows (T = 64) at c ^ ((r >> 1) & 7): the 16 rows one fragment read touches per pass fill
// all 16 chunk slots of a 256-byte bank line.
template <int T>
DX_DEVICE int vt_swz(int row) {
  if constexpr (T == 32) return (row >> 2) & 3;
  else return (row >> 1) & 7;  // 128-byte rows
}
template <int T>
DX_DEVICE int vt_off(int row, int chunk) { return row * T + ((chunk ^ vt_swz<T>(row)) << 3); }

// MFMA row vk of a 32-key block reads key kperm(vk). The output register r of
// lane-half hh then holds key 16 (r >> 3) + 8 hh + (r & 7).
DX_DEVICE int kperm(int vk) { return 16 * (vk >> 4) + 8 * ((vk >> 2) & 1) + 4 * ((vk >> 3) & 1) + (vk & 3); }

// Direct-to-LDS loads: instruction j of a wave's share fills 1 KB of LDS (64 lanes x 16 bytes) at a
// wave-uniform base; each lane fetches the global chunk whose swizzled slot it fills.
typedef __attribute__((address_space(3))) void lds_void;

DX_DEVICE __amdgpu_buffer_rsrc_t make_rsrc(const uint16_t *base, long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}

// 16 bytes per lane from a buffer resource into LDS at lds + 16 * lane. The builtin is compiled in the
// device pass only: this clang drops a kernel's host-side symbols when the host pass sees it.
DX_DEVICE void lds_load16(__amdgpu_buffer_rsrc_t rsrc, uint16_t *lds, int voffset) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void *)lds, 16, voffset, 0, 0, 0);
#endif
}

// Schedule n (LDS read, MFMA) pairs with the reads LEAD ahead: enough to cover LDS latency, few
// enough that the operand registers in flight stay small.
template <int N>
DX_DEVICE void stream_sched() {
  constexpr int LEAD = 3;
  __builtin_amdgcn_sched_group_barrier(0x100, LEAD, 0);
#pragma unroll
  for (int t = 0; t < N - LEAD; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, LEAD, 0);
}

template <int D>
DX_DEVICE int k_swz(int row) {
  if constexpr (D / 8 >= 16) return row & 15;
  else return (row >> 1) & 7;
}

// bf16 path: WAVES waves (two per SIMD, the short or long form above), wave w = 32 query rows of head
// g * G + w % G. Each 64-key tile is processed in two 32-key halves (QK^T, softmax, PV per half) so a wave
// needs only 16 score registers and the other wave on its SIMD can run MFMAs while this one is in the
// softmax.
// Keys per tile: 32 at head_dim 256 (a 64-key tile would halve the ring depth), 64 below.
template <int D>
constexpr int tile_keys() { return D >= 256 ? 32 : 64; }

template <bool B>
struct Flag {
  static constexpr bool value = B;
};

// KM: a per-key mask (key_bits, key_words 32-bit words per sequence; bit j of word w of sequence b is key
// 32 w + j) hides keys beyond the causal / window rule. Tiles that hold a masked key take the masked body,
// and a query row that sees no key is written as zeros.
template <int D, int G, int MODE, bool KM, int WAVES, int NSTAGE>
__global__ void __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2, 2)))
attn_bf16_kernel(const uint16_t *__restrict__ Q, const uint16_t *__restrict__ K, const uint16_t *__restrict__ Vt,
                 uint16_t *__restrict__ O, const int32_t *__restrict__ seq_start,
                 const int32_t *__restrict__ seq_len, const int32_t *__restrict__ vt_start, long vt_seq_stride,
                 int max_seq_len, long q_stride, long k_stride, long vt_ld, long o_stride, float scale,
                 float softcap, int window, int causal, const uint32_t *__restrict__ key_bits, int key_words) {
  constexpr int TK = tile_keys<D>();
  constexpr int RG = WAVES / G;         // 32-row groups per head
  constexpr int BQ = 32 * RG;           // query rows per workgroup
  constexpr int KST = TK * D;           // elements of the K tile [TK][D]; the V^T tile [D][TK] follows
  constexpr int STAGE = 2 * TK * D;
  constexpr int NI = TK * D / 256;      // direct-to-LDS instructions per tile (K then V^T), 1 KB each
  constexpr int WI = NI / WAVES;        // per wave
  constexpr int NKS = D / 16;
  constexpr int NDB = D / 32;
  constexpr int CPR = D / 8;            // 16-byte chunks per K row
  static_assert(WI >= 2 && WI % 2 == 0 && NI % WAVES == 0, "tile too small for the wave count");
  static_assert(WAVES * 32 * D <= NSTAGE * STAGE, "the ring must hold every wave's 32 x D output tile");
  __shared__ __attribute__((aligned(1024))) uint16_t smem[NSTAGE * STAGE];

  // Grid order, the query tile index counted from the last (heaviest first):
  // - max_seq_len > SHORT_SEQ: (query tile, KV head, sequence), dealt out so that each XCD runs whole
  //   (sequence, KV head) units. Workgroups go to the 8 XCDs round-robin in dispatch order, each with its
  //   own L2, so dispatch p runs on XCD p % 8; unit u = 8 k + x takes XCD x's k-th run of query tiles.
  //   Every query tile of a unit reads the same K and V^T from key 0 (or the window start), so they hit
  //   in one L2 instead of being fetched once per XCD (9B batch: -7 to -9% per layer; 27B 4 x 16384:
  //   -6 to -14%). An XCD still walks its units in descriptor order, which the forward driver sorts
  //   longest first. Unit counts that are not a multiple of 8 keep the plain order.
  // - otherwise: (KV head, sequence, query tile), the heaviest tiles of every sequence first. With short
  //   sequences a single tile is a large share of a CU's work, so the order above leaves a tail
  //   (8 x 2048: 15% slower that way), while each (sequence, head)'s K and V^T fit in an XCD's L2.
  //   On ragged lengths up to 16K this order costs 25-35% instead: the concurrent streams scatter.
  const bool tile_major = max_seq_len <= SHORT_SEQ;
  int g, b, qt;
  if (tile_major) {
    g = blockIdx.x;
    b = blockIdx.y;
    qt = blockIdx.z;
  } else if ((gridDim.y * gridDim.z) % 8 == 0) {
    const long p = blockIdx.x + (long)gridDim.x * (blockIdx.y + (long)gridDim.y * blockIdx.z);
    const long idx = p >> 3, u = idx / gridDim.x * 8 + (p & 7);
    qt = (int)(idx % gridDim.x);
    g = (int)(u % gridDim.y);
    b = (int)(u / gridDim.y);
  } else {
    qt = blockIdx.x;
    g = blockIdx.y;
    b = blockIdx.z;
  }
  const int len = min(max(seq_len[b], 0), max_seq_len);
  const int ntiles = (max_seq_len + BQ - 1) / BQ;
  const int q0 = (ntiles - 1 - qt) * BQ;
  if (q0 >= len) return;
  const long start = seq_start[b];
  const long vts = vt_start ? (long)vt_start[b] : (long)b * vt_seq_stride;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lrow = lane & 31, lhalf = lane >> 5;
  const int rg = wave / G, h = g * G + wave % G;
  const int qw0 = q0 + rg * 32, qw1 = qw0 + 31;
  const int qi = qw0 + lrow;

  bf16x8 qf[NKS];
  {
    const uint16_t *qp = Q + (start + min(qi, len - 1)) * q_stride + (long)h * D + lhalf * 8;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) qf[ks] = as_bf16x8(*reinterpret_cast<const u32x4 *>(qp + ks * 16));
  }
  if constexpr (MODE == MODE_FIXED) {
    // q <- bf16(c1 q): the QK^T MFMAs then give the exponent c1 s of the fixed-shift softmax below
    const float c1 = 2.f * LOG2E * scale / softcap;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      u32x4 w = __builtin_bit_cast(u32x4, qf[ks]);
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = pack_bf2(lo_bf(w[i]) * c1, hi_bf(w[i]) * c1);
      qf[ks] = as_bf16x8(w);
    }
  }

  const int qlast = min(q0 + BQ, len) - 1;
  int klo, khi;
  if (causal) {
    khi = qlast + 1;
    klo = window > 0 ? max(0, q0 - window + 1) : 0;
  } else {
    khi = window > 0 ? min(len, qlast + window + 1) : len;
    klo = window > 0 ? max(0, q0 - window) : 0;
  }
  const int kt0 = klo / TK, kt1 = (khi + TK - 1) / TK;

  // K rows past len read as zero (outside the resource); V^T columns stay inside this sequence's
  // 64-aligned block, whose tail dx_transpose_v zero-fills. Each tile's resources are rebased at the
  // tile (scalar work), so the per-lane offsets below are loop-invariant.
  const uint16_t *kbase0 = K + start * k_stride + (long)g * D;
  const uint16_t *vbase0 = Vt + (long)g * D * vt_ld + vts;
  const long kbytes = (long)len * k_stride * 2;
  const long vbytes = ((long)(D - 1) * vt_ld + ((len + 63) & ~63)) * 2;
  // Wave w fills K instructions [w WI/2, (w + 1) WI/2) and as many V^T instructions. K instruction i
  // fills K slots [64 i, 64 i + 64): row p / CPR, chunk (p % CPR) ^ k_swz(row); V^T instruction i
  // fills row p / (TK / 8), chunk (p % (TK / 8)) ^ vt_swz(row).
  constexpr int WH = WI / 2;
  int koff[WH], voff[WH];
#pragma unroll
  for (int j = 0; j < WH; ++j) {
    const int p = (wave * WH + j) * 64 + lane;
    const int krow = p / CPR, kc = (p % CPR) ^ k_swz<D>(krow);
    koff[j] = (int)(krow * k_stride * 2) + kc * 16;
    const int vrow = p / (TK / 8), vc = (p % (TK / 8)) ^ vt_swz<TK>(vrow);
    voff[j] = (int)(vrow * vt_ld * 2) + vc * 16;
  }
  auto issue = [&](int kt, int st) {
    uint16_t *base = smem + st * STAGE;
    const long kb = (long)kt * TK;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase0 + kb * k_stride, max(kbytes - kb * k_stride * 2, 0L));
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase0 + kb, vbytes - kb * 2);
#pragma unroll
    for (int j = 0; j < WH; ++j) {
      lds_load16(rk, base + (wave * WH + j) * 512, koff[j]);
      lds_load16(rv, base + KST + (wave * WH + j) * 512, voff[j]);
    }
  };

  floatx16 o[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float lsum = 0.f;
  float mrun = NEG_BIG;

  const float c2inv = 1.f / (-2.f * LOG2E * softcap);
  const float c3 = 0.5f * LOG2E * softcap;

  // Which 32-key blocks this wave's rows see: active = some key visible, masked = some key hidden.
  auto block_state = [&](const int kbase, bool &need_mask) {
    bool active = qw0 < len;
    need_mask = kbase + 32 > len;
    if (causal) {
      active = active && kbase <= qw1 && !(window > 0 && kbase + 31 <= qw0 - window);
      need_mask = need_mask || kbase + 31 > qw0 || (window > 0 && kbase <= qw1 - window);
    } else if (window > 0) {
      active = active && kbase <= qw1 + window && kbase + 31 >= qw0 - window;
      need_mask = need_mask || kbase < qw1 - window || kbase + 31 > qw0 + window;
    }
    return active;
  };
  // Visible keys of row qi form one interval [vlo, vhi].
  int vlo, vhi;
  if (causal) {
    vhi = min(qi, len - 1);
    vlo = window > 0 ? qi - window + 1 : 0;
  } else {
    vhi = window > 0 ? min(qi + window, len - 1) : len - 1;
    vlo = window > 0 ? qi - window : 0;
  }

  // One 32-key block kb of the tile in stage sk (K, then V^T at sk + KST): S^T = K Q^T, softmax,
  // O^T += V^T P^T. MASKED evaluates the causal / window / length mask and skips blocks no row sees.
  auto block = [&](const uint16_t *sk, const int kbase, const int kb, auto masked) {
    constexpr bool M = decltype(masked)::value;
    if constexpr (M) {
      bool need_mask;
      if (!block_state(kbase, need_mask)) return;
    }
    floatx16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
    {
      // for ks and ks + 8 the swizzled slots differ by the same 16 chunks: 8 lane offsets serve all 16
      const int krow = kb * 32 + kperm(lrow);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int lo = (((ks & 7) * 2 + lhalf) ^ k_swz<D>(krow)) << 3;
        s = mfma32(as_bf16x8(*reinterpret_cast<const u32x4 *>(sk + krow * D + (ks & ~7) * 16 + lo)), qf[ks], s);
      }
      stream_sched<NKS>();  // keep only a few K fragments live at once
    }
    // key of score r: kbase + 16 (r >> 3) + 8 lhalf + (r & 7); visible iff inside [vlo, vhi] (and, with a
    // key mask, its bit is set: kbase is a multiple of 32, so the block's 32 keys are one mask word)
    const int mlo = vlo - kbase - 8 * lhalf, mhi = vhi - kbase - 8 * lhalf;
    uint32_t kbits = 0xffffffffu;
    if constexpr (KM && M) kbits = key_bits[(long)b * key_words + (kbase >> 5)] >> (8 * lhalf);
    auto keep = [&](int r) {
      const int j = 16 * (r >> 3) + (r & 7);
      if constexpr (KM) return j >= mlo && j <= mhi && ((kbits >> j) & 1u);
      else return j >= mlo && j <= mhi;
    };
    if constexpr (MODE == MODE_FIXED) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = fast_exp2(s[r]);  // s[r] = c1 * score: q was scaled by c1 at load
        float p = fast_exp2(fast_rcp(__builtin_fmaf(e, c2inv, c2inv)) + c3);
        if constexpr (M) p = keep(r) ? p : 0.f;
        s[r] = p;
        lsum += p;
      }
    } else {
      float tmax = NEG_BIG;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float t = s[r] * scale;
        if (softcap > 0.f) t = softcap * tanhf(t / softcap);
        t *= LOG2E;
        if constexpr (M) t = keep(r) ? t : NEG_BIG;
        s[r] = t;
        tmax = fmaxf(tmax, t);
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float mnew = fmaxf(mrun, tmax);
      const float alpha = fast_exp2(mrun - mnew);
      mrun = mnew;
      lsum *= alpha;
#pragma unroll
      for (int i = 0; i < NDB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(s[r] - mnew);
        if constexpr (M) p = keep(r) ? p : 0.f;
        s[r] = p;
        lsum += p;
      }
    }
    bf16x8 pf[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      u32x4 w;
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = pack_bf2(s[8 * h2 + 2 * i], s[8 * h2 + 2 * i + 1]);
      pf[h2] = as_bf16x8(w);
    }
    const uint16_t *sv = sk + KST;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int vrow = db * 32 + lrow;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
        o[db] = mfma32(as_bf16x8(*reinterpret_cast<const u32x4 *>(sv + vt_off<TK>(vrow, kb * 4 + 2 * h2 + lhalf))),
                       pf[h2], o[db]);
    }
    stream_sched<2 * NDB>();
  };

  // Ring of NSTAGE tiles: tile kt sits in stage (kt - kt0) % NSTAGE, and tile kt + NSTAGE - 1 is
  // fetched while tile kt is multiplied (clamped: the last tiles reload themselves harmlessly).
  auto tile = [&](const int kt, auto masked) {
    issue(min(kt + NSTAGE - 1, kt1 - 1), (kt - kt0 + NSTAGE - 1) % NSTAGE);
    const uint16_t *sk = smem + ((kt - kt0) % NSTAGE) * STAGE;
#pragma unroll
    for (int kb = 0; kb < TK / 32; ++kb) block(sk, kt * TK + kb * 32, kb, masked);
    // tile kt + 1 has landed in every wave's share (the NSTAGE - 2 younger tiles may stay in flight)
    // and every wave is done reading tile kt, whose stage the next iteration refills. A plain s_barrier:
    // __syncthreads would also wait for the younger tiles' loads (its fence waits for all LDS writes).
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((NSTAGE - 2) * WI) : "memory");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };

  // Tiles [ta, tb) hold no key this wave's rows cannot see (all blocks active, none masked): they run
  // without any mask code. The tiles before and after take the masked body. Every wave runs one
  // iteration (one barrier) per tile, whichever body.
  int ta = kt1, tb = kt1;
  if (qw1 < len) {
    int lo_u = 0, hi_u = len - 32;  // first / last kbase of an unmasked block
    if (causal) {
      hi_u = min(hi_u, qw0 - 31);
      if (window > 0) lo_u = qw1 - window + 1;
    } else if (window > 0) {
      lo_u = qw1 - window;
      hi_u = min(hi_u, qw0 + window - 31);
    }
    lo_u = max(lo_u, 0);
    const int a = max(kt0, (lo_u + TK - 1) / TK);
    const int last = hi_u - (TK - 32);  // kbase of the tile's first block
    const int b = last < 0 ? kt0 : min(kt1, last / TK + 1);
    if (a < b) {
      ta = a;
      tb = b;
    }
  }

#pragma unroll
  for (int i = 0; i < NSTAGE - 1; ++i) issue(min(kt0 + i, kt1 - 1), i);
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((NSTAGE - 2) * WI) : "memory");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (KM) {
    // A tile of [ta, tb) whose keys the mask keeps entirely takes the unmasked body as well. Its mask
    // words are requested one tile ahead (scalar loads, which the tile's barrier wait covers).
    const uint32_t *const kw = key_bits + (long)b * key_words;
    auto full = [&](int kt) {
      bool f = true;
#pragma unroll
      for (int i = 0; i < TK / 32; ++i) f = f && kw[kt * (TK / 32) + i] == 0xffffffffu;
      return f;
    };
    for (int kt = kt0; kt < kt1; ++kt) {
      if (kt >= ta && kt < tb && full(kt)) {
        // a run of interior tiles whose keys the mask keeps, each next tile's words read before this one
        for (bool more = true; more; ++kt) {
          more = kt + 1 < tb && full(kt + 1);
          tile(kt, Flag<false>());
        }
        if (kt == kt1) break;
      }
      tile(kt, Flag<true>());
    }
  } else {
    for (int kt = kt0; kt < kt1; ++kt) {
      if (kt == ta) {
        for (; kt < tb; ++kt) tile(kt, Flag<false>());
        if (kt == kt1) break;
      }
      tile(kt, Flag<true>());
    }
  }
  // Every wave's ring loads have landed and no wave reads the ring any more: it now stages the output.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // Each lane holds 4-value pieces of its row qi scattered over the head's D columns; stored directly,
  // every store instruction would touch 32 rows (32 cache lines, 8 bytes each). The wave writes its
  // 32 x D bf16 tile to its own LDS region (row r's 16-byte chunk c at slot c ^ (r % CPR)), then each
  // store instruction writes whole contiguous rows, 16 bytes per lane.
  lsum += __shfl_xor(lsum, 32, 64);
  float inv = 1.f / lsum;
  if constexpr (KM) inv = lsum > 0.f ? inv : 0.f;
  // Lane indices derived anew here, through an opaque copy: values shared with the prologue would stay
  // live across the key loop, and the loop's schedule then keeps fewer fragment reads in flight.
  int el = (int)threadIdx.x & 63;
  asm volatile("" : "+v"(el));
  const int erow = el & 31, ehalf = el >> 5;
  uint16_t *stage = smem + wave * 32 * D;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      u32x2 w;
      w[0] = pack_bf2(o[db][grp * 4 + 0] * inv, o[db][grp * 4 + 1] * inv);
      w[1] = pack_bf2(o[db][grp * 4 + 2] * inv, o[db][grp * 4 + 3] * inv);
      const int chunk = db * 4 + grp;  // 16-byte chunk of the row; this lane fills its half ehalf
      *reinterpret_cast<u32x2 *>(stage + erow * D + ((chunk ^ (erow % CPR)) << 3) + ehalf * 4) = w;
    }
  __syncthreads();
  constexpr int RPI = 64 / CPR;  // rows per store instruction
#pragma unroll
  for (int i = 0; i < 32 / RPI; ++i) {
    const int r = i * RPI + el / CPR, c = el % CPR;
    if (qw0 + r < len)
      *reinterpret_cast<u32x4 *>(O + (start + qw0 + r) * o_stride + (long)h * D + c * 8) =
          *reinterpret_cast<const u32x4 *>(stage + r * D + ((c ^ (r % CPR)) << 3));
  }
}

// fp32 path: VALU flash attention, TPQ threads per query row.
template <int D, int TPQ>
__global__ void __launch_bounds__(THREADS)
attn_f32_kernel(const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
                float *__restrict__ O, const int32_t *__restrict__ seq_start, const int32_t *__restrict__ seq_len,
                int max_seq_len, int hq, int hkv, long q_stride, long k_stride, long v_stride, long o_stride,
                float scale, float softcap, int window, int causal, const uint8_t *__restrict__ key_mask) {
  constexpr int QPB = THREADS / TPQ;
  constexpr int DPT = D / TPQ;
  constexpr int TK = 32;
  __shared__ __attribute__((aligned(16))) float ks[TK * D];
  __shared__ __attribute__((aligned(16))) float vs[TK * D];

  const int b = blockIdx.y, h = blockIdx.z, g = h / (hq / hkv);
  const int len = min(max(seq_len[b], 0), max_seq_len);
  const int ntiles = (max_seq_len + QPB - 1) / QPB;
  const int q0 = (ntiles - 1 - (int)blockIdx.x) * QPB;
  if (q0 >= len) return;
  const long start = seq_start[b];
  const int tid = threadIdx.x, part = tid % TPQ;
  const int qi = q0 + tid / TPQ;

  float q[DPT], o[DPT];
  {
    const float *qp = Q + (start + min(qi, len - 1)) * q_stride + (long)h * D + part * DPT;
#pragma unroll
    for (int d = 0; d < DPT; ++d) {
      q[d] = qp[d];
      o[d] = 0.f;
    }
  }
  const int qlast = min(q0 + QPB, len) - 1;
  int klo, khi;
  if (causal) {
    khi = qlast + 1;
    klo = window > 0 ? max(0, q0 - window + 1) : 0;
  } else {
    khi = window > 0 ? min(len, qlast + window + 1) : len;
    klo = window > 0 ? max(0, q0 - window) : 0;
  }
  float m = NEG_BIG, l = 0.f;
  for (int k0 = (klo / TK) * TK; k0 < khi; k0 += TK) {
    __syncthreads();
    for (int idx = tid; idx < TK * D / 4; idx += THREADS) {
      const int row = idx / (D / 4), c = idx % (D / 4);
      const long key = start + min(k0 + row, len - 1);
      reinterpret_cast<float4 *>(ks)[idx] = *reinterpret_cast<const float4 *>(K + key * k_stride + (long)g * D + c * 4);
      reinterpret_cast<float4 *>(vs)[idx] = *reinterpret_cast<const float4 *>(V + key * v_stride + (long)g * D + c * 4);
    }
    __syncthreads();
    float sc[TK];
    uint32_t vis = 0;
    float tmax = NEG_BIG;
#pragma unroll
    for (int j = 0; j < TK; ++j) {
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < DPT; ++d) s = fmaf(q[d], ks[j * D + part * DPT + d], s);
#pragma unroll
      for (int off = 1; off < TPQ; off <<= 1) s += __shfl_xor(s, off, 64);
      s *= scale;
      if (softcap > 0.f) s = softcap * tanhf(s / softcap);
      // key_mask (nullable) hides keys of row start + key; read only for keys inside the sequence
      const bool v = visible(qi, k0 + j, len, window, causal) && (!key_mask || key_mask[start + k0 + j]);
      vis |= (uint32_t)v << j;
      sc[j] = s;
      if (v) tmax = fmaxf(tmax, s);
    }
    const float mnew = fmaxf(m, tmax);
    const float alpha = expf(m - mnew);
    l *= alpha;
#pragma unroll
    for (int d = 0; d < DPT; ++d) o[d] *= alpha;
#pragma unroll
    for (int j = 0; j < TK; ++j) {
      const float p = ((vis >> j) & 1u) ? expf(sc[j] - mnew) : 0.f;
      l += p;
#pragma unroll
      for (int d = 0; d < DPT; ++d) o[d] = fmaf(p, vs[j * D + part * DPT + d], o[d]);
    }
    m = mnew;
  }
  if (qi < len) {
    float *op = O + (start + qi) * o_stride + (long)h * D + part * DPT;
#pragma unroll
    for (int d = 0; d < DPT; ++d) op[d] = l > 0.f ? o[d] / l : 0.f;  // a row that sees no key: zeros
  }
}

// fp32 path on the matrix core, head_dim <= 128: v_mfma_f32_32x32x2_f32 (fp32 products and sums).
// A workgroup takes 32 query rows of one head. Its F_WAVES waves split the 32-key blocks (wave w takes
// blocks w, w + F_WAVES, ...), each staging its block in an LDS region of its own, and merge their
// online-softmax states (running max, row sum, O) at the end, so no barrier runs inside the key loop.
//   S^T = K Q^T: D / 2 MFMAs, MFMA j contracting head dims j (lanes 0-31) and D / 2 + j (lanes
//   32-63). Lane l then holds query l % 32 and keys (r / 4) 8 + (l / 32) 4 + r % 4 of the block.
//   O^T += V^T P^T: MFMA step i contracts the two keys the lane halves hold in register i, so each lane
//   feeds its own probabilities as the B operand and reads V[key][d] for its half's key.
// The next block's K and V are requested from global memory into registers at the start of this block
// and go to LDS once the region's previous reads are done (K after this block's PV, V at the start of the
// next block; LDS operations of one wave complete in order), so each load has a whole block to land.
constexpr int F_WAVES = 4;

DX_DEVICE floatx16 mfma32_f32(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int D>
__global__ void __launch_bounds__(64 * F_WAVES) __attribute__((amdgpu_waves_per_eu(1, 1)))
attn_f32_mfma_kernel(const float *__restrict__ Q, const float *__restrict__ K, const float *__restrict__ V,
                     float *__restrict__ O, const int32_t *__restrict__ seq_start, const int32_t *__restrict__ seq_len,
                     int max_seq_len, int hq, int hkv, long q_stride, long k_stride, long v_stride, long o_stride,
                     float scale, float softcap, int window, int causal, const uint8_t *__restrict__ key_mask) {
  static_assert(D == 64 || D == 128, "fp32 matrix-core attention covers head_dim 64 and 128");
  constexpr int KP = D + 4;    // K row pitch (floats): 16 lanes reading 16 bytes of 16 rows cover all 64 banks
  constexpr int VP = D + 8;    // V row pitch: the lane halves read rows 4 apart, on disjoint banks
  constexpr int REGION = 32 * KP + 32 * VP;  // floats per wave
  constexpr int DH = D / 2;
  constexpr int NDB = D / 32;
  constexpr int LPL = 32 * (D / 4) / 64;     // 16-byte chunks of a 32 x D block per lane
  constexpr int OP = 33;                     // merge: O^T [D][32] at pitch 33, then m [32] and l [32]
  static_assert(D * OP + 64 <= REGION, "merge state fits the wave's region");
  __shared__ __attribute__((aligned(16))) float smem[F_WAVES * REGION];

  const int b = blockIdx.y, h = blockIdx.z, g = h / (hq / hkv);
  const int len = min(max(seq_len[b], 0), max_seq_len);
  const int ntiles = (max_seq_len + 31) / 32;
  const int q0 = (ntiles - 1 - (int)blockIdx.x) * 32;  // heaviest (last) query tiles first
  if (q0 >= len) return;
  const long start = seq_start[b];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lrow = lane & 31, hh = lane >> 5;
  const int qi = q0 + lrow;
  float *const ks = smem + wave * REGION;
  float *const vs = ks + 32 * KP;

  float qf[DH];
  {
    const float *qp = Q + (start + min(qi, len - 1)) * q_stride + (long)h * D + hh * DH;
#pragma unroll
    for (int j = 0; j < DH; j += 4) {
      const float4 v = *reinterpret_cast<const float4 *>(qp + j);
      qf[j] = v.x;
      qf[j + 1] = v.y;
      qf[j + 2] = v.z;
      qf[j + 3] = v.w;
    }
  }
  const int qlast = min(q0 + 31, len - 1);
  int klo, khi;
  if (causal) {
    khi = qlast + 1;
    klo = window > 0 ? max(0, q0 - window + 1) : 0;
  } else {
    khi = window > 0 ? min(len, qlast + window + 1) : len;
    klo = window > 0 ? max(0, q0 - window) : 0;
  }
  const int kb0 = klo / 32, kb1 = (khi + 31) / 32;

  // chunk c = lane + 64 t of a block: key row c / (D / 4) = t RPT + lane / (D / 4), columns
  // 4 (lane % (D / 4)) .. + 3. Each block's K and V rows come through buffer resources based at the
  // block's first key, so the per-lane offsets are loop-invariant and rows past the sequence read zeros
  // (their scores are masked).
  constexpr int RPT = 64 / (D / 4);  // key rows per chunk step t
  const int crow = lane / (D / 4), ccol = (lane % (D / 4)) * 4;
  const int koff = (int)((crow * k_stride + ccol) * 4), voff = (int)((crow * v_stride + ccol) * 4);
  const float *const kseq = K + start * k_stride + (long)g * D;
  const float *const vseq = V + start * v_stride + (long)g * D;
  float4 kr[LPL], vr[LPL];
  auto rsrc = [&](const float *base, long stride, int kb) {
    // the block's rows only (32-bit byte counts); wave-uniform, which the compiler is told so that the
    // descriptor stays in scalar registers (a vector one costs a waterfall loop around every load)
    const long rows = __builtin_amdgcn_readfirstlane(min(max(len - kb * 32, 0), 32));
    return __builtin_amdgcn_make_buffer_rsrc((void *)(base + (long)kb * 32 * stride), (short)0,
                                             (int)(rows * stride * 4), 0x00020000);
  };
  auto fetch_k = [&](int kb) {
    const __amdgpu_buffer_rsrc_t r = rsrc(kseq, k_stride, kb);
#pragma unroll
    for (int t = 0; t < LPL; ++t)
      kr[t] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, koff, (int)(t * RPT * k_stride * 4), 0));
  };
  auto fetch_v = [&](int kb) {
    const __amdgpu_buffer_rsrc_t r = rsrc(vseq, v_stride, kb);
#pragma unroll
    for (int t = 0; t < LPL; ++t)
      vr[t] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, (int)(t * RPT * v_stride * 4), 0));
  };
  auto put_k = [&]() {
#pragma unroll
    for (int t = 0; t < LPL; ++t) *reinterpret_cast<float4 *>(ks + (t * RPT + crow) * KP + ccol) = kr[t];
  };
  auto put_v = [&]() {
#pragma unroll
    for (int t = 0; t < LPL; ++t) *reinterpret_cast<float4 *>(vs + (t * RPT + crow) * VP + ccol) = vr[t];
  };

  floatx16 o[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m = NEG_BIG, l = 0.f;  // running max (log2 units) and this lane's share of the row sum
  const float cap2 = softcap > 0.f ? 2.f * LOG2E / softcap : 0.f;

  int kb = kb0 + wave;
  if (kb < kb1) {
    fetch_k(kb);
    put_k();
    fetch_v(kb);
  }
  for (; kb < kb1; kb += F_WAVES) {
    put_v();
    const int nb = kb + F_WAVES;
    const bool more = nb < kb1;
    if (more) {  // the next block's K and V load during this whole block
      fetch_k(nb);
      fetch_v(nb);
    }
    floatx16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
    {
      // every K fragment of the block is requested before the first MFMA: one LDS round trip per block
      // instead of one per four MFMAs of the dependent chain
      const float *kp = ks + lrow * KP + hh * DH;
      float4 kv[DH / 4];
#pragma unroll
      for (int j = 0; j < DH / 4; ++j) kv[j] = *reinterpret_cast<const float4 *>(kp + 4 * j);
      __builtin_amdgcn_sched_barrier(0);  // the scheduler would otherwise sink each read to its MFMAs
#pragma unroll
      for (int j = 0; j < DH / 4; ++j) {
        s = mfma32_f32(kv[j].x, qf[4 * j], s);
        s = mfma32_f32(kv[j].y, qf[4 * j + 1], s);
        s = mfma32_f32(kv[j].z, qf[4 * j + 2], s);
        s = mfma32_f32(kv[j].w, qf[4 * j + 3], s);
      }
    }
    // score r is key kb 32 + (r / 4) 8 + 4 hh + r % 4 of query qi. The softcap and key-mask tests are
    // taken once per block, outside the per-score loops.
    const int kbase = kb * 32 + 4 * hh;
    if (softcap > 0.f) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[r] * scale;
        x = softcap - 2.f * softcap * fast_rcp(1.f + fast_exp2(x * cap2));  // cap tanh(x / cap)
        s[r] = x * LOG2E;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = s[r] * scale;
        s[r] = x * LOG2E;
      }
    }
    uint32_t vis = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) vis |= (uint32_t)visible(qi, kbase + (r >> 2) * 8 + (r & 3), len, window, causal) << r;
    if (key_mask) {
#pragma unroll
      for (int r = 0; r < 16; ++r)  // read only for visible keys, which lie inside the sequence
        if (((vis >> r) & 1u) && !key_mask[start + kbase + (r >> 2) * 8 + (r & 3)]) vis &= ~(1u << r);
    }
    float tmax = NEG_BIG;
#pragma unroll
    for (int r = 0; r < 16; ++r) tmax = ((vis >> r) & 1u) ? fmaxf(tmax, s[r]) : tmax;
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mnew = fmaxf(m, tmax);
    const float alpha = fast_exp2(m - mnew);
    m = mnew;
    l *= alpha;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {  // some row's running max moved
#pragma unroll
      for (int i = 0; i < NDB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = ((vis >> r) & 1u) ? fast_exp2(s[r] - mnew) : 0.f;
      s[r] = p;
      l += p;
    }
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        o[db] = mfma32_f32(vs[((i >> 2) * 8 + 4 * hh + (i & 3)) * VP + db * 32 + lrow], s[i], o[db]);
    if (more) put_k();
  }

  // merge the waves' states: wave w writes O^T, m and the row sum into its region, then every thread
  // combines (query, head-dim) elements, consecutive threads taking consecutive head dims
  l += __shfl_xor(l, 32, 64);
  __syncthreads();  // every wave is done with its K / V region
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) ks[(db * 32 + (r >> 2) * 8 + 4 * hh + (r & 3)) * OP + lrow] = o[db][r];
  if (hh == 0) {
    ks[D * OP + lrow] = m;
    ks[D * OP + 32 + lrow] = l;
  }
  __syncthreads();
  for (int idx = tid; idx < 32 * D; idx += 64 * F_WAVES) {
    const int q = idx / D, d = idx % D;
    if (q0 + q >= len) continue;
    float mx = NEG_BIG;
#pragma unroll
    for (int w = 0; w < F_WAVES; ++w) mx = fmaxf(mx, smem[w * REGION + D * OP + q]);
    float acc = 0.f, sum = 0.f;
#pragma unroll
    for (int w = 0; w < F_WAVES; ++w) {
      const float *st = smem + w * REGION;
      const float f = fast_exp2(st[D * OP + q] - mx);
      acc += st[d * OP + q] * f;
      sum += st[D * OP + 32 + q] * f;
    }
    O[(start + q0 + q) * o_stride + (long)h * D + d] = sum > 0.f ? acc / sum : 0.f;  // no visible key: zeros
  }
}

// V rows -> V^T tiles. Grid: (64-row tiles of the longest sequence, sequences,
// kv heads x D/64). Rows past seq_len up to the next multiple of 64 are
// written as zeros, so P.V never multiplies a zero probability by stale data.
__global__ void __launch_bounds__(THREADS)
transpose_v_kernel(const uint16_t *__restrict__ V, uint16_t *__restrict__ Vt, const int32_t *__restrict__ seq_start,
                   const int32_t *__restrict__ seq_len, const int32_t *__restrict__ vt_start, long vt_seq_stride,
                   int max_seq_len, int d, long v_stride, long vt_ld) {
  __shared__ uint16_t tile[64][66];
  const int b = blockIdx.y;
  const int len = min(max(seq_len[b], 0), max_seq_len);
  const int p0 = blockIdx.x * 64;
  if (p0 >= len) return;
  const int dblocks = d / 64;
  const int g = blockIdx.z / dblocks, d0 = (blockIdx.z % dblocks) * 64;
  const long start = seq_start[b];
  const long vts = vt_start ? (long)vt_start[b] : (long)b * vt_seq_stride;
  const int tid = threadIdx.x;
  {
    const int row = tid >> 2, c = (tid & 3) * 16;
    u32x4 a = {0, 0, 0, 0}, bb = {0, 0, 0, 0};
    if (p0 + row < len) {
      const uint16_t *src = V + (start + p0 + row) * v_stride + (long)g * d + d0 + c;
      a = *reinterpret_cast<const u32x4 *>(src);
      bb = *reinterpret_cast<const u32x4 *>(src + 8);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      tile[row][c + 2 * i] = (uint16_t)(a[i] & 0xffff);
      tile[row][c + 2 * i + 1] = (uint16_t)(a[i] >> 16);
      tile[row][c + 8 + 2 * i] = (uint16_t)(bb[i] & 0xffff);
      tile[row][c + 8 + 2 * i + 1] = (uint16_t)(bb[i] >> 16);
    }
  }
  __syncthreads();
  {
    const int dr = tid >> 2, c = (tid & 3) * 16;
    u32x4 a, bb;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = (uint32_t)tile[c + 2 * i][dr] | ((uint32_t)tile[c + 2 * i + 1][dr] << 16);
      bb[i] = (uint32_t)tile[c + 8 + 2 * i][dr] | ((uint32_t)tile[c + 8 + 2 * i + 1][dr] << 16);
    }
    uint16_t *dst = Vt + ((long)g * d + d0 + dr) * vt_ld + vts + p0 + c;
    *reinterpret_cast<u32x4 *>(dst) = a;
    *reinterpret_cast<u32x4 *>(dst + 8) = bb;
  }
}

// Block (s, y): V^T rows [4 y, 4 y + 4) of sequence s, columns [seq_len, seq_len rounded up to 64) <- 0.
__global__ void __launch_bounds__(THREADS)
vt_zero_tails_kernel(uint16_t *__restrict__ Vt, const int32_t *__restrict__ seq_len,
                     const int32_t *__restrict__ vt_start, int vt_rows, long vt_ld) {
  const int len = max(seq_len[blockIdx.x], 0);
  const int row = blockIdx.y * (THREADS / 64) + (int)threadIdx.x / 64, j = len + (int)threadIdx.x % 64;
  if (row < vt_rows && j < ((len + 63) & ~63)) Vt[(long)row * vt_ld + vt_start[blockIdx.x] + j] = 0;
}

template <int D, int G, int W, int NS>
hipError_t launch_bf16_dgw(const AttnArgs &a, hipStream_t s) {
  constexpr int BQ = 32 * (W / G);
  const unsigned ntiles = (a.max_seq_len + BQ - 1) / BQ;
  const dim3 grid = a.max_seq_len <= SHORT_SEQ ? dim3(a.hkv, a.num_seqs, ntiles) : dim3(ntiles, a.hkv, a.num_seqs);
  const bool fixed = a.softcap > 0.f && a.softcap <= 56.f;
  auto kern = a.key_bits ? (fixed ? attn_bf16_kernel<D, G, MODE_FIXED, true, W, NS>
                                  : attn_bf16_kernel<D, G, MODE_ONLINE, true, W, NS>)
                         : (fixed ? attn_bf16_kernel<D, G, MODE_FIXED, false, W, NS>
                                  : attn_bf16_kernel<D, G, MODE_ONLINE, false, W, NS>);
  kern<<<grid, dim3(64 * W), 0, s>>>(
      static_cast<const uint16_t *>(a.q), static_cast<const uint16_t *>(a.k), static_cast<const uint16_t *>(a.v),
      static_cast<uint16_t *>(a.out), a.seq_start, a.seq_len, a.vt_start, a.vt_seq_stride, a.max_seq_len,
      a.q_stride, a.k_stride, a.v_stride, a.out_stride, a.scale, a.softcap, a.window, a.causal, a.key_bits,
      a.key_words);
  return hipGetLastError();
}

// Keys a query row sees on average: the window, or half the longest sequence when causal and unwindowed.
inline long mean_key_span(const AttnArgs &a) {
  const long n = a.max_seq_len;
  const long w = a.window;
  if (a.causal) return w > 0 ? (w < n ? w : n) : n / 2;
  return w > 0 ? (2 * w < n ? 2 * w : n) : n;
}

template <int D, int G>
hipError_t launch_bf16_dg(const AttnArgs &a, hipStream_t s) {
  if constexpr (D == 128)
    if (mean_key_span(a) <= 2048) return launch_bf16_dgw<D, G, 4, 2>(a, s);
  return launch_bf16_dgw<D, G, 8, 4>(a, s);
}

template <int D>
hipError_t launch_bf16_d(const AttnArgs &a, hipStream_t s) {
  switch (a.hq / a.hkv) {
    case 1: return launch_bf16_dg<D, 1>(a, s);
    case 2: return launch_bf16_dg<D, 2>(a, s);
    case 4: return launch_bf16_dg<D, 4>(a, s);
  }
  return hipErrorInvalidValue;
}

template <int D, int TPQ>
hipError_t launch_f32_d(const AttnArgs &a, hipStream_t s) {
  constexpr int QPB = THREADS / TPQ;
  const dim3 grid((a.max_seq_len + QPB - 1) / QPB, a.num_seqs, a.hq);
  attn_f32_kernel<D, TPQ><<<grid, dim3(THREADS), 0, s>>>(
      static_cast<const float *>(a.q), static_cast<const float *>(a.k), static_cast<const float *>(a.v),
      static_cast<float *>(a.out), a.seq_start, a.seq_len, a.max_seq_len, a.hq, a.hkv, a.q_stride, a.k_stride,
      a.v_stride, a.out_stride, a.scale, a.softcap, a.window, a.causal, a.key_mask);
  return hipGetLastError();
}

template <int D>
hipError_t launch_f32_mfma_d(const AttnArgs &a, hipStream_t s) {
  const dim3 grid((a.max_seq_len + 31) / 32, a.num_seqs, a.hq);
  attn_f32_mfma_kernel<D><<<grid, dim3(64 * F_WAVES), 0, s>>>(
      static_cast<const float *>(a.q), static_cast<const float *>(a.k), static_cast<const float *>(a.v),
      static_cast<float *>(a.out), a.seq_start, a.seq_len, a.max_seq_len, a.hq, a.hkv, a.q_stride, a.k_stride,
      a.v_stride, a.out_stride, a.scale, a.softcap, a.window, a.causal, a.key_mask);
  return hipGetLastError();
}

// Thread t packs word t % words of sequence t / words: bit j <- key_mask[seq_start + 32 w + j] != 0 for keys
// inside the sequence, 0 past its length.
__global__ void __launch_bounds__(THREADS)
pack_key_bits_kernel(const uint8_t *__restrict__ key_mask, const int32_t *__restrict__ seq_start,
                     const int32_t *__restrict__ seq_len, int num_seqs, int max_seq_len, int words,
                     uint32_t *__restrict__ bits) {
  const long t = (long)blockIdx.x * THREADS + threadIdx.x;
  if (t >= (long)num_seqs * words) return;
  const int b = (int)(t / words), w = (int)(t % words);
  const int len = min(max(seq_len[b], 0), max_seq_len);
  const long start = seq_start[b];
  uint32_t word = 0;
  for (int j = 0; j < 32; ++j) {
    const int key = 32 * w + j;
    if (key < len && key_mask[start + key]) word |= 1u << j;
  }
  bits[t] = word;
}

}  // namespace

hipError_t dx_pack_key_bits_launch(const uint8_t *key_mask, const int32_t *seq_start, const int32_t *seq_len,
                                   int num_seqs, int max_seq_len, int words, uint32_t *bits, hipStream_t s) {
  const long total = (long)num_seqs * words;
  pack_key_bits_kernel<<<dim3((unsigned)((total + THREADS - 1) / THREADS)), dim3(THREADS), 0, s>>>(
      key_mask, seq_start, seq_len, num_seqs, max_seq_len, words, bits);
  return hipGetLastError();
}

hipError_t dx_attn_bf16(const AttnArgs &a, hipStream_t s) {
  switch (a.d) {
    case 64: return launch_bf16_d<64>(a, s);
    case 128: return launch_bf16_d<128>(a, s);
    case 256: return launch_bf16_d<256>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t dx_attn_f32(const AttnArgs &a, hipStream_t s) {
  switch (a.d) {
    case 64: return launch_f32_mfma_d<64>(a, s);
    case 128: return launch_f32_mfma_d<128>(a, s);
    // head_dim 256 keeps the VALU kernel (the matrix-core one would hold 128 query registers per lane),
    // 16 threads per query
    case 256: return launch_f32_d<256, 16>(a, s);
  }
  return hipErrorInvalidValue;
}

hipError_t dx_vt_zero_tails_launch(uint16_t *vt, const int32_t *seq_len, const int32_t *vt_start, int num_seqs,
                                   int vt_rows, long vt_ld, hipStream_t s) {
  const dim3 grid((unsigned)num_seqs, (unsigned)((vt_rows + THREADS / 64 - 1) / (THREADS / 64)));
  vt_zero_tails_kernel<<<grid, dim3(THREADS), 0, s>>>(vt, seq_len, vt_start, vt_rows, vt_ld);
  return hipGetLastError();
}

hipError_t dx_transpose_v_launch(const uint16_t *v, uint16_t *vt, const int32_t *seq_start, const int32_t *seq_len,
                                 const int32_t *vt_start, long vt_seq_stride, int num_seqs, int max_seq_len, int hkv,
                                 int d, long v_stride, long vt_ld, hipStream_t s) {
  const dim3 grid((max_seq_len + 63) / 64, num_seqs, hkv * (d / 64));
  transpose_v_kernel<<<grid, dim3(THREADS), 0, s>>>(v, vt, seq_start, seq_len, vt_start, vt_seq_stride, max_seq_len,
                                                   d, v_stride, vt_ld);
  return hipGetLastError();
}
