// bf16 "NT" GEMM on gfx950 MFMA: C[m, n] = sum_k A[m, k] * B[n, k].
//
// A is activations [M, K] and B is a weight in PyTorch [out, in] layout, so
// both operands are K-contiguous and every MFMA operand is one 16-byte LDS
// read. Block tile BM x BN x 64 over 4 waves (2 x 2), each wave BM/2 x BN/2 in
// 32x32x16 MFMA blocks with fp32 accumulators. Two LDS stages; the next K tile
// is fetched into registers while the current one feeds the MFMAs.
//
// LDS layout: row-major [rows][64] bf16, 16-byte chunk c of row r stored at
// chunk position c ^ ((r >> 1) & 7). A 32-lane operand read touches 32 rows at
// one logical chunk; with a 128-byte row pitch the XOR spreads 16 consecutive
// rows over all 16 chunk slots of a 256-byte bank line.
//
// Epilogues: bf16 store (staged through LDS for 16-byte row stores), fp32
// store, and the gated activation for a gate|up weight packed in 64-row
// blocks (dx_pack_gate_up), which writes act = bf16(bf16(act(g)) * u) with
// g, u rounded to bf16 first — the rounding points of the reference's fused
// MLP epilogue (src/deciax/kernels/swiglu.py:100-101).
#include "common.h"
#include "kernels.h"

namespace {

constexpr int BK = 64;
constexpr int THREADS = 256;

enum { EPI_BF16 = 0, EPI_F32 = 1, EPI_GATED = 2 };

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2). Renumber so each XCD gets a contiguous run of logical tiles, then walk
// tiles in groups of GROUP_M tile-rows so concurrently running tiles share A
// rows and B columns inside one L2.
DX_DEVICE void tile_coords(int pid, int nblocks, int num_m, int num_n, int &tm, int &tn) {
  const int per = nblocks / 8, rem = nblocks % 8;
  const int xcd = pid % 8, idx = pid / 8;
  const int lpid = xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
  constexpr int GROUP_M = 8;
  const int group_size = GROUP_M * num_n;
  const int group = lpid / group_size;
  const int first_m = group * GROUP_M;
  const int gm = min(num_m - first_m, GROUP_M);
  const int in = lpid % group_size;
  tm = first_m + in % gm;
  tn = in / gm;
}

DX_DEVICE int swz(int row, int chunk) { return row * 64 + ((chunk ^ ((row >> 1) & 7)) << 3); }

template <int BM, int BN, int EPI>
__global__ void __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_nt_kernel(const uint16_t *__restrict__ A, const uint16_t *__restrict__ B, void *__restrict__ C,
               int M, int N, int K, long lda, long ldb, long ldc, int act) {
  constexpr int TM = BM / 64;  // 32x32 blocks per wave along m
  constexpr int TN = BN / 64;  // along n
  constexpr int ACH = BM * BK / 8 / THREADS;
  constexpr int BCH = BN * BK / 8 / THREADS;
  constexpr int STAGE = (BM + BN) * BK;
  constexpr int OUT_W = EPI == EPI_GATED ? BN / 2 : BN;
  constexpr int OUT_PITCH = OUT_W + 8;
  constexpr int SMEM = (2 * STAGE > BM * OUT_PITCH) ? 2 * STAGE : BM * OUT_PITCH;
  __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM];

  const int num_m = (M + BM - 1) / BM, num_n = N / BN;
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, num_m, num_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const uint16_t *a_src[ACH];
  const uint16_t *b_src[BCH];
  int a_dst[ACH], b_dst[BCH];
#pragma unroll
  for (int j = 0; j < ACH; ++j) {
    const int id = tid + THREADS * j, row = id >> 3, c = id & 7;
    const int grow = min(m0 + row, M - 1);  // tail rows re-read the last row; never stored
    a_src[j] = A + (long)grow * lda + c * 8;
    a_dst[j] = swz(row, c);
  }
#pragma unroll
  for (int j = 0; j < BCH; ++j) {
    const int id = tid + THREADS * j, row = id >> 3, c = id & 7;
    b_src[j] = B + (long)(n0 + row) * ldb + c * 8;
    b_dst[j] = BM * BK + swz(row, c);
  }

  u32x4 ra[ACH], rb[BCH];
  auto gload = [&](int kt) {
#pragma unroll
    for (int j = 0; j < ACH; ++j) ra[j] = *reinterpret_cast<const u32x4 *>(a_src[j] + kt * BK);
#pragma unroll
    for (int j = 0; j < BCH; ++j) rb[j] = *reinterpret_cast<const u32x4 *>(b_src[j] + kt * BK);
  };
  auto sstore = [&](int stage) {
    uint16_t *base = smem + stage * STAGE;
#pragma unroll
    for (int j = 0; j < ACH; ++j) *reinterpret_cast<u32x4 *>(base + a_dst[j]) = ra[j];
#pragma unroll
    for (int j = 0; j < BCH; ++j) *reinterpret_cast<u32x4 *>(base + b_dst[j]) = rb[j];
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int lrow = lane & 31, lhalf = lane >> 5;
  auto compute = [&](int stage) {
    const uint16_t *sa = smem + stage * STAGE;
    const uint16_t *sb = sa + BM * BK;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int c = ks * 2 + lhalf;
      bf16x8 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * (BM / 2) + i * 32 + lrow;
        af[i] = as_bf16x8(*reinterpret_cast<const u32x4 *>(sa + swz(row, c)));
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int row = wn * (BN / 2) + j * 32 + lrow;
        bfr[j] = as_bf16x8(*reinterpret_cast<const u32x4 *>(sb + swz(row, c)));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma32(af[i], bfr[j], acc[i][j]);
    }
  };

  const int KT = K / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    if (kt + 1 < KT) gload(kt + 1);
    compute(kt & 1);
    if (kt + 1 < KT) sstore((kt + 1) & 1);
    __syncthreads();
  }

  if constexpr (EPI == EPI_F32) {
    float *Cf = reinterpret_cast<float *>(C);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + wm * (BM / 2) + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
          const int col = n0 + wn * (BN / 2) + j * 32 + lrow;
          if (row < M) Cf[(long)row * ldc + col] = acc[i][j][r];
        }
    return;
  } else {
    // Stage the bf16 tile through LDS, then store 16-byte row chunks.
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = wm * (BM / 2) + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
        if constexpr (EPI == EPI_BF16) {
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int col = wn * (BN / 2) + j * 32 + lrow;
            smem[row * OUT_PITCH + col] = f2bf(acc[i][j][r]);
          }
        } else {
          // Wave columns [0, BN/4) are gate, [BN/4, BN/2) the matching up.
#pragma unroll
          for (int j = 0; j < TN / 2; ++j) {
            const float g = round_bf(acc[i][j][r]);
            const float u = round_bf(acc[i][j + TN / 2][r]);
            const float a = round_bf(act == DX_ACT_SILU ? silu(g) : gelu_tanh(g));
            const int col = wn * (BN / 4) + j * 32 + lrow;
            smem[row * OUT_PITCH + col] = f2bf(a * u);
          }
        }
      }
    __syncthreads();
    uint16_t *Cb = reinterpret_cast<uint16_t *>(C);
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

template <int BM, int BN, int EPI>
hipError_t launch(const uint16_t *A, const uint16_t *B, void *C, long M, long N, long K, long lda, long ldb,
                  long ldc, int act, hipStream_t s) {
  const long num_m = (M + BM - 1) / BM, num_n = N / BN;
  gemm_nt_kernel<BM, BN, EPI><<<dim3((unsigned)(num_m * num_n)), dim3(THREADS), 0, s>>>(
      A, B, C, (int)M, (int)N, (int)K, lda, ldb, ldc, act);
  return hipGetLastError();
}

template <int EPI>
hipError_t dispatch(const uint16_t *A, const uint16_t *B, void *C, long M, long N, long K, long lda, long ldb,
                    long ldc, int act, hipStream_t s) {
  // Small M: halve the row tile so more workgroups exist.
  if (M <= 1024) return launch<128, 256, EPI>(A, B, C, M, N, K, lda, ldb, ldc, act, s);
  return launch<256, 256, EPI>(A, B, C, M, N, K, lda, ldb, ldc, act, s);
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
