// FP8 block-scaled GEMM for gfx950 (the DeepGEMM `fp8_gemm_nt` call of
// quail/backends/quail/executor/attention.py:479-490).
//
//   C[m, n] = bf16( sum_kb  sA[kb, m] * sW[n / 128, kb] * sum_{k in kb} A[m, k] * W[n, k] )
//
//   A  : M x K e4m3fn, row-major, leading dimension lda (bytes)
//   sA : per-token 128-column scales, stored (K/128) x M ("column-major
//        scales", attention.py:534-537): sA[kb * sa_ld + m]
//   W  : N x K e4m3fn, row-major (the checkpoint's (out, in) layout)
//   sW : (N/128) x (K/128) fp32 `weight_scale_inv` (attention.py:471-477)
//   C  : M x N bf16, row-major, leading dimension ldc (elements)
//
// Design (MI355X / CDNA4):
//   * one 128-wide K step is one scale group; per step each wave runs two
//     v_mfma_f32_32x32x64_f8f6f4 per 32x32 output tile into a temporary and
//     promotes it into the fp32 accumulator with the product of the two
//     scales ("promotion": the scales change every 128 of K, so they cannot
//     be applied once after the loop);
//   * the MFMA "A" operand is the weight tile and "B" the token tile, so the
//     32x32 output tile holds one token per lane column: the token scale
//     sA[kb, m] is one value per lane per tile and the weight scale one
//     value per wave;
//   * operand tiles travel HBM -> LDS with global_load_lds_dwordx4 (no VGPR
//     staging), double buffered; rows are 128 B with the 16-B chunk index
//     XOR-swizzled by (row & 7), so fragment reads are bank-conflict free;
//   * workgroups are remapped so each XCD (8 per MI355X, each with its own
//     L2) runs a contiguous band of tiles that share operands.
#include "qx_common.h"
#include "qx_status.h"

namespace qx {
namespace {

typedef __attribute__((address_space(3))) void lds_void;

template <int BM, int BN, int WAVES_N, int WAVES_M>
struct GemmCfg {
  static constexpr int kThreads = 64 * WAVES_N * WAVES_M;
  static constexpr int kTN = BN / WAVES_N / 32;  // 32-row weight tiles per wave
  static constexpr int kTM = BM / WAVES_M / 32;  // 32-row token tiles per wave
  static constexpr int kABytes = BM * 128;
  static constexpr int kWBytes = BN * 128;
  static constexpr int kStage = kABytes + kWBytes;
  static constexpr int kLds = 2 * kStage;
  static_assert(kTN >= 1 && kTM >= 1, "wave tile must hold a 32x32 MFMA tile");
  static_assert(BM % (8 * WAVES_N * WAVES_M) == 0 && BN % (8 * WAVES_N * WAVES_M) == 0,
                "each wave loads whole 8-row slabs");
};

// Issue this wave's share of one K step's tile loads (rows of 128 B) from
// global memory straight into LDS. Each instruction moves 8 rows: lane i
// writes LDS bytes [i*16, i*16+16) of the 1 KiB slab, i.e. row i/8, physical
// chunk i%8, and therefore reads logical chunk (i%8) ^ (row & 7).
template <int ROWS, int WAVES>
__device__ __forceinline__ void load_tile(const uint8_t* __restrict__ g, int64_t ld, int row0,
                                          int row_max, int64_t k_off, uint8_t* lds, int wave,
                                          int lane) {
  constexpr int kSlabs = ROWS / 8 / WAVES;
  const int r_in = lane >> 3;
  const int p = lane & 7;
#pragma unroll
  for (int j = 0; j < kSlabs; ++j) {
    const int slab = wave * kSlabs + j;
    const int row = slab * 8 + r_in;
    const int c = p ^ (row & 7);
    int grow = row0 + row;
    grow = grow < row_max ? grow : row_max;  // tail rows re-read the last row
    const uint8_t* src = g + (int64_t)grow * ld + k_off + c * 16;
    __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(lds + slab * 1024), 16, 0, 0);
  }
}

// One lane's 32-byte fragment of row `row` for K-half `half` (bytes
// [half*64 + (lane/32)*32, +32) of the 128-B row), read through the swizzle.
__device__ __forceinline__ v8i read_frag(const uint8_t* lds, int row, int half, int lane) {
  const int c0 = half * 4 + (lane >> 5) * 2;
  const int sw = row & 7;
  const v4i* base = reinterpret_cast<const v4i*>(lds + row * 128);
  v4i lo = base[c0 ^ sw];
  v4i hi = base[(c0 + 1) ^ sw];
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

template <int BM, int BN, int WAVES_N, int WAVES_M>
__global__ __launch_bounds__(64 * WAVES_N * WAVES_M, 1) void gemm_fp8_bs_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sA, const uint8_t* __restrict__ W,
    const float* __restrict__ sW, uint16_t* __restrict__ C, int M, int N, int K, int64_t lda,
    int64_t ldc, int64_t sa_ld, int tiles_m, int tiles_n, int group_m) {
  using Cfg = GemmCfg<BM, BN, WAVES_N, WAVES_M>;
  constexpr int TN = Cfg::kTN, TM = Cfg::kTM;
  constexpr int WAVES = WAVES_N * WAVES_M;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Cfg::kLds];

  // ---- tile scheduling: XCD-contiguous bands, grouped along M ----------
  const int total = tiles_m * tiles_n;
  int id = blockIdx.x;
  {
    // workgroup i runs on XCD i % 8; give XCD x the ids [x*per, (x+1)*per)
    const int per = (total + 7) / 8;
    const int xcd = id & 7, local = id >> 3;
    const int full = total - (per - 1) * 8;  // XCDs that hold `per` ids
    id = xcd < full ? xcd * per + local : full * per + (xcd - full) * (per - 1) + local;
  }
  const int width = group_m * tiles_n;
  const int group = id / width;
  const int first_m = group * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int tile_m = first_m + (id % width) % gsize;
  const int tile_n = (id % width) / gsize;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wn = wave % WAVES_N;
  const int wm = wave / WAVES_N;
  const int m0 = tile_m * BM;
  const int n0 = tile_n * BN;
  const int KT = K >> 7;

  v16f acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;

  // this lane's tokens (one per token tile) and the scale rows it reads
  int tok[TM];
#pragma unroll
  for (int b = 0; b < TM; ++b) {
    int m = m0 + wm * TM * 32 + b * 32 + (lane & 31);
    tok[b] = m < M ? m : M - 1;
  }
  int wblk[TN];
#pragma unroll
  for (int a = 0; a < TN; ++a) wblk[a] = ((n0 + wn * TN * 32 + a * 32) >> 7) * KT;

  // prologue: stage 0
  load_tile<BM, WAVES>(A, lda, m0, M - 1, 0, smem, wave, lane);
  load_tile<BN, WAVES>(W, K, n0, N - 1, 0, smem + Cfg::kABytes, wave, lane);

  float sa_next[TM];
#pragma unroll
  for (int b = 0; b < TM; ++b) sa_next[b] = sA[tok[b]];

  for (int kt = 0; kt < KT; ++kt) {
    const int stage = kt & 1;
    float sa[TM];
#pragma unroll
    for (int b = 0; b < TM; ++b) sa[b] = sa_next[b];
    float sw[TN];
#pragma unroll
    for (int a = 0; a < TN; ++a) sw[a] = sW[wblk[a] + kt];

    __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS-bound loads landed
    __syncthreads();                // ... and every other wave's
    if (kt + 1 < KT) {
      uint8_t* nxt = smem + (stage ^ 1) * Cfg::kStage;
      const int64_t k_off = (int64_t)(kt + 1) * 128;
      load_tile<BM, WAVES>(A, lda, m0, M - 1, k_off, nxt, wave, lane);
      load_tile<BN, WAVES>(W, K, n0, N - 1, k_off, nxt + Cfg::kABytes, wave, lane);
#pragma unroll
      for (int b = 0; b < TM; ++b) sa_next[b] = sA[(int64_t)(kt + 1) * sa_ld + tok[b]];
    }

    const uint8_t* sa_lds = smem + stage * Cfg::kStage;
    const uint8_t* sw_lds = sa_lds + Cfg::kABytes;
    v8i wf[2][TN], af[2][TM];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int a = 0; a < TN; ++a)
        wf[h][a] = read_frag(sw_lds, wn * TN * 32 + a * 32 + (lane & 31), h, lane);
#pragma unroll
      for (int b = 0; b < TM; ++b)
        af[h][b] = read_frag(sa_lds, wm * TM * 32 + b * 32 + (lane & 31), h, lane);
    }
#pragma unroll
    for (int a = 0; a < TN; ++a) {
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        v16f p = {};
        p = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[0][a], af[0][b], p, 0, 0, 0, 0, 0, 0);
        p = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[1][a], af[1][b], p, 0, 0, 0, 0, 0, 0);
        const float s = sa[b] * sw[a];
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][b][e] = fmaf(p[e], s, acc[a][b][e]);
      }
    }
  }

  // ---- epilogue: lane holds token column (lane & 31); rows are weights --
#pragma unroll
  for (int b = 0; b < TM; ++b) {
    const int m = m0 + wm * TM * 32 + b * 32 + (lane & 31);
    if (m >= M) continue;
    uint16_t* crow = C + (int64_t)m * ldc;
#pragma unroll
    for (int a = 0; a < TN; ++a) {
      const int nbase = n0 + wn * TN * 32 + a * 32 + (lane >> 5) * 4;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint2 v;
        v.x = pack2_bf16(acc[a][b][g * 4 + 0], acc[a][b][g * 4 + 1]);
        v.y = pack2_bf16(acc[a][b][g * 4 + 2], acc[a][b][g * 4 + 3]);
        *reinterpret_cast<uint2*>(crow + nbase + g * 8) = v;
      }
    }
  }
}

template <int BM, int BN, int WN, int WM>
int launch(const void* A, const float* sA, const void* W, const float* sW, void* C, int M, int N,
           int K, int64_t lda, int64_t ldc, int64_t sa_ld, int group_m, hipStream_t stream) {
  using Cfg = GemmCfg<BM, BN, WN, WM>;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  const int total = tiles_m * tiles_n;
  hipLaunchKernelGGL((gemm_fp8_bs_kernel<BM, BN, WN, WM>), dim3(total), dim3(Cfg::kThreads), 0,
                     stream, (const uint8_t*)A, sA, (const uint8_t*)W, sW, (uint16_t*)C, M, N, K,
                     lda, ldc, sa_ld, tiles_m, tiles_n, group_m < 1 ? 1 : group_m);
  QX_LAUNCH_STATUS();
}

}  // namespace
}  // namespace qx

extern "C" {

// Tile configurations: 0 = 128 tokens x 256 weights (default), 1 = 256 x 256,
// 2 = 128 x 128. Chosen by the caller per shape; all give the same result.
int qx_gemm_fp8_blockscaled(const void* A, const float* sA, const void* W, const float* sW,
                            void* C, int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldc,
                            int64_t sa_ld, int config, hipStream_t stream) {
  QX_CHECK(A && sA && W && sW && C, "gemm: null pointer");
  QX_CHECK(M >= 0 && N > 0 && K > 0, "gemm: bad shape M=%lld N=%lld K=%lld", (long long)M,
           (long long)N, (long long)K);
  QX_CHECK(K % 128 == 0, "gemm: K=%lld is not a multiple of 128", (long long)K);
  QX_CHECK(N % 128 == 0, "gemm: N=%lld is not a multiple of 128", (long long)N);
  QX_CHECK(lda >= K && lda % 16 == 0, "gemm: lda=%lld must be >= K and 16-byte aligned",
           (long long)lda);
  QX_CHECK(ldc >= N && ldc % 4 == 0, "gemm: ldc=%lld", (long long)ldc);
  QX_CHECK(sa_ld >= M, "gemm: sa_ld=%lld < M", (long long)sa_ld);
  QX_CHECK(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31), "gemm: dims exceed int32");
  QX_CHECK(((uintptr_t)A & 15) == 0 && ((uintptr_t)W & 15) == 0, "gemm: A/W not 16-byte aligned");
  QX_CHECK(((uintptr_t)C & 7) == 0, "gemm: C not 8-byte aligned");
  if (M == 0) return QX_OK;
  const int m = (int)M, n = (int)N, k = (int)K;
  switch (config) {
    case 0:
      QX_CHECK(n % 256 == 0, "gemm config 0 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch<128, 256, 2, 2>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8, stream);
    case 1:
      QX_CHECK(n % 256 == 0, "gemm config 1 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch<256, 256, 2, 2>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 4, stream);
    case 2:
      return qx::launch<128, 128, 2, 2>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8, stream);
    default:
      QX_CHECK(false, "gemm: unknown config %d", config);
  }
}

}  // extern "C"
