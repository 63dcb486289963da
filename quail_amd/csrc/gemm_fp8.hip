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
//   * v_mfma_f32_32x32x64_f8f6f4 does the products; the MFMA "A" operand is
//     the weight tile and "B" the token tile, so a 32x32 output tile holds
//     one token per lane column: the token scale is one value per lane per
//     tile and the weight scale one value per wave;
//   * the scales change every 128 of K. Instead of promoting each 128-K
//     partial from a temporary, the accumulator is kept in units of the
//     current block's scale s = sA * sW: entering block kb it is multiplied
//     by s_(kb-1) / s_kb and the MFMAs accumulate the raw FP8 products into
//     it; the epilogue multiplies by the last block's scale. That is
//     sum_kb s_kb P_kb as the reference defines it, with no temporaries and
//     16 VALU multiplies per 32x32 tile per 128 of K. A block whose weight
//     scale is 0 contributes nothing and is skipped;
//   * operand tiles go HBM -> LDS with global_load_lds_dwordx4 (no VGPR
//     staging) in 64-byte K slices through a STAGES-deep ring, so up to
//     STAGES-1 slices are in flight while one is consumed. A slice row is
//     64 B (4 chunks of 16 B), chunk-swizzled by ((row >> 2) & 3) so the 16
//     rows of one ds_read_b128 phase cover all 64 LDS banks;
//   * workgroups are remapped so each XCD (8 per MI355X, each with its own
//     L2) runs a contiguous band of tiles that share operands.
#include <type_traits>

#include "qx_common.h"
#include "qx_status.h"

namespace qx {
namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kSlice = 64;  // bytes of K per pipeline stage (one MFMA k-step)

// Cache policy of the operand loads into LDS: device scope (sc1). The
// vector L1 keeps no copy of these streamed rows (every workgroup reads its
// operands once), which measured 10% faster on the widest Qwen3 projection
// than the default policy and no slower elsewhere.
constexpr int kOperandLoadPolicy = 16;

__device__ __forceinline__ int swz(int row) { return (row >> 2) & 3; }


template <int BM, int BN, int WAVES_N, int WAVES_M, int STAGES>
struct GemmCfg {
  static constexpr int kWaves = WAVES_N * WAVES_M;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kTN = BN / WAVES_N / 32;  // 32-row weight tiles per wave
  static constexpr int kTM = BM / WAVES_M / 32;  // 32-row token tiles per wave
  static constexpr int kABytes = BM * kSlice;
  static constexpr int kWBytes = BN * kSlice;
  static constexpr int kStage = kABytes + kWBytes;
  static constexpr int kLds = STAGES * kStage;
  static constexpr int kASlabs = BM / 16 / kWaves;  // 1 KiB (16-row) slabs per wave
  static constexpr int kWSlabs = BN / 16 / kWaves;
  // vector-memory ops one wave issues per stage: slabs + its token scales
  static constexpr int kOpsPerStage = kASlabs + kWSlabs + kTM;
  static_assert(kTN >= 1 && kTM >= 1, "wave tile must hold a 32x32 MFMA tile");
  static_assert(BM % (16 * kWaves) == 0 && BN % (16 * kWaves) == 0,
                "each wave loads whole 16-row slabs");
  static_assert(128 % (BN / WAVES_N) == 0 || (BN / WAVES_N) == 128,
                "a wave's weight rows stay inside one 128-row scale block");
  static_assert(kLds <= 160 * 1024, "LDS");
  static_assert(STAGES >= 2, "stages");
  static_assert((STAGES - 2) * kOpsPerStage < 64, "vmcnt");
};

// This wave's share of one stage: 16-row slabs of 64 B. Lane i writes LDS
// bytes [i*16, i*16+16) of its slab: row i/4, physical chunk i%4, so it
// reads logical chunk (i%4) ^ swz(row).
template <int SLABS>
__device__ __forceinline__ void load_slabs(const uint8_t* __restrict__ g, int64_t ld, int row0,
                                           int row_max, int64_t k_off, uint8_t* lds, int first,
                                           int lane) {
  const int r_in = lane >> 2;
  const int p = lane & 3;
#pragma unroll
  for (int j = 0; j < SLABS; ++j) {
    const int slab = first + j;
    const int row = slab * 16 + r_in;
    const int c = p ^ swz(row);
    int grow = row0 + row;
    grow = grow < row_max ? grow : row_max;  // tail rows re-read the last row
    const uint8_t* src = g + (int64_t)grow * ld + k_off + c * 16;
    __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(lds + slab * 1024), 16, 0,
                                     kOperandLoadPolicy);
  }
}

// A lane's 32-byte MFMA fragment: bytes [(lane/32)*32, +32) of a 64-B row.
__device__ __forceinline__ v8i read_frag(const uint8_t* lds, int row, int lane) {
  const int c0 = (lane >> 5) * 2;
  const int sw = swz(row);
  const v4i* base = reinterpret_cast<const v4i*>(lds + row * kSlice);
  const v4i lo = base[c0 ^ sw];
  const v4i hi = base[(c0 + 1) ^ sw];
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

template <int BM, int BN, int WAVES_N, int WAVES_M, int STAGES>
__global__ __launch_bounds__(64 * WAVES_N * WAVES_M)
__attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_fp8_bs_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sA, const uint8_t* __restrict__ W,
    const float* __restrict__ sW, uint16_t* __restrict__ C, int M, int N, int K, int64_t lda,
    int64_t ldc, int64_t sa_ld, int tiles_m, int tiles_n, int group_m) {
  using Cfg = GemmCfg<BM, BN, WAVES_N, WAVES_M, STAGES>;
  constexpr int TN = Cfg::kTN, TM = Cfg::kTM;
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

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int wn = wave % WAVES_N;
  const int wm = wave / WAVES_N;
  const int m0 = tile_m * BM;
  const int n0 = tile_n * BN;
  const int KT = K >> 7;        // scale blocks
  const int KS = K / kSlice;    // pipeline slices (two per scale block)

  v16f acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;

  int tok[TM];
#pragma unroll
  for (int b = 0; b < TM; ++b) {
    const int m = m0 + wm * TM * 32 + b * 32 + (lane & 31);
    tok[b] = m < M ? m : M - 1;
  }
  const float* sw_row = sW + (int64_t)((n0 + wn * TN * 32) >> 7) * KT;

  // sa_ring[s][b]: token scales of the scale block of the slice in stage s.
  // The K loop below is unrolled by STAGES, so every stage index is a
  // compile-time constant and the ring stays in registers.
  float sa_ring[STAGES][TM];
  auto issue = [&](int slice, int stage) {
    uint8_t* buf = smem + stage * Cfg::kStage;
    const int64_t k_off = (int64_t)slice * kSlice;
    load_slabs<Cfg::kASlabs>(A, lda, m0, M - 1, k_off, buf, wave * Cfg::kASlabs, lane);
    load_slabs<Cfg::kWSlabs>(W, K, n0, N - 1, k_off, buf + Cfg::kABytes, wave * Cfg::kWSlabs,
                             lane);
    const int64_t kb = slice >> 1;
#pragma unroll
    for (int b = 0; b < TM; ++b) sa_ring[stage][b] = sA[kb * sa_ld + tok[b]];
  };

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < KS) issue(s, s);

  float s_prev[TM];
#pragma unroll
  for (int b = 0; b < TM; ++b) s_prev[b] = 0.0f;
  bool skip = false;

  for (int base = 0; base < KS; base += STAGES) {
#pragma unroll
    for (int stage = 0; stage < STAGES; ++stage) {
      const int ks = base + stage;
      if (ks < KS) {
        // slices ks+1 .. ks+STAGES-2 may stay in flight
        if (ks + STAGES - 2 < KS) {
          wait_vmcnt<(STAGES - 2) * Cfg::kOpsPerStage>();
        } else {
          wait_vmcnt<0>();
        }
        lds_barrier();
        if (ks + STAGES - 1 < KS) issue(ks + STAGES - 1, (stage + STAGES - 1) % STAGES);

        if ((ks & 1) == 0) {
          // entering scale block kb: acc <- acc * s_prev / s_kb
          const float sw = sw_row[ks >> 1];
          skip = sw == 0.0f;  // wave-uniform
          if (!skip) {
#pragma unroll
            for (int b = 0; b < TM; ++b) {
              const float s_cur = sa_ring[stage][b] * sw;
              const float r = s_prev[b] / s_cur;  // 0 until the first block
#pragma unroll
              for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[a][b][e] *= r;
              s_prev[b] = s_cur;
            }
          }
        }
        if (!skip) {
          const uint8_t* a_lds = smem + stage * Cfg::kStage;
          const uint8_t* w_lds = a_lds + Cfg::kABytes;
          v8i wf[TN], af[TM];
#pragma unroll
          for (int a = 0; a < TN; ++a)
            wf[a] = read_frag(w_lds, wn * TN * 32 + a * 32 + (lane & 31), lane);
#pragma unroll
          for (int b = 0; b < TM; ++b)
            af[b] = read_frag(a_lds, wm * TM * 32 + b * 32 + (lane & 31), lane);
#pragma unroll
          for (int a = 0; a < TN; ++a)
#pragma unroll
            for (int b = 0; b < TM; ++b)
              acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                  wf[a], af[b], acc[a][b], 0, 0, 0, 0, 0, 0);
        }
      }
    }
  }

  // ---- epilogue: lane holds token column (lane & 31); rows are weights --
#pragma unroll
  for (int b = 0; b < TM; ++b) {
    const int m = m0 + wm * TM * 32 + b * 32 + (lane & 31);
    if (m >= M) continue;
    const float s = s_prev[b];
    uint16_t* crow = C + (int64_t)m * ldc;
#pragma unroll
    for (int a = 0; a < TN; ++a) {
      const int nbase = n0 + wn * TN * 32 + a * 32 + (lane >> 5) * 4;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint2 v;
        v.x = pack2_bf16(acc[a][b][g * 4 + 0] * s, acc[a][b][g * 4 + 1] * s);
        v.y = pack2_bf16(acc[a][b][g * 4 + 2] * s, acc[a][b][g * 4 + 3] * s);
        *reinterpret_cast<uint2*>(crow + nbase + g * 8) = v;
      }
    }
  }
}


// ---------------------------------------------------------------------------
// Variant with local-read prefetch: the MFMA fragments of slice ks+1 are read
// from LDS while the MFMAs of slice ks run, so a wave leaving the barrier has
// its MFMA operands in registers already. The token scales of each slice are
// staged in LDS by the same direct loads (one dword per lane), so no register
// array is indexed by a run-time stage. STAGES >= 3 (slice ks+1 must be waited
// for while slice ks+2 may still be in flight).
template <int BM, int BN, int WAVES_N, int WAVES_M, int STAGES>
struct PlrCfg {
  static constexpr int kWaves = WAVES_N * WAVES_M;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kTN = BN / WAVES_N / 32;
  static constexpr int kTM = BM / WAVES_M / 32;
  static constexpr int kABytes = BM * kSlice;
  static constexpr int kWBytes = BN * kSlice;
  static constexpr int kSaBytes = kWaves * 256;  // each wave stages 64 token scales
  static constexpr int kStage = kABytes + kWBytes + kSaBytes;
  static constexpr int kLds = STAGES * kStage;
  static constexpr int kASlabs = BM / 16 / kWaves;
  static constexpr int kWSlabs = BN / 16 / kWaves;
  static constexpr int kOpsPerStage = kASlabs + kWSlabs + 1;
  static_assert(STAGES >= 3, "local-read prefetch needs three stages");
  static_assert(kTN >= 1 && kTM >= 1, "wave tile");
  static_assert(BM % (16 * kWaves) == 0 && BN % (16 * kWaves) == 0, "slabs");
  static_assert(128 % (BN / WAVES_N) == 0 || (BN / WAVES_N) == 128, "weight scale block");
  static_assert(BM <= 64 * kWaves, "token scales staged by the waves");
  static_assert(kLds <= 160 * 1024, "LDS");
  static_assert((STAGES - 3) * kOpsPerStage < 64, "vmcnt");
};

template <int BM, int BN, int WAVES_N, int WAVES_M, int STAGES>
__global__ __launch_bounds__(64 * WAVES_N * WAVES_M)
__attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_fp8_plr_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sA, const uint8_t* __restrict__ W,
    const float* __restrict__ sW, uint16_t* __restrict__ C, int M, int N, int K, int64_t lda,
    int64_t ldc, int64_t sa_ld, int tiles_m, int tiles_n, int group_m) {
  using Cfg = PlrCfg<BM, BN, WAVES_N, WAVES_M, STAGES>;
  constexpr int TN = Cfg::kTN, TM = Cfg::kTM;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Cfg::kLds];

  const int total = tiles_m * tiles_n;
  int id = blockIdx.x;
  {
    const int per = (total + 7) / 8;
    const int xcd = id & 7, local = id >> 3;
    const int full = total - (per - 1) * 8;
    id = xcd < full ? xcd * per + local : full * per + (xcd - full) * (per - 1) + local;
  }
  const int width = group_m * tiles_n;
  const int group = id / width;
  const int first_m = group * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int tile_m = first_m + (id % width) % gsize;
  const int tile_n = (id % width) / gsize;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave % WAVES_N;
  const int wm = wave / WAVES_N;
  const int m0 = tile_m * BM;
  const int n0 = tile_n * BN;
  const int KT = K >> 7;
  const int KS = K / kSlice;

  v16f acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;

  const float* sw_row = sW + (int64_t)((n0 + wn * TN * 32) >> 7) * KT;
  // the token whose scale this lane stages (tile rows wave*64 + lane)
  int sa_tok = m0 + wave * 64 + lane;
  sa_tok = min(sa_tok, min(m0 + BM, M) - 1);

  auto issue = [&](int slice) {
    uint8_t* buf = smem + (slice % STAGES) * Cfg::kStage;
    const int64_t k_off = (int64_t)slice * kSlice;
    const float* src = sA + (int64_t)(slice >> 1) * sa_ld + sa_tok;
    __builtin_amdgcn_global_load_lds((const void*)src,
                                     (lds_void*)(buf + Cfg::kABytes + Cfg::kWBytes + wave * 256),
                                     4, 0, 0);
    load_slabs<Cfg::kASlabs>(A, lda, m0, M - 1, k_off, buf, wave * Cfg::kASlabs, lane);
    load_slabs<Cfg::kWSlabs>(W, K, n0, N - 1, k_off, buf + Cfg::kABytes, wave * Cfg::kWSlabs,
                             lane);
  };
  auto read_frags = [&](int slice, v8i (&wf)[TN], v8i (&af)[TM]) {
    const uint8_t* a_lds = smem + (slice % STAGES) * Cfg::kStage;
    const uint8_t* w_lds = a_lds + Cfg::kABytes;
#pragma unroll
    for (int a = 0; a < TN; ++a) wf[a] = read_frag(w_lds, wn * TN * 32 + a * 32 + (lane & 31), lane);
#pragma unroll
    for (int b = 0; b < TM; ++b) af[b] = read_frag(a_lds, wm * TM * 32 + b * 32 + (lane & 31), lane);
  };

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < KS) issue(s);
  __builtin_amdgcn_s_waitcnt(0);  // the prologue waits once for everything
  lds_barrier();

  float s_prev[TM];
#pragma unroll
  for (int b = 0; b < TM; ++b) s_prev[b] = 0.0f;
  bool skip = false;

  v8i wf0[TN], af0[TM], wf1[TN], af1[TM];
  read_frags(0, wf0, af0);

  // one slice: wait for and read slice ks+1 while slice ks's MFMAs run
  auto step = [&](int ks, v8i (&wf)[TN], v8i (&af)[TM], v8i (&wfn)[TN], v8i (&afn)[TM]) {
    const bool next = ks + 1 < KS;
    if (next) {
      // slice ks+1 landed; slices ks+2 .. ks+STAGES-2 may stay in flight
      if (ks + STAGES - 2 < KS) {
        wait_vmcnt<(STAGES - 3) * Cfg::kOpsPerStage>();
      } else {
        wait_vmcnt<0>();
      }
      lds_barrier();
      if (ks + STAGES - 1 < KS) issue(ks + STAGES - 1);
      read_frags(ks + 1, wfn, afn);
    }
    if ((ks & 1) == 0) {
      const float sw = sw_row[ks >> 1];
      skip = sw == 0.0f;  // wave-uniform
      if (!skip) {
        const float* sa_lds = reinterpret_cast<const float*>(
            smem + (ks % STAGES) * Cfg::kStage + Cfg::kABytes + Cfg::kWBytes);
#pragma unroll
        for (int b = 0; b < TM; ++b) {
          const float s_cur = sa_lds[wm * TM * 32 + b * 32 + (lane & 31)] * sw;
          const float r = s_prev[b] / s_cur;  // 0 until the first block
#pragma unroll
          for (int a = 0; a < TN; ++a)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[a][b][e] *= r;
          s_prev[b] = s_cur;
        }
      }
    }
    if (!skip) {
#pragma unroll
      for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[a], af[b], acc[a][b], 0,
                                                                      0, 0, 0, 0, 0);
    }
  };
  for (int ks = 0; ks < KS; ks += 2) {
    step(ks, wf0, af0, wf1, af1);
    if (ks + 1 < KS) step(ks + 1, wf1, af1, wf0, af0);
  }

#pragma unroll
  for (int b = 0; b < TM; ++b) {
    const int m = m0 + wm * TM * 32 + b * 32 + (lane & 31);
    if (m >= M) continue;
    const float s = s_prev[b];
    uint16_t* crow = C + (int64_t)m * ldc;
#pragma unroll
    for (int a = 0; a < TN; ++a) {
      const int nbase = n0 + wn * TN * 32 + a * 32 + (lane >> 5) * 4;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint2 v;
        v.x = pack2_bf16(acc[a][b][g * 4 + 0] * s, acc[a][b][g * 4 + 1] * s);
        v.y = pack2_bf16(acc[a][b][g * 4 + 2] * s, acc[a][b][g * 4 + 3] * s);
        *reinterpret_cast<uint2*>(crow + nbase + g * 8) = v;
      }
    }
  }
}

template <int BM, int BN, int WN, int WM, int ST>
int launch_plr(const void* A, const float* sA, const void* W, const float* sW, void* C, int M,
               int N, int K, int64_t lda, int64_t ldc, int64_t sa_ld, int group_m,
               hipStream_t stream) {
  using Cfg = PlrCfg<BM, BN, WN, WM, ST>;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  const int total = tiles_m * tiles_n;
  hipLaunchKernelGGL((gemm_fp8_plr_kernel<BM, BN, WN, WM, ST>), dim3(total), dim3(Cfg::kThreads),
                     0, stream, (const uint8_t*)A, sA, (const uint8_t*)W, sW, (uint16_t*)C, M, N,
                     K, lda, ldc, sa_ld, tiles_m, tiles_n, group_m < 1 ? 1 : group_m);
  QX_LAUNCH_STATUS();
}


// ---- 128-byte slices: one 128-K scale block per pipeline stage ------------
// Rows of 128 B (8 chunks of 16 B), chunk-swizzled by ((row >> 1) & 7); a
// 1 KiB direct-load slab is 8 rows; a lane's MFMA fragment for K-half h is
// bytes [h*64 + (lane/32)*32, +32).
__device__ __forceinline__ int swz128(int row) { return (row >> 1) & 7; }

// hi_shift moves tile rows >= 128 by that many global rows (the gate_up
// tile of the SwiGLU epilogue); a slab never straddles row 128.
template <int SLABS>
__device__ __forceinline__ void load_slabs128(const uint8_t* __restrict__ g, int64_t ld, int row0,
                                              int row_max, int64_t k_off, uint8_t* lds,
                                              int first, int lane, int hi_shift = 0) {
  const int r_in = lane >> 3;
  const int p = lane & 7;
#pragma unroll
  for (int j = 0; j < SLABS; ++j) {
    const int slab = first + j;
    const int row = slab * 8 + r_in;
    const int c = p ^ swz128(row);
    int grow = row0 + row + (slab >= 16 ? hi_shift : 0);
    grow = grow < row_max ? grow : row_max;
    const uint8_t* src = g + (int64_t)grow * ld + k_off + c * 16;
    __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(lds + slab * 1024), 16, 0,
                                     kOperandLoadPolicy);
  }
}

// load_slabs128 for a tile whose rows are all in bounds, split in two: the
// per-lane byte offsets within a tile (the same for every tile), computed
// once, and the loads of one K block from a wave-uniform base
template <int SLABS>
__device__ __forceinline__ void slab_offsets128(int64_t ld, int first, int lane, int hi_shift,
                                                int64_t (&off)[SLABS]) {
  const int r_in = lane >> 3;
  const int p = lane & 7;
#pragma unroll
  for (int j = 0; j < SLABS; ++j) {
    const int slab = first + j;
    const int row = slab * 8 + r_in;
    off[j] = (int64_t)(row + (slab >= 16 ? hi_shift : 0)) * ld + (p ^ swz128(row)) * 16;
  }
}

template <int SLABS>
__device__ __forceinline__ void load_slab_offsets128(const uint8_t* base, const int64_t (&off)[SLABS],
                                                     uint8_t* lds, int first) {
#pragma unroll
  for (int j = 0; j < SLABS; ++j)
    __builtin_amdgcn_global_load_lds((const void*)(base + off[j]),
                                     (lds_void*)(lds + (first + j) * 1024), 16, 0,
                                     kOperandLoadPolicy);
}

__device__ __forceinline__ v8i read_frag128(const uint8_t* lds, int row, int h, int lane) {
  const int c0 = h * 4 + (lane >> 5) * 2;
  const int sw = swz128(row);
  const v4i* base = reinterpret_cast<const v4i*>(lds + row * 128);
  const v4i lo = base[c0 ^ sw];
  const v4i hi = base[(c0 + 1) ^ sw];
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

template <int BM, int BN, int WAVES_N, int WAVES_M, int STAGES>
struct Cfg128 {
  static constexpr int kWaves = WAVES_N * WAVES_M;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kTN = BN / WAVES_N / 32;
  static constexpr int kTM = BM / WAVES_M / 32;
  static constexpr int kABytes = BM * 128;
  static constexpr int kWBytes = BN * 128;
  // the tile's token scales of the block: 64 slots per wave, the first
  // kSaPerWave of them used
  static constexpr int kSaBytes = 256 * WAVES_N * WAVES_M;
  static constexpr int kStage = kABytes + kWBytes + kSaBytes;
  static constexpr int kLds = STAGES * kStage;
  static constexpr int kASlabs = BM / 8 / kWaves;
  static constexpr int kWSlabs = BN / 8 / kWaves;
  static constexpr int kSaPerWave = BM / kWaves;
  static constexpr int kOpsPerStage = kASlabs + kWSlabs + 1;
  static_assert(kTN >= 1 && kTM >= 1, "wave tile");
  static_assert(BM % (8 * kWaves) == 0 && BN % (8 * kWaves) == 0, "slabs");
  static_assert(kSaPerWave >= 1 && kSaPerWave <= 64 && BM % kWaves == 0, "scale loads");
  static_assert(128 % (BN / WAVES_N) == 0 || (BN / WAVES_N) == 128, "weight scale block");
  static_assert(kLds <= 160 * 1024, "LDS");
  static_assert(STAGES >= 2 && (STAGES - 2) * kOpsPerStage < 64, "stages");
};

// Epilogue of the 128-K-stage tile kernels (acc in units of the last
// block's scale s_prev): stage the bf16 tile in LDS and write it back.
template <int BM, int BN, int WAVES_N, int WAVES_M, int LDS_BYTES, bool SWIGLU, int TN, int TM>
__device__ __forceinline__ void tile_epilogue(uint8_t* smem, const v16f (&acc)[TN][TM],
                                              const float (&s_prev)[TM], int lane, int wave, int m0,
                                              int n0, int M, uint16_t* __restrict__ C,
                                              int64_t ldc, uint8_t* __restrict__ Q, int64_t q_ld,
                                              float* __restrict__ Qs, int64_t qs_ld) {
  constexpr int kWaves = WAVES_N * WAVES_M;
  const int wn = wave % WAVES_N;
  const int wm = wave / WAVES_N;
  // Epilogue through LDS. A lane's accumulators are one token's values at
  // 4 runs of 4 columns, so storing them directly makes every store
  // instruction touch 32 rows of C (8 bytes each); the bf16 tile is staged
  // in LDS instead (rows = tokens, each row padded by 16 bytes so the 32
  // rows one write instruction touches spread over the banks) and written
  // back one whole tile row per BN/8 lanes, 16 bytes per lane.
  // The stores are non-temporal: C is not read again by this launch, and
  // keeping it out of L2 leaves L2 to the operand rows other workgroups
  // are about to read (measured 1-8% faster per Qwen3-4B shape).
  constexpr int kRowBytes = BN * 2 + 16;
  constexpr int kChunks = BN / 8;
  static_assert(BM * kRowBytes <= LDS_BYTES, "epilogue tile fits the stage buffers");
  static_assert(64 % kChunks == 0 && BM % kWaves == 0 &&
                    (BM / kWaves) % (64 / kChunks) == 0,
                "epilogue rows");
  __syncthreads();  // every wave is done with the last stage's operands
#pragma unroll
  for (int b = 0; b < TM; ++b) {
    const int row = wm * TM * 32 + b * 32 + (lane & 31);
    const float s = s_prev[b];
    uint8_t* lrow = smem + row * kRowBytes;
#pragma unroll
    for (int a = 0; a < TN; ++a) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int off = (wn * TN * 32 + a * 32 + (lane >> 5) * 4 + g * 8) * 2;
        uint2 v;
        v.x = pack2_bf16(acc[a][b][g * 4 + 0] * s, acc[a][b][g * 4 + 1] * s);
        v.y = pack2_bf16(acc[a][b][g * 4 + 2] * s, acc[a][b][g * 4 + 3] * s);
        *reinterpret_cast<uint2*>(lrow + off) = v;
      }
    }
  }
  __syncthreads();
  constexpr int kRowsPerWave = BM / kWaves;
  if constexpr (SWIGLU) {
    // 16 lanes per tile row, 8 gate and 8 up values each (the SiLU-quant
    // kernel's grouping: one 128-column quant group per 16 lanes)
    static_assert(BN == 256 && kRowsPerWave % 4 == 0, "128 gate + 128 up columns per tile");
    const int j0 = n0 >> 1;
    const int seg = lane & 15;
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 4; ++i) {
      const int row = wave * kRowsPerWave + i * 4 + (lane >> 4);
      const int m = m0 + row;
      const uint8_t* lrow = smem + row * kRowBytes;
      const uint4 g = *reinterpret_cast<const uint4*>(lrow + seg * 16);
      const uint4 u = *reinterpret_cast<const uint4*>(lrow + 256 + seg * 16);
      const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
      float y[8];
      float amax = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        y[2 * k] = silu_mul(lo_bf16(gw[k]), lo_bf16(uw[k]));
        y[2 * k + 1] = silu_mul(hi_bf16(gw[k]), hi_bf16(uw[k]));
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(y[k]));
      amax = group_max<16>(amax);
      const float scale = fp8_scale(amax);
      const float rs = recip(scale);
      if (m < M) {
        const v2i o = {(int)pack4_fp8(div_by(y[0], scale, rs), div_by(y[1], scale, rs),
                                      div_by(y[2], scale, rs), div_by(y[3], scale, rs)),
                       (int)pack4_fp8(div_by(y[4], scale, rs), div_by(y[5], scale, rs),
                                      div_by(y[6], scale, rs), div_by(y[7], scale, rs))};
        __builtin_nontemporal_store(o, reinterpret_cast<v2i*>(Q + (int64_t)m * q_ld + j0 + seg * 8));
        if (seg == 0) Qs[(int64_t)(j0 >> 7) * qs_ld + m] = scale;
      }
    }
  } else {
    constexpr int kRowsPerOp = 64 / kChunks;
    const bool wide = ((ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
    const int c = lane % kChunks;
#pragma unroll
    for (int i = 0; i < kRowsPerWave / kRowsPerOp; ++i) {
      const int row = wave * kRowsPerWave + i * kRowsPerOp + lane / kChunks;
      const int m = m0 + row;
      const uint4 v = *reinterpret_cast<const uint4*>(smem + row * kRowBytes + c * 16);
      if (m < M) {
        uint16_t* dst = C + (int64_t)m * ldc + n0 + c * 8;
        if (wide) {
          const v4i w = {(int)v.x, (int)v.y, (int)v.z, (int)v.w};
          __builtin_nontemporal_store(w, reinterpret_cast<v4i*>(dst));
        } else {
          reinterpret_cast<uint2*>(dst)[0] = make_uint2(v.x, v.y);
          reinterpret_cast<uint2*>(dst)[1] = make_uint2(v.z, v.w);
        }
      }
    }
  }
}

// WARM: with each stage's loads, also touch one 4-byte word of every
// 128-byte row segment of the block one stage further ahead (into a small
// LDS sink nothing reads), so that block's rows are on their way into L2
// when their real loads are issued.
//
// SWIGLU: W (N x K) is a gate_up weight, rows [gate (N/2) | up (N/2)], and
// tile t covers output columns j0 = 128t.. of both halves: its first 128
// weight rows are gate rows j0.., the next 128 up rows N/2 + j0... The
// epilogue then writes silu(gate) * up, FP8-quantized per 128 columns (one
// group per tile), to Q (M x N/2 e4m3, leading dimension q_ld) and its
// scales to Qs (column-major, Qs[group * qs_ld + m]) instead of C; the bf16
// rounding of gate and up is the unfused GEMM's, and the SiLU and quant
// arithmetic the SiLU-quant kernel's, so the result is bit-identical to
// qx_gemm_fp8_blockscaled followed by qx_silu_mul_quant.
template <int BM, int BN, int WAVES_N, int WAVES_M, int STAGES, bool WARM, bool SWIGLU = false>
__global__ __launch_bounds__(64 * WAVES_N * WAVES_M) void gemm_fp8_k128_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sA, const uint8_t* __restrict__ W,
    const float* __restrict__ sW, uint16_t* __restrict__ C, int M, int N, int K, int64_t lda,
    int64_t ldc, int64_t sa_ld, int tiles_m, int tiles_n, int group_m, uint8_t* __restrict__ Q,
    int64_t q_ld, float* __restrict__ Qs, int64_t qs_ld) {
  using Cfg = Cfg128<BM, BN, WAVES_N, WAVES_M, STAGES>;
  constexpr int TN = Cfg::kTN, TM = Cfg::kTM;
  constexpr int kWarm = WARM ? (BM + BN + 64 * Cfg::kWaves - 1) / (64 * Cfg::kWaves) : 0;
  constexpr int kSink = WARM ? Cfg::kWaves * 256 : 0;
  // vector loads per stage, not counting the weight-scale load (a scalar
  // load where the compiler sees its uniform address; undercounting only
  // makes a wait stricter)
  constexpr int kOps = Cfg::kOpsPerStage + kWarm;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Cfg::kLds + kSink];

  const int total = tiles_m * tiles_n;
  int id = blockIdx.x;
  {
    const int per = (total + 7) / 8;
    const int xcd = id & 7, local = id >> 3;
    const int full = total - (per - 1) * 8;
    id = xcd < full ? xcd * per + local : full * per + (xcd - full) * (per - 1) + local;
  }
  const int width = group_m * tiles_n;
  const int group = id / width;
  const int first_m = group * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int tile_m = first_m + (id % width) % gsize;
  const int tile_n = (id % width) / gsize;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
  // SWIGLU: the tile's weight rows are gate rows j0.. then up rows N/2 + j0..
  const int w_row0 = SWIGLU ? (n0 >> 1) : n0;
  const int w_hi_shift = SWIGLU ? (N >> 1) - 128 : 0;
  static_assert(!SWIGLU || (BN == 256 && WAVES_N == 2), "SwiGLU tiles: 128 gate + 128 up rows");
  const float* sw_row =
      sW + (int64_t)((SWIGLU ? w_row0 + wn * ((N >> 1)) : n0 + wn * TN * 32) >> 7) * KT;

  float sw_ring[STAGES];
  auto issue = [&](int kb, int stage) {
    uint8_t* buf = smem + stage * Cfg::kStage;
    const int64_t k_off = (int64_t)kb * 128;
    load_slabs128<Cfg::kASlabs>(A, lda, m0, M - 1, k_off, buf, wave * Cfg::kASlabs, lane);
    load_slabs128<Cfg::kWSlabs>(W, K, w_row0, N - 1, k_off, buf + Cfg::kABytes,
                                wave * Cfg::kWSlabs, lane, w_hi_shift);
    // token scales of the tile for this block, beside its operands: lane i of
    // wave w loads the scale of tile row w * kSaPerWave + i into slot
    // w * 64 + i (lanes past kSaPerWave repeat a row into unused slots)
    {
      const int t = min(m0 + wave * Cfg::kSaPerWave + lane % Cfg::kSaPerWave, M - 1);
      __builtin_amdgcn_global_load_lds((const void*)(sA + (int64_t)kb * sa_ld + t),
                                       (lds_void*)(buf + Cfg::kABytes + Cfg::kWBytes + wave * 256),
                                       4, 0, 0);
    }
    sw_ring[stage] = __builtin_nontemporal_load(sw_row + kb);
    if (WARM) {
      // block kb + 1 (clamped to the last block): row g of [A rows | W rows]
      const int64_t w_off = (int64_t)min(kb + 1, KT - 1) * 128;
#pragma unroll
      for (int j = 0; j < kWarm; ++j) {
        const int g = j * 64 * Cfg::kWaves + wave * 64 + lane;
        const uint8_t* src;
        if (g < BM) {
          src = A + (int64_t)min(m0 + g, M - 1) * lda + w_off;
        } else {
          src = W + (int64_t)min(n0 + min(g - BM, BN - 1), N - 1) * K + w_off;
        }
        __builtin_amdgcn_global_load_lds((const void*)src,
                                         (lds_void*)(smem + Cfg::kLds + wave * 256), 4, 0, 0);
      }
    }
  };
#pragma unroll
  for (int st = 0; st < STAGES - 1; ++st)
    if (st < KT) issue(st, st);

  float s_prev[TM];
#pragma unroll
  for (int b = 0; b < TM; ++b) s_prev[b] = 0.0f;

  for (int base = 0; base < KT; base += STAGES) {
#pragma unroll
    for (int stage = 0; stage < STAGES; ++stage) {
      const int kb = base + stage;
      if (kb < KT) {
        // this block's loads are done; the warm loads issued last with
        // them, and the later stages' loads, may still be in flight
        if (kb + STAGES - 2 < KT) {
          wait_vmcnt<(STAGES - 2) * kOps + kWarm>();
        } else {
          wait_vmcnt<0>();
        }
        lds_barrier();
        if (kb + STAGES - 1 < KT) issue(kb + STAGES - 1, (stage + STAGES - 1) % STAGES);
        const float sw = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sw_ring[stage])));
        if (sw != 0.0f) {  // wave-uniform; a zero weight-scale block adds nothing
#pragma unroll
          for (int b = 0; b < TM; ++b) {
            const float* sa_lds =
                reinterpret_cast<const float*>(smem + stage * Cfg::kStage + Cfg::kABytes +
                                               Cfg::kWBytes);
            const int row = wm * TM * 32 + b * 32 + (lane & 31);
            const float s_cur =
                sa_lds[(row / Cfg::kSaPerWave) * 64 + row % Cfg::kSaPerWave] * sw;
            const float r = s_prev[b] / s_cur;
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
              for (int e = 0; e < 16; ++e) acc[a][b][e] *= r;
            s_prev[b] = s_cur;
          }
          const uint8_t* a_lds = smem + stage * Cfg::kStage;
          const uint8_t* w_lds = a_lds + Cfg::kABytes;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            v8i wf[TN], af[TM];
#pragma unroll
            for (int a = 0; a < TN; ++a)
              wf[a] = read_frag128(w_lds, wn * TN * 32 + a * 32 + (lane & 31), h, lane);
#pragma unroll
            for (int b = 0; b < TM; ++b)
              af[b] = read_frag128(a_lds, wm * TM * 32 + b * 32 + (lane & 31), h, lane);
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
              for (int b = 0; b < TM; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    wf[a], af[b], acc[a][b], 0, 0, 0, 0, 0, 0);
          }
        }
      }
    }
  }

  tile_epilogue<BM, BN, WAVES_N, WAVES_M, Cfg::kLds, SWIGLU>(smem, acc, s_prev, lane, wave, m0,
                                                            n0, M, C, ldc, Q, q_ld, Qs, qs_ld);
}

// ---- staggered rescale ---------------------------------------------------------
// gemm_fp8_k128_kernel<256, 256, 2, 4, 2> with the block-scale rescale moved
// away from the MFMAs that produce and consume each accumulator. VALU work
// on an accumulator right after the MFMA that wrote it, or right before the
// MFMA that reads it, serialises with the matrix core; a few MFMAs between
// them and it overlaps. A wave's 8 tiles are two token halves b = 0, 1 of 4
// weight tiles each; per block the MFMAs run h0 b0 | h0 b1 | h1 b0 | h1 b1
// (4 each), the b1 tiles are rescaled for block kb while the h0 b0 MFMAs of
// kb issue, and the b0 tiles for block kb + 1 while the h1 b1 MFMAs of kb
// issue, so four MFMAs separate every rescale from the MFMAs on either side.
// The rescale of the b0 tiles needs block kb + 1's scales during block kb:
// each lane loads its two tokens' scales two blocks ahead into registers,
// and the weight scale is loaded with the stage. Per output element the
// operations and their order are unchanged (rescale, then the block's MFMAs
// in K order): bit-identical to the other configurations.
template <bool SWIGLU>
__global__ __launch_bounds__(512) void gemm_fp8_k128s_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sA, const uint8_t* __restrict__ W,
    const float* __restrict__ sW, uint16_t* __restrict__ C, int M, int N, int K, int64_t lda,
    int64_t ldc, int64_t sa_ld, int tiles_m, int tiles_n, int group_m, uint8_t* __restrict__ Q,
    int64_t q_ld, float* __restrict__ Qs, int64_t qs_ld) {
  constexpr int BM = 256, BN = 256, WAVES_N = 2, WAVES_M = 4, STAGES = 2;
  using Cfg = Cfg128<BM, BN, WAVES_N, WAVES_M, STAGES>;
  constexpr int TN = Cfg::kTN, TM = Cfg::kTM;
  static_assert(TN == 4 && TM == 2, "two token halves of four weight tiles");
  constexpr int kStage = Cfg::kABytes + Cfg::kWBytes;
  // the stage buffers, or the epilogue's padded bf16 tile, whichever is larger
  constexpr int kEpilogueBytes = BM * (BN * 2 + 16);
  constexpr int kLds = STAGES * kStage > kEpilogueBytes ? STAGES * kStage : kEpilogueBytes;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kLds];

  const int total = tiles_m * tiles_n;
  int id = blockIdx.x;
  {
    const int per = (total + 7) / 8;
    const int xcd = id & 7, local = id >> 3;
    const int full = total - (per - 1) * 8;
    id = xcd < full ? xcd * per + local : full * per + (xcd - full) * (per - 1) + local;
  }
  const int width = group_m * tiles_n;
  const int first_m = (id / width) * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int m0 = (first_m + (id % width) % gsize) * BM;
  const int n0 = ((id % width) / gsize) * BN;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave % WAVES_N;
  const int wm = wave / WAVES_N;
  const int KT = K >> 7;
  const int w_row0 = SWIGLU ? (n0 >> 1) : n0;
  const int w_hi_shift = SWIGLU ? (N >> 1) - 128 : 0;
  const float* sw_row =
      sW + (int64_t)((SWIGLU ? w_row0 + wn * (N >> 1) : n0 + wn * TN * 32) >> 7) * KT;
  // this lane's two token rows (tail rows read the last row's scales)
  const int t0 = min(m0 + wm * TM * 32 + (lane & 31), M - 1);
  const int t1 = min(m0 + wm * TM * 32 + 32 + (lane & 31), M - 1);

  v16f acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;
  float s_prev[TM] = {0.0f, 0.0f};
  float sw_ring[STAGES];

  auto issue = [&](int kb, int stage) __attribute__((always_inline)) {
    uint8_t* buf = smem + stage * kStage;
    const int64_t k_off = (int64_t)kb * 128;
    load_slabs128<Cfg::kASlabs>(A, lda, m0, M - 1, k_off, buf, wave * Cfg::kASlabs, lane);
    load_slabs128<Cfg::kWSlabs>(W, K, w_row0, N - 1, k_off, buf + Cfg::kABytes,
                                wave * Cfg::kWSlabs, lane, w_hi_shift);
    sw_ring[stage] = __builtin_nontemporal_load(sw_row + kb);
  };
  // token scales of blocks kb (cur), kb + 1 (nxt), kb + 2 (nxt2), by half
  float ta_cur[2], ta_nxt[2], ta_nxt2[2];
  auto load_ta = [&](int kb, float (&dst)[2]) __attribute__((always_inline)) {
    const float* row = sA + (int64_t)min(kb, KT - 1) * sa_ld;  // wave-uniform
    dst[0] = row[t0];
    dst[1] = row[t1];
  };

  issue(0, 0);
  load_ta(0, ta_cur);
  load_ta(1, ta_nxt);
  // block 0's scale of the b0 tiles (their rescale by 0 / s of zero
  // accumulators is a no-op); a zero weight-scale block keeps s_prev
  {
    const float sw0 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sw_ring[0])));
    if (sw0 != 0.0f) s_prev[0] = ta_cur[0] * sw0;
  }

  for (int base = 0; base < KT; base += STAGES) {
#pragma unroll
    for (int stage = 0; stage < STAGES; ++stage) {
      const int kb = base + stage;
      if (kb < KT) {
        wait_vmcnt<0>();  // block kb's operands (and older scale loads) are in
        lds_barrier();
        if (kb + 1 < KT) issue(kb + 1, stage ^ 1);
        load_ta(kb + 2, ta_nxt2);
        const float sw = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sw_ring[stage])));
        const bool run = sw != 0.0f;  // wave-uniform
        const uint8_t* a_lds = smem + stage * kStage;
        const uint8_t* w_lds = a_lds + Cfg::kABytes;
        // the b1 tiles' factor for block kb
        float r1 = 1.0f;
        if (run) {
          const float s_cur = ta_cur[1] * sw;
          r1 = s_prev[1] / s_cur;
          s_prev[1] = s_cur;
        }
        // the b0 tiles' factor for block kb + 1 (1 if there is none or it adds nothing)
        float r0 = 1.0f;
        if (kb + 1 < KT) {
          const float swn =
              __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sw_ring[stage ^ 1])));
          if (swn != 0.0f) {
            const float s_cur = ta_nxt[0] * swn;
            r0 = s_prev[0] / s_cur;
            s_prev[0] = s_cur;
          }
        }
        // A block whose weight scale is 0 adds nothing: its MFMAs run on
        // zero token fragments (acc + 0 leaves acc's bits: the accumulators
        // start at +0 and never hold -0), so every block is one instruction
        // stream and skipping it would give the same result.
        const v8i zero = {0, 0, 0, 0, 0, 0, 0, 0};
        {
          v8i wf[TN], af[TM];
#pragma unroll
          for (int a = 0; a < TN; ++a)
            wf[a] = read_frag128(w_lds, wn * TN * 32 + a * 32 + (lane & 31), 0, lane);
#pragma unroll
          for (int b = 0; b < TM; ++b)
            af[b] = run ? read_frag128(a_lds, wm * TM * 32 + b * 32 + (lane & 31), 0, lane) : zero;
          // h0 b0, with the b1 rescale
#pragma unroll
          for (int a = 0; a < TN; ++a) {
            acc[a][0] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[a], af[0], acc[a][0],
                                                                       0, 0, 0, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[a][1][e] *= r1;
          }
#pragma unroll
          for (int a = 0; a < TN; ++a) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
          }
          // h0 b1
#pragma unroll
          for (int a = 0; a < TN; ++a)
            acc[a][1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[a], af[1], acc[a][1],
                                                                       0, 0, 0, 0, 0, 0);
#pragma unroll
          for (int a = 0; a < TN; ++a)
            wf[a] = read_frag128(w_lds, wn * TN * 32 + a * 32 + (lane & 31), 1, lane);
#pragma unroll
          for (int b = 0; b < TM; ++b)
            af[b] = run ? read_frag128(a_lds, wm * TM * 32 + b * 32 + (lane & 31), 1, lane) : zero;
          // h1 b0
#pragma unroll
          for (int a = 0; a < TN; ++a)
            acc[a][0] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[a], af[0], acc[a][0],
                                                                       0, 0, 0, 0, 0, 0);
          // h1 b1, with the b0 rescale for block kb + 1
#pragma unroll
          for (int a = 0; a < TN; ++a) {
            acc[a][1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[a], af[1], acc[a][1],
                                                                       0, 0, 0, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[a][0][e] *= r0;
          }
#pragma unroll
          for (int a = 0; a < TN; ++a) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);
          }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          ta_cur[h] = ta_nxt[h];
          ta_nxt[h] = ta_nxt2[h];
        }
      }
    }
  }

  tile_epilogue<BM, BN, WAVES_N, WAVES_M, kLds, SWIGLU>(
      smem, acc, s_prev, lane, wave, m0, n0, M, C, ldc, Q, q_ld, Qs, qs_ld);
}

template <bool SWIGLU>
int launch128s(const void* A, const float* sA, const void* W, const float* sW, void* C, int M,
               int N, int K, int64_t lda, int64_t ldc, int64_t sa_ld, void* Q, int64_t q_ld,
               float* Qs, int64_t qs_ld, hipStream_t stream) {
  const int tiles_m = (M + 255) / 256;
  const int tiles_n = N / 256;
  hipLaunchKernelGGL((gemm_fp8_k128s_kernel<SWIGLU>), dim3(tiles_m * tiles_n), dim3(512), 0,
                     stream, (const uint8_t*)A, sA, (const uint8_t*)W, sW, (uint16_t*)C, M, N, K,
                     lda, ldc, sa_ld, tiles_m, tiles_n, 4, (uint8_t*)Q, q_ld, Qs, qs_ld);
  QX_LAUNCH_STATUS();
}

template <int BM, int BN, int WN, int WM, int ST, bool WARM = false>
int launch128(const void* A, const float* sA, const void* W, const float* sW, void* C, int M,
              int N, int K, int64_t lda, int64_t ldc, int64_t sa_ld, int group_m,
              hipStream_t stream) {
  using Cfg = Cfg128<BM, BN, WN, WM, ST>;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  const int total = tiles_m * tiles_n;
  hipLaunchKernelGGL((gemm_fp8_k128_kernel<BM, BN, WN, WM, ST, WARM>), dim3(total),
                     dim3(Cfg::kThreads), 0, stream, (const uint8_t*)A, sA, (const uint8_t*)W, sW,
                     (uint16_t*)C, M, N, K, lda, ldc, sa_ld, tiles_m, tiles_n,
                     group_m < 1 ? 1 : group_m, nullptr, 0, nullptr, 0);
  QX_LAUNCH_STATUS();
}

// the gate_up GEMM with the SiLU-quant epilogue (N = 2 x intermediate)
int launch128_swiglu(const void* A, const float* sA, const void* W, const float* sW, void* Q,
                     int64_t q_ld, float* Qs, int64_t qs_ld, int M, int N, int K, int64_t lda,
                     int64_t sa_ld, hipStream_t stream) {
  using Cfg = Cfg128<256, 256, 2, 4, 2>;
  const int tiles_m = (M + 255) / 256;
  const int tiles_n = N / 256;
  hipLaunchKernelGGL((gemm_fp8_k128_kernel<256, 256, 2, 4, 2, false, true>),
                     dim3(tiles_m * tiles_n), dim3(Cfg::kThreads), 0, stream, (const uint8_t*)A,
                     sA, (const uint8_t*)W, sW, nullptr, M, N, K, lda, (int64_t)0, sa_ld, tiles_m,
                     tiles_n, 4, (uint8_t*)Q, q_ld, Qs, qs_ld);
  QX_LAUNCH_STATUS();
}

// ---- persistent tiles with the K pipeline running across them ---------------
// Measured on the one-tile-per-workgroup kernel (config 10): a tile's time is
// ~13 us plus 1.77 us per 128-K block (M = 16384, N = 6144, K = 640 .. 10240),
// i.e. at K = 2560 a quarter of it is the pipeline fill and the epilogue,
// which every CU reaches at the same moment (all tiles take equally long),
// so the first-stage loads and the C stores of all CUs arrive in one burst
// while the matrix cores wait. Here one workgroup per CU walks its tiles and
// the next tile's first block is loaded during the current tile's last
// block, so it is in LDS by the time the epilogue ends; the epilogue stages
// the tile through the last block's stage buffer only (two passes of 128
// rows), leaving the prefetched block alone, with LDS-only barriers (no wait
// on the loads in flight). 256 x 256 tiles, 8 waves, two 128-K stages; the
// same arithmetic as config 10 in the same order (bit-identical).
__device__ __forceinline__ void lgkm_barrier() {
  // lgkmcnt(0) with vmcnt and expcnt unconstrained, then the barrier
  __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));
  asm volatile("s_barrier" ::: "memory");
}

template <bool SWIGLU>
__global__ __launch_bounds__(512) void gemm_fp8_k128q_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sA, const uint8_t* __restrict__ W,
    const float* __restrict__ sW, uint16_t* __restrict__ C, int M, int N, int K, int64_t lda,
    int64_t ldc, int64_t sa_ld, int tiles_m, int tiles_n, int group_m, uint8_t* __restrict__ Q,
    int64_t q_ld, float* __restrict__ Qs, int64_t qs_ld) {
  constexpr int BM = 256, BN = 256, WAVES_N = 2, WAVES_M = 4;
  using Cfg = Cfg128<BM, BN, WAVES_N, WAVES_M, 2>;
  constexpr int TN = Cfg::kTN, TM = Cfg::kTM;
  constexpr int kRowBytes = BN * 2 + 16;   // padded staging row (bank spread)
  constexpr int kPassRows = WAVES_M * 32;  // tile rows staged per epilogue pass
  constexpr int kRowsPerWave = kPassRows / Cfg::kWaves;
  static_assert(kPassRows * kRowBytes <= Cfg::kStage, "an epilogue pass fits one stage");
  static_assert(TM * kPassRows == BM, "passes cover the tile");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Cfg::kLds];

  // this workgroup's tiles: a contiguous band of tile ids per XCD (i mod 8),
  // walked with stride (workgroups per XCD); ids map to tiles in groups of
  // group_m token tiles, as in the one-tile-per-workgroup kernels
  const int total = tiles_m * tiles_n;
  const int xcd = blockIdx.x & 7;
  const int per_xcd = gridDim.x >> 3;  // the grid is a multiple of 8
  const int local = blockIdx.x >> 3;
  const int per = (total + 7) / 8;
  const int full = total - (per - 1) * 8;
  const int band0 = xcd < full ? xcd * per : full * per + (xcd - full) * (per - 1);
  const int band = xcd < full ? per : per - 1;
  const int my_tiles = local < band ? (band - local + per_xcd - 1) / per_xcd : 0;
  const int width = group_m * tiles_n;
  auto origin = [&](int iter, int& m0_, int& n0_) {
    const int id = band0 + local + iter * per_xcd;
    const int first_m = (id / width) * group_m;
    const int gsize = min(tiles_m - first_m, group_m);
    m0_ = (first_m + (id % width) % gsize) * BM;
    n0_ = ((id % width) / gsize) * BN;
  };
  const int KT = K >> 7;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave % WAVES_N;
  const int wm = wave / WAVES_N;

  float sw0 = 0.0f, sw1 = 0.0f;  // the weight scale of the block in stage 0 / 1
  // per-lane offsets of the operand rows within a tile, the same for every
  // tile: a block's loads add a wave-uniform base (the one-tile kernel's
  // hoisted addresses); only a token tile past the last row clamps per lane
  int64_t a_off[Cfg::kASlabs], w_off[Cfg::kWSlabs];
  slab_offsets128<Cfg::kASlabs>(lda, wave * Cfg::kASlabs, lane, 0, a_off);
  slab_offsets128<Cfg::kWSlabs>(K, wave * Cfg::kWSlabs, lane, SWIGLU ? (N >> 1) - 128 : 0, w_off);
  auto issue = [&](int m0_, int n0_, int kb, int stage) {
    uint8_t* buf = smem + stage * Cfg::kStage;
    const int64_t k_off = (int64_t)kb * 128;
    const int w_row0 = SWIGLU ? (n0_ >> 1) : n0_;
    if (m0_ + BM <= M) {  // wave-uniform
      load_slab_offsets128<Cfg::kASlabs>(A + (int64_t)m0_ * lda + k_off, a_off, buf,
                                         wave * Cfg::kASlabs);
    } else {
      load_slabs128<Cfg::kASlabs>(A, lda, m0_, M - 1, k_off, buf, wave * Cfg::kASlabs, lane);
    }
    load_slab_offsets128<Cfg::kWSlabs>(W + (int64_t)w_row0 * K + k_off, w_off,
                                       buf + Cfg::kABytes, wave * Cfg::kWSlabs);
    const int t = min(m0_ + wave * Cfg::kSaPerWave + lane % Cfg::kSaPerWave, M - 1);
    __builtin_amdgcn_global_load_lds((const void*)(sA + (int64_t)kb * sa_ld + t),
                                     (lds_void*)(buf + Cfg::kABytes + Cfg::kWBytes + wave * 256),
                                     4, 0, 0);
    const float* sw_row =
        sW + (int64_t)((SWIGLU ? w_row0 + wn * (N >> 1) : n0_ + wn * TN * 32) >> 7) * KT;
    const float sw = __builtin_nontemporal_load(sw_row + kb);
    if (stage) {
      sw1 = sw;
    } else {
      sw0 = sw;
    }
  };

  v16f acc[TN][TM];
  float s_prev[TM];
  int m0 = 0, n0 = 0;
  if (my_tiles > 0) {
    origin(0, m0, n0);
    issue(m0, n0, 0, 0);
  }
  // block kb of a tile sits in stage kb & 1 (K / 128 is even), so the next
  // tile's first block goes into stage 0 while the last one (stage 1) runs
  for (int it = 0; it < my_tiles; ++it) {
    int nm0 = m0, nn0 = n0;
    const bool has_next = it + 1 < my_tiles;
    if (has_next) origin(it + 1, nm0, nn0);
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;
#pragma unroll
    for (int b = 0; b < TM; ++b) s_prev[b] = 0.0f;
    for (int kb0 = 0; kb0 < KT; kb0 += 2) {
#pragma unroll
      for (int stage = 0; stage < 2; ++stage) {
        const int kb = kb0 + stage;
        wait_vmcnt<0>();  // this block's operands (and earlier stores) are done
        lds_barrier();
        // the next block: this tile's, or after its last, the next tile's
        // first (its addresses replace this tile's, all of whose blocks are
        // issued by then)
        if (kb + 1 < KT || has_next) {
          const bool same = kb + 1 < KT;
          issue(same ? m0 : nm0, same ? n0 : nn0, same ? kb + 1 : 0, stage ^ 1);
        }
        const float sw =
            __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(stage ? sw1 : sw0)));
        if (sw != 0.0f) {  // wave-uniform; a zero weight-scale block adds nothing
          const uint8_t* a_lds = smem + stage * Cfg::kStage;
          const uint8_t* w_lds = a_lds + Cfg::kABytes;
          const float* sa_lds = reinterpret_cast<const float*>(w_lds + Cfg::kWBytes);
#pragma unroll
          for (int b = 0; b < TM; ++b) {
            const int row = wm * TM * 32 + b * 32 + (lane & 31);
            const float s_cur =
                sa_lds[(row / Cfg::kSaPerWave) * 64 + row % Cfg::kSaPerWave] * sw;
            const float r = s_prev[b] / s_cur;
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
              for (int e = 0; e < 16; ++e) acc[a][b][e] *= r;
            s_prev[b] = s_cur;
          }
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            v8i wf[TN], af[TM];
#pragma unroll
            for (int a = 0; a < TN; ++a)
              wf[a] = read_frag128(w_lds, wn * TN * 32 + a * 32 + (lane & 31), h, lane);
#pragma unroll
            for (int b = 0; b < TM; ++b)
              af[b] = read_frag128(a_lds, wm * TM * 32 + b * 32 + (lane & 31), h, lane);
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
              for (int b = 0; b < TM; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    wf[a], af[b], acc[a][b], 0, 0, 0, 0, 0, 0);
          }
        }
      }
    }

    // epilogue through stage 1 (the tile's last block), pass b holding rows
    // wm * TM * 32 + b * 32 + (0..31) of every wave
    uint8_t* buf = smem + Cfg::kStage;
    const bool wide = ((ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
#pragma unroll
    for (int b = 0; b < TM; ++b) {
      // b == 0: every wave is done with the last block's operands; b > 0:
      // with the previous pass's rows
      lgkm_barrier();
      {
        const float s = s_prev[b];
        uint8_t* lrow = buf + (wm * 32 + (lane & 31)) * kRowBytes;
#pragma unroll
        for (int a = 0; a < TN; ++a)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int off = (wn * TN * 32 + a * 32 + (lane >> 5) * 4 + g * 8) * 2;
            uint2 v;
            v.x = pack2_bf16(acc[a][b][g * 4 + 0] * s, acc[a][b][g * 4 + 1] * s);
            v.y = pack2_bf16(acc[a][b][g * 4 + 2] * s, acc[a][b][g * 4 + 3] * s);
            *reinterpret_cast<uint2*>(lrow + off) = v;
          }
      }
      lgkm_barrier();
      if constexpr (SWIGLU) {
        // 16 lanes per row: 8 gate and 8 up values each, one quant group
        const int j0 = n0 >> 1;
        const int seg = lane & 15;
#pragma unroll
        for (int i = 0; i < kRowsPerWave / 4; ++i) {
          const int prow = wave * kRowsPerWave + i * 4 + (lane >> 4);
          const int m = m0 + (prow >> 5) * TM * 32 + b * 32 + (prow & 31);
          const uint8_t* lrow = buf + prow * kRowBytes;
          const uint4 g = *reinterpret_cast<const uint4*>(lrow + seg * 16);
          const uint4 u = *reinterpret_cast<const uint4*>(lrow + 256 + seg * 16);
          const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
          float y[8];
          float amax = 0.0f;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            y[2 * k] = silu_mul(lo_bf16(gw[k]), lo_bf16(uw[k]));
            y[2 * k + 1] = silu_mul(hi_bf16(gw[k]), hi_bf16(uw[k]));
          }
#pragma unroll
          for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(y[k]));
          amax = group_max<16>(amax);
          const float scale = fp8_scale(amax);
          const float rs = recip(scale);
          if (m < M) {
            const v2i o = {(int)pack4_fp8(div_by(y[0], scale, rs), div_by(y[1], scale, rs),
                                          div_by(y[2], scale, rs), div_by(y[3], scale, rs)),
                           (int)pack4_fp8(div_by(y[4], scale, rs), div_by(y[5], scale, rs),
                                          div_by(y[6], scale, rs), div_by(y[7], scale, rs))};
            __builtin_nontemporal_store(o, reinterpret_cast<v2i*>(Q + (int64_t)m * q_ld + j0 +
                                                                 seg * 8));
            if (seg == 0) Qs[(int64_t)(j0 >> 7) * qs_ld + m] = scale;
          }
        }
      } else {
        constexpr int kChunks = BN / 8;
        constexpr int kRowsPerOp = 64 / kChunks;
        const int c = lane % kChunks;
#pragma unroll
        for (int i = 0; i < kRowsPerWave / kRowsPerOp; ++i) {
          const int prow = wave * kRowsPerWave + i * kRowsPerOp + lane / kChunks;
          const int m = m0 + (prow >> 5) * TM * 32 + b * 32 + (prow & 31);
          const uint4 v = *reinterpret_cast<const uint4*>(buf + prow * kRowBytes + c * 16);
          if (m < M) {
            uint16_t* dst = C + (int64_t)m * ldc + n0 + c * 8;
            if (wide) {
              const v4i w = {(int)v.x, (int)v.y, (int)v.z, (int)v.w};
              __builtin_nontemporal_store(w, reinterpret_cast<v4i*>(dst));
            } else {
              reinterpret_cast<uint2*>(dst)[0] = make_uint2(v.x, v.y);
              reinterpret_cast<uint2*>(dst)[1] = make_uint2(v.z, v.w);
            }
          }
        }
      }
    }
    m0 = nm0;
    n0 = nn0;
  }
}


// ---- ping-pong variant ------------------------------------------------------
// The 8 waves form two groups, waves 0-3 and 4-7 (one of each per SIMD), that
// run the same code a phase apart: group 1 passes one extra barrier at the
// start (and group 0 one at the end). A 128-K block is four steps, each ended
// by a barrier, one "prepare" and one "compute" step per 64-K half h:
// prepare reads the half's 6 MFMA fragments from LDS into registers (with
// h = 0, also the block's token scales and the rescale factors); compute
// issues the half's 8 MFMAs (with h = 0, each tile's accumulators are
// rescaled just before its first MFMA). So in every phase one wave per SIMD
// feeds the matrix core while the other does its LDS work.
// Phases are numbered from group 0's first step. Every wave loads its share
// of block j + 1 at the start of its step 4j (group 0 in phase 4j, group 1 in
// phase 4j + 1) and waits for it at the end of its step 4j + 2 (phases 4j + 2
// and 4j + 3); the first reader of block j + 1 runs in phase 4j + 4. The
// stage buffer it fills held block j - 1, last read by group 1 in phase
// 4j - 1. (With LOADERS = 4 only group 0 loads, waiting at the end of its
// step 4j + 3, which leaves the loads a phase more.) Per output element the
// operations and their order are those of the other configurations
// (rescale, then the block's MFMAs in K order): the result is bit-identical.
template <int BM, int BN, int LOADERS>
__global__ __launch_bounds__(512) void gemm_fp8_pp_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sA, const uint8_t* __restrict__ W,
    const float* __restrict__ sW, uint16_t* __restrict__ C, int M, int N, int K, int64_t lda,
    int64_t ldc, int64_t sa_ld, int tiles_m, int tiles_n, int group_m) {
  constexpr int WAVES_N = 2, WAVES_M = 4, STAGES = 2;
  using Cfg = Cfg128<BM, BN, WAVES_N, WAVES_M, STAGES>;
  constexpr int TN = Cfg::kTN, TM = Cfg::kTM;
  constexpr int kASlabs = BM / 8 / LOADERS, kWSlabs = BN / 8 / LOADERS;
  constexpr int kSaPerWave = BM / LOADERS;
  static_assert(Cfg::kWaves == 8, "two groups of four waves");
  static_assert(LOADERS == 4 || LOADERS == 8, "group 0 or every wave loads");
  static_assert(kSaPerWave <= 64 && BM % (8 * LOADERS) == 0 && BN % (8 * LOADERS) == 0,
                "loads per wave");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Cfg::kLds];

  const int total = tiles_m * tiles_n;
  int id = blockIdx.x;
  {
    const int per = (total + 7) / 8;
    const int xcd = id & 7, local = id >> 3;
    const int full = total - (per - 1) * 8;
    id = xcd < full ? xcd * per + local : full * per + (xcd - full) * (per - 1) + local;
  }
  const int width = group_m * tiles_n;
  const int first_m = (id / width) * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int m0 = (first_m + (id % width) % gsize) * BM;
  const int n0 = ((id % width) / gsize) * BN;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave % WAVES_N;
  const int wm = wave / WAVES_N;
  const bool loader = wave < LOADERS;
  const bool first_group = wave < 4;
  const int KT = K >> 7;

  v16f acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;
  float s_prev[TM], ratio[TM];
#pragma unroll
  for (int b = 0; b < TM; ++b) s_prev[b] = ratio[b] = 0.0f;
  const float* sw_row = sW + (int64_t)((n0 + wn * TN * 32) >> 7) * KT;
  float sw_stage[STAGES];
  v8i wf[TN], af[TM];
  bool run = false;  // the block being prepared or computed has a nonzero weight scale

  // operands and token scales of block kb (group 0), the weight scale (every wave)
  auto issue = [&](int kb, auto stage_c) __attribute__((always_inline)) {
    constexpr int stage = decltype(stage_c)::value;
    if (loader) {
      uint8_t* buf = smem + stage * Cfg::kStage;
      const int64_t k_off = (int64_t)kb * 128;
      load_slabs128<kASlabs>(A, lda, m0, M - 1, k_off, buf, wave * kASlabs, lane);
      load_slabs128<kWSlabs>(W, K, n0, N - 1, k_off, buf + Cfg::kABytes, wave * kWSlabs, lane);
      const int t = min(m0 + wave * kSaPerWave + lane % kSaPerWave, M - 1);
      __builtin_amdgcn_global_load_lds((const void*)(sA + (int64_t)kb * sa_ld + t),
                                       (lds_void*)(buf + Cfg::kABytes + Cfg::kWBytes + wave * 256),
                                       4, 0, 0);
    }
    sw_stage[stage] = __builtin_nontemporal_load(sw_row + kb);
  };

  // prepare half h of the block in `stage`
  auto prep = [&](auto stage_c, auto h_c) __attribute__((always_inline)) {
    constexpr int stage = decltype(stage_c)::value;
    constexpr int h = decltype(h_c)::value;
    const uint8_t* a_lds = smem + stage * Cfg::kStage;
    const uint8_t* w_lds = a_lds + Cfg::kABytes;
    if (h == 0) {
      const float sw =
          __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sw_stage[stage])));
      run = sw != 0.0f;
      if (run) {
        const float* sa_lds = reinterpret_cast<const float*>(w_lds + Cfg::kWBytes);
#pragma unroll
        for (int b = 0; b < TM; ++b) {
          const int row = wm * TM * 32 + b * 32 + (lane & 31);
          const float s_cur = sa_lds[(row / kSaPerWave) * 64 + row % kSaPerWave] * sw;
          ratio[b] = s_prev[b] / s_cur;
          s_prev[b] = s_cur;
        }
      }
    }
    if (run) {
#pragma unroll
      for (int a = 0; a < TN; ++a)
        wf[a] = read_frag128(w_lds, wn * TN * 32 + a * 32 + (lane & 31), h, lane);
#pragma unroll
      for (int b = 0; b < TM; ++b)
        af[b] = read_frag128(a_lds, wm * TM * 32 + b * 32 + (lane & 31), h, lane);
    }
    // the stage is refilled a few phases on; its reads must be done by then
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  };

  auto compute = [&](auto h_c) __attribute__((always_inline)) {
    constexpr int h = decltype(h_c)::value;
    if (run) {
#pragma unroll
      for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b) {
          if (h == 0) {
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[a][b][e] *= ratio[b];
          }
          acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[a], af[b], acc[a][b], 0,
                                                                     0, 0, 0, 0, 0);
        }
      if (h == 0) {
        // each tile's 16 multiplies, then its MFMA: the next tile's
        // multiplies issue while the MFMA runs
#pragma unroll
        for (int i = 0; i < TN * TM; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);  // VALU
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        }
      }
    }
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  auto block = [&](int j, auto stage_c) __attribute__((always_inline)) {
    constexpr int stage = decltype(stage_c)::value;
    if (j + 1 < KT) issue(j + 1, std::integral_constant<int, stage ^ 1>());
    prep(stage_c, I0());
    lds_barrier();
    compute(I0());
    lds_barrier();
    prep(stage_c, I1());
    if (LOADERS == 8) wait_vmcnt<0>();
    lds_barrier();
    compute(I1());
    if (LOADERS == 4) wait_vmcnt<0>();
    lds_barrier();
  };

  issue(0, I0());
  wait_vmcnt<0>();
  lds_barrier();
  if (!first_group) lds_barrier();  // group 1 runs one phase behind
  for (int j = 0; j < KT; j += 2) {
    block(j, I0());
    if (j + 1 < KT) block(j + 1, I1());
  }
  if (first_group) lds_barrier();

  // epilogue, as in gemm_fp8_k128_kernel: the tile staged in LDS (padded
  // rows), then whole rows stored, non-temporal
  constexpr int kRowBytes = BN * 2 + 16;
  constexpr int kChunks = BN / 8;
  static_assert(BM * kRowBytes <= Cfg::kLds, "epilogue tile fits the stage buffers");
  static_assert(64 % kChunks == 0 && (BM / Cfg::kWaves) % (64 / kChunks) == 0, "epilogue rows");
  __syncthreads();
#pragma unroll
  for (int b = 0; b < TM; ++b) {
    const int row = wm * TM * 32 + b * 32 + (lane & 31);
    const float s = s_prev[b];
    uint8_t* lrow = smem + row * kRowBytes;
#pragma unroll
    for (int a = 0; a < TN; ++a) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int off = (wn * TN * 32 + a * 32 + (lane >> 5) * 4 + g * 8) * 2;
        uint2 v;
        v.x = pack2_bf16(acc[a][b][g * 4 + 0] * s, acc[a][b][g * 4 + 1] * s);
        v.y = pack2_bf16(acc[a][b][g * 4 + 2] * s, acc[a][b][g * 4 + 3] * s);
        *reinterpret_cast<uint2*>(lrow + off) = v;
      }
    }
  }
  __syncthreads();
  constexpr int kRowsPerOp = 64 / kChunks;
  constexpr int kRowsPerWave = BM / Cfg::kWaves;
  const bool wide = ((ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  const int c = lane % kChunks;
#pragma unroll
  for (int i = 0; i < kRowsPerWave / kRowsPerOp; ++i) {
    const int row = wave * kRowsPerWave + i * kRowsPerOp + lane / kChunks;
    const int m = m0 + row;
    const uint4 v = *reinterpret_cast<const uint4*>(smem + row * kRowBytes + c * 16);
    if (m < M) {
      uint16_t* dst = C + (int64_t)m * ldc + n0 + c * 8;
      if (wide) {
        const v4i w = {(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        __builtin_nontemporal_store(w, reinterpret_cast<v4i*>(dst));
      } else {
        reinterpret_cast<uint2*>(dst)[0] = make_uint2(v.x, v.y);
        reinterpret_cast<uint2*>(dst)[1] = make_uint2(v.z, v.w);
      }
    }
  }
}

template <int BM, int BN, int LOADERS>
int launch_pp(const void* A, const float* sA, const void* W, const float* sW, void* C, int M,
              int N, int K, int64_t lda, int64_t ldc, int64_t sa_ld, int group_m,
              hipStream_t stream) {
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  hipLaunchKernelGGL((gemm_fp8_pp_kernel<BM, BN, LOADERS>), dim3(tiles_m * tiles_n), dim3(512), 0,
                     stream,
                     (const uint8_t*)A, sA, (const uint8_t*)W, sW, (uint16_t*)C, M, N, K, lda,
                     ldc, sa_ld, tiles_m, tiles_n, group_m < 1 ? 1 : group_m);
  QX_LAUNCH_STATUS();
}

// ---- ping-pong variant over 64-K stages ---------------------------------------
// As gemm_fp8_pp_kernel, but the LDS ring holds four 64-K half-blocks (each
// with its block's token scales), so loads run three half-blocks ahead
// (96 KiB in flight per CU instead of 64). Steps per half-block q: prepare q
// (issue the loads of q + 3, read q's 6 fragments; for an even q also the
// block's scales and rescale factors), then compute q. Phases are numbered
// from group 0's first step (group 1 runs one phase behind):
//   * q + 3 loads into slot (q + 3) % 4 at the start of group 0's phase 2q
//     (group 1: 2q + 1); that slot held q - 1, last read by group 1's
//     prepare in phase 2q - 1;
//   * every wave waits for its loads of q + 1 at the end of its prepare step
//     of q (phases 2q and 2q + 1); q + 1 is first read in phase 2q + 2.
template <int BM, int BN>
__global__ __launch_bounds__(512) void gemm_fp8_pp64_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sA, const uint8_t* __restrict__ W,
    const float* __restrict__ sW, uint16_t* __restrict__ C, int M, int N, int K, int64_t lda,
    int64_t ldc, int64_t sa_ld, int tiles_m, int tiles_n, int group_m) {
  constexpr int WAVES_N = 2, WAVES_M = 4, kWaves = 8, RING = 4, AHEAD = 3;
  constexpr int TN = BN / WAVES_N / 32, TM = BM / WAVES_M / 32;
  constexpr int kABytes = BM * 64, kWBytes = BN * 64, kSaBytes = 256 * kWaves;
  constexpr int kStage = kABytes + kWBytes + kSaBytes;
  constexpr int kLds = RING * kStage;
  constexpr int kASlabs = BM / 16 / kWaves, kWSlabs = BN / 16 / kWaves;
  constexpr int kSaPerWave = BM / kWaves;
  constexpr int kOps = kASlabs + kWSlabs + 1;  // vector loads per wave per half-block
  static_assert(TN >= 1 && TM >= 1 && BM % (16 * kWaves) == 0 && BN % (16 * kWaves) == 0,
                "slabs");
  static_assert(BN / WAVES_N == 128, "a wave's weight rows are one 128-row scale block");
  static_assert(kSaPerWave <= 64, "token scales");
  static_assert(kLds <= 160 * 1024, "LDS");
  static_assert((AHEAD - 1) * kOps < 64 && AHEAD <= RING - 1, "vmcnt, ring");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kLds];

  const int total = tiles_m * tiles_n;
  int id = blockIdx.x;
  {
    const int per = (total + 7) / 8;
    const int xcd = id & 7, local = id >> 3;
    const int full = total - (per - 1) * 8;
    id = xcd < full ? xcd * per + local : full * per + (xcd - full) * (per - 1) + local;
  }
  const int width = group_m * tiles_n;
  const int first_m = (id / width) * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int m0 = (first_m + (id % width) % gsize) * BM;
  const int n0 = ((id % width) / gsize) * BN;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave % WAVES_N;
  const int wm = wave / WAVES_N;
  const bool first_group = wave < 4;
  const int Q = K >> 6;  // half-blocks

  v16f acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;
  float s_prev[TM], ratio[TM];
#pragma unroll
  for (int b = 0; b < TM; ++b) s_prev[b] = ratio[b] = 0.0f;
  const float* sw_row = sW + (int64_t)((n0 + wn * TN * 32) >> 7) * (K >> 7);
  float sw_ring[2];  // weight scale of the blocks, by block parity
  v8i wf[TN], af[TM];
  bool run = false;

  auto issue = [&](int q, auto slot_c) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    uint8_t* buf = smem + slot * kStage;
    const int kb = q >> 1;
    const int64_t k_off = (int64_t)q * 64;
    load_slabs<kASlabs>(A, lda, m0, M - 1, k_off, buf, wave * kASlabs, lane);
    load_slabs<kWSlabs>(W, K, n0, N - 1, k_off, buf + kABytes, wave * kWSlabs, lane);
    const int t = min(m0 + wave * kSaPerWave + lane % kSaPerWave, M - 1);
    __builtin_amdgcn_global_load_lds((const void*)(sA + (int64_t)kb * sa_ld + t),
                                     (lds_void*)(buf + kABytes + kWBytes + wave * 256), 4, 0, 0);
    // slot parity is the half-block's parity: even slots start a block
    if ((slot & 1) == 0) sw_ring[(slot >> 1) & 1] = __builtin_nontemporal_load(sw_row + kb);
  };

  auto prep = [&](auto slot_c) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    const uint8_t* a_lds = smem + slot * kStage;
    const uint8_t* w_lds = a_lds + kABytes;
    if ((slot & 1) == 0) {
      const float sw = __int_as_float(
          __builtin_amdgcn_readfirstlane(__float_as_int(sw_ring[(slot >> 1) & 1])));
      run = sw != 0.0f;
      if (run) {
        const float* sa_lds = reinterpret_cast<const float*>(w_lds + kWBytes);
#pragma unroll
        for (int b = 0; b < TM; ++b) {
          const int row = wm * TM * 32 + b * 32 + (lane & 31);
          const float s_cur = sa_lds[(row / kSaPerWave) * 64 + row % kSaPerWave] * sw;
          ratio[b] = s_prev[b] / s_cur;
          s_prev[b] = s_cur;
        }
      }
    }
    if (run) {
#pragma unroll
      for (int a = 0; a < TN; ++a) wf[a] = read_frag(w_lds, wn * TN * 32 + a * 32 + (lane & 31), lane);
#pragma unroll
      for (int b = 0; b < TM; ++b) af[b] = read_frag(a_lds, wm * TM * 32 + b * 32 + (lane & 31), lane);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  };

  auto compute = [&](auto h_c) __attribute__((always_inline)) {
    constexpr int h = decltype(h_c)::value;
    if (run) {
#pragma unroll
      for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b) {
          if (h == 0) {
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[a][b][e] *= ratio[b];
          }
          acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[a], af[b], acc[a][b], 0,
                                                                     0, 0, 0, 0, 0);
        }
      if (h == 0) {
#pragma unroll
        for (int i = 0; i < TN * TM; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);  // VALU
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        }
      }
    }
  };

  auto half_block = [&](int q, auto slot_c) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    const bool more = q + AHEAD < Q;
    if (more) issue(q + AHEAD, std::integral_constant<int, (slot + AHEAD) % RING>());
    prep(slot_c);
    if (more) {
      wait_vmcnt<(AHEAD - 1) * kOps>();  // q + 1 has landed
    } else {
      wait_vmcnt<0>();
    }
    lds_barrier();
    compute(std::integral_constant<int, slot & 1>());
    lds_barrier();
  };

  using std::integral_constant;
#pragma unroll
  for (int q = 0; q < AHEAD; ++q) {
    if (q < Q) {
      if (q == 0) issue(0, integral_constant<int, 0>());
      if (q == 1) issue(1, integral_constant<int, 1>());
      if (q == 2) issue(2, integral_constant<int, 2>());
    }
  }
  if (Q >= AHEAD) {
    wait_vmcnt<(AHEAD - 1) * kOps>();
  } else {
    wait_vmcnt<0>();
  }
  lds_barrier();
  if (!first_group) lds_barrier();  // group 1 runs one phase behind
  for (int q = 0; q < Q; q += RING) {
    half_block(q, integral_constant<int, 0>());
    half_block(q + 1, integral_constant<int, 1>());  // Q is even
    if (q + 2 < Q) {
      half_block(q + 2, integral_constant<int, 2>());
      half_block(q + 3, integral_constant<int, 3>());
    }
  }
  if (first_group) lds_barrier();

  // epilogue as in gemm_fp8_k128_kernel
  constexpr int kRowBytes = BN * 2 + 16;
  constexpr int kChunks = BN / 8;
  static_assert(BM * kRowBytes <= kLds, "epilogue tile fits the ring");
  static_assert(64 % kChunks == 0 && (BM / kWaves) % (64 / kChunks) == 0, "epilogue rows");
  __syncthreads();
#pragma unroll
  for (int b = 0; b < TM; ++b) {
    const int row = wm * TM * 32 + b * 32 + (lane & 31);
    const float s = s_prev[b];
    uint8_t* lrow = smem + row * kRowBytes;
#pragma unroll
    for (int a = 0; a < TN; ++a) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int off = (wn * TN * 32 + a * 32 + (lane >> 5) * 4 + g * 8) * 2;
        uint2 v;
        v.x = pack2_bf16(acc[a][b][g * 4 + 0] * s, acc[a][b][g * 4 + 1] * s);
        v.y = pack2_bf16(acc[a][b][g * 4 + 2] * s, acc[a][b][g * 4 + 3] * s);
        *reinterpret_cast<uint2*>(lrow + off) = v;
      }
    }
  }
  __syncthreads();
  constexpr int kRowsPerOp = 64 / kChunks;
  constexpr int kRowsPerWave = BM / kWaves;
  const bool wide = ((ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  const int c = lane % kChunks;
#pragma unroll
  for (int i = 0; i < kRowsPerWave / kRowsPerOp; ++i) {
    const int row = wave * kRowsPerWave + i * kRowsPerOp + lane / kChunks;
    const int m = m0 + row;
    const uint4 v = *reinterpret_cast<const uint4*>(smem + row * kRowBytes + c * 16);
    if (m < M) {
      uint16_t* dst = C + (int64_t)m * ldc + n0 + c * 8;
      if (wide) {
        const v4i w = {(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        __builtin_nontemporal_store(w, reinterpret_cast<v4i*>(dst));
      } else {
        reinterpret_cast<uint2*>(dst)[0] = make_uint2(v.x, v.y);
        reinterpret_cast<uint2*>(dst)[1] = make_uint2(v.z, v.w);
      }
    }
  }
}

template <int BM, int BN>
int launch_pp64(const void* A, const float* sA, const void* W, const float* sW, void* C, int M,
                int N, int K, int64_t lda, int64_t ldc, int64_t sa_ld, int group_m,
                hipStream_t stream) {
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  hipLaunchKernelGGL((gemm_fp8_pp64_kernel<BM, BN>), dim3(tiles_m * tiles_n), dim3(512), 0,
                     stream, (const uint8_t*)A, sA, (const uint8_t*)W, sW, (uint16_t*)C, M, N, K,
                     lda, ldc, sa_ld, tiles_m, tiles_n, group_m < 1 ? 1 : group_m);
  QX_LAUNCH_STATUS();
}

// ---- persistent variant -----------------------------------------------------
// One workgroup per CU walks its XCD's band of tiles (the same bands and
// group_m order as the one-tile-per-workgroup kernel). The pipeline runs over
// the flattened (tile, 128-K block) sequence, so the next tile's first block
// loads into the free stage while the current tile's last block computes and
// its epilogue stores, where a fresh workgroup would start with an empty
// pipeline. The epilogue stages C through the stage buffer it has just
// consumed (its token scales included: they are read before the MFMAs), in
// TM passes of WAVES_M * 32 rows. Each output element sums the
// same products in the same order as the other configurations.
template <int BM, int BN, int WAVES_N, int WAVES_M>
__global__ __launch_bounds__(64 * WAVES_N * WAVES_M) void gemm_fp8_k128p_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sA, const uint8_t* __restrict__ W,
    const float* __restrict__ sW, uint16_t* __restrict__ C, int M, int N, int K, int64_t lda,
    int64_t ldc, int64_t sa_ld, int tiles_m, int tiles_n, int group_m) {
  constexpr int STAGES = 2;
  using Cfg = Cfg128<BM, BN, WAVES_N, WAVES_M, STAGES>;
  constexpr int TN = Cfg::kTN, TM = Cfg::kTM;
  constexpr int kRowBytes = BN * 2 + 16;  // padded: the 32 rows of one write spread over the banks
  constexpr int kChunks = BN / 8;
  constexpr int kPassRows = WAVES_M * 32;
  constexpr int kRowsPerOp = 64 / kChunks;
  constexpr int kRowsPerWave = kPassRows / Cfg::kWaves;
  static_assert(kPassRows * kRowBytes <= Cfg::kStage, "epilogue pass fits a stage");
  static_assert(64 % kChunks == 0 && kPassRows % Cfg::kWaves == 0 &&
                    kRowsPerWave % kRowsPerOp == 0,
                "epilogue rows");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Cfg::kLds];

  const int total = tiles_m * tiles_n;
  const int xcd = blockIdx.x & 7;
  const int per_xcd = gridDim.x >> 3;  // the grid is a multiple of 8
  const int local = blockIdx.x >> 3;
  const int per = (total + 7) / 8;
  const int full = total - (per - 1) * 8;
  const int band0 = xcd < full ? xcd * per : full * per + (xcd - full) * (per - 1);
  const int band = xcd < full ? per : per - 1;
  const int my_tiles = local < band ? (band - local + per_xcd - 1) / per_xcd : 0;
  const int KT = K >> 7;
  const int steps = my_tiles * KT;
  const int width = group_m * tiles_n;
  auto origin = [&](int iter, int& m0_, int& n0_) {
    const int id = band0 + local + iter * per_xcd;
    const int first_m = (id / width) * group_m;
    const int gsize = min(tiles_m - first_m, group_m);
    m0_ = (first_m + (id % width) % gsize) * BM;
    n0_ = ((id % width) / gsize) * BN;
  };

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave % WAVES_N;
  const int wm = wave / WAVES_N;

  v16f acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;
  float s_prev[TM];
#pragma unroll
  for (int b = 0; b < TM; ++b) s_prev[b] = 0.0f;
  float sw_ring[STAGES];

  auto issue = [&](int m0_, int n0_, int kb, int stage) {
    uint8_t* buf = smem + stage * Cfg::kStage;
    const int64_t k_off = (int64_t)kb * 128;
    load_slabs128<Cfg::kASlabs>(A, lda, m0_, M - 1, k_off, buf, wave * Cfg::kASlabs, lane);
    load_slabs128<Cfg::kWSlabs>(W, K, n0_, N - 1, k_off, buf + Cfg::kABytes, wave * Cfg::kWSlabs,
                                lane);
    const int t = min(m0_ + wave * Cfg::kSaPerWave + lane % Cfg::kSaPerWave, M - 1);
    __builtin_amdgcn_global_load_lds((const void*)(sA + (int64_t)kb * sa_ld + t),
                                     (lds_void*)(buf + Cfg::kABytes + Cfg::kWBytes + wave * 256),
                                     4, 0, 0);
    sw_ring[stage] =
        __builtin_nontemporal_load(sW + (int64_t)((n0_ + wn * TN * 32) >> 7) * KT + kb);
  };

  auto epilogue = [&](int m0_, int n0_, int stage) {
    uint8_t* buf = smem + stage * Cfg::kStage;
    const bool wide = ((ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
    const int c = lane % kChunks;
#pragma unroll
    for (int b = 0; b < TM; ++b) {
      // b == 0: every wave is done with this stage's operands; b > 0: with
      // the previous pass's rows
      __syncthreads();
      {
        const int prow = wm * 32 + (lane & 31);
        const float s = s_prev[b];
        uint8_t* lrow = buf + prow * kRowBytes;
#pragma unroll
        for (int a = 0; a < TN; ++a) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int off = (wn * TN * 32 + a * 32 + (lane >> 5) * 4 + g * 8) * 2;
            uint2 v;
            v.x = pack2_bf16(acc[a][b][g * 4 + 0] * s, acc[a][b][g * 4 + 1] * s);
            v.y = pack2_bf16(acc[a][b][g * 4 + 2] * s, acc[a][b][g * 4 + 3] * s);
            *reinterpret_cast<uint2*>(lrow + off) = v;
          }
        }
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kRowsPerWave / kRowsPerOp; ++i) {
        const int prow = wave * kRowsPerWave + i * kRowsPerOp + lane / kChunks;
        const int m = m0_ + (prow >> 5) * TM * 32 + b * 32 + (prow & 31);
        const uint4 v = *reinterpret_cast<const uint4*>(buf + prow * kRowBytes + c * 16);
        if (m < M) {
          uint16_t* dst = C + (int64_t)m * ldc + n0_ + c * 8;
          if (wide) {
            const v4i w = {(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            __builtin_nontemporal_store(w, reinterpret_cast<v4i*>(dst));
          } else {
            reinterpret_cast<uint2*>(dst)[0] = make_uint2(v.x, v.y);
            reinterpret_cast<uint2*>(dst)[1] = make_uint2(v.z, v.w);
          }
        }
      }
    }
  };

  // the step being loaded (l_*) runs one ahead of the step being computed (c_*)
  int l_iter = 0, l_kb = 0, lm0 = 0, ln0 = 0;
  int c_iter = 0, c_kb = 0, cm0 = 0, cn0 = 0;
  if (steps > 0) {
    origin(0, lm0, ln0);
    cm0 = lm0;
    cn0 = ln0;
    issue(lm0, ln0, 0, 0);
    if (++l_kb == KT) {
      l_kb = 0;
      if (++l_iter < my_tiles) origin(l_iter, lm0, ln0);
    }
  }
  for (int s0 = 0; s0 < steps; s0 += STAGES) {
#pragma unroll
    for (int stage = 0; stage < STAGES; ++stage) {
      if (s0 + stage < steps) {
        wait_vmcnt<0>();  // this step's operands (and any earlier stores) are done
        lds_barrier();
        if (s0 + stage + 1 < steps) {
          issue(lm0, ln0, l_kb, stage ^ 1);
          if (++l_kb == KT) {
            l_kb = 0;
            if (++l_iter < my_tiles) origin(l_iter, lm0, ln0);
          }
        }
        const float sw =
            __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sw_ring[stage])));
        if (sw != 0.0f) {  // wave-uniform; a zero weight-scale block adds nothing
          const float* sa_lds = reinterpret_cast<const float*>(smem + stage * Cfg::kStage +
                                                               Cfg::kABytes + Cfg::kWBytes);
#pragma unroll
          for (int b = 0; b < TM; ++b) {
            const int row = wm * TM * 32 + b * 32 + (lane & 31);
            const float s_cur = sa_lds[(row / Cfg::kSaPerWave) * 64 + row % Cfg::kSaPerWave] * sw;
            const float r = s_prev[b] / s_cur;
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
              for (int e = 0; e < 16; ++e) acc[a][b][e] *= r;
            s_prev[b] = s_cur;
          }
          const uint8_t* a_lds = smem + stage * Cfg::kStage;
          const uint8_t* w_lds = a_lds + Cfg::kABytes;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            v8i wf[TN], af[TM];
#pragma unroll
            for (int a = 0; a < TN; ++a)
              wf[a] = read_frag128(w_lds, wn * TN * 32 + a * 32 + (lane & 31), h, lane);
#pragma unroll
            for (int b = 0; b < TM; ++b)
              af[b] = read_frag128(a_lds, wm * TM * 32 + b * 32 + (lane & 31), h, lane);
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
              for (int b = 0; b < TM; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    wf[a], af[b], acc[a][b], 0, 0, 0, 0, 0, 0);
          }
        }
        if (++c_kb == KT) {
          epilogue(cm0, cn0, stage);
          c_kb = 0;
          if (++c_iter < my_tiles) origin(c_iter, cm0, cn0);
#pragma unroll
          for (int b = 0; b < TM; ++b) {
            s_prev[b] = 0.0f;
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
              for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;
          }
        }
      }
    }
  }
}

// Workgroups of the persistent kernel: one per CU, a multiple of 8 (one
// band per XCD); the CU count is read once per device.
inline int persistent_grid(int total) {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n;
  }
  return (total < cus[dev] ? total : cus[dev]) & ~7;
}

// the persistent kernel with the cross-tile pipeline (config 22; the SwiGLU
// epilogue with Q != nullptr); too few tiles to share out, or an odd number
// of 128-K blocks, fall back to one workgroup per tile
template <bool SWIGLU>
int launch128q(const void* A, const float* sA, const void* W, const float* sW, void* C, int M,
               int N, int K, int64_t lda, int64_t ldc, int64_t sa_ld, void* Q, int64_t q_ld,
               float* Qs, int64_t qs_ld, hipStream_t stream) {
  const int tiles_m = (M + 255) / 256;
  const int tiles_n = N / 256;
  const int grid = persistent_grid(tiles_m * tiles_n);
  if (grid < 8 || (K / 128) % 2) {  // the stage of a block is its parity within the tile
    if (SWIGLU)
      return launch128_swiglu(A, sA, W, sW, Q, q_ld, Qs, qs_ld, M, N, K, lda, sa_ld, stream);
    return launch128<256, 256, 2, 4, 2>(A, sA, W, sW, C, M, N, K, lda, ldc, sa_ld, 4, stream);
  }
  hipLaunchKernelGGL((gemm_fp8_k128q_kernel<SWIGLU>), dim3(grid), dim3(512), 0, stream,
                     (const uint8_t*)A, sA, (const uint8_t*)W, sW, (uint16_t*)C, M, N, K, lda,
                     ldc, sa_ld, tiles_m, tiles_n, 4, (uint8_t*)Q, q_ld, Qs, qs_ld);
  QX_LAUNCH_STATUS();
}

template <int BM, int BN, int WN, int WM>
int launch128p(const void* A, const float* sA, const void* W, const float* sW, void* C, int M,
               int N, int K, int64_t lda, int64_t ldc, int64_t sa_ld, int group_m,
               hipStream_t stream) {
  using Cfg = Cfg128<BM, BN, WN, WM, 2>;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  const int grid = persistent_grid(tiles_m * tiles_n);
  if (grid < 8)  // too few tiles to share out: one workgroup per tile
    return launch128<BM, BN, WN, WM, 2>(A, sA, W, sW, C, M, N, K, lda, ldc, sa_ld, group_m,
                                        stream);
  hipLaunchKernelGGL((gemm_fp8_k128p_kernel<BM, BN, WN, WM>), dim3(grid), dim3(Cfg::kThreads), 0,
                     stream, (const uint8_t*)A, sA, (const uint8_t*)W, sW, (uint16_t*)C, M, N, K,
                     lda, ldc, sa_ld, tiles_m, tiles_n, group_m < 1 ? 1 : group_m);
  QX_LAUNCH_STATUS();
}

template <int BM, int BN, int WN, int WM, int ST>
int launch(const void* A, const float* sA, const void* W, const float* sW, void* C, int M, int N,
           int K, int64_t lda, int64_t ldc, int64_t sa_ld, int group_m, hipStream_t stream) {
  using Cfg = GemmCfg<BM, BN, WN, WM, ST>;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  const int total = tiles_m * tiles_n;
  hipLaunchKernelGGL((gemm_fp8_bs_kernel<BM, BN, WN, WM, ST>), dim3(total), dim3(Cfg::kThreads), 0,
                     stream, (const uint8_t*)A, sA, (const uint8_t*)W, sW, (uint16_t*)C, M, N, K,
                     lda, ldc, sa_ld, tiles_m, tiles_n, group_m < 1 ? 1 : group_m);
  QX_LAUNCH_STATUS();
}

}  // namespace
}  // namespace qx

extern "C" {

// Tile configurations (tokens x weights); every one gives the same result,
// bit for bit. 64-K stages: 0: 256x256, 8 waves, 4 stages; 1: 256x256, 4
// waves, 4; 2: 128x128, 4 waves, 4; 3: 128x256, 4 waves, 3; 4: 256x128, 4
// waves, 3; 5: 256x128, 4 waves, 2; 6: 256x128, 4 waves, 4; 7-9: the same
// with the next slice's fragments read during the current MFMAs. 128-K
// stages (one scale block each): 10: 256x256, 8 waves (the default); 11:
// 256x128, 4 waves; 12: 128x128; 13: 10 with L2 warming; 14, 15: 128x256;
// 16, 17: persistent 256x256 / 256x128; 18, 19: 256x256 ping-pong (group 0
// loads / every wave loads); 20: ping-pong over four 64-K stages; 21: 10
// with the rescale staggered away from the MFMAs.
// gate_up projection + SiLU-gated product + per-128 FP8 quant in one launch:
// W / sW are the gate_up weight (2I x K, rows [gate | up]) and its scales;
// I = intermediate width.
int qx_gemm_fp8_swiglu_quant(const void* A, const float* sA, const void* W, const float* sW,
                             void* Q, int64_t q_ld, float* Qs, int64_t qs_ld, int64_t M,
                             int64_t I, int64_t K, int64_t lda, int64_t sa_ld, int config,
                             hipStream_t stream) {
  QX_CHECK(A && sA && W && sW && Q && Qs, "gemm_swiglu: null pointer");
  QX_CHECK(M >= 0 && I > 0 && K > 0, "gemm_swiglu: bad shape M=%lld I=%lld K=%lld",
           (long long)M, (long long)I, (long long)K);
  QX_CHECK(K % 128 == 0 && I % 128 == 0, "gemm_swiglu: K=%lld, I=%lld not multiples of 128",
           (long long)K, (long long)I);
  QX_CHECK(lda >= K && lda % 16 == 0, "gemm_swiglu: lda=%lld", (long long)lda);
  QX_CHECK(q_ld >= I && q_ld % 8 == 0 && ((uintptr_t)Q & 7) == 0, "gemm_swiglu: q_ld=%lld",
           (long long)q_ld);
  QX_CHECK(qs_ld >= M && sa_ld >= M, "gemm_swiglu: scale strides");
  QX_CHECK(M < (1LL << 31) && 2 * I < (1LL << 31) && K < (1LL << 31), "gemm_swiglu: dims");
  QX_CHECK(((uintptr_t)A & 15) == 0 && ((uintptr_t)W & 15) == 0, "gemm_swiglu: alignment");
  QX_CHECK(config == 10 || config == 22, "gemm_swiglu: config %d (10 or 22)", config);
  if (M == 0) return QX_OK;
  if (config == 22)
    return qx::launch128q<true>(A, sA, W, sW, nullptr, (int)M, (int)(2 * I), (int)K, lda, 0,
                                sa_ld, Q, q_ld, Qs, qs_ld, stream);
  return qx::launch128_swiglu(A, sA, W, sW, Q, q_ld, Qs, qs_ld, (int)M, (int)(2 * I), (int)K, lda,
                              sa_ld, stream);
}

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
      return qx::launch<256, 256, 2, 4, 4>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 4, stream);
    case 1:
      QX_CHECK(n % 256 == 0, "gemm config 1 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch<256, 256, 2, 2, 4>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 4, stream);
    case 2:
      return qx::launch<128, 128, 2, 2, 4>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8, stream);
    case 3:
      QX_CHECK(n % 256 == 0, "gemm config 3 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch<128, 256, 2, 2, 3>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8, stream);
    case 4:
      return qx::launch<256, 128, 1, 4, 3>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8, stream);
    case 5:
      return qx::launch<256, 128, 1, 4, 2>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8, stream);
    case 6:
      return qx::launch<256, 128, 1, 4, 4>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8, stream);
    case 7:
      QX_CHECK(n % 256 == 0, "gemm config 7 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch_plr<256, 256, 2, 4, 4>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 4,
                                               stream);
    case 8:
      return qx::launch_plr<256, 128, 1, 4, 3>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8,
                                               stream);
    case 9:
      return qx::launch_plr<128, 128, 2, 2, 4>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8,
                                               stream);
    case 10:
      QX_CHECK(n % 256 == 0, "gemm config 10 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch128<256, 256, 2, 4, 2>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 4,
                                              stream);
    case 11:
      return qx::launch128<256, 128, 1, 4, 2>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8,
                                              stream);
    case 12:
      return qx::launch128<128, 128, 2, 2, 2>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8,
                                              stream);
    case 14:
      QX_CHECK(n % 256 == 0, "gemm config 14 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch128<128, 256, 2, 4, 2>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8,
                                              stream);
    case 15:
      QX_CHECK(n % 256 == 0, "gemm config 15 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch128<128, 256, 4, 2, 2>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8,
                                              stream);
    case 13:
      QX_CHECK(n % 256 == 0, "gemm config 13 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch128<256, 256, 2, 4, 2, true>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld,
                                                    4, stream);
    case 16:
      QX_CHECK(n % 256 == 0, "gemm config 16 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch128p<256, 256, 2, 4>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 4, stream);
    case 17:
      return qx::launch128p<256, 128, 1, 4>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8, stream);
    case 18:
      QX_CHECK(n % 256 == 0, "gemm config 18 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch_pp<256, 256, 4>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 4, stream);
    case 19:
      QX_CHECK(n % 256 == 0, "gemm config 19 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch_pp<256, 256, 8>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 4, stream);
    case 21:
      QX_CHECK(n % 256 == 0, "gemm config 21 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch128s<false>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, nullptr, 0, nullptr,
                                   0, stream);
    case 20:
      QX_CHECK(n % 256 == 0, "gemm config 20 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch_pp64<256, 256>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 4, stream);
    case 22:
      QX_CHECK(n % 256 == 0, "gemm config 22 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch128q<false>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, nullptr, 0,
                                   nullptr, 0, stream);
    default:
      QX_CHECK(false, "gemm: unknown config %d", config);
  }
}

}  // extern "C"
