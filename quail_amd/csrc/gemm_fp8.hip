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
//   * the MFMA "A" operand is the weight tile and "B" the token tile, so an
//     output tile holds one token per lane column: the token scale is one
//     value per lane per tile and the weight scale one value per wave;
//   * the scales change every 128 of K. Two arithmetic families compute
//     sum_kb s_kb P_kb (s = sA * sW, P_kb the block's FP8 products):
//       - rescale (configs 10, 11, 12, 22; v_mfma_scale_f32_32x32x64_f8f6f4
//         with unit scales): the accumulator is kept in units of the
//         current block's scale; entering block kb it is multiplied by
//         s_(kb-1) / s_kb and the MFMAs accumulate the raw products into it;
//         the epilogue multiplies by the last block's scale. No temporaries;
//       - promotion (configs 30 and 31, 256 x 256 and 256 x 320 tiles;
//         v_mfma_scale_f32_16x16x128_f8f6f4 with unit scales): each
//         block's products are summed from zero by one MFMA per 16 x 16
//         tile and promoted into an fp32 total on the VALU,
//         total += s_kb * P_kb;
//   * operand tiles go HBM -> LDS with global_load_lds_dwordx4 (no VGPR
//     staging), one 128-K scale block per pipeline stage (two stages), so
//     the next block's loads are in flight while one is consumed. A stage
//     row is 128 B (8 chunks of 16 B), chunk-swizzled so that the rows one
//     ds_read_b128 phase touches cover all 64 LDS banks: by ((row >> 1) & 7)
//     for the 32x32 fragments, by (row & 7) for the 16x16 ones;
//   * workgroups are remapped so each XCD (8 per MI355X, each with its own
//     L2) runs a contiguous band of tiles that share operands.
#include <type_traits>

#include "qx_common.h"
#include "qx_status.h"

namespace qx {
namespace {

typedef __attribute__((address_space(3))) void lds_void;


// Cache policy of the operand loads into LDS: device scope (sc1). The
// vector L1 keeps no copy of these streamed rows (every workgroup reads its
// operands once), which measured 10% faster on the widest Qwen3 projection
// than the default policy and no slower elsewhere.
constexpr int kOperandLoadPolicy = 16;

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
        const v2i o = {(int)pack4_fp8(silu_quot(y[0], rs), silu_quot(y[1], rs),
                                      silu_quot(y[2], rs), silu_quot(y[3], rs)),
                       (int)pack4_fp8(silu_quot(y[4], rs), silu_quot(y[5], rs),
                                      silu_quot(y[6], rs), silu_quot(y[7], rs))};
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

// SWIGLU: W (N x K) is a gate_up weight, rows [gate (N/2) | up (N/2)], and
// tile t covers output columns j0 = 128t.. of both halves: its first 128
// weight rows are gate rows j0.., the next 128 up rows N/2 + j0... The
// epilogue then writes silu(gate) * up, FP8-quantized per 128 columns (one
// group per tile), to Q (M x N/2 e4m3, leading dimension q_ld) and its
// scales to Qs (column-major, Qs[group * qs_ld + m]) instead of C; the bf16
// rounding of gate and up is the unfused GEMM's, and the SiLU and quant
// arithmetic the SiLU-quant kernel's, so the result is bit-identical to
// qx_gemm_fp8_blockscaled followed by qx_silu_mul_quant.
template <int BM, int BN, int WAVES_N, int WAVES_M, int STAGES, bool SWIGLU = false>
__global__ __launch_bounds__(64 * WAVES_N * WAVES_M) void gemm_fp8_k128_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sA, const uint8_t* __restrict__ W,
    const float* __restrict__ sW, uint16_t* __restrict__ C, int M, int N, int K, int64_t lda,
    int64_t ldc, int64_t sa_ld, int tiles_m, int tiles_n, int group_m, uint8_t* __restrict__ Q,
    int64_t q_ld, float* __restrict__ Qs, int64_t qs_ld) {
  using Cfg = Cfg128<BM, BN, WAVES_N, WAVES_M, STAGES>;
  constexpr int TN = Cfg::kTN, TM = Cfg::kTM;
  static_assert(128 % (BN / WAVES_N) == 0 || (BN / WAVES_N) == 128,
                "a wave's weight rows lie in one scale block");
  // vector loads per stage, not counting the weight-scale load (a scalar
  // load where the compiler sees its uniform address; undercounting only
  // makes a wait stricter)
  constexpr int kOps = Cfg::kOpsPerStage;
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
        // this block's loads are done; the later stages' loads may still
        // be in flight
        if (kb + STAGES - 2 < KT) {
          wait_vmcnt<(STAGES - 2) * kOps>();
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

template <int BM, int BN, int WN, int WM, int ST>
int launch128(const void* A, const float* sA, const void* W, const float* sW, void* C, int M,
              int N, int K, int64_t lda, int64_t ldc, int64_t sa_ld, int group_m,
              hipStream_t stream) {
  using Cfg = Cfg128<BM, BN, WN, WM, ST>;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  const int total = tiles_m * tiles_n;
  hipLaunchKernelGGL((gemm_fp8_k128_kernel<BM, BN, WN, WM, ST>), dim3(total),
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
  hipLaunchKernelGGL((gemm_fp8_k128_kernel<256, 256, 2, 4, 2, true>),
                     dim3(tiles_m * tiles_n), dim3(Cfg::kThreads), 0, stream, (const uint8_t*)A,
                     sA, (const uint8_t*)W, sW, nullptr, M, N, K, lda, (int64_t)0, sa_ld, tiles_m,
                     tiles_n, 4, (uint8_t*)Q, q_ld, Qs, qs_ld);
  QX_LAUNCH_STATUS();
}

// ---- 256 x 320 tiles: whole waves where N = 2560 -----------------------------
// Qwen3-4B's o_proj and down projections (N = 2560) make ceil(M/256) x 10
// tiles of 256 x 256: 2.5 waves of the 256 CUs for a 16k-row pack, 1.25 at
// M = 8192, the last one half empty. 256 x 320 tiles make ceil(M/256) x 8:
// exactly 2 waves (1 at M = 8192), each tile 1.25x the work and 10% fewer
// operand bytes per FLOP. Each wave covers 160 weight rows, which straddle
// two 128-row scale blocks: its 32-row tiles a < split lie in the first,
// the rest in the second, and the accumulator rescale keeps one s_prev per
// block. Every element sees the same operations in the same order as with
// 256 x 256 tiles (s = sA * sW, acc *= s_prev / s, acc * s_last in the
// epilogue; a block whose weight scale is 0 skipped), so the results are
// bit-identical. The bf16 tile (256 x 640 B) does not fit the stage buffers
// at once and leaves in two passes of 128 rows.
// Zero rows [r0, r1) of 128 B at rows (a weight block whose scale is 0).
__device__ __noinline__ void zero_weight_rows(uint8_t* rows, int r0, int r1, int lane) {
  for (int r = r0; r < r1; r += 8)
    *reinterpret_cast<v4i*>(rows + (r + (lane >> 3)) * 128 + (lane & 7) * 16) = v4i{0, 0, 0, 0};
  __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
}

// The K loop and epilogue of one 256 x 320 tile for a wave whose first SPLIT
// 32-row weight tiles lie in its first scale block (SPLIT is fixed per wave
// for the whole tile, so the selection is resolved at compile time).
template <int STAGES, int SPLIT>
__device__ __forceinline__ void n320_tile(
    uint8_t* smem, const uint8_t* __restrict__ A, const float* __restrict__ sA,
    const uint8_t* __restrict__ W, const float* __restrict__ sw_row0, uint16_t* __restrict__ C,
    int M, int N, int K, int64_t lda, int64_t ldc, int64_t sa_ld, int m0, int n0, int lane,
    int wave) {
  constexpr int BM = 256, BN = 320, WAVES_N = 2, WAVES_M = 4;
  using Cfg = Cfg128<BM, BN, WAVES_N, WAVES_M, STAGES>;
  constexpr int TN = Cfg::kTN, TM = Cfg::kTM;
  static_assert(TN == 5 && TM == 2 && SPLIT >= 1 && SPLIT <= 4, "160 x 64 wave tiles");
  constexpr int kOps = Cfg::kOpsPerStage;
  const int wn = wave % WAVES_N;
  const int wm = wave / WAVES_N;
  const int KT = K >> 7;
  const float* sw_row1 = sw_row0 + KT;

  v16f acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;

  // 32-bit per-lane offsets of the wave's slab rows within the tile (one
  // register per slab instead of a 64-bit address; the launcher checks that
  // 256 * lda and 320 * K fit), added to the block's wave-uniform base
  uint32_t a_off[Cfg::kASlabs], w_off[Cfg::kWSlabs];
  {
    const int r_in = lane >> 3, p = lane & 7;
#pragma unroll
    for (int j = 0; j < Cfg::kASlabs; ++j) {
      const int row = (wave * Cfg::kASlabs + j) * 8 + r_in;
      const int grow = min(m0 + row, M - 1);  // rows past M repeat the last one
      a_off[j] = (uint32_t)((grow - m0) * lda + (p ^ swz128(row)) * 16);
    }
#pragma unroll
    for (int j = 0; j < Cfg::kWSlabs; ++j) {
      const int row = (wave * Cfg::kWSlabs + j) * 8 + r_in;  // n0 + row < N
      w_off[j] = (uint32_t)((int64_t)row * K + (p ^ swz128(row)) * 16);
    }
  }
  const uint8_t* a_tile = A + (int64_t)m0 * lda;
  const uint8_t* w_tile = W + (int64_t)n0 * K;

  float sw_ring[STAGES][2];
  // the next block's A slabs and scales go out after the barrier, its
  // weight slabs behind the first K half's MFMAs (the address unit then
  // takes them while the matrix core runs: 2-4% faster than all at once)
  auto issue_w = [&](int kb, int stage) {
    uint8_t* buf = smem + stage * Cfg::kStage;
    const uint8_t* w_blk = w_tile + kb * 128;
#pragma unroll
    for (int j = 0; j < Cfg::kWSlabs; ++j)
      __builtin_amdgcn_global_load_lds(
          (const void*)(w_blk + w_off[j]),
          (lds_void*)(buf + Cfg::kABytes + (wave * Cfg::kWSlabs + j) * 1024), 16, 0,
          kOperandLoadPolicy);
  };
  auto issue = [&](int kb, int stage, bool with_w = true) {
    uint8_t* buf = smem + stage * Cfg::kStage;
    const uint8_t* a_blk = a_tile + kb * 128;
#pragma unroll
    for (int j = 0; j < Cfg::kASlabs; ++j)
      __builtin_amdgcn_global_load_lds((const void*)(a_blk + a_off[j]),
                                       (lds_void*)(buf + (wave * Cfg::kASlabs + j) * 1024), 16, 0,
                                       kOperandLoadPolicy);
    if (with_w) issue_w(kb, stage);
    {
      const int t = min(m0 + wave * Cfg::kSaPerWave + lane % Cfg::kSaPerWave, M - 1);
      __builtin_amdgcn_global_load_lds((const void*)(sA + (int64_t)kb * sa_ld + t),
                                       (lds_void*)(buf + Cfg::kABytes + Cfg::kWBytes + wave * 256),
                                       4, 0, 0);
    }
    sw_ring[stage][0] = __builtin_nontemporal_load(sw_row0 + kb);
    sw_ring[stage][1] = __builtin_nontemporal_load(sw_row1 + kb);
  };
#pragma unroll
  for (int st = 0; st < STAGES - 1; ++st)
    if (st < KT) issue(st, st);

  float s_prev[2][TM];
#pragma unroll
  for (int b = 0; b < TM; ++b) s_prev[0][b] = s_prev[1][b] = 0.0f;

  for (int base = 0; base < KT; base += STAGES) {
#pragma unroll
    for (int stage = 0; stage < STAGES; ++stage) {
      const int kb = base + stage;
      if (kb < KT) {
        if (kb + STAGES - 2 < KT) {
          wait_vmcnt<(STAGES - 2) * kOps>();
        } else {
          wait_vmcnt<0>();
        }
        lds_barrier();
        if (kb + STAGES - 1 < KT) issue(kb + STAGES - 1, (stage + STAGES - 1) % STAGES, false);
        const float sw0 =
            __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sw_ring[stage][0])));
        const float sw1 =
            __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sw_ring[stage][1])));
        const bool live0 = sw0 != 0.0f, live1 = sw1 != 0.0f;  // wave-uniform
        uint8_t* a_lds = smem + stage * Cfg::kStage;
        uint8_t* w_lds = a_lds + Cfg::kABytes;
        if (!(live0 && live1)) {
          // A block whose weight scale is 0 adds nothing: the wave zeroes
          // its weight rows of that block in this stage (the other waves
          // reading them write the same zeros), its tiles' accumulators are
          // rescaled by exactly 1 and keep their s_prev, and their MFMAs add
          // +0 to sums that start at +0: bit for bit what skipping does for
          // finite activation codes (a NaN code gives 0 * NaN = NaN here, 0
          // where the block is skipped). Rare (real checkpoints have no
          // all-zero weight blocks).
          // (out of line: the main loop keeps its registers)
          zero_weight_rows(w_lds + wn * TN * 32 * 128, live0 ? SPLIT * 32 : 0,
                           live1 ? SPLIT * 32 : TN * 32, lane);
        }
        const float* sa_lds = reinterpret_cast<const float*>(a_lds + Cfg::kABytes + Cfg::kWBytes);
#pragma unroll
        for (int b = 0; b < TM; ++b) {
          const int row = wm * TM * 32 + b * 32 + (lane & 31);
          const float sa = sa_lds[(row / Cfg::kSaPerWave) * 64 + row % Cfg::kSaPerWave];
          // the same expressions as the 256 x 256 kernel, per scale block
          const float s0 = sa * sw0, s1 = sa * sw1;
          const float q0 = live0 ? s_prev[0][b] / s0 : 1.0f;
          const float q1 = live1 ? s_prev[1][b] / s1 : 1.0f;
#pragma unroll
          for (int a = 0; a < TN; ++a) {
            const float r = a < SPLIT ? q0 : q1;
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[a][b][e] *= r;
          }
          s_prev[0][b] = live0 ? s0 : s_prev[0][b];
          s_prev[1][b] = live1 ? s1 : s_prev[1][b];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          // 160 accumulators leave room for one K half's fragments, not two:
          // the second half's reads wait until the first half's MFMAs issue
          if (h) __builtin_amdgcn_sched_barrier(0);
          if (h && kb + STAGES - 1 < KT)
            issue_w(kb + STAGES - 1, (stage + STAGES - 1) % STAGES);
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

  // epilogue: two passes of 128 tile rows (waves wm = 2p, 2p + 1 stage
  // theirs), rows padded by 16 bytes, written back 16 bytes per lane,
  // non-temporal (as the 256 x 256 kernel's)
  constexpr int kRowBytes = BN * 2 + 16;
  constexpr int kPassRows = BM / 2;
  constexpr int kChunks = BN / 8;
  static_assert(kPassRows * kRowBytes <= Cfg::kLds, "an epilogue pass fits the stage buffers");
  static_assert((kPassRows * kChunks) % Cfg::kThreads == 0, "epilogue chunks");
  const bool wide = ((ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    __syncthreads();  // the operands (pass 0) or the previous pass's rows are consumed
    if ((wm >> 1) == pass) {
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        const int row = (wm & 1) * TM * 32 + b * 32 + (lane & 31);
        uint8_t* lrow = smem + row * kRowBytes;
#pragma unroll
        for (int a = 0; a < TN; ++a) {
          const float s = a < SPLIT ? s_prev[0][b] : s_prev[1][b];
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
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPassRows * kChunks / Cfg::kThreads; ++i) {
      const int idx = i * Cfg::kThreads + threadIdx.x;
      const int row = idx / kChunks, c = idx % kChunks;
      const int m = m0 + pass * kPassRows + row;
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

template <int STAGES>
__global__ __launch_bounds__(512) void gemm_fp8_n320_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sA, const uint8_t* __restrict__ W,
    const float* __restrict__ sW, uint16_t* __restrict__ C, int M, int N, int K, int64_t lda,
    int64_t ldc, int64_t sa_ld, int tiles_m, int tiles_n, int group_m) {
  using Cfg = Cfg128<256, 320, 2, 4, STAGES>;
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
  const int m0 = tile_m * 256;
  const int n0 = tile_n * 320;
  // the wave's weight rows [wrow0, wrow0 + 160): tiles a < split lie in
  // scale block wrow0 / 128, the others in the next one; wrow0 % 128 is 0
  // or 32 (even tile_n) and 64 or 96 (odd), so split is 4, 3, 2 or 1
  const int wrow0 = n0 + (wave % 2) * 160;
  const int split = (128 - (wrow0 & 127)) >> 5;
  const float* sw_row0 = sW + (int64_t)(wrow0 >> 7) * (K >> 7);
#define QX_N320_TILE(S)                                                                          \
  n320_tile<STAGES, S>(smem, A, sA, W, sw_row0, C, M, N, K, lda, ldc, sa_ld, m0, n0, lane, wave)
  switch (split) {
    case 4: QX_N320_TILE(4); break;
    case 3: QX_N320_TILE(3); break;
    case 2: QX_N320_TILE(2); break;
    default: QX_N320_TILE(1); break;
  }
#undef QX_N320_TILE
}

int launch_n320(const void* A, const float* sA, const void* W, const float* sW, void* C, int M,
                int N, int K, int64_t lda, int64_t ldc, int64_t sa_ld, hipStream_t stream) {
  using Cfg = Cfg128<256, 320, 2, 4, 2>;
  const int tiles_m = (M + 255) / 256;
  const int tiles_n = N / 320;
  hipLaunchKernelGGL((gemm_fp8_n320_kernel<2>), dim3(tiles_m * tiles_n), dim3(Cfg::kThreads), 0,
                     stream, (const uint8_t*)A, sA, (const uint8_t*)W, sW, (uint16_t*)C, M, N, K,
                     lda, ldc, sa_ld, tiles_m, tiles_n, 4);
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
            const v2i o = {(int)pack4_fp8(silu_quot(y[0], rs), silu_quot(y[1], rs),
                                          silu_quot(y[2], rs), silu_quot(y[3], rs)),
                           (int)pack4_fp8(silu_quot(y[4], rs), silu_quot(y[5], rs),
                                          silu_quot(y[6], rs), silu_quot(y[7], rs))};
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


// ---- promotion form: one 16x16x128 MFMA per 128-K block ---------------------
// DeepGEMM's arithmetic (the reference's fp8_gemm_nt): each 128-K block's
// products are summed from zero into a partial, and the partial is promoted
// into an fp32 total, total += (sA * sW) * partial. With
// v_mfma_f32_16x16x128_f8f6f4 one MFMA covers a whole scale block of one
// 16 x 16 output tile: its C operand is the inline constant 0, its result a
// 4-register partial that only the promoting FMA reads. The totals are
// never an MFMA operand, so the promotion runs on the VALU beside the
// matrix core instead of waiting on it (rescaling the MFMA accumulators in
// place, configs 10-22, serialises the two). Same tile walk, operand
// staging and epilogue as config 22; a wave covers 128 weight rows x 64
// tokens as 8 x 4 tiles of 16 x 16.
//
// Fragment of a 16-row tile for the 16x16x128 MFMA: lane l holds row l % 16
// and the 32 bytes of K in 16-byte chunks q and q + 4 of the row, q = l / 16
// (bytes [16 q, +16) and [64 + 16 q, +16)). The weight (A) and token (B)
// operands use the same K order, so each lane pair multiplies matching K.
// In LDS this kernel's rows hold chunk c at position c ^ (row % 8). Measured
// with a read probe (8 waves per CU, 16 ds_read_b128 per trip): this layout
// reads at the rate of contiguous 16-byte reads; chunks 2q, 2q + 1 under
// the ((row >> 1) % 8) swizzle of the 32x32 kernels ran 1.55x slower (bank
// conflicts: 3.6 cycles per LDS instruction by the SQ counter).
__device__ __forceinline__ int swz16(int row) { return row & 7; }

__device__ __forceinline__ v8i read_frag16(const uint8_t* lds, int row, int q) {
  const int sw = swz16(row);
  const v4i* base = reinterpret_cast<const v4i*>(lds + row * 128);
  const v4i lo = base[q ^ sw];
  const v4i hi = base[(q + 4) ^ sw];
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

// BN = 320 (config 31, plain output only): each wave's 160 weight rows
// straddle two 128-row scale blocks, the first `split` of its 16-row tiles
// in the first (8, 6, 4 or 2, by the tile column's parity and the wave's
// half); the block's second weight scale rides in the same direct load, and
// a tile's promotion takes the scale of its block. The 656-byte staging rows
// of a 320-column tile leave in four passes of one token tile per wave.
template <bool SWIGLU, int BN>
__global__ __launch_bounds__(512) void gemm_fp8_promo_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ sA, const uint8_t* __restrict__ W,
    const float* __restrict__ sW, uint16_t* __restrict__ C, int M, int N, int K, int64_t lda,
    int64_t ldc, int64_t sa_ld, int tiles_m, int tiles_n, int group_m, uint8_t* __restrict__ Q,
    int64_t q_ld, float* __restrict__ Qs, int64_t qs_ld) {
  static_assert(BN == 256 || (BN == 320 && !SWIGLU), "256-wide tiles, or 320-wide plain");
  constexpr int BM = 256, WAVES_N = 2, WAVES_M = 4;
  using Cfg = Cfg128<BM, BN, WAVES_N, WAVES_M, 2>;
  constexpr int TN = BN / WAVES_N / 16;  // 8 (10) weight tiles of 16 rows per wave
  constexpr int TM = BM / WAVES_M / 16;  // 4 token tiles of 16 per wave
  constexpr int kRowBytes = BN * 2 + 16;   // padded staging row (bank spread)
  constexpr int kTPP = BN == 256 ? 2 : 1;  // token tiles of every wave per epilogue pass
  constexpr int kPassRows = WAVES_M * 16 * kTPP;
  constexpr int kPasses = TM / kTPP;
  constexpr int kWS = Cfg::kWSlabs;        // weight slabs per wave per block: 4 (5)
  constexpr int kRowsPerWave = kPassRows / Cfg::kWaves;
  static_assert(kPassRows * kRowBytes <= Cfg::kStage, "an epilogue pass fits one stage");
  static_assert(kPasses * kPassRows == BM, "passes cover the tile");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Cfg::kLds];

  // this workgroup's tiles: a contiguous band of tile ids per XCD (i mod 8),
  // walked with stride (workgroups per XCD), as in config 22
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
  const int r16 = lane & 15, q16 = lane >> 4;

  // Operand loads of one block: slab j of a wave is tile rows
  // row0 + 8 j, row0 = 32 wave + lane / 8 (A and W alike, 4 slabs each);
  // lane p = lane % 8 of a row writes LDS position p, which holds global
  // chunk p ^ (row % 8) = p ^ (lane / 8), the same for every slab. The
  // per-lane part of an address is a 32-bit offset over a wave-uniform base
  // (the launcher checks that a tile's rows span less than 4 GiB); token
  // rows past M clamp to M - 1.
  static_assert(Cfg::kASlabs == 4 && (kWS == 4 || kWS == 5), "slab walk");
  static_assert(Cfg::kSaPerWave + 2 <= 64, "scale slots past the token scales");
  const int row0 = wave * 32 + (lane >> 3);
  const uint32_t chunk = (uint32_t)(((lane & 7) ^ swz16(row0)) * 16);
  // a wave's weight slabs are rows w_row0 + 8 jw (row % 8 = lane / 8 as for A)
  const int w_row0 = wave * kWS * 8 + (lane >> 3);
  const uint32_t w_lane = (uint32_t)w_row0 * (uint32_t)K + chunk;
  // the block to load: its tile, 128-K block and stage
  struct Blk {
    const uint8_t* a;  // the tile's first token row at the block's K
    const uint8_t* w;  // the tile's first weight row at the block's K
    const float* sa;   // the block's scale of the tile's first token
    const float* sw;   // the wave's (first) weight scale of the block
    uint8_t* buf;
    int m_last;        // the tile's last token row (rows past it clamp)
  };
  auto block_of = [&](int m0_, int n0_, int kb, int stage) {
    Blk b;
    const int64_t k_off = (int64_t)kb * 128;
    const int w_row0 = SWIGLU ? (n0_ >> 1) : n0_;
    b.buf = smem + stage * Cfg::kStage;
    b.m_last = M - 1 - m0_;
    b.a = A + (int64_t)m0_ * lda + k_off;
    b.w = W + (int64_t)w_row0 * K + k_off;
    b.sa = sA + (int64_t)kb * sa_ld + m0_;
    b.sw = sW + (int64_t)((SWIGLU ? w_row0 + wn * (N >> 1) : n0_ + wn * (BN / WAVES_N)) >> 7) * KT + kb;
    return b;
  };
  // load op j of a block: A slabs (j < 4), weight slabs (4 <= j < 4 + kWS),
  // then the token scales and the weight scales, in one direct load: lane
  // i < 32 of a wave brings token scale i of its 32 rows, the lanes past
  // them the wave's weight scale (odd lanes, with 320-wide tiles, that of
  // its second block; a scalar load here would stall every LDS wait of the
  // block behind it: the scalar and LDS counters are one)
  constexpr int kLoadOps = Cfg::kASlabs + Cfg::kWSlabs + 1;
  const int sa_row = wave * Cfg::kSaPerWave + lane % Cfg::kSaPerWave;
  auto load_op = [&](const Blk& b, int j) {
    if (j < 4) {
      const int row = row0 + 8 * j;
      const uint32_t crow = (uint32_t)(row < b.m_last ? row : b.m_last);
      const uint32_t off = crow * (uint32_t)lda + chunk;
      __builtin_amdgcn_global_load_lds((const void*)(b.a + off),
                                       (lds_void*)(b.buf + (wave * 4 + j) * 1024), 16, 0,
                                       kOperandLoadPolicy);
    } else if (j < 4 + kWS) {
      const int jw = j - 4;
      // uniform row shift of slab jw (SwiGLU: rows 128.. are up rows)
      const int shift = 8 * jw + (SWIGLU && wave * 4 + jw >= 16 ? (N >> 1) - 128 : 0);
      __builtin_amdgcn_global_load_lds(
          (const void*)(b.w + (int64_t)shift * K + w_lane),
          (lds_void*)(b.buf + Cfg::kABytes + (wave * kWS + jw) * 1024), 16, 0,
          kOperandLoadPolicy);
    } else {
      const int t = min(sa_row, b.m_last);
      // lanes past the wave's token scales carry its weight scale(s)
      const float* src = lane < Cfg::kSaPerWave ? b.sa + t
                                                : (BN == 320 && (lane & 1) ? b.sw + KT : b.sw);
      __builtin_amdgcn_global_load_lds((const void*)src,
                                       (lds_void*)(b.buf + Cfg::kABytes + Cfg::kWBytes + wave * 256),
                                       4, 0, 0);
    }
  };
  v4f tot[TN][TM];
  int m0 = 0, n0 = 0;
  // the block most recently issued: within a tile the next one is its K
  // neighbour (every address one block further on, the other stage), so
  // block_of's full address arithmetic runs once per tile
  Blk issued{};
  if (my_tiles > 0) {
    origin(0, m0, n0);
    issued = block_of(m0, n0, 0, 0);
#pragma unroll
    for (int j = 0; j < kLoadOps; ++j) load_op(issued, j);
  }
  // Blocks alternate between the two stages across tiles. The next block's
  // fragments are read, and the block after it is loaded, while the last
  // weight tile's MFMAs of the current block run: every wave has read its
  // last operand of the current block by then, so one barrier there frees
  // the block's stage for the loads and lets the next block start with its
  // fragments in registers (a barrier and the fragment reads at each
  // block's start left the matrix cores idle there: 1-6% slower, same
  // bits). A tile's first block (after the epilogue, which stages the tile
  // through the stage of its last block) starts with the barrier and its
  // reads.
  constexpr int kLast = (TN - 1) * TM;  // the last weight tile's first MFMA
  constexpr int kEarly = TM - 1;        // loads issued in that tile's other slots
  static_assert(kLoadOps > kEarly, "load split");
  int stage = 0;
  v8i wf, wf_next, af[TM];
  for (int it = 0; it < my_tiles; ++it) {
    int nm0 = m0, nn0 = n0;
    const bool has_next = it + 1 < my_tiles;
    if (has_next) origin(it + 1, nm0, nn0);
    // the wave's weight tiles in its first scale block (all of them, 256 wide)
    const int split = BN == 320 ? (128 - ((n0 + wn * (BN / WAVES_N)) & 127)) / 16 : TN;
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b) tot[a][b] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // the block after `from` (block kb of this tile) into stage `to`: its K
    // neighbour, or after the tile's last the next tile's first; after the
    // workgroup's last block, block kb again (into a free stage: loads with
    // no branch around them, drained before the end)
    auto after = [&](const Blk& from, int kb, int to) {
      Blk b = from;
      if (kb + 1 < KT) {
        b.a += 128;
        b.w += 128;
        b.sa += sa_ld;
        b.sw += 1;
        b.buf = smem + to * Cfg::kStage;
      } else {
        b = has_next ? block_of(nm0, nn0, 0, to) : block_of(m0, n0, kb, to);
      }
      return b;
    };
    // block kb of the tile. pre: its fragments were read during the
    // previous block, and its first kEarly loads issued there; fetch: the
    // block after the next is this tile's (or the next tile's first), so
    // its loads start during this block's last weight tile
    // (wave-uniform flags: one copy of the block's code, whose registers
    // the 256-VGPR budget holds)
    for (int kb = 0; kb < KT; ++kb) {
      const bool pre = kb > 0;
      const bool fetch = kb + 1 < KT;
      const uint8_t* a_lds = smem + stage * Cfg::kStage;
      const uint8_t* w_lds = a_lds + Cfg::kABytes;
      const float* sa_lds = reinterpret_cast<const float*>(w_lds + Cfg::kWBytes);
      const uint8_t* a_nxt = smem + (stage ^ 1) * Cfg::kStage;
      const uint8_t* w_nxt = a_nxt + Cfg::kABytes;
      // weight fragments kAhead tiles ahead (one ahead in the 320-wide
      // kernel, whose 160 totals leave no registers for a third fragment:
      // measured 6-8% faster than two ahead there, or than a one-MFMA lag)
      constexpr int kAhead = BN == 256 ? 2 : 1;
      // the block whose loads this block issues (pre: begun in the previous)
      Blk nb = issued;
      if (!pre) {
        // this block's operands are done: a tile's first block (but the
        // workgroup's first) was waited for before the previous tile's
        // epilogue stores, which drain under this block instead
        if (it == 0) wait_vmcnt<0>();
        lds_barrier();
        nb = after(issued, kb, stage ^ 1);
        issued = nb;
        // its first loads here (the later ones go one per MFMA, as after a
        // prefetched block, whose first ones the previous block issued)
#pragma unroll
        for (int j = 0; j < kEarly; ++j) load_op(nb, j);
        // the fragments in the order the first MFMAs use them: weight tile
        // 0, the token tiles, weight tile 1 (reading the weight fragments
        // two tiles ahead hides the LDS latency that one ahead left
        // exposed: 3-5% faster)
        wf = read_frag16(w_lds, wn * TN * 16 + r16, q16);
#pragma unroll
        for (int b = 0; b < TM; ++b) af[b] = read_frag16(a_lds, wm * TM * 16 + b * 16 + r16, q16);
      }
      // weight tile 1 (read here after a prefetched block too: the registers
      // that would hold it during the previous block's last tile are not free)
      if constexpr (kAhead == 2) wf_next = read_frag16(w_lds, wn * TN * 16 + 16 + r16, q16);
      // the block's scales (the wave's weight scale came with its token
      // scales, in the slot past them)
      const float sw = sa_lds[wave * 64 + Cfg::kSaPerWave];
      const float sw1 = BN == 320 ? sa_lds[wave * 64 + Cfg::kSaPerWave + 1] : 0.0f;
      float s[TM], s1[TM];
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        const int row = wm * TM * 16 + b * 16 + r16;
        const float sr = sa_lds[(row / Cfg::kSaPerWave) * 64 + row % Cfg::kSaPerWave];
        s[b] = sr * sw;
        s1[b] = BN == 320 ? sr * sw1 : 0.0f;
      }
      // MFMA t (weight tile a = t / TM, token tile b = t % TM) writes
      // partial slot t % 3; each scheduling slot issues one MFMA and the
      // promotion of the partial two MFMAs older, so three partials are
      // live and the FMAs never wait on the MFMA just issued. Weight
      // fragment a + kAhead is read at the start of fragment a's MFMAs.
      constexpr int kLag = 2;
      v4f part[kLag + 1];
      auto promote = [&](int t) {
        // the scale of the tile's weight block (wave-uniform choice)
        const float sc = BN == 320 && t / TM >= split ? s1[t % TM] : s[t % TM];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          tot[t / TM][t % TM][e] =
              __builtin_fmaf(sc, part[t % (kLag + 1)][e], tot[t / TM][t % TM][e]);
      };
      v8i wf_next2;
      // the block loaded during this block's last weight tile (formed here:
      // a branch among the slots would let the compiler move the
      // promotions away from their MFMAs)
      const Blk nb2 = fetch ? after(issued, kb + 1, stage) : issued;
      issued = nb2;
#pragma unroll
      for (int t = 0; t < TN * TM; ++t) {
        const int a = t / TM, b = t % TM;
        if constexpr (kAhead == 1) {
          if (b == 0 && a + 1 < TN)
            wf_next = read_frag16(w_lds, wn * TN * 16 + (a + 1) * 16 + r16, q16);
        }
        part[t % (kLag + 1)] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            wf, af[b], v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0, 0, 0, 0);
        if (t >= kLag) promote(t - kLag);
        if constexpr (kAhead == 2) {
          // after the MFMA that takes fragment a: the compiler's wait for
          // that fragment drains every LDS read in flight (the direct loads
          // leave its LDS counting imprecise), so a read issued ahead of the
          // MFMA would be waited for there too (0-2% slower)
          if (b == 0 && a + 2 < TN) {
            __builtin_amdgcn_sched_barrier(0);
            wf_next2 = read_frag16(w_lds, wn * TN * 16 + (a + 2) * 16 + r16, q16);
          }
        }
        // the loads, one per MFMA over the block's first slots: all of them
        // issued at once after the barrier queue every wave behind the
        // address unit while the matrix core waits (measured 7-14% slower),
        // spread one per two or three MFMAs they land too close to the next
        // barrier (3-8% slower)
        if (t + kEarly < kLoadOps) load_op(nb, t + kEarly);
        if (t >= kLast) {
          // the next block's reads after this slot's MFMA: the registers
          // they fill are the ones it reads
          __builtin_amdgcn_sched_barrier(0);
          if (t == kLast) {
            // this wave's loads of the next block have landed, and its
            // reads of this block's operands are consumed (the weight
            // fragment of this tile fed the MFMA just issued): after the
            // barrier the next block is in LDS for every wave and this
            // block's stage is free. In a tile's last block the next is
            // the next tile's first, read here to no use (its first
            // block reads it again after the epilogue, which stages the
            // tile through this block's stage), and the loads below
            // rewrite its first rows with the same bytes: the code of
            // the slots has no branch, which would let the compiler move
            // the promotions away from their MFMAs
            wait_vmcnt<0>();
            lds_barrier();
            wf_next = read_frag16(w_nxt, wn * TN * 16 + r16, q16);
          }
          // token fragment b of the next block, into the registers of
          // this block's, whose last MFMA was just issued
          af[b] = read_frag16(a_nxt, wm * TM * 16 + b * 16 + r16, q16);
          if (t > kLast) load_op(nb2, t - kLast - 1);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (b == TM - 1 && a + 1 < TN) {
          wf = wf_next;
          if constexpr (kAhead == 2) wf_next = wf_next2;
        }
      }
#pragma unroll
      for (int t = TN * TM - kLag; t < TN * TM; ++t) promote(t);
      wf = wf_next;
      stage ^= 1;
    }

    // epilogue through the stage of the tile's last block. Lane l holds
    // token b * 16 + l % 16 of the wave's 64 and weight rows
    // a * 16 + 4 (l / 16) .. + 3 of its 128 (160). Pass p stages token tiles
    // kTPP p .. kTPP p + kTPP - 1 of every wave: staging row
    // wm * 16 kTPP + (b - kTPP p) * 16 + l % 16.
    // the next tile's first block (issued during this tile's last) lands
    // before any of this tile's stores is issued: every CU reaches its
    // epilogue at about the same time, and waiting for the stores' burst at
    // the next block cost 6-13% of a launch
    wait_vmcnt<0>();
    uint8_t* buf = smem + (stage ^ 1) * Cfg::kStage;
    const bool wide = ((ldc & 7) == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      // pass 0: every wave is done with the last block's operands; later
      // passes: with the previous pass's rows
      lgkm_barrier();
#pragma unroll
      for (int bb = 0; bb < kTPP; ++bb) {
        const int b = pass * kTPP + bb;
        uint8_t* lrow = buf + (wm * 16 * kTPP + bb * 16 + r16) * kRowBytes;
#pragma unroll
        for (int a = 0; a < TN; ++a) {
          const int off = (wn * TN * 16 + a * 16 + q16 * 4) * 2;
          uint2 v;
          v.x = pack2_bf16(tot[a][b][0], tot[a][b][1]);
          v.y = pack2_bf16(tot[a][b][2], tot[a][b][3]);
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
          const int m = m0 + (prow >> 5) * TM * 16 + pass * 32 + (prow & 31);  // kTPP = 2
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
            const v2i o = {(int)pack4_fp8(silu_quot(y[0], rs), silu_quot(y[1], rs),
                                          silu_quot(y[2], rs), silu_quot(y[3], rs)),
                           (int)pack4_fp8(silu_quot(y[4], rs), silu_quot(y[5], rs),
                                          silu_quot(y[6], rs), silu_quot(y[7], rs))};
            __builtin_nontemporal_store(o, reinterpret_cast<v2i*>(Q + (int64_t)m * q_ld + j0 +
                                                                 seg * 8));
            if (seg == 0) Qs[(int64_t)(j0 >> 7) * qs_ld + m] = scale;
          }
        }
      } else {
        // 16-byte chunks of the wave's staged rows, 64 per store instruction
        constexpr int kChunks = BN / 8;
        static_assert(kRowsPerWave * kChunks % 64 == 0, "whole store instructions");
        constexpr int kRowsG = 16 * kTPP;  // staging rows per wave group
        // 320 wide: the lane's rows and chunks are formed here for each
        // tile; kept from the kernel's start they outlived the block loop in
        // spilled registers (100 B per lane, 13 MB of scratch writes per
        // launch), 1-4% slower. The 256-wide kernels have the registers.
        const int el = BN == 320 ? opaque(lane) : lane;
#pragma unroll
        for (int i = 0; i < kRowsPerWave * kChunks / 64; ++i) {
          const int idx = i * 64 + el;
          const int prow = wave * kRowsPerWave + idx / kChunks;
          const int c = idx % kChunks;
          const int m = m0 + (prow / kRowsG) * TM * 16 + pass * kRowsG + prow % kRowsG;
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
  wait_vmcnt<0>();  // the repeated last block's loads
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
// the promotion-form kernel (config 30, 256 x 256 tiles; the SwiGLU
// epilogue with Q != nullptr; config 31, 256 x 320 tiles): one workgroup per
// CU, at least one per XCD
template <bool SWIGLU, int BN>
int launch_promo(const void* A, const float* sA, const void* W, const float* sW, void* C, int M,
                 int N, int K, int64_t lda, int64_t ldc, int64_t sa_ld, void* Q, int64_t q_ld,
                 float* Qs, int64_t qs_ld, hipStream_t stream) {
  const int tiles_m = (M + 255) / 256;
  const int tiles_n = N / BN;
  int grid = persistent_grid(tiles_m * tiles_n);
  if (grid < 8) grid = 8;
  hipLaunchKernelGGL((gemm_fp8_promo_kernel<SWIGLU, BN>), dim3(grid), dim3(512), 0, stream,
                     (const uint8_t*)A, sA, (const uint8_t*)W, sW, (uint16_t*)C, M, N, K, lda,
                     ldc, sa_ld, tiles_m, tiles_n, 4, (uint8_t*)Q, q_ld, Qs, qs_ld);
  QX_LAUNCH_STATUS();
}
}  // namespace
}  // namespace qx

extern "C" {

// Tile configurations (tokens x weights). The rescale family, bit-identical
// to each other since each output element sums the same products in the
// same order: 10: 256 x 256 tiles, 8 waves, two 128-K stages, one workgroup
// per tile (widths that are a multiple of 256); 11: 256 x 128 tiles, 4
// waves (any width that is a multiple of 128); 12: 256 x 320 tiles, 8 waves
// (widths that are a multiple of 320); 22: config 10's tiles on a
// persistent grid with the K pipeline running across tiles (falls back to
// 10 when there are too few tiles or an odd number of 128-K blocks). The
// promotion family, bit-identical to each other: 30 (256 x 256 tiles) and
// 31 (256 x 320 tiles), both persistent.
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
  QX_CHECK(config == 10 || config == 22 || config == 30,
           "gemm_swiglu: config %d (10, 22 or 30)", config);
  if (M == 0) return QX_OK;
  if (config == 30) {
    QX_CHECK(256 * lda < (1LL << 32) && (I + 128) * K < (1LL << 32),
             "gemm_swiglu config 30: a tile's rows must span less than 4 GiB (lda=%lld, K=%lld)",
             (long long)lda, (long long)K);
    return qx::launch_promo<true, 256>(A, sA, W, sW, nullptr, (int)M, (int)(2 * I), (int)K, lda, 0,
                                  sa_ld, Q, q_ld, Qs, qs_ld, stream);
  }
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
    case 10:
      QX_CHECK(n % 256 == 0, "gemm config 10 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch128<256, 256, 2, 4, 2>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 4,
                                              stream);
    case 11:
      return qx::launch128<256, 128, 1, 4, 2>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, 8,
                                              stream);
    case 12:
      QX_CHECK(n % 320 == 0, "gemm config 12 needs N %% 320 == 0 (N=%d)", n);
      QX_CHECK(256 * lda < (1LL << 32) && 320LL * k < (1LL << 32),
               "gemm config 12: a tile's rows must span less than 4 GiB (lda=%lld, K=%d)",
               (long long)lda, k);
      return qx::launch_n320(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, stream);
    case 22:
      QX_CHECK(n % 256 == 0, "gemm config 22 needs N %% 256 == 0 (N=%d)", n);
      return qx::launch128q<false>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, nullptr, 0,
                                   nullptr, 0, stream);
    case 30:
      QX_CHECK(n % 256 == 0, "gemm config 30 needs N %% 256 == 0 (N=%d)", n);
      QX_CHECK(256 * lda < (1LL << 32) && 256LL * k < (1LL << 32),
               "gemm config 30: a tile's rows must span less than 4 GiB (lda=%lld, K=%d)",
               (long long)lda, k);
      return qx::launch_promo<false, 256>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, nullptr, 0,
                                          nullptr, 0, stream);
    case 31:
      QX_CHECK(n % 320 == 0, "gemm config 31 needs N %% 320 == 0 (N=%d)", n);
      QX_CHECK(256 * lda < (1LL << 32) && 320LL * k < (1LL << 32),
               "gemm config 31: a tile's rows must span less than 4 GiB (lda=%lld, K=%d)",
               (long long)lda, k);
      return qx::launch_promo<false, 320>(A, sA, W, sW, C, m, n, k, lda, ldc, sa_ld, nullptr, 0,
                                          nullptr, 0, stream);
    default:
      QX_CHECK(false, "gemm: unknown config %d (10, 11, 12, 22, 30 or 31)", config);
  }
}

}  // extern "C"
