// Full-vocabulary label log-probabilities: the normalize=True path of the
// AI.CLASSIFY readout (quail/backends/quail/executor/readout.py:143-200),
// which computes, per block of rows, bf16 logits = normed @ head^T over the
// whole vocabulary (F.linear in bf16), then
//   out[row, j] = float(logits[row, target_j]) - logsumexp(float(logits[row, :])).
//
// Two launches, no (n x V) logits in memory:
//   * vocab_lse_kernel: a workgroup owns 128 head rows and up to 128 rows of
//     `normed`, streamed through LDS 64 K elements at a time by direct
//     loads of whole 128-byte lines (v_mfma_f32_32x32x16_bf16, head rows as
//     the A operand, tokens as B, K read in a permuted order that is the
//     same for both operands, so each dot product is a plain fp32 sum),
//     rounds its logits to bf16 as F.linear's output is, and reduces them
//     to a per-token (max, sum of exp) partial; the waves' partials merge
//     in LDS into one per (head-row block, token). The lane holding a target
//     id's logit writes it.
//   * vocab_finish_kernel: one wave per token merges the blocks' partials
//     into the logsumexp and subtracts it from the target logits.
// The head (V x H bf16, 778 MB for Qwen3) is read once per 128 tokens, so a
// launch over a pack's final rows is bound by streaming it from HBM.
#include <mutex>

#include "qx_common.h"
#include "qx_status.h"

namespace qx {
namespace {

constexpr int kWaves = 8;
constexpr int kMaxTargets = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// merge two (max, sum of exp(x - max)) pairs
__device__ __forceinline__ float2 lse_merge(float2 a, float2 b) {
  const float m = fmaxf(a.x, b.x);
  if (m == -INFINITY) return make_float2(-INFINITY, 0.0f);
  return make_float2(m, a.y * __builtin_amdgcn_exp2f((a.x - m) * kLog2e) +
                            b.y * __builtin_amdgcn_exp2f((b.x - m) * kLog2e));
}

__device__ __forceinline__ float bf16_round(float v) {
  return static_cast<float>(static_cast<__bf16>(v));
}

constexpr int kStages = 3;

// 128-byte LDS rows of 8 16-byte chunks, chunk-swizzled by (row >> 1) & 7:
// the 16 rows one quarter-wave's ds_read_b128 touches then cover all banks
__device__ __forceinline__ int vswz(int row) { return (row >> 1) & 7; }

// one 1 KiB direct load: 8 rows x 128 bytes of a row-major bf16 matrix,
// rows clamped to row_max; lane i fills LDS chunk i % 8 of row i / 8. The
// loads are inline assembly the compiler does not track (lds_dma16): with
// the builtin it waits for every load in flight before each LDS read of
// any stage. STREAM: device scope, no L1 copy (the head is read once).
template <bool STREAM>
__device__ __forceinline__ void load_slab(const uint16_t* __restrict__ g, int64_t ld, int row0,
                                          int row_max, int k, uint8_t* lds, int slab, int lane) {
  const int row = slab * 8 + (lane >> 3);
  const int c = (lane & 7) ^ vswz(row);
  const uint16_t* src = g + (int64_t)min(row0 + row, row_max) * ld + k + c * 8;
  if (STREAM) {
    lds_dma16_stream(src, lds + slab * 1024);
  } else {
    lds_dma16(src, lds + slab * 1024);
  }
}

// A workgroup of 4 waves covers 128 head rows (32 per wave) and TM 32-token
// tiles; 64 K elements per stage (head 16 KiB + tokens 4 KiB per tile),
// three stages. The MFMA fragment of k-step s for lane half hh is K
// elements [32 hh + 8 s, +8) of the chunk (16-byte chunk 4 hh + s), the
// same permutation for both operands.
template <int TM>
__global__ __launch_bounds__(256) void vocab_lse_kernel(
    const uint16_t* __restrict__ x, int64_t x_ld, const uint16_t* __restrict__ head,
    int64_t h_ld, const int64_t* __restrict__ targets, int t, float2* __restrict__ part,
    float* __restrict__ tlogit, int n, int V, int H) {
  constexpr int kWavesLds = 4;
  constexpr int kHeadBytes = 128 * 128;
  constexpr int kStage = kHeadBytes + TM * 32 * 128;
  constexpr int kSlabs = kStage / 1024;
  static_assert(kSlabs % kWavesLds == 0, "slabs per wave");
  constexpr int kSlabsPerWave = kSlabs / kWavesLds;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kStages * kStage];
  __shared__ float2 red[kWavesLds][32 * TM];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hh = lane >> 5;
  const int r = lane & 31;
  const int vb = blockIdx.x * 128;
  const int tok0 = blockIdx.y * (32 * TM);
  const int KC = H >> 6;

  auto issue = [&](int kc, int stage) {
    uint8_t* buf = smem + stage * kStage;
#pragma unroll
    for (int j = 0; j < kSlabsPerWave; ++j) {
      const int slab = wave * kSlabsPerWave + j;
      if (slab < 16) {
        load_slab<true>(head, h_ld, vb, V - 1, kc * 64, buf, slab, lane);
      } else {
        load_slab<false>(x, x_ld, tok0, n - 1, kc * 64, buf + kHeadBytes, slab - 16, lane);
      }
    }
  };

  v16f acc[TM];
#pragma unroll
  for (int b = 0; b < TM; ++b) acc[b] = v16f{};
#pragma unroll
  for (int st = 0; st < kStages - 1; ++st)
    if (st < KC) issue(st, st);
  for (int kc = 0; kc < KC; ++kc) {
    const int stage = kc % kStages;
    if (kc + 1 < KC) {
      wait_vmcnt<kSlabsPerWave>();  // chunk kc landed; kc + 1 may be in flight
    } else {
      wait_vmcnt<0>();
    }
    // every wave's chunk kc has landed, and its reads of the stage about to
    // be refilled (chunk kc - 1, consumed by its MFMAs) are done
    lds_barrier();
    if (kc + kStages - 1 < KC) issue(kc + kStages - 1, (kc + kStages - 1) % kStages);
    const uint8_t* hl = smem + stage * kStage;
    const uint8_t* tl = hl + kHeadBytes;
    const int hrow = wave * 32 + r;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int c = hh * 4 + s;
      const v8bf a = *reinterpret_cast<const v8bf*>(hl + hrow * 128 + ((c ^ vswz(hrow)) << 4));
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        const int trow = b * 32 + r;
        const v8bf bt = *reinterpret_cast<const v8bf*>(tl + trow * 128 + ((c ^ vswz(trow)) << 4));
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bt, acc[b], 0, 0, 0);
      }
    }
  }

  // lane (hh, r) of tile b holds token tok0 + 32 b + r at head rows
  // v0 + 4 hh + 8 g + e (g, e in 0..3)
  const int v0 = vb + wave * 32;
#pragma unroll
  for (int b = 0; b < TM; ++b) {
    float v[16];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = v0 + hh * 4 + (i >> 2) * 8 + (i & 3);
      v[i] = row < V ? bf16_round(acc[b][i]) : -INFINITY;
      m = fmaxf(m, v[i]);
    }
    float s = 0.0f;
    if (m != -INFINITY) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s += __builtin_amdgcn_exp2f((v[i] - m) * kLog2e);
    }
    const auto om = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m),
                                                     false, false);
    const auto os = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s),
                                                     false, false);
    // the swap hands every lane both halves' values, the lower half's in
    // slot 0 and the upper half's in slot 1: merging them in that order
    // gives both halves the same bits
    const float2 merged = lse_merge(make_float2(__uint_as_float(om[0]), __uint_as_float(os[0])),
                                    make_float2(__uint_as_float(om[1]), __uint_as_float(os[1])));
    if (hh == 0) red[wave][b * 32 + r] = merged;
    const int tok = tok0 + b * 32 + r;
    for (int it = 0; it < t; ++it) {
      const int64_t tg = targets[it];
      const int i = (int)(tg - v0);
      if (i >= 0 && i < 32 && ((i >> 2) & 1) == hh && tok < n) {
        float val = v[0];
#pragma unroll
        for (int q = 1; q < 16; ++q)
          if (q == ((i >> 3) << 2) + (i & 3)) val = v[q];
        tlogit[(int64_t)tok * t + it] = val;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x < 32 * TM) {
    const int j = threadIdx.x;
    float2 acc2 = red[0][j];
#pragma unroll
    for (int w = 1; w < kWavesLds; ++w) acc2 = lse_merge(acc2, red[w][j]);
    if (tok0 + j < n) part[(int64_t)blockIdx.x * n + tok0 + j] = acc2;
  }
}

__global__ __launch_bounds__(64) void vocab_finish_kernel(const float2* __restrict__ part,
                                                          int nblk, const float* __restrict__ tlogit,
                                                          int t, float* __restrict__ out,
                                                          int64_t out_ld, int n) {
  const int tok = blockIdx.x;
  const int lane = threadIdx.x;
  float2 acc = make_float2(-INFINITY, 0.0f);
  for (int b = lane; b < nblk; b += 64) acc = lse_merge(acc, part[(int64_t)b * n + tok]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float2 o = make_float2(__shfl_xor(acc.x, off), __shfl_xor(acc.y, off));
    acc = lse_merge(acc, o);
  }
  // the butterfly leaves each lane a sum in its own association order, which
  // may differ in the last bit: every target takes lane 0's
  const float lse = __shfl(acc.x + __log2f(acc.y) * kLn2, 0);
  if (lane < t) out[(int64_t)tok * out_ld + lane] = tlogit[(int64_t)tok * t + lane] - lse;
}

// head rows per workgroup
int block_rows(int64_t) { return 128; }

int64_t workspace_bytes(int64_t n, int64_t V, int64_t t) {
  const int64_t nblk = (V + block_rows(n) - 1) / block_rows(n);
  return nblk * n * (int64_t)sizeof(float2) + ((n * t * 4 + 255) / 256) * 256;
}

}  // namespace
}  // namespace qx

namespace qx {
namespace {

// Both entry points: argument checks, then the two launches over `workspace`
// (workspace_bytes(n, V, t) bytes, every byte written before it is read).
int vocab_run(const void* normed, int64_t n_ld, const void* head, int64_t h_ld,
              const int64_t* targets, int64_t t, float* out, int64_t out_ld, int64_t n, int64_t V,
              int64_t H, void* workspace, int64_t workspace_size, hipStream_t stream) {
  QX_CHECK(normed && head && targets && out && workspace, "vocab_logprobs: null pointer");
  QX_CHECK(t >= 1 && t <= kMaxTargets, "vocab_logprobs: %lld targets (1..16)", (long long)t);
  QX_CHECK(H > 0 && H % 64 == 0, "vocab_logprobs: hidden %lld not a multiple of 64",
           (long long)H);
  QX_CHECK(V >= 1 && V < (1LL << 31) && n >= 0 && n < (1LL << 31), "vocab_logprobs: sizes");
  QX_CHECK(n_ld >= H && h_ld >= H && n_ld % 8 == 0 && h_ld % 8 == 0 && out_ld >= t,
           "vocab_logprobs: strides");
  QX_CHECK(((uintptr_t)normed & 15) == 0 && ((uintptr_t)head & 15) == 0 &&
               ((uintptr_t)workspace & 15) == 0,
           "vocab_logprobs: alignment");
  QX_CHECK(workspace_size >= workspace_bytes(n, V, t), "vocab_logprobs: workspace of %lld "
           "bytes, needs %lld", (long long)workspace_size, (long long)workspace_bytes(n, V, t));
  if (n == 0) return QX_OK;
  const int rows = block_rows(n);
  const int nblk = (int)((V + rows - 1) / rows);
  float2* part = reinterpret_cast<float2*>(workspace);
  float* tlogit = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) +
                                           (int64_t)nblk * n * sizeof(float2));
  const int tm = n <= 32 ? 1 : n <= 64 ? 2 : 4;
  const dim3 grid(nblk, (unsigned)((n + 32 * tm - 1) / (32 * tm)));
  const auto* xp = reinterpret_cast<const uint16_t*>(normed);
  const auto* hp = reinterpret_cast<const uint16_t*>(head);
  if (tm == 1) {
    hipLaunchKernelGGL(vocab_lse_kernel<1>, grid, dim3(256), 0, stream, xp, n_ld, hp, h_ld,
                       targets, (int)t, part, tlogit, (int)n, (int)V, (int)H);
  } else if (tm == 2) {
    hipLaunchKernelGGL(vocab_lse_kernel<2>, grid, dim3(256), 0, stream, xp, n_ld, hp, h_ld,
                       targets, (int)t, part, tlogit, (int)n, (int)V, (int)H);
  } else {
    hipLaunchKernelGGL(vocab_lse_kernel<4>, grid, dim3(256), 0, stream, xp, n_ld, hp, h_ld,
                       targets, (int)t, part, tlogit, (int)n, (int)V, (int)H);
  }
  {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  hipLaunchKernelGGL(vocab_finish_kernel, dim3((unsigned)n), dim3(64), 0, stream, part, nblk,
                     tlogit, (int)t, out, out_ld, (int)n);
  QX_LAUNCH_STATUS();
}

// The allocation-free entry point's workspace: one array per GPU, held until
// the process ends. In host code `scratch` names a host-side stand-in, not a
// device address: its address on each device comes from hipGetSymbolAddress,
// taken once per device with that device current.
constexpr int64_t kScratchBytes = 8 << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex scratch_mutex;
void* scratch_ptr[kMaxDevices] = {};

// this device's address of `scratch` (nullptr and the error text on failure)
void* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("vocab_logprobs_noalloc: no current device (or device id %d >= %d)", dev,
              kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      set_error("vocab_logprobs_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
      return nullptr;
    }
    scratch_ptr[dev] = ptr;
  }
  return scratch_ptr[dev];
}

}  // namespace
}  // namespace qx

extern "C" {

int64_t qx_vocab_logprobs_workspace(int64_t n, int64_t V, int64_t t) {
  if (n < 0 || V < 1 || t < 1) return -1;
  return qx::workspace_bytes(n, V, t);
}

int qx_vocab_logprobs(const void* normed, int64_t n_ld, const void* head, int64_t h_ld,
                      const int64_t* targets, int64_t t, float* out, int64_t out_ld, int64_t n,
                      int64_t V, int64_t H, void* workspace, int64_t workspace_bytes,
                      hipStream_t stream) {
  return qx::vocab_run(normed, n_ld, head, h_ld, targets, t, out, out_ld, n, V, H, workspace,
                       workspace_bytes, stream);
}

int64_t qx_vocab_logprobs_noalloc_max_bytes(void) { return qx::kScratchBytes; }

int qx_vocab_logprobs_noalloc(const void* normed, int64_t n_ld, const void* head, int64_t h_ld,
                              const int64_t* targets, int64_t t, float* out, int64_t out_ld,
                              int64_t n, int64_t V, int64_t H, hipStream_t stream) {
  QX_CHECK(n >= 0 && V >= 1 && t >= 1, "vocab_logprobs_noalloc: sizes");
  const int64_t need = qx::workspace_bytes(n, V, t);
  QX_CHECK(need <= qx::kScratchBytes, "vocab_logprobs_noalloc: %lld rows x %lld vocabulary "
           "need %lld bytes of workspace, more than its %lld (call qx_vocab_logprobs with a "
           "workspace, or fewer rows per call)", (long long)n, (long long)V, (long long)need,
           (long long)qx::kScratchBytes);
  void* ws = qx::scratch_on_current_device();
  if (!ws) return QX_EINVAL;
  return qx::vocab_run(normed, n_ld, head, h_ld, targets, t, out, out_ld, n, V, H, ws,
                       qx::kScratchBytes, stream);
}

}  // extern "C"
