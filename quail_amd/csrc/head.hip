// Last-token answer head: the readouts of
// quail/backends/quail/executor/readout.py.
//
//   logits[i, j] = normed[i, :] . rows[j, :]   (fp32 accumulation)
//
// mode 0 (AnswerRows.logits / AsyncLabelLogprobs with normalize=False,
//         readout.py:44-48, :188-191): logits rounded to bf16, as a bf16
//         F.linear returns them, then widened to fp32;
// mode 1 (AsyncScores, readout.py:331-336): fp32 logits of the fp32 inputs.
//
// Then, when `cls` is given (cls[j] = 1 for a TRUE/yes spelling, 0 for a
// FALSE/no spelling, -1 for neither), per row:
//   yes = max_{cls=1} logits, no = max_{cls=0} logits,
//   bits = yes > no (AI.IF), score = sigmoid((yes - no) / temperature) (AI.SCORE).
// One wave per row; lanes stride the hidden dimension in 16-byte chunks.
#include "qx_common.h"
#include "qx_status.h"

namespace qx {
namespace {

constexpr int kMaxLabels = 16;

__global__ __launch_bounds__(256) void answer_head_kernel(
    const uint16_t* __restrict__ normed, int64_t n_ld, const uint16_t* __restrict__ rows,
    int64_t r_ld, int t, int n, int H, int mode, const int* __restrict__ cls, float inv_temp,
    float* __restrict__ logits, uint8_t* __restrict__ bits, float* __restrict__ yes_no,
    float* __restrict__ score) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  float acc[kMaxLabels];
#pragma unroll
  for (int j = 0; j < kMaxLabels; ++j) acc[j] = 0.f;
  const uint16_t* x = normed + (int64_t)row * n_ld;
  for (int c = lane; c < (H >> 3); c += 64) {
    uint4 a = *reinterpret_cast<const uint4*>(x + c * 8);
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
    float xv[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      xv[2 * k] = lo_bf16(aw[k]);
      xv[2 * k + 1] = hi_bf16(aw[k]);
    }
#pragma unroll
    for (int j = 0; j < kMaxLabels; ++j) {
      if (j < t) {
        uint4 b = *reinterpret_cast<const uint4*>(rows + (int64_t)j * r_ld + c * 8);
        const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc[j] = fmaf(xv[2 * k], lo_bf16(bw[k]), acc[j]);
          acc[j] = fmaf(xv[2 * k + 1], hi_bf16(bw[k]), acc[j]);
        }
      }
    }
  }
  float yes = -INFINITY, no = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMaxLabels; ++j) {
    if (j < t) {
      float v = group_sum<64>(acc[j]);
      if (mode == 0) v = round_bf16(v);
      if (logits && lane == 0) logits[(int64_t)row * t + j] = v;
      if (cls) {
        const int c = cls[j];
        if (c == 1) yes = fmaxf(yes, v);
        if (c == 0) no = fmaxf(no, v);
      }
    }
  }
  if (cls && lane == 0) {
    if (bits) bits[row] = yes > no ? 1 : 0;
    if (yes_no) {
      yes_no[2 * (int64_t)row] = yes;
      yes_no[2 * (int64_t)row + 1] = no;
    }
    if (score) score[row] = 1.0f / (1.0f + expf(-(yes - no) * inv_temp));
  }
}

}  // namespace
}  // namespace qx

extern "C" {

int qx_answer_head(const void* normed, int64_t n_ld, const void* rows, int64_t r_ld, int64_t t,
                   int64_t n, int64_t H, int mode, const int* cls, float temperature,
                   float* logits, uint8_t* bits, float* yes_no, float* score,
                   hipStream_t stream) {
  QX_CHECK(normed && rows, "answer_head: null pointer");
  QX_CHECK(t >= 1 && t <= qx::kMaxLabels, "answer_head: %lld label rows (1..16)", (long long)t);
  QX_CHECK(H % 8 == 0 && n_ld % 8 == 0 && r_ld % 8 == 0, "answer_head: strides");
  QX_CHECK(mode == 0 || mode == 1, "answer_head: mode %d", mode);
  QX_CHECK(cls || !(bits || yes_no || score), "answer_head: class outputs need cls");
  QX_CHECK(temperature > 0.f, "answer_head: temperature must be positive");
  if (n == 0) return QX_OK;
  hipLaunchKernelGGL(qx::answer_head_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, stream,
                     (const uint16_t*)normed, n_ld, (const uint16_t*)rows, r_ld, (int)t, (int)n,
                     (int)H, mode, cls, 1.0f / temperature, logits, bits, yes_no, score);
  QX_LAUNCH_STATUS();
}

}  // extern "C"
