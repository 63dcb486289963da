// HBM-streaming kernels of the Qwen3 prefill pass (one wave per row or
// row-block, 16-byte coalesced loads, fp32 arithmetic, the reference's
// rounding points). Each follows a reference kernel:
//
//   qx_add_rmsnorm_quant   Triton add_rms_norm_quant       attention.py:796-829
//   qx_rmsnorm_quant       vLLM rms_norm + group quant     attention.py:539-556, 517-532
//   qx_embed_rmsnorm_quant embed_tokens + the layer-0 norm qwen3.py:123, 47-49
//   qx_qk_norm_rope        Triton qk_norm_rope             attention.py:833-879
//   qx_silu_mul_quant      Triton silu_mul_quant           attention.py:771-793
//   qx_group_quant         vLLM per_token_group_quant_fp8  attention.py:517-532
//   qx_kv_scatter          Triton kv_row_scatter           attention.py:885-897
//   qx_add_rmsnorm         vLLM fused_add_rms_norm         attention.py:558-562
//   qx_embed               vLLM embed_tokens               qwen3.py:123
//
// FP8 scales are written "column-major": scale of (token t, group g) at
// scales[g * s_ld + t], the (K/128, n) storage the reference views as (n, K/128).
#include "qx_common.h"
#include "qx_status.h"

namespace qx {
namespace {

constexpr int kRowThreads = 256;  // 4 rows (one per wave) per workgroup

// ---------------------------------------------------------------------------
// Row norm + quant. One wave per token row; lane holds chunks of 8 columns
// (16 B of bf16): chunk c = lane + 64 * i. A 128-column group is 16 chunks,
// held by 16 consecutive lanes of one pass.
//
// MODE 0: y = fp32 (x + res) * rstd * w   (Triton add_rms_norm_quant; res <- bf16(x + res))
// MODE 1: y = bf16(bf16(x * rstd) * w)    (vLLM rms_norm, bf16 output, then quant)
// MODE 2: as MODE 1 with x gathered from an embedding table and copied to res
template <int NITER, int MODE>
__global__ __launch_bounds__(kRowThreads) void norm_quant_kernel(
    const uint16_t* __restrict__ x, int64_t x_ld, uint16_t* __restrict__ res, int64_t res_ld,
    const int64_t* __restrict__ ids, const uint16_t* __restrict__ w, uint8_t* __restrict__ q,
    int64_t q_ld, float* __restrict__ scales, int64_t s_ld, int n, int H, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (kRowThreads / 64) + (threadIdx.x >> 6);
  if (row >= n) return;
  const int nch = H >> 3;
  const uint16_t* xrow;
  if (MODE == 2) {
    xrow = x + ids[row] * x_ld;
  } else {
    xrow = x + (int64_t)row * x_ld;
  }
  float v[NITER][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NITER; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      uint4 a = *reinterpret_cast<const uint4*>(xrow + c * 8);
      uint32_t aw[4] = {a.x, a.y, a.z, a.w};
      if (MODE == 0) {
        uint16_t* rrow = res + (int64_t)row * res_ld;
        uint4 r = *reinterpret_cast<const uint4*>(rrow + c * 8);
        uint32_t rw[4] = {r.x, r.y, r.z, r.w};
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          float s0 = lo_bf16(aw[k]) + lo_bf16(rw[k]);
          float s1 = hi_bf16(aw[k]) + hi_bf16(rw[k]);
          v[i][2 * k] = s0;
          v[i][2 * k + 1] = s1;
          o[k] = pack2_bf16(s0, s1);
        }
        *reinterpret_cast<uint4*>(rrow + c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          v[i][2 * k] = lo_bf16(aw[k]);
          v[i][2 * k + 1] = hi_bf16(aw[k]);
        }
        if (MODE == 2) {
          *reinterpret_cast<uint4*>(res + (int64_t)row * res_ld + c * 8) = a;
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) ss += v[i][k] * v[i][k];
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[i][k] = 0.f;
    }
  }
  ss = group_sum<64>(ss);
  const float rstd = 1.0f / sqrtf(ss / (float)H + eps);
  uint8_t* qrow = q + (int64_t)row * q_ld;
#pragma unroll
  for (int i = 0; i < NITER; ++i) {
    const int c = lane + 64 * i;
    if (i * 64 >= nch) break;  // wave-uniform
    const bool live = c < nch;
    float y[8];
    float amax = 0.f;
    if (live) {
      uint4 wv = *reinterpret_cast<const uint4*>(w + c * 8);
      uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float w0 = lo_bf16(ww[k]), w1 = hi_bf16(ww[k]);
        if (MODE == 0) {
          y[2 * k] = v[i][2 * k] * rstd * w0;
          y[2 * k + 1] = v[i][2 * k + 1] * rstd * w1;
        } else {
          y[2 * k] = round_bf16(round_bf16(v[i][2 * k] * rstd) * w0);
          y[2 * k + 1] = round_bf16(round_bf16(v[i][2 * k + 1] * rstd) * w1);
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(y[k]));
    }
    amax = group_max<16>(amax);
    const float scale = fp8_scale(amax);
    const float rs = recip(scale);
    if (live) {
      uint2 o;
      o.x = pack4_fp8(div_by(y[0], scale, rs), div_by(y[1], scale, rs), div_by(y[2], scale, rs),
                      div_by(y[3], scale, rs));
      o.y = pack4_fp8(div_by(y[4], scale, rs), div_by(y[5], scale, rs), div_by(y[6], scale, rs),
                      div_by(y[7], scale, rs));
      *reinterpret_cast<uint2*>(qrow + c * 8) = o;
      if ((lane & 15) == 0) scales[(int64_t)(c >> 4) * s_ld + row] = scale;
    }
  }
}

template <int MODE>
int launch_norm_quant(const void* x, int64_t x_ld, void* res, int64_t res_ld, const int64_t* ids,
                      const void* w, void* q, int64_t q_ld, float* scales, int64_t s_ld, int n,
                      int H, float eps, hipStream_t stream) {
  const int niter = (H / 8 + 63) / 64;
  dim3 grid((n + 3) / 4), block(kRowThreads);
#define QX_NQ_CASE(NI)                                                                     \
  case NI:                                                                                 \
    hipLaunchKernelGGL((norm_quant_kernel<NI, MODE>), grid, block, 0, stream,              \
                       (const uint16_t*)x, x_ld, (uint16_t*)res, res_ld, ids,              \
                       (const uint16_t*)w, (uint8_t*)q, q_ld, scales, s_ld, n, H, eps);    \
    break;
  switch (niter) {
    QX_NQ_CASE(1)
    QX_NQ_CASE(2)
    QX_NQ_CASE(3)
    QX_NQ_CASE(4)
    QX_NQ_CASE(5)
    QX_NQ_CASE(6)
    QX_NQ_CASE(7)
    QX_NQ_CASE(8)
    QX_NQ_CASE(9)
    QX_NQ_CASE(10)
    QX_NQ_CASE(11)
    QX_NQ_CASE(12)
    QX_NQ_CASE(13)
    QX_NQ_CASE(14)
    QX_NQ_CASE(15)
    QX_NQ_CASE(16)
    default:
      QX_CHECK(false, "norm_quant: hidden %d exceeds 8192", H);
  }
#undef QX_NQ_CASE
  QX_LAUNCH_STATUS();
}

// ---------------------------------------------------------------------------
// vLLM fused_add_rms_norm over selected rows: z = bf16(h + r); r <- z;
// out = bf16(bf16(z * rstd) * w). rows == nullptr selects rows 0..n-1;
// otherwise output row i reads input row rows[i] (the final_indices gather
// of qwen3.py:130-134) and the updated residual is written to res_out[i].
template <int NITER>
// out may alias h and res_out may alias r (vLLM updates both in place): every
// lane reads its columns of h and r before it writes them.
__global__ __launch_bounds__(kRowThreads) void add_rmsnorm_kernel(
    const uint16_t* h, int64_t h_ld, const uint16_t* r, int64_t r_ld,
    const int64_t* __restrict__ rows, const uint16_t* __restrict__ w, uint16_t* out,
    int64_t out_ld, uint16_t* res_out, int64_t res_out_ld, int n, int H, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * (kRowThreads / 64) + (threadIdx.x >> 6);
  if (row >= n) return;
  const int64_t src = rows ? rows[row] : row;
  const int nch = H >> 3;
  float v[NITER][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NITER; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      uint4 a = *reinterpret_cast<const uint4*>(h + src * h_ld + c * 8);
      uint4 b = *reinterpret_cast<const uint4*>(r + src * r_ld + c * 8);
      uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w}, o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float z0 = round_bf16(lo_bf16(aw[k]) + lo_bf16(bw[k]));
        float z1 = round_bf16(hi_bf16(aw[k]) + hi_bf16(bw[k]));
        v[i][2 * k] = z0;
        v[i][2 * k + 1] = z1;
        o[k] = pack2_bf16(z0, z1);
      }
      if (res_out)
        *reinterpret_cast<uint4*>(res_out + (int64_t)row * res_out_ld + c * 8) =
            make_uint4(o[0], o[1], o[2], o[3]);
#pragma unroll
      for (int k = 0; k < 8; ++k) ss += v[i][k] * v[i][k];
    }
  }
  ss = group_sum<64>(ss);
  const float rstd = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
  for (int i = 0; i < NITER; ++i) {
    const int c = lane + 64 * i;
    if (c < nch) {
      uint4 wv = *reinterpret_cast<const uint4*>(w + c * 8);
      uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w}, o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float y0 = round_bf16(v[i][2 * k] * rstd) * lo_bf16(ww[k]);
        float y1 = round_bf16(v[i][2 * k + 1] * rstd) * hi_bf16(ww[k]);
        o[k] = pack2_bf16(y0, y1);
      }
      *reinterpret_cast<uint4*>(out + (int64_t)row * out_ld + c * 8) =
          make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

// ---------------------------------------------------------------------------
// Per-head RMSNorm of q and k with the shared (D,) weights, then neox RoPE
// from cos_sin[pos] = [cos D/2 | sin D/2] (attention.py:833-879), fp32
// throughout, bf16 output. A head is handled by D/8 lanes; each lane holds 4
// columns of the first half (a) and the matching 4 of the second half (b).
// POOL: the row's K goes to pool row dst[row] of kp (ko unused) and its V
// (the qkv columns after the K heads) to the same row of vp, as bf16 or,
// with V_F16, as fp16 (pack2_f16_sat, as qx_kv_scatter converts it);
// dst[row] < 0 writes neither. With dst2, the same K and V rows also go to
// row dst2[row] (when >= 0) of kp2 / vp2.
template <int D, bool CS_F32, bool POOL, bool V_F16 = false>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ qkv, int64_t qkv_ld, uint16_t* __restrict__ qo, int64_t qo_ld,
    uint16_t* __restrict__ ko, int64_t ko_ld, const void* __restrict__ cs,
    const int64_t* __restrict__ pos, const uint16_t* __restrict__ qw,
    const uint16_t* __restrict__ kw, int n, int HQ, int HK, float eps,
    uint16_t* __restrict__ kp, uint16_t* __restrict__ vp, const int64_t* __restrict__ dst,
    uint16_t* __restrict__ kp2, uint16_t* __restrict__ vp2, const int64_t* __restrict__ dst2) {
  constexpr int LPH = D / 8;       // lanes per head
  constexpr int HALF = D / 2;
  constexpr int HPB = 256 / LPH;   // heads per pass of the workgroup
  const int row = blockIdx.x;
  const int slot = threadIdx.x / LPH;
  const int j = threadIdx.x % LPH;
  const uint16_t* xrow = qkv + (int64_t)row * qkv_ld;
  const int total = HQ + HK;
  const int64_t kv_row = (int64_t)HK * D;
  // with no q output the pass writes K and V only (the attention normalizes
  // and rotates q as it loads it): the first k_threads lanes take the K
  // heads and the rest copy V alongside (when the K heads leave any)
  const bool kv_only = POOL && qo == nullptr;
  const int k_threads = kv_only && HK < HPB ? HK * LPH : 256;
  const int v_first = k_threads < 256 ? k_threads : 0;
  int64_t drow = 0, drow2 = -1;
  if (POOL) {
    drow = dst[row];
    drow2 = dst2 ? dst2[row] : -1;
    if ((drow >= 0 || drow2 >= 0) && (int)threadIdx.x >= v_first) {
      const uint4* vs = reinterpret_cast<const uint4*>(xrow + total * D);
      uint4* vd = drow >= 0 ? reinterpret_cast<uint4*>(vp + drow * kv_row) : nullptr;
      uint4* vd2 = drow2 >= 0 ? reinterpret_cast<uint4*>(vp2 + drow2 * kv_row) : nullptr;
      for (int c = threadIdx.x - v_first; c < (int)(kv_row >> 3); c += 256 - v_first) {
        const uint4 w = V_F16 ? bf16x8_to_f16(vs[c]) : vs[c];
        if (drow >= 0) vd[c] = w;
        if (drow2 >= 0) vd2[c] = w;
      }
    }
  }
  // whole LPH-lane groups: the group_sum exchanges stay inside live groups
  if ((int)threadIdx.x >= k_threads) return;
  const int64_t p = pos[row];
  float cosv[4], sinv[4];
  if (CS_F32) {
    const float* c = reinterpret_cast<const float*>(cs) + p * D;
    float4 c4 = *reinterpret_cast<const float4*>(c + j * 4);
    float4 s4 = *reinterpret_cast<const float4*>(c + HALF + j * 4);
    cosv[0] = c4.x; cosv[1] = c4.y; cosv[2] = c4.z; cosv[3] = c4.w;
    sinv[0] = s4.x; sinv[1] = s4.y; sinv[2] = s4.z; sinv[3] = s4.w;
  } else {
    const uint16_t* c = reinterpret_cast<const uint16_t*>(cs) + p * D;
    bf16x4_to_f32(*reinterpret_cast<const uint2*>(c + j * 4), cosv);
    bf16x4_to_f32(*reinterpret_cast<const uint2*>(c + HALF + j * 4), sinv);
  }
  const int first = qo ? 0 : HQ;
  for (int h0 = first; h0 < total; h0 += HPB) {
    const int h = h0 + slot;
    const bool live = h < total;  // uniform across the LPH lanes of a head
    const bool is_q = h < HQ;
    const uint16_t* wt = is_q ? qw : kw;
    const int hin = live ? h : 0;
    float a[4], b[4], wa[4], wb[4], oa[4], ob[4];
    bf16x4_to_f32(*reinterpret_cast<const uint2*>(xrow + hin * D + j * 4), a);
    bf16x4_to_f32(*reinterpret_cast<const uint2*>(xrow + hin * D + HALF + j * 4), b);
    const float ss = group_sum<LPH>(norm_part4(a, b));
    const float rstd = norm_rstd<D>(ss, eps);
    bf16x4_to_f32(*reinterpret_cast<const uint2*>(wt + j * 4), wa);
    bf16x4_to_f32(*reinterpret_cast<const uint2*>(wt + HALF + j * 4), wb);
    norm_rope4(a, b, wa, wb, cosv, sinv, rstd, oa, ob);
    if (live && (is_q || !POOL || drow >= 0)) {
      uint16_t* out = is_q    ? qo + (int64_t)row * qo_ld + h * D
                      : POOL ? kp + drow * kv_row + (h - HQ) * D
                             : ko + (int64_t)row * ko_ld + (h - HQ) * D;
      *reinterpret_cast<uint2*>(out + j * 4) = make_uint2(pack2_bf16(oa[0], oa[1]), pack2_bf16(oa[2], oa[3]));
      *reinterpret_cast<uint2*>(out + HALF + j * 4) =
          make_uint2(pack2_bf16(ob[0], ob[1]), pack2_bf16(ob[2], ob[3]));
    }
    if (POOL && live && !is_q && drow2 >= 0) {
      uint16_t* out = kp2 + drow2 * kv_row + (h - HQ) * D;
      *reinterpret_cast<uint2*>(out + j * 4) = make_uint2(pack2_bf16(oa[0], oa[1]), pack2_bf16(oa[2], oa[3]));
      *reinterpret_cast<uint2*>(out + HALF + j * 4) =
          make_uint2(pack2_bf16(ob[0], ob[1]), pack2_bf16(ob[2], ob[3]));
    }
  }
}

// ---------------------------------------------------------------------------
// Per-token 128-group quant of a bf16 matrix, optionally of silu(g) * u.
// One wave per (row, 512 columns): lane holds 8 columns; a group is 16 lanes.
// SILU: input row is [g (I) | u (I)], y = g * sigmoid(g) * u in fp32
// (attention.py:771-793); otherwise y = x (vLLM per_token_group_quant_fp8).
template <bool SILU>
__global__ __launch_bounds__(256) void group_quant_kernel(const uint16_t* __restrict__ x,
                                                          int64_t x_ld, uint8_t* __restrict__ q,
                                                          int64_t q_ld, float* __restrict__ scales,
                                                          int64_t s_ld, int n, int I, int blocks) {
  const int lane = threadIdx.x & 63;
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= n * blocks) return;
  const int row = wid / blocks;
  const int blk = wid % blocks;
  const int col = blk * 512 + lane * 8;
  const bool live = col < I;
  const uint16_t* xrow = x + (int64_t)row * x_ld;
  float y[8];
  float amax = 0.f;
  if (live) {
    uint4 g = *reinterpret_cast<const uint4*>(xrow + col);
    uint32_t gw[4] = {g.x, g.y, g.z, g.w};
    if (SILU) {
      uint4 u = *reinterpret_cast<const uint4*>(xrow + I + col);
      uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        y[2 * k] = silu_mul(lo_bf16(gw[k]), lo_bf16(uw[k]));
        y[2 * k + 1] = silu_mul(hi_bf16(gw[k]), hi_bf16(uw[k]));
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        y[2 * k] = lo_bf16(gw[k]);
        y[2 * k + 1] = hi_bf16(gw[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(y[k]));
  }
  amax = group_max<16>(amax);
  const float scale = fp8_scale(amax);
  const float rs = recip(scale);
  // the SiLU rows divide as the gate_up GEMM's fused epilogue does
  auto quot = [&](float v) { return SILU ? silu_quot(v, rs) : div_by(v, scale, rs); };
  if (live) {
    uint2 o;
    o.x = pack4_fp8(quot(y[0]), quot(y[1]), quot(y[2]), quot(y[3]));
    o.y = pack4_fp8(quot(y[4]), quot(y[5]), quot(y[6]), quot(y[7]));
    *reinterpret_cast<uint2*>(q + (int64_t)row * q_ld + col) = o;
    if ((lane & 15) == 0) scales[(int64_t)(col >> 7) * s_ld + row] = scale;
  }
}

// ---------------------------------------------------------------------------
// pool[dst[i]] = rows[src[i]] for K and V; dst < 0 writes nothing
// (attention.py:885-897); without src and dst, row i goes to row i. One
// wave per pair; rows are row_elems 16-bit values. V_F16: V source rows are
// bf16 and the V pool holds fp16 (pack2_f16_sat: round to nearest even,
// saturated at +-65504); otherwise both are copied as they are.
template <bool V_F16>
__global__ __launch_bounds__(256) void kv_scatter_kernel(
    const uint16_t* __restrict__ k, int64_t k_ld, const uint16_t* __restrict__ v, int64_t v_ld,
    uint16_t* __restrict__ kp, uint16_t* __restrict__ vp, const int64_t* __restrict__ src,
    const int64_t* __restrict__ dst, int count, int row_elems) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= count) return;
  const int64_t d = dst ? dst[i] : i;
  if (d < 0) return;
  const int64_t s = src ? src[i] : i;
  const uint4* ks = reinterpret_cast<const uint4*>(k + s * k_ld);
  const uint4* vs = reinterpret_cast<const uint4*>(v + s * v_ld);
  uint4* kd = reinterpret_cast<uint4*>(kp + d * row_elems);
  uint4* vd = reinterpret_cast<uint4*>(vp + d * row_elems);
  const int nch = row_elems >> 3;
  for (int c = lane; c < nch; c += 64) {
    kd[c] = ks[c];
    vd[c] = V_F16 ? bf16x8_to_f16(vs[c]) : vs[c];
  }
}

__global__ __launch_bounds__(256) void embed_kernel(const uint16_t* __restrict__ table,
                                                    int64_t t_ld, const int64_t* __restrict__ ids,
                                                    uint16_t* __restrict__ out, int64_t o_ld,
                                                    int n, int H) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n) return;
  const uint4* s = reinterpret_cast<const uint4*>(table + ids[row] * t_ld);
  uint4* d = reinterpret_cast<uint4*>(out + (int64_t)row * o_ld);
  for (int c = lane; c < (H >> 3); c += 64) d[c] = s[c];
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace
}  // namespace qx

using namespace qx;

extern "C" {

int qx_add_rmsnorm_quant(const void* x, int64_t x_ld, void* res, int64_t res_ld, const void* w,
                         void* q, int64_t q_ld, float* scales, int64_t s_ld, int64_t n, int64_t H,
                         float eps, hipStream_t stream) {
  QX_CHECK(x && res && w && q && scales, "add_rmsnorm_quant: null pointer");
  QX_CHECK(H > 0 && H % 128 == 0 && H <= 8192, "add_rmsnorm_quant: hidden %lld", (long long)H);
  QX_CHECK(x_ld % 8 == 0 && res_ld % 8 == 0 && q_ld % 8 == 0, "add_rmsnorm_quant: strides");
  QX_CHECK(aligned16(x) && aligned16(res) && aligned16(w), "add_rmsnorm_quant: alignment");
  QX_CHECK(s_ld >= n, "add_rmsnorm_quant: s_ld < n");
  if (n == 0) return QX_OK;
  return launch_norm_quant<0>(x, x_ld, res, res_ld, nullptr, w, q, q_ld, scales, s_ld, (int)n,
                              (int)H, eps, stream);
}

int qx_rmsnorm_quant(const void* x, int64_t x_ld, const void* w, void* q, int64_t q_ld,
                     float* scales, int64_t s_ld, int64_t n, int64_t H, float eps,
                     hipStream_t stream) {
  QX_CHECK(x && w && q && scales, "rmsnorm_quant: null pointer");
  QX_CHECK(H > 0 && H % 128 == 0 && H <= 8192, "rmsnorm_quant: hidden %lld", (long long)H);
  QX_CHECK(x_ld % 8 == 0 && q_ld % 8 == 0, "rmsnorm_quant: strides");
  QX_CHECK(aligned16(x) && aligned16(w), "rmsnorm_quant: alignment");
  QX_CHECK(s_ld >= n, "rmsnorm_quant: s_ld < n");
  if (n == 0) return QX_OK;
  return launch_norm_quant<1>(x, x_ld, nullptr, 0, nullptr, w, q, q_ld, scales, s_ld, (int)n,
                              (int)H, eps, stream);
}

int qx_embed_rmsnorm_quant(const void* table, int64_t t_ld, const int64_t* ids, void* res,
                           int64_t res_ld, const void* w, void* q, int64_t q_ld, float* scales,
                           int64_t s_ld, int64_t n, int64_t H, float eps, hipStream_t stream) {
  QX_CHECK(table && ids && res && w && q && scales, "embed_rmsnorm_quant: null pointer");
  QX_CHECK(H > 0 && H % 128 == 0 && H <= 8192, "embed_rmsnorm_quant: hidden %lld", (long long)H);
  QX_CHECK(t_ld % 8 == 0 && res_ld % 8 == 0 && q_ld % 8 == 0, "embed_rmsnorm_quant: strides");
  QX_CHECK(aligned16(table) && aligned16(res) && aligned16(w), "embed_rmsnorm_quant: alignment");
  QX_CHECK(s_ld >= n, "embed_rmsnorm_quant: s_ld < n");
  if (n == 0) return QX_OK;
  return launch_norm_quant<2>(table, t_ld, res, res_ld, ids, w, q, q_ld, scales, s_ld, (int)n,
                              (int)H, eps, stream);
}

int qx_add_rmsnorm(const void* h, int64_t h_ld, const void* r, int64_t r_ld, const int64_t* rows,
                   const void* w, void* out, int64_t out_ld, void* res_out, int64_t res_out_ld,
                   int64_t n, int64_t H, float eps, hipStream_t stream) {
  QX_CHECK(h && r && w && out, "add_rmsnorm: null pointer");
  QX_CHECK(H > 0 && H % 8 == 0 && H <= 8192, "add_rmsnorm: hidden %lld", (long long)H);
  QX_CHECK(h_ld % 8 == 0 && r_ld % 8 == 0 && out_ld % 8 == 0 && res_out_ld % 8 == 0,
           "add_rmsnorm: strides");
  if (n == 0) return QX_OK;
  const int niter = ((int)H / 8 + 63) / 64;
  dim3 grid(((int)n + 3) / 4), block(kRowThreads);
#define QX_AR_CASE(NI)                                                                       \
  case NI:                                                                                   \
    hipLaunchKernelGGL(add_rmsnorm_kernel<NI>, grid, block, 0, stream, (const uint16_t*)h,  \
                       h_ld, (const uint16_t*)r, r_ld, rows, (const uint16_t*)w,             \
                       (uint16_t*)out, out_ld, (uint16_t*)res_out, res_out_ld, (int)n,      \
                       (int)H, eps);                                                         \
    break;
  switch (niter) {
    QX_AR_CASE(1)
    QX_AR_CASE(2)
    QX_AR_CASE(3)
    QX_AR_CASE(4)
    QX_AR_CASE(5)
    QX_AR_CASE(6)
    QX_AR_CASE(7)
    QX_AR_CASE(8)
    QX_AR_CASE(9)
    QX_AR_CASE(10)
    QX_AR_CASE(11)
    QX_AR_CASE(12)
    QX_AR_CASE(13)
    QX_AR_CASE(14)
    QX_AR_CASE(15)
    QX_AR_CASE(16)
    default:
      QX_CHECK(false, "add_rmsnorm: hidden too large");
  }
#undef QX_AR_CASE
  QX_LAUNCH_STATUS();
}

namespace {
int qk_norm_rope_launch(const void* qkv, int64_t qkv_ld, void* q_out, int64_t q_ld, void* k_out,
                        int64_t k_ld, const void* cos_sin, int cs_is_f32,
                        const int64_t* positions, const void* q_w, const void* k_w, int64_t n,
                        int64_t HQ, int64_t HK, int64_t D, float eps, void* k_pool, void* v_pool,
                        const int64_t* dst, void* k_pool2, void* v_pool2, const int64_t* dst2,
                        int v_f16, hipStream_t stream) {
  QX_CHECK(D == 64 || D == 128, "qk_norm_rope: head_dim %lld (64 or 128)", (long long)D);
  QX_CHECK(HQ > 0 && HK > 0, "qk_norm_rope: heads");
  QX_CHECK(qkv_ld % 4 == 0 && q_ld % 4 == 0 && k_ld % 4 == 0, "qk_norm_rope: strides");
  if (n == 0) return QX_OK;
  dim3 grid((unsigned)n), block(256);
#define QX_QK(DD, F32, P, VF)                                                                  \
  hipLaunchKernelGGL((qk_norm_rope_kernel<DD, F32, P, VF>), grid, block, 0, stream,            \
                     (const uint16_t*)qkv, qkv_ld, (uint16_t*)q_out, q_ld, (uint16_t*)k_out,  \
                     k_ld, cos_sin, positions, (const uint16_t*)q_w, (const uint16_t*)k_w,    \
                     (int)n, (int)HQ, (int)HK, eps, (uint16_t*)k_pool, (uint16_t*)v_pool, dst, \
                     (uint16_t*)k_pool2, (uint16_t*)v_pool2, dst2)
#define QX_QK_D(DD, P, VF) \
  if (cs_is_f32) QX_QK(DD, true, P, VF); else QX_QK(DD, false, P, VF);
  if (dst && v_f16) {
    if (D == 128) { QX_QK_D(128, true, true) } else { QX_QK_D(64, true, true) }
  } else if (dst) {
    if (D == 128) { QX_QK_D(128, true, false) } else { QX_QK_D(64, true, false) }
  } else {
    if (D == 128) { QX_QK_D(128, false, false) } else { QX_QK_D(64, false, false) }
  }
#undef QX_QK_D
#undef QX_QK
  QX_LAUNCH_STATUS();
}
}  // namespace

int qx_qk_norm_rope(const void* qkv, int64_t qkv_ld, void* q_out, int64_t q_ld, void* k_out,
                    int64_t k_ld, const void* cos_sin, int cs_is_f32, const int64_t* positions,
                    const void* q_w, const void* k_w, int64_t n, int64_t HQ, int64_t HK, int64_t D,
                    float eps, hipStream_t stream) {
  QX_CHECK(qkv && q_out && k_out && cos_sin && positions && q_w && k_w,
           "qk_norm_rope: null pointer");
  return qk_norm_rope_launch(qkv, qkv_ld, q_out, q_ld, k_out, k_ld, cos_sin, cs_is_f32,
                             positions, q_w, k_w, n, HQ, HK, D, eps, nullptr, nullptr, nullptr,
                             nullptr, nullptr, nullptr, 0, stream);
}

int qx_qk_norm_rope_kv(const void* qkv, int64_t qkv_ld, void* q_out, int64_t q_ld, void* k_pool,
                       void* v_pool, const int64_t* dst, void* k_pool2, void* v_pool2,
                       const int64_t* dst2, const void* cos_sin, int cs_is_f32,
                       const int64_t* positions, const void* q_w, const void* k_w, int64_t n,
                       int64_t HQ, int64_t HK, int64_t D, float eps, int v_f16,
                       hipStream_t stream) {
  QX_CHECK(qkv && k_pool && v_pool && dst && cos_sin && positions && q_w && k_w,
           "qk_norm_rope_kv: null pointer");
  QX_CHECK(!dst2 || (k_pool2 && v_pool2), "qk_norm_rope_kv: second destination pools");
  QX_CHECK(qkv_ld % 8 == 0 && aligned16(qkv) && aligned16(k_pool) && aligned16(v_pool) &&
               (!dst2 || (aligned16(k_pool2) && aligned16(v_pool2))),
           "qk_norm_rope_kv: alignment");
  return qk_norm_rope_launch(qkv, qkv_ld, q_out, q_ld, nullptr, 0, cos_sin, cs_is_f32, positions,
                             q_w, k_w, n, HQ, HK, D, eps, k_pool, v_pool, dst, k_pool2, v_pool2,
                             dst2, v_f16, stream);
}

int qx_silu_mul_quant(const void* gate_up, int64_t gu_ld, void* q, int64_t q_ld, float* scales,
                      int64_t s_ld, int64_t n, int64_t I, hipStream_t stream) {
  QX_CHECK(gate_up && q && scales, "silu_mul_quant: null pointer");
  QX_CHECK(I > 0 && I % 128 == 0, "silu_mul_quant: intermediate %lld", (long long)I);
  QX_CHECK(gu_ld % 8 == 0 && q_ld % 8 == 0 && aligned16(gate_up), "silu_mul_quant: strides");
  QX_CHECK(s_ld >= n, "silu_mul_quant: s_ld < n");
  if (n == 0) return QX_OK;
  const int blocks = (int)((I + 511) / 512);
  const int64_t waves = n * blocks;
  hipLaunchKernelGGL(group_quant_kernel<true>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     stream, (const uint16_t*)gate_up, gu_ld, (uint8_t*)q, q_ld, scales, s_ld,
                     (int)n, (int)I, blocks);
  QX_LAUNCH_STATUS();
}

int qx_group_quant(const void* x, int64_t x_ld, void* q, int64_t q_ld, float* scales,
                   int64_t s_ld, int64_t n, int64_t K, hipStream_t stream) {
  QX_CHECK(x && q && scales, "group_quant: null pointer");
  QX_CHECK(K > 0 && K % 128 == 0, "group_quant: width %lld", (long long)K);
  QX_CHECK(x_ld % 8 == 0 && q_ld % 8 == 0 && aligned16(x), "group_quant: strides");
  QX_CHECK(s_ld >= n, "group_quant: s_ld < n");
  if (n == 0) return QX_OK;
  const int blocks = (int)((K + 511) / 512);
  const int64_t waves = n * blocks;
  hipLaunchKernelGGL(group_quant_kernel<false>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0,
                     stream, (const uint16_t*)x, x_ld, (uint8_t*)q, q_ld, scales, s_ld, (int)n,
                     (int)K, blocks);
  QX_LAUNCH_STATUS();
}

int qx_kv_scatter(const void* k, int64_t k_ld, const void* v, int64_t v_ld, void* k_pool,
                  void* v_pool, const int64_t* src, const int64_t* dst, int64_t count,
                  int64_t row_elems, int v_to_f16, hipStream_t stream) {
  QX_CHECK(k && v && k_pool && v_pool && (src != nullptr) == (dst != nullptr),
           "kv_scatter: null pointer");
  QX_CHECK(row_elems > 0 && row_elems % 8 == 0, "kv_scatter: row %lld", (long long)row_elems);
  QX_CHECK(k_ld % 8 == 0 && v_ld % 8 == 0 && aligned16(k) && aligned16(v) && aligned16(k_pool) &&
               aligned16(v_pool),
           "kv_scatter: alignment");
  if (count == 0) return QX_OK;
  if (v_to_f16)
    hipLaunchKernelGGL(kv_scatter_kernel<true>, dim3((unsigned)((count + 3) / 4)), dim3(256), 0,
                       stream, (const uint16_t*)k, k_ld, (const uint16_t*)v, v_ld,
                       (uint16_t*)k_pool, (uint16_t*)v_pool, src, dst, (int)count,
                       (int)row_elems);
  else
    hipLaunchKernelGGL(kv_scatter_kernel<false>, dim3((unsigned)((count + 3) / 4)), dim3(256), 0,
                       stream, (const uint16_t*)k, k_ld, (const uint16_t*)v, v_ld,
                       (uint16_t*)k_pool, (uint16_t*)v_pool, src, dst, (int)count,
                       (int)row_elems);
  QX_LAUNCH_STATUS();
}

int qx_embed(const void* table, int64_t t_ld, const int64_t* ids, void* out, int64_t o_ld,
             int64_t n, int64_t H, hipStream_t stream) {
  QX_CHECK(table && ids && out, "embed: null pointer");
  QX_CHECK(H % 8 == 0 && t_ld % 8 == 0 && o_ld % 8 == 0 && aligned16(table) && aligned16(out),
           "embed: alignment");
  if (n == 0) return QX_OK;
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, stream,
                     (const uint16_t*)table, t_ld, ids, (uint16_t*)out, o_ld, (int)n, (int)H);
  QX_LAUNCH_STATUS();
}

}  // extern "C"
