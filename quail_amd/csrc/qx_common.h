// Device helpers shared by the gfx950 kernels of libquail_mi355x.
//
// Number formats follow the reference's arithmetic:
//   * bf16 is stored as uint16_t and rounded from fp32 to nearest even, as
//     torch's `.to(torch.bfloat16)` and Triton's `.to(tl.bfloat16)` do.
//   * FP8 is OCP e4m3fn (max 448), the format of Qwen3 FP8 checkpoints
//     (quail/specs/qwen3.py:16). Values are clamped to +-448 before the
//     hardware round-to-nearest-even conversion, which is the reference's
//     `clamp(x / s, -448, 448).to(e4m3)` (attention.py:782-786).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qx {

constexpr float kFp8Max = 448.0f;
constexpr float kScaleFloor = 1e-10f;  // attention.py:781 `max(amax, 1e-10)`
constexpr int kGroup = 128;            // per-token FP8 group (attention.py GROUP)

typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;  // NaN stays NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Round an fp32 value through bf16 and back (the reference stores bf16
// intermediates between kernels): gfx950's conversion (v_cvt_pk_bf16_f32,
// round to nearest even, the same bits as f32_to_bf16 for every non-NaN
// value; a NaN stays a NaN), two instructions where f32_to_bf16 takes five.
__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f)));
}

// Four fp32 values -> four packed e4m3fn bytes (little-endian order).
// Every caller passes values divided by their group's scale, amax / 448
// (div_by with fp8_scale), so |x| <= 448 up to an ulp of the quotient,
// which the conversion rounds to +-448: the reference's clamp to +-448
// (attention.py:786-787) changes nothing there and is not repeated. NaN
// converts to the NaN code, as the clamp would have kept it.
__device__ __forceinline__ uint32_t pack4_fp8(float a, float b, float c, float d) {
  int v = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  v = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, v, true);
  return static_cast<uint32_t>(v);
}

// Unpack two bf16 held in one 32-bit word.
__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16 (round to nearest even): one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  const bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// fp32 clamped to fp16's finite range; NaN stays NaN (fminf / fmaxf return
// the operand that is not NaN, so NaN is passed around the clamp)
__device__ __forceinline__ float clamp_f16_range(float x) {
  return x != x ? x : fminf(fmaxf(x, -65504.0f), 65504.0f);
}

// Two fp32 -> packed fp16, round to nearest even, saturated at +-65504 (a
// value past fp16's range, infinities included, becomes its largest finite
// value; NaN stays NaN, as it does in the reference's bf16 pools).
__device__ __forceinline__ uint32_t pack2_f16_sat(float lo, float hi) {
  const f16x2 v = {(_Float16)clamp_f16_range(lo), (_Float16)clamp_f16_range(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// The 8 bf16 of a 16-byte chunk as fp16 (pack2_f16_sat).
__device__ __forceinline__ uint4 bf16x8_to_f16(uint4 w) {
  w.x = pack2_f16_sat(lo_bf16(w.x), hi_bf16(w.x));
  w.y = pack2_f16_sat(lo_bf16(w.y), hi_bf16(w.y));
  w.z = pack2_f16_sat(lo_bf16(w.z), hi_bf16(w.z));
  w.w = pack2_f16_sat(lo_bf16(w.w), hi_bf16(w.w));
  return w;
}

// v of another lane of the same 16-lane DPP row: CTRL is a DPP control
// (quad_perm 0x00-0xff, row_mirror 0x140, row_half_mirror 0x141); a VALU
// operand modifier, no LDS permute.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Butterfly reductions across `width` consecutive lanes of a wave64. The
// max over an aligned group of 16 (one DPP row) takes four DPP moves:
// lane ^ 1 and lane ^ 2 (quad_perm [1,0,3,2], [2,3,0,1]) leave each quad's
// max on its lanes, the mirror within the half row pairs each quad with
// the other one, the mirror within the row each half with the other. Max
// is order-free (fmaxf drops a NaN operand either way), so the result is
// the permute butterfly's.
template <int width>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (width == 16) {
    v = fmaxf(v, dpp_f32<0xb1>(v));
    v = fmaxf(v, dpp_f32<0x4e>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    return fmaxf(v, dpp_f32<0x140>(v));
  } else {
#pragma unroll
    for (int o = width / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
  }
}

template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = width / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Max / sum of x over lanes l and l ^ 32 (the two halves of a wave64),
// through one v_permlane32_swap instead of an LDS permute: after the swap
// the pair holds (x[l], x[l + 32]) on lanes l < 32 and (x[l - 32], x[l]) on
// the others.
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Workgroup barrier with no memory fence. __syncthreads() (and an
// LDS-scoped fence) make the compiler drain every vector-memory load in
// flight before s_barrier, including the global->LDS prefetches of later
// pipeline stages. Kernels using this barrier wait for their own LDS-bound
// loads explicitly (s_waitcnt vmcnt) and consume every ds_read result before
// the barrier; the "memory" clobber keeps the compiler from moving memory
// accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// v as an opaque value where this call stands: the compiler cannot move
// what is computed from it out of an enclosing loop, so per-lane addresses
// that a loop's tail uses are recomputed there instead of being kept live
// (or spilled) across the loop's body.
__device__ __forceinline__ int opaque(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

// s_waitcnt with vmcnt <= n and the other counters unconstrained (gfx9
// encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14));
}

typedef __attribute__((address_space(3))) uint8_t lds_u8;

// Direct HBM -> LDS load of 16 bytes per lane (lane i writes lds + 16 i),
// written as inline assembly so that the compiler does not track it as an
// LDS write: it would otherwise wait for every such load in flight before
// any later LDS read, including reads of other buffers. Callers order these
// loads with explicit s_waitcnt vmcnt and barriers. Loads the compiler does
// not count can only make its own vmcnt waits stricter (vector memory loads
// complete in order). M0 is saved and restored around the load.
__device__ __forceinline__ void lds_dma16(const void* src, const uint8_t* lds) {
  const uint32_t addr = (uint32_t)(uintptr_t)(lds_u8*)lds;
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 1\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(addr), "v"(src)
      : "memory");
}

// The same with device scope (sc1: the vector L1 keeps no copy), for
// operands every workgroup streams once.
__device__ __forceinline__ void lds_dma16_stream(const void* src, const uint8_t* lds) {
  const uint32_t addr = (uint32_t)(uintptr_t)(lds_u8*)lds;
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 1\n\t"
      "global_load_lds_dwordx4 %2, off sc1\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(addr), "v"(src)
      : "memory");
}

// 4 bytes per lane (lane i writes lds + 4 i), untracked like lds_dma16.
__device__ __forceinline__ void lds_dma4(const void* src, const uint8_t* lds) {
  const uint32_t addr = (uint32_t)(uintptr_t)(lds_u8*)lds;
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 1\n\t"
      "global_load_lds_dword %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(addr), "v"(src)
      : "memory");
}

// y / s from the hardware reciprocal r = rcp(s) and one FMA correction of
// the quotient (the residual y - q0 s is exact in an FMA), which gives the
// correctly rounded quotient except in rare ties of double rounding; three
// instructions instead of IEEE division's ten. Callers pass r once per group.
__device__ __forceinline__ float div_by(float y, float s, float r) {
  const float q0 = y * r;
  return fmaf(fmaf(-q0, s, y), r, q0);
}

// 1 / s to within an ulp: the hardware reciprocal refined by one Newton step.
__device__ __forceinline__ float recip(float s) {
  const float r = __builtin_amdgcn_rcpf(s);
  return fmaf(fmaf(-r, s, 1.0f), r, r);
}

// silu(g) * u in fp32 (attention.py:771-793): sigmoid(g) = 1 / (1 + e^-g),
// e^-g = 2^(-g log2 e) on v_exp_f32 and the reciprocal on v_rcp_f32 (each
// within an ulp, as the reference's approximate exp and division are);
// past |g| ~ 88 the exponential saturates to 0 or inf and sigmoid to 1 or
// 0. Shared by the SiLU-quant kernel and the gate_up GEMM's fused epilogue
// so both give the same bits.
__device__ __forceinline__ float silu_mul(float g, float u) {
  constexpr float kLog2e = 1.4426950408889634f;
  const float d = 1.0f + __builtin_amdgcn_exp2f(-g * kLog2e);
  return g * __builtin_amdgcn_rcpf(d) * u;
}

// y / s for the SiLU-quant rows as y times the scale's reciprocal r (within
// an ulp and a half of the quotient; the fp8 code then differs from the
// correctly rounded quotient's for about one value in a million, as the
// reference's approximate division may). Shared like silu_mul.
__device__ __forceinline__ float silu_quot(float y, float r) { return y * r; }

// qk-norm and neox RoPE (attention.py:833-879) in pieces shared by the
// qk-norm-rope pass and the attention's Q load, so both give the same bits;
// no fused multiply-adds: each product and sum rounds on its own. A head's
// column j-group is a[k] = x[4j + k] and b[k] = x[D/2 + 4j + k], k < 4.
//
// sum over k of a[k]^2 + b[k]^2, in k order
__device__ __forceinline__ float norm_part4(const float (&a)[4], const float (&b)[4]) {
#pragma clang fp contract(off)
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) ss += a[k] * a[k] + b[k] * b[k];
  return ss;
}

// 1 / sqrt(mean square + eps) of a head of D columns from its sum of squares
template <int D>
__device__ __forceinline__ float norm_rstd(float ss, float eps) {
#pragma clang fp contract(off)
  return 1.0f / sqrtf(ss / (float)D + eps);
}

// xa = a * rstd * wa, xb = b * rstd * wb; oa = xa cos - xb sin,
// ob = xb cos + xa sin (cos / sin of columns 4j + k)
__device__ __forceinline__ void norm_rope4(const float (&a)[4], const float (&b)[4],
                                           const float (&wa)[4], const float (&wb)[4],
                                           const float (&cosv)[4], const float (&sinv)[4],
                                           float rstd, float (&oa)[4], float (&ob)[4]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float xa = a[k] * rstd * wa[k];
    const float xb = b[k] * rstd * wb[k];
    oa[k] = xa * cosv[k] - xb * sinv[k];
    ob[k] = xb * cosv[k] + xa * sinv[k];
  }
}

// Four bf16 held in two words, as fp32.
__device__ __forceinline__ void bf16x4_to_f32(uint2 w, float (&x)[4]) {
  x[0] = lo_bf16(w.x); x[1] = hi_bf16(w.x); x[2] = lo_bf16(w.y); x[3] = hi_bf16(w.y);
}

// Per-group FP8 scale: max(amax, 1e-10) / 448 (attention.py:780-781),
// correctly rounded as the division is, in four operations instead of the
// division's ten: x / 448 = (x / 7) * 2^-6 exactly for these x (normal,
// and so are the quotients), and x / 7 is x * RN(1/7) corrected by one
// fma of the remainder, which gives the correctly rounded quotient for
// every fp32 significand (checked exhaustively). inf stays inf (the
// remainder of inf is NaN).
__device__ __forceinline__ float fp8_scale(float amax) {
#pragma clang fp contract(off)
  static_assert(kFp8Max == 448.0f, "448 = 7 * 2^6");
  constexpr float kSeventh = 1.0f / 7.0f;
  const float x = fmaxf(amax, kScaleFloor);
  const float q0 = x * kSeventh;
  const float q = __builtin_fmaf(__builtin_fmaf(-q0, 7.0f, x), kSeventh, q0);
  return (q0 == __builtin_inff() ? q0 : q) * 0.015625f;
}

}  // namespace qx

// Status codes of every extern "C" entry point.
#ifndef QX_OK
#define QX_OK 0
#define QX_EINVAL (-1)
#endif

// Record a launch error (if any) as the entry point's return value.
#define QX_LAUNCH_STATUS()                          \
  do {                                              \
    hipError_t _e = hipGetLastError();              \
    return _e == hipSuccess ? QX_OK : (int)_e;      \
  } while (0)
