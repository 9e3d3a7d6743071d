// Shared device helpers for the gfx950 DiT estimator kernels.
//
// Conventions used by every kernel in this library:
//   * GEMM operands, attention operands and the weights are IEEE fp16 (type `f16` below);
//   * the residual stream and all boundary tensors are fp32;
//   * MFMA fragments follow the CDNA 16x16 / 32x32 accumulator layouts:
//       16x16x32 : lane l holds D[4*(l/16) + j][l%16], j = 0..3
//       32x32x16 : lane l holds D[8*(i/4) + 4*(l/32) + i%4][l%32], i = 0..15
//     Operand slots are loaded with the same (lane, slot) -> k rule for A and
//     B, so the result does not depend on the hardware's k order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fcv {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

__device__ __forceinline__ float h2f(f16 v) { return (float)v; }

// fp32 -> fp16 conversions, round to nearest even from the fp32 values as computed.  The empty
// asm pins those values: left to itself the backend fuses a product that feeds a conversion
// into v_fma_mix, which rounds the exact product once instead of twice, and it does so in some
// template instantiations and not in others, so an output's bits would depend on the GEMM tile
// shape (and so on the batch a document is packed with).  The asm emits no instruction.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ f16x2 f2h2(float a, float b) {
  asm("" : "+v"(a), "+v"(b));
  return f16x2{(f16)a, (f16)b};
}
__device__ __forceinline__ f16 f2h(float v) { return f2h2(v, v)[0]; }
__device__ __forceinline__ f16x4 f2h4(float a, float b, float c, float d) {
  const f16x2 lo = f2h2(a, b), hi = f2h2(c, d);
  return f16x4{lo[0], lo[1], hi[0], hi[1]};
}

__device__ __forceinline__ f32x4 mfma16(const f16x8& a, const f16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(const f16x8& a, const f16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Reductions over the 64 lanes of a wave without LDS round trips: DPP inside each row of 16
// lanes (quad swaps, half-row mirror, row mirror), then v_permlane16_swap (rows 0<->1, 2<->3)
// and v_permlane32_swap (halves).  Every lane ends with the same value, combined in a fixed
// order.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}
__device__ __forceinline__ float swap16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_f<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  return swap32_sum(swap16_sum(v));
}

// Hardware transcendentals (v_exp_f32 = 2^x, v_rcp_f32 = 1/x; about 1 ulp each).
__device__ __forceinline__ float hw_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float hw_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// tanh-approximated GELU (torch nn.GELU(approximate="tanh")):
//   0.5 x (1 + tanh(u)) = x / (1 + e^(-2u)),  u = sqrt(2/pi) (x + 0.044715 x^3),
// with -2 u log2(e) = x (c0 + c1 x^2): three VALU operations before the exponential.
// For x -> -inf, e^(-2u) overflows to inf and the result is -0; for x -> +inf it is x.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float c0 = -2.302208198144325f;    // -2 log2(e) sqrt(2/pi)
  const float c1 = -0.1029432395800235f;   // c0 * 0.044715
  return x * hw_rcp(1.0f + hw_exp2(x * fmaf(c1, x * x, c0)));
}

// Mish: x * tanh(softplus(x)).  With e = e^x, tanh(log(1 + e)) = n / (n + 2), n = e (e + 2).
// Above 20 torch's softplus returns x itself, and tanh(x) rounds to 1 in fp32.
__device__ __forceinline__ float mish(float x) {
  if (x > 20.0f) return x;
  const float e = hw_exp2(1.4426950408889634f * x);
  const float n = e * (e + 2.0f);
  return x * n * hw_rcp(n + 2.0f);
}

__device__ __forceinline__ float silu(float x) { return x * hw_rcp(1.0f + hw_exp2(-1.4426950408889634f * x)); }

}  // namespace fcv
