// moe_device.h -- device helpers shared by the gfx950 MoE kernels.
//
// Activations are fp32, fp16 (_Float16) or bf16 (raw uint16_t bits; bf16 <->
// fp32 conversion is done on bits, round-to-nearest-even, the same rounding as
// the reference's float32_to_bfloat16_bits, test/ops/op_test_utils.py:235-245).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

constexpr int kWave = 64;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Element tags.
struct F32 { using storage = float; static constexpr int kId = 1; };
struct F16 { using storage = _Float16; static constexpr int kId = 10; };
struct BF16 { using storage = uint16_t; static constexpr int kId = 16; };
// OCP Microscaling (MX v1.0) E8M0 block scale: 2^(e - 127), e = 255 is NaN.
struct E8M0 { using storage = uint8_t; static constexpr int kId = 2; };

__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  return e == 0 ? __uint_as_float(0x00400000u) : (e == 255 ? __uint_as_float(0x7FC00000u) : __uint_as_float(e << 23));
}

// OCP MX FP4 E2M1 element (sign, 2 exponent bits with bias 1, 1 mantissa
// bit): 0, 0.5, 1, 1.5, 2, 3, 4, 6 and their negatives.
__device__ __forceinline__ float e2m1_to_f32(uint32_t n) {
  const uint32_t e = (n >> 1) & 3u, m = n & 1u;
  const float mag = e == 0 ? 0.5f * static_cast<float>(m) : __builtin_ldexpf(1.0f + 0.5f * static_cast<float>(m), static_cast<int>(e) - 1);
  return (n & 8u) ? -mag : mag;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
// Round to nearest even (gfx950 converts in hardware, v_cvt_pk_bf16_f32; NaN
// stays a quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

template <typename Tag>
__device__ __forceinline__ float to_f32(typename Tag::storage v);
template <>
__device__ __forceinline__ float to_f32<F32>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<F16>(_Float16 v) { return static_cast<float>(v); }
template <>
__device__ __forceinline__ float to_f32<BF16>(uint16_t v) { return bf16_to_f32(v); }
template <>
__device__ __forceinline__ float to_f32<E8M0>(uint8_t v) { return e8m0_to_f32(v); }

template <typename Tag>
__device__ __forceinline__ typename Tag::storage from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<F32>(float v) { return v; }
template <>
__device__ __forceinline__ _Float16 from_f32<F16>(float v) { return static_cast<_Float16>(v); }
template <>
__device__ __forceinline__ uint16_t from_f32<BF16>(float v) { return f32_to_bf16(v); }

// Load one element of a runtime-typed buffer (scales, biases) as fp32.
__device__ __forceinline__ float load_any(const void* p, int elem_type, int64_t i) {
  if (elem_type == 1) return static_cast<const float*>(p)[i];
  if (elem_type == 10) return static_cast<float>(static_cast<const _Float16*>(p)[i]);
  return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// ---- wave reductions (64 lanes, butterfly over __shfl_xor) ----
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// ---- activations (fp32) ----
enum Act : int { kRelu = 0, kGelu = 1, kSilu = 2, kIdentity = 3, kSwiglu = 4 };

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

// FAST: sigmoid from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32;
// about 1 ulp each, far below the 16-bit output rounding of the MFMA paths).
// Saturates correctly: exp2 overflows to +inf -> 0, underflows to 0 -> 1.
template <bool FAST>
__device__ __forceinline__ float sigmoid_t(float x) {
  if constexpr (FAST) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
  } else {
    return sigmoid_f(x);
  }
}

template <bool FAST = false>
__device__ __forceinline__ float act_single(float x, int act) {
  switch (act) {
    case kRelu: return x > 0.0f ? x : 0.0f;
    case kGelu: return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
    case kSilu: return x * sigmoid_t<FAST>(x);
    default: return x;
  }
}

// SwiGLU with clamp: G = min(g, limit), L = clamp(l, -limit, limit),
// out = G * sigmoid(alpha * G) * (L + beta).
template <bool FAST = false>
__device__ __forceinline__ float swiglu_f(float g, float l, float alpha, float beta, float limit) {
  g = fminf(g, limit);
  l = fminf(fmaxf(l, -limit), limit);
  return g * sigmoid_t<FAST>(alpha * g) * (l + beta);
}

// Combines a gate value and (if gated) a linear value into one activation.
// gated == false: act(g).  activation == swiglu: swiglu(g, l).  Otherwise
// act(g) * l (fc3 gating).  FAST selects the hardware sigmoid (16-bit outputs).
template <bool FAST = false>
__device__ __forceinline__ float apply_act(float g, float l, bool gated, int act, float alpha, float beta,
                                           float limit) {
  if (!gated) return act_single<FAST>(g, act);
  if (act == kSwiglu) return swiglu_f<FAST>(g, l, alpha, beta, limit);
  return act_single<FAST>(g, act) * l;
}

}  // namespace moe
