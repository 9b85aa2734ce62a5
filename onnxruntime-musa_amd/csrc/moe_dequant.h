// moe_dequant.h -- in-register dequantisation of QMoE weights into MFMA
// operands (8 consecutive k of one weight row -> 8 x 16-bit in 4 dwords).
//
// Encoding (symmetric): int8 w = (q - 128) * s; int4 w = (nibble - 8) * s with
// the even-k element in the low nibble of each byte.
//
// "Exact" converters produce the integer (q - zero_point) as fp16/bf16, which
// is exact in both formats; the scale is then applied to fp32 MFMA partial
// sums.  "Scaled" converters fold the scale in before the MFMA (one rounding
// of (q - zp) * s to the 16-bit type), used where one MFMA's K range spans
// several scale blocks.
//
// fp16 converters use the magic-exponent trick: 0x6400 | q is the fp16 value
// 1024 + q for q < 1024, so one byte-permute/or builds two operands and one
// packed subtract removes the bias.
#pragma once

#include "moe_device.h"
#include "moe_launch.h"

namespace moe {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t h2_bits(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ half2_t bits_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }

// int4 dword (k0..k7) -> fp16 pairs of (nibble - 8), exact.  The nibble
// bytes are first put in k order (one permute per 4 k), then each output
// dword takes two of them under 0x64 high bytes (the magic 1024 + q) with a
// second permute against a constant, and one packed subtract removes 1032.
__device__ __forceinline__ u32x4_t dq4_f16_exact(uint32_t v) {
  const uint32_t x = v & 0x0F0F0F0Fu;         // k0, k2, k4, k6
  const uint32_t y = (v >> 4) & 0x0F0F0F0Fu;  // k1, k3, k5, k7
  const uint32_t z0 = __builtin_amdgcn_perm(y, x, 0x05010400u);  // bytes k0 k1 k2 k3
  const uint32_t z1 = __builtin_amdgcn_perm(y, x, 0x07030602u);  // bytes k4 k5 k6 k7
  const uint32_t c = 0x64646464u;
  const half2_t bias = {static_cast<_Float16>(1032.0f), static_cast<_Float16>(1032.0f)};
  u32x4_t r;
  r[0] = h2_bits(bits_h2(__builtin_amdgcn_perm(c, z0, 0x04010400u)) - bias);
  r[1] = h2_bits(bits_h2(__builtin_amdgcn_perm(c, z0, 0x04030402u)) - bias);
  r[2] = h2_bits(bits_h2(__builtin_amdgcn_perm(c, z1, 0x04010400u)) - bias);
  r[3] = h2_bits(bits_h2(__builtin_amdgcn_perm(c, z1, 0x04030402u)) - bias);
  return r;
}

// int8 dwords (k0..k3, k4..k7) -> fp16 pairs of (q - 128), exact.
__device__ __forceinline__ u32x4_t dq8_f16_exact(uint32_t v0, uint32_t v1) {
  const uint32_t c = 0x64646464u;
  const half2_t bias = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
  u32x4_t r;
  r[0] = h2_bits(bits_h2(__builtin_amdgcn_perm(c, v0, 0x04010400u)) - bias);
  r[1] = h2_bits(bits_h2(__builtin_amdgcn_perm(c, v0, 0x04030402u)) - bias);
  r[2] = h2_bits(bits_h2(__builtin_amdgcn_perm(c, v1, 0x04010400u)) - bias);
  r[3] = h2_bits(bits_h2(__builtin_amdgcn_perm(c, v1, 0x04030402u)) - bias);
  return r;
}

// Packs the bf16 images of two fp32 values whose low 16 bits are zero (small
// integers), lo in bits 0-15.
__device__ __forceinline__ uint32_t pack_bf16_exact(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

__device__ __forceinline__ u32x4_t dq4_bf16_exact(uint32_t v) {
  u32x4_t r;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint32_t byte = (v >> (8 * b)) & 0xFFu;
    const float lo = static_cast<float>(byte & 0xFu) - 8.0f;
    const float hi = static_cast<float>(byte >> 4) - 8.0f;
    r[b] = pack_bf16_exact(lo, hi);
  }
  return r;
}

__device__ __forceinline__ u32x4_t dq8_bf16_exact(uint32_t v0, uint32_t v1) {
  u32x4_t r;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    r[b] = pack_bf16_exact(static_cast<float>((v0 >> (16 * b)) & 0xFFu) - 128.0f,
                           static_cast<float>((v0 >> (16 * b + 8)) & 0xFFu) - 128.0f);
    r[2 + b] = pack_bf16_exact(static_cast<float>((v1 >> (16 * b)) & 0xFFu) - 128.0f,
                               static_cast<float>((v1 >> (16 * b + 8)) & 0xFFu) - 128.0f);
  }
  return r;
}

// Rounds two fp32 values to the 16-bit activation type and packs them.
template <typename AT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<F16>(float lo, float hi) {
  const half2_t h = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
  return h2_bits(h);
}
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <>
__device__ __forceinline__ uint32_t pack2<BF16>(float lo, float hi) {
  const bf16x2_t h = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};  // one v_cvt_pk_bf16_f32
  return __builtin_bit_cast(uint32_t, h);
}

// Scaled converters: 8 weights times per-element-group scale s -> 16-bit,
// one rounding of (q - zp) * s: the byte converts exactly to fp32 and one
// fma against the exact constant -zp * s (zp is a power of two) forms the
// product.
template <typename AT>
__device__ __forceinline__ u32x4_t dq4_scaled(uint32_t v, float s) {
  const uint32_t x = v & 0x0F0F0F0Fu;         // k0, k2, k4, k6
  const uint32_t y = (v >> 4) & 0x0F0F0F0Fu;  // k1, k3, k5, k7
  const float ns = -8.0f * s;
  u32x4_t r;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float lo = static_cast<float>((x >> (8 * b)) & 0xFFu);  // v_cvt_f32_ubyte<b>
    const float hi = static_cast<float>((y >> (8 * b)) & 0xFFu);
    r[b] = pack2<AT>(__builtin_fmaf(lo, s, ns), __builtin_fmaf(hi, s, ns));
  }
  return r;
}

template <typename AT>
__device__ __forceinline__ u32x4_t dq8_scaled(uint32_t v0, uint32_t v1, float s) {
  const float ns = -128.0f * s;
  u32x4_t r;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    r[b] = pack2<AT>(__builtin_fmaf(static_cast<float>((v0 >> (16 * b)) & 0xFFu), s, ns),
                     __builtin_fmaf(static_cast<float>((v0 >> (16 * b + 8)) & 0xFFu), s, ns));
    r[2 + b] = pack2<AT>(__builtin_fmaf(static_cast<float>((v1 >> (16 * b)) & 0xFFu), s, ns),
                         __builtin_fmaf(static_cast<float>((v1 >> (16 * b + 8)) & 0xFFu), s, ns));
  }
  return r;
}

template <typename AT>
__device__ __forceinline__ u32x4_t dq4_exact(uint32_t v);
template <>
__device__ __forceinline__ u32x4_t dq4_exact<F16>(uint32_t v) { return dq4_f16_exact(v); }
template <>
__device__ __forceinline__ u32x4_t dq4_exact<BF16>(uint32_t v) { return dq4_bf16_exact(v); }

template <typename AT>
__device__ __forceinline__ u32x4_t dq8_exact(uint32_t v0, uint32_t v1);
template <>
__device__ __forceinline__ u32x4_t dq8_exact<F16>(uint32_t v0, uint32_t v1) {
  return dq8_f16_exact(v0, v1);
}
template <>
__device__ __forceinline__ u32x4_t dq8_exact<BF16>(uint32_t v0, uint32_t v1) {
  return dq8_bf16_exact(v0, v1);
}

// 16x16x32 MFMA on 8 x 16-bit operands held as 4 dwords.
template <typename AT>
__device__ __forceinline__ floatx4_t mfma16x16x32(u32x4_t a, u32x4_t b, floatx4_t c);
template <>
__device__ __forceinline__ floatx4_t mfma16x16x32<F16>(u32x4_t a, u32x4_t b, floatx4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                                __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ floatx4_t mfma16x16x32<BF16>(u32x4_t a, u32x4_t b, floatx4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// 32x32x16 MFMA.
template <typename AT>
__device__ __forceinline__ floatx16_t mfma32x32x16(u32x4_t a, u32x4_t b, floatx16_t c);
template <>
__device__ __forceinline__ floatx16_t mfma32x32x16<F16>(u32x4_t a, u32x4_t b, floatx16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a),
                                                __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ floatx16_t mfma32x32x16<BF16>(u32x4_t a, u32x4_t b, floatx16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}


// "Biased" converters for the decode kernels: the 16-bit value of (B + q)
// with the zero point left in (B = 1024 for fp16, 128 for bf16), one fewer
// instruction per two weights than the exact form.  The kernel multiplies the
// activations by an all-ones operand in the same MFMA pipe to get their sums
// and removes (B + zp) * sum afterwards.
__device__ __forceinline__ u32x4_t dq4_f16_biased(uint32_t v) {  // 1024 + q
  const uint32_t x = v & 0x0F0F0F0Fu, y = (v >> 4) & 0x0F0F0F0Fu;
  const uint32_t z0 = __builtin_amdgcn_perm(y, x, 0x05010400u), z1 = __builtin_amdgcn_perm(y, x, 0x07030602u);
  const uint32_t c = 0x64646464u;
  return u32x4_t{__builtin_amdgcn_perm(c, z0, 0x04010400u), __builtin_amdgcn_perm(c, z0, 0x04030402u),
                 __builtin_amdgcn_perm(c, z1, 0x04010400u), __builtin_amdgcn_perm(c, z1, 0x04030402u)};
}
__device__ __forceinline__ u32x4_t dq4_bf16_biased(uint32_t v) {  // 128 + q
  const uint32_t x = v & 0x0F0F0F0Fu, y = (v >> 4) & 0x0F0F0F0Fu;
  const uint32_t z0 = __builtin_amdgcn_perm(y, x, 0x05010400u), z1 = __builtin_amdgcn_perm(y, x, 0x07030602u);
  const uint32_t c = 0x43434343u;
  return u32x4_t{__builtin_amdgcn_perm(c, z0, 0x04010400u), __builtin_amdgcn_perm(c, z0, 0x04030402u),
                 __builtin_amdgcn_perm(c, z1, 0x04010400u), __builtin_amdgcn_perm(c, z1, 0x04030402u)};
}
__device__ __forceinline__ u32x4_t dq8_f16_biased(uint32_t v0, uint32_t v1) {  // 1024 + q
  const uint32_t c = 0x64646464u;
  return u32x4_t{__builtin_amdgcn_perm(c, v0, 0x04010400u), __builtin_amdgcn_perm(c, v0, 0x04030402u),
                 __builtin_amdgcn_perm(c, v1, 0x04010400u), __builtin_amdgcn_perm(c, v1, 0x04030402u)};
}

// Whether the biased form exists for (activation type, weight format), and
// the value (B + zero point) it leaves in every weight.
template <typename AT, int WF>
struct Biased {
  static constexpr bool kOk = (AT::kId == 10 && (WF == kInt4 || WF == kInt8)) || (AT::kId == 16 && WF == kInt4);
  static constexpr float kOffset = AT::kId == 10 ? (WF == kInt4 ? 1032.0f : 1152.0f) : 136.0f;
  static constexpr uint32_t kOnes = AT::kId == 10 ? 0x3C003C00u : 0x3F803F80u;  // 1.0 pairs
};

// ---- raw buffer access ----
// Offset past every buffer range: a raw buffer load there returns 0 and makes
// no memory access.
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ u32x4_t bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 0));
}

// Weight operand of MFMA step s from a lane's 16-byte weight vectors: the
// 8 k of step s as 16-bit values (FOLD: times sc; otherwise exact integers).
template <typename AT, int WF, bool FOLD>
__device__ __forceinline__ u32x4_t weight_operand(const u32x4_t* v, int s, float sc) {
  if constexpr (WF == kInt4) {
    if constexpr (FOLD) return dq4_scaled<AT>(v[0][s], sc);
    else return dq4_exact<AT>(v[0][s]);
  } else if constexpr (WF == kInt8) {
    const uint32_t a = v[s >> 1][(s & 1) * 2], b = v[s >> 1][(s & 1) * 2 + 1];
    if constexpr (FOLD) return dq8_scaled<AT>(a, b, sc);
    else return dq8_exact<AT>(a, b);
  } else {
    return v[s];
  }
}

// Biased weight operand of MFMA step s (decode chunk layout).
template <typename AT, int WF>
__device__ __forceinline__ u32x4_t weight_biased(const u32x4_t* v, int s) {
  if constexpr (WF == kInt4) {
    if constexpr (AT::kId == 10) return dq4_f16_biased(v[0][s]);
    else return dq4_bf16_biased(v[0][s]);
  } else {
    return dq8_f16_biased(v[s >> 1][(s & 1) * 2], v[s >> 1][(s & 1) * 2 + 1]);
  }
}

// MXFP4 (OCP MX v1.0 FP4 E2M1, even k in the low nibble) dword (k0..k7) ->
// 16-bit pairs (k0 k1) .. (k6 k7) of e2m1(nibble) * sc, with the gfx950
// FP4 conversion (one instruction per byte).  Every E2M1 value times a
// power of two is exact in fp16 / bf16 inside the type's range.
template <typename AT>
__device__ __forceinline__ u32x4_t fp4_scaled(uint32_t v, float sc) {
  if constexpr (AT::kId == 10) {
    return u32x4_t{h2_bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 0)),
                   h2_bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 1)),
                   h2_bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 2)),
                   h2_bits(__builtin_amdgcn_cvt_scalef32_pk_f16_fp4(v, sc, 3))};
  } else {
    return u32x4_t{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 0)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 1)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 2)),
                   __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, sc, 3))};
  }
}

// Weight row (within one expert) that tile t of feature f reads.
__device__ __forceinline__ int64_t tile_row(int64_t f, bool lin, bool fc1_gated, int gate_mode, int64_t nfeat) {
  if (fc1_gated && gate_mode == kGateInterleaved) return 2 * f + (lin ? 1 : 0);
  if (fc1_gated && gate_mode == kGateChunked) return f + (lin ? nfeat : 0);
  return f;
}

}  // namespace moe
