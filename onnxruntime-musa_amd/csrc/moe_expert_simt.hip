// moe_expert_simt.hip -- generic expert FFN kernels (any activation dtype,
// any weight format) and the finalize gather-reduce.
//
// These serve the fp32 activation path (the small fp32 MoE config: fp32
// accumulation, max-abs 1e-4 against the oracle) and are the functional
// fallback for shapes the MFMA paths do not cover.  One wavefront computes one
// output feature of one dispatched row: lanes stride over K with coalesced
// loads, each lane accumulates in fp32, a butterfly sum reduces the wave.
#include "moe_device.h"
#include "moe_launch.h"

namespace moe {
namespace {

// fp32 value of element (n, kk) of expert e's [N, K] weight matrix.
struct WeightView {
  const void* w;
  const void* s;
  int32_t wfmt, act_type, scale_type;
  int64_t N, K, block_size;
  int32_t mx;  // MXFP4: E2M1 nibbles, E8M0 scale bytes per block of 32

  __device__ __forceinline__ float get(int64_t e, int64_t n, int64_t kk) const {
    if (wfmt == kDense) return load_any(w, act_type, (e * N + n) * K + kk);
    const uint8_t* q = static_cast<const uint8_t*>(w);
    const int64_t nblk = block_size > 0 ? K / block_size : 1;
    if (mx) {
      const uint8_t b = q[(e * N + n) * (K / 2) + (kk >> 1)];
      const uint8_t sc = static_cast<const uint8_t*>(s)[(e * N + n) * nblk + kk / block_size];
      return e2m1_to_f32((kk & 1) ? (b >> 4) : (b & 0x0F)) * e8m0_to_f32(sc);
    }
    const float sc =
        load_any(s, scale_type, (e * N + n) * nblk + (block_size > 0 ? kk / block_size : 0));
    int v;
    if (wfmt == kInt8) {
      v = static_cast<int>(q[(e * N + n) * K + kk]) - 128;
    } else {
      const uint8_t b = q[(e * N + n) * (K / 2) + (kk >> 1)];
      v = static_cast<int>((kk & 1) ? (b >> 4) : (b & 0x0F)) - 8;
    }
    return static_cast<float>(v) * sc;
  }
};

__device__ __forceinline__ float load_act(const void* p, int t, int64_t i) {
  return load_any(p, t, i);
}

// fc1 (+fc3) + bias + activation: act[r, i].
__global__ void __launch_bounds__(256) fc1_simt_kernel(ExpertArgs a) {
  const int lane = threadIdx.x % kWave;
  const int64_t i = static_cast<int64_t>(blockIdx.y) * (blockDim.x / kWave) + threadIdx.x / kWave;
  const int64_t r = blockIdx.x;
  if (i >= a.I) return;
  const int32_t f = a.perm[r];
  const int64_t tok = f / a.k;
  const int64_t e = a.topk_ids[f];
  const bool gated = a.gate_mode != kGateNone;
  const int64_t N1 = (a.gate_mode == kGateInterleaved || a.gate_mode == kGateChunked) ? 2 * a.I : a.I;
  int64_t ng = i, nl = 0;
  if (a.gate_mode == kGateInterleaved) { ng = 2 * i; nl = 2 * i + 1; }
  else if (a.gate_mode == kGateChunked) { ng = i; nl = a.I + i; }
  else if (a.gate_mode == kGateFc3) { ng = i; nl = i; }
  const WeightView w1{a.w1, a.s1, a.wfmt, a.act_type, a.scale_type, N1, a.H, a.block_size, a.mx};
  const WeightView w3{a.w3, a.s3, a.wfmt, a.act_type, a.scale_type, a.I, a.H, a.block_size, a.mx};
  float sg = 0.0f, sl = 0.0f;
  for (int64_t kk = lane; kk < a.H; kk += kWave) {
    const float xv = load_act(a.x, a.act_type, tok * a.H + kk);
    sg += xv * w1.get(e, ng, kk);
    if (a.gate_mode == kGateFc3) sl += xv * w3.get(e, nl, kk);
    else if (gated) sl += xv * w1.get(e, nl, kk);
  }
  sg = wave_sum(sg);
  sl = wave_sum(sl);
  if (lane == 0) {
    if (a.b1) sg += load_any(a.b1, a.act_type, e * N1 + ng);
    if (a.gate_mode == kGateFc3) {
      if (a.b3) sl += load_any(a.b3, a.act_type, e * a.I + nl);
    } else if (gated && a.b1) {
      sl += load_any(a.b1, a.act_type, e * N1 + nl);
    }
    const float v = apply_act(sg, sl, gated, a.activation, a.alpha, a.beta, a.limit);
    const int64_t o = r * a.I + i;
    if (a.act_type == MOE_ELEM_FLOAT) static_cast<float*>(a.act)[o] = v;
    else if (a.act_type == MOE_ELEM_FLOAT16) static_cast<_Float16*>(a.act)[o] = static_cast<_Float16>(v);
    else static_cast<uint16_t*>(a.act)[o] = f32_to_bf16(v);
  }
}

// fc2 + bias: y2[r, h] (fp32).
__global__ void __launch_bounds__(256) fc2_simt_kernel(ExpertArgs a) {
  const int lane = threadIdx.x % kWave;
  const int64_t h = static_cast<int64_t>(blockIdx.y) * (blockDim.x / kWave) + threadIdx.x / kWave;
  const int64_t r = blockIdx.x;
  if (h >= a.H) return;
  const int64_t e = a.topk_ids[a.perm[r]];
  const WeightView w2{a.w2, a.s2, a.wfmt, a.act_type, a.scale_type, a.H, a.I, a.block_size, a.mx};
  float s = 0.0f;
  for (int64_t kk = lane; kk < a.I; kk += kWave)
    s += load_act(a.act, a.act_type, r * a.I + kk) * w2.get(e, h, kk);
  s = wave_sum(s);
  if (lane == 0) {
    if (a.b2) s += load_any(a.b2, a.act_type, e * a.H + h);
    a.y2[r * a.H + h] = s;
  }
}

// out[t, h] = sum_j w[t, j] * y2[inv_perm[t*k + j], h], summed in slot order
// (y2 itself the fixed-order sum of its partial planes when fc2 split K).
template <typename OT>
__global__ void __launch_bounds__(256) finalize_kernel(ExpertArgs a) {
  const int64_t t = blockIdx.x;
  const int64_t h0 = (static_cast<int64_t>(blockIdx.y) * blockDim.x + threadIdx.x) * 4;
  if (h0 >= a.H) return;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (a.y2_half) {  // one plane in the output type (fp16 or bf16)
    using YS = typename OT::storage;
    const YS* y2h = reinterpret_cast<const YS*>(a.y2);
    for (int64_t j = 0; j < a.k; ++j) {
      const int64_t f = t * a.k + j;
      const float w = a.topk_w[f];
      const YS* y = y2h + static_cast<int64_t>(a.inv_perm[f]) * a.H;
      for (int c = 0; c < 4 && h0 + c < a.H; ++c) acc[c] += w * to_f32<OT>(y[h0 + c]);
    }
    typename OT::storage* out = static_cast<typename OT::storage*>(a.out);
    for (int c = 0; c < 4 && h0 + c < a.H; ++c) out[t * a.H + h0 + c] = from_f32<OT>(acc[c]);
    return;
  }
  const int64_t plane = a.T * a.k * a.H;
  // Up to kFinLoads (slot, plane) values per thread: every load is issued
  // before the first sum (a decode layer's y2 planes are in L2, so the
  // time is load latency), then the sums run in the order of the loop below.
  constexpr int kFinLoads = 16;
  if ((a.H % 4) == 0 && a.k * a.y2_planes <= kFinLoads) {
    const int np = a.y2_planes, nl = static_cast<int>(a.k) * np;
    float4 v[kFinLoads];
#pragma unroll
    for (int i = 0; i < kFinLoads; ++i) {
      if (i < nl) {
        const int j = i / np, z = i - j * np;
        v[i] = *reinterpret_cast<const float4*>(a.y2 + z * plane + static_cast<int64_t>(a.inv_perm[t * a.k + j]) * a.H + h0);
      }
    }
    float4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kFinLoads; ++i) {
      if (i < nl) {
        const int j = i / np, z = i - j * np;
        if (z == 0) {
          s = v[i];
        } else {
          s.x += v[i].x;
          s.y += v[i].y;
          s.z += v[i].z;
          s.w += v[i].w;
        }
        if (z == np - 1) {
          const float w = a.topk_w[t * a.k + j];
          acc[0] += w * s.x;
          acc[1] += w * s.y;
          acc[2] += w * s.z;
          acc[3] += w * s.w;
        }
      }
    }
    typename OT::storage* out = static_cast<typename OT::storage*>(a.out);
#pragma unroll
    for (int c = 0; c < 4; ++c) out[t * a.H + h0 + c] = from_f32<OT>(acc[c]);
    return;
  }
  for (int64_t j = 0; j < a.k; ++j) {
    const int64_t f = t * a.k + j;
    const float w = a.topk_w[f];
    const float* y = a.y2 + static_cast<int64_t>(a.inv_perm[f]) * a.H;
    if (h0 + 4 <= a.H && (a.H % 4) == 0) {
      float4 v = *reinterpret_cast<const float4*>(y + h0);
      for (int z = 1; z < a.y2_planes; ++z) {  // partial sums over K, fixed order
        const float4 u = *reinterpret_cast<const float4*>(y + z * plane + h0);
        v.x += u.x;
        v.y += u.y;
        v.z += u.z;
        v.w += u.w;
      }
      acc[0] += w * v.x;
      acc[1] += w * v.y;
      acc[2] += w * v.z;
      acc[3] += w * v.w;
    } else {
      for (int c = 0; c < 4 && h0 + c < a.H; ++c) {
        float v = y[h0 + c];
        for (int z = 1; z < a.y2_planes; ++z) v += y[z * plane + h0 + c];
        acc[c] += w * v;
      }
    }
  }
  typename OT::storage* out = static_cast<typename OT::storage*>(a.out);
  for (int c = 0; c < 4 && h0 + c < a.H; ++c) out[t * a.H + h0 + c] = from_f32<OT>(acc[c]);
}

// One plane in the output type (16-bit prefill without a K split), H a
// multiple of 8: one thread per (token, 8 features), 16-byte loads and
// stores, the same sums in the same order as finalize_kernel.
template <typename OT>
__global__ void __launch_bounds__(256) finalize_half8_kernel(ExpertArgs a) {
  using YS = typename OT::storage;
  const int64_t t = blockIdx.x;
  const int64_t h0 = (static_cast<int64_t>(blockIdx.y) * blockDim.x + threadIdx.x) * 8;
  if (h0 >= a.H) return;
  const YS* y2h = reinterpret_cast<const YS*>(a.y2);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int64_t j = 0; j < a.k; ++j) {
    const int64_t f = t * a.k + j;
    const float w = a.topk_w[f];
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(y2h + static_cast<int64_t>(a.inv_perm[f]) * a.H + h0);
#pragma unroll
    for (int c = 0; c < 8; ++c)
      acc[c] += w * to_f32<OT>(__builtin_bit_cast(YS, static_cast<uint16_t>(v[c / 2] >> (16 * (c % 2)))));
  }
  u32x4_t o;
#pragma unroll
  for (int c = 0; c < 4; ++c)
    o[c] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<OT>(acc[2 * c]))) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<OT>(acc[2 * c + 1]))) << 16);
  *reinterpret_cast<u32x4_t*>(static_cast<YS*>(a.out) + t * a.H + h0) = o;
}

}  // namespace

hipError_t launch_fc1_simt(const ExpertArgs& a, hipStream_t stream) {
  const int64_t rows = a.T * a.k;
  if (rows == 0) return hipSuccess;
  dim3 grid(static_cast<unsigned>(rows), static_cast<unsigned>((a.I + 3) / 4));
  hipLaunchKernelGGL(fc1_simt_kernel, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_fc2_simt(const ExpertArgs& a, hipStream_t stream) {
  const int64_t rows = a.T * a.k;
  if (rows == 0) return hipSuccess;
  dim3 grid(static_cast<unsigned>(rows), static_cast<unsigned>((a.H + 3) / 4));
  hipLaunchKernelGGL(fc2_simt_kernel, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_finalize(const ExpertArgs& a, hipStream_t stream) {
  if (a.T == 0) return hipSuccess;
  if (a.y2_half && (a.act_type == MOE_ELEM_FLOAT16 || a.act_type == MOE_ELEM_BFLOAT16) && a.H % 8 == 0) {
    const dim3 grid8(static_cast<unsigned>(a.T), static_cast<unsigned>((a.H + 2047) / 2048));
    if (a.act_type == MOE_ELEM_FLOAT16) hipLaunchKernelGGL(finalize_half8_kernel<F16>, grid8, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL(finalize_half8_kernel<BF16>, grid8, dim3(256), 0, stream, a);
    return hipGetLastError();
  }
  dim3 grid(static_cast<unsigned>(a.T), static_cast<unsigned>((a.H + 1023) / 1024));
  switch (a.act_type) {
    case MOE_ELEM_FLOAT: hipLaunchKernelGGL(finalize_kernel<F32>, grid, dim3(256), 0, stream, a); break;
    case MOE_ELEM_FLOAT16: hipLaunchKernelGGL(finalize_kernel<F16>, grid, dim3(256), 0, stream, a); break;
    case MOE_ELEM_BFLOAT16: hipLaunchKernelGGL(finalize_kernel<BF16>, grid, dim3(256), 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace moe
