// moe_softmax.hip -- the ONNX Softmax op (opset 13 semantics: one axis) for
// gfx950, the router's normalisation as a stand-alone op: y = exp(x - max) *
// (1 / sum exp(x - max)) along the axis, accumulated in fp32 (fp64 for
// double inputs), as the reference's kernel computes it
// (musa/ep/src/kernels/math/softmax_impl.mu:49-84).
//
// The input is viewed as [outer, dim, inner].  With inner == 1 one wavefront
// takes a row.  Rows up to 4096 long stay in registers between the max, sum
// and write steps, so each is read once.  For longer rows each lane keeps a
// running maximum and a sum of exponentials rescaled whenever its maximum
// rises, the lanes' pairs merge in a butterfly, and a second pass writes --
// two reads of the row instead of three (max, sum, write).
// Otherwise (inner > 1) one thread takes an (outer, inner) position and walks dim, so
// that neighbouring threads read neighbouring inner elements.
#include <stdint.h>

#include "moe_device.h"
#include "moe_launch.h"

namespace moe {
namespace {

template <typename T, typename A>
__device__ __forceinline__ A sm_load(const T* p, int64_t i);
template <>
__device__ __forceinline__ float sm_load<float, float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float sm_load<_Float16, float>(const _Float16* p, int64_t i) { return static_cast<float>(p[i]); }
template <>
__device__ __forceinline__ float sm_load<uint16_t, float>(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
template <>
__device__ __forceinline__ double sm_load<double, double>(const double* p, int64_t i) { return p[i]; }

template <typename T, typename A>
__device__ __forceinline__ void sm_store(T* p, int64_t i, A v);
template <>
__device__ __forceinline__ void sm_store<float, float>(float* p, int64_t i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void sm_store<_Float16, float>(_Float16* p, int64_t i, float v) { p[i] = static_cast<_Float16>(v); }
template <>
__device__ __forceinline__ void sm_store<uint16_t, float>(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
template <>
__device__ __forceinline__ void sm_store<double, double>(double* p, int64_t i, double v) { p[i] = v; }

__device__ __forceinline__ float sm_exp(float v) { return expf(v); }
__device__ __forceinline__ double sm_exp(double v) { return exp(v); }

template <typename A>
__device__ __forceinline__ A sm_wave_max(A v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const A u = __shfl_xor(v, o, kWave);
    v = u > v ? u : v;
  }
  return v;
}
template <typename A>
__device__ __forceinline__ A sm_wave_sum(A v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Rows longer than 64 * kCachedMaxNv take softmax_rows_kernel (128 values
// per lane would pass the 256 VGPRs of a wave and spill).
constexpr int kCachedMaxNv = 64;

// inner == 1 and dim <= 64 NV: one wavefront per row, the row held in
// registers (NV elements per lane, d = lane + 64 i), so it is read once: the
// exponentials computed for the sum are the ones written.
template <typename T, typename A, int NV>
__global__ void __launch_bounds__(256) softmax_rows_cached_kernel(const T* __restrict__ in, T* __restrict__ out,
                                                                  int64_t rows, int64_t dim) {
  const int lane = threadIdx.x & 63;
  const int64_t wpb = blockDim.x / kWave;
  const int d = static_cast<int>(dim);
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * wpb + threadIdx.x / kWave; r < rows;
       r += static_cast<int64_t>(gridDim.x) * wpb) {
    const T* x = in + r * dim;
    A v[NV];
    A m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + kWave * i;
      v[i] = c < d ? sm_load<T, A>(x, c) : static_cast<A>(-INFINITY);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) m = v[i] > m ? v[i] : m;
    m = sm_wave_max(m);
    A s = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (lane + kWave * i < d) {
        v[i] = sm_exp(v[i] - m);
        s += v[i];
      }
    }
    const A inv = static_cast<A>(1) / sm_wave_sum(s);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + kWave * i;
      if (c < d) sm_store<T, A>(out + r * dim, c, v[i] * inv);
    }
  }
}

// inner == 1, longer rows: one wavefront per row, the
// online max-and-sum pass then the write pass
template <typename T, typename A>
__global__ void __launch_bounds__(256) softmax_rows_kernel(const T* __restrict__ in, T* __restrict__ out,
                                                           int64_t rows, int64_t dim) {
  const int lane = threadIdx.x & 63;
  const int64_t wpb = blockDim.x / kWave;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * wpb + threadIdx.x / kWave; r < rows;
       r += static_cast<int64_t>(gridDim.x) * wpb) {
    const T* x = in + r * dim;
    A m = -INFINITY, s = 0;
    for (int64_t d = lane; d < dim; d += kWave) {
      const A v = sm_load<T, A>(x, d);
      if (v > m) {
        s = s * sm_exp(m - v) + static_cast<A>(1);  // exp(-inf) = 0 on a lane's first element
        m = v;
      } else if (m != -INFINITY) {  // -inf elements before any finite one add nothing
        s += sm_exp(v - m);
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const A om = __shfl_xor(m, o, kWave), os = __shfl_xor(s, o, kWave);
      const A nm = om > m ? om : m;
      // a side with nothing summed yet (s = 0, m = -inf) adds nothing
      s = (m == nm ? s : (s == 0 ? static_cast<A>(0) : s * sm_exp(m - nm))) +
          (om == nm ? os : (os == 0 ? static_cast<A>(0) : os * sm_exp(om - nm)));
      m = nm;
    }
    const A inv = static_cast<A>(1) / s;
    for (int64_t d = lane; d < dim; d += kWave) sm_store<T, A>(out + r * dim, d, sm_exp(sm_load<T, A>(x, d) - m) * inv);
  }
}

// inner > 1: one thread per (outer, inner) position
template <typename T, typename A>
__global__ void __launch_bounds__(256) softmax_strided_kernel(const T* __restrict__ in, T* __restrict__ out,
                                                              int64_t outer, int64_t dim, int64_t inner) {
  const int64_t n = outer * inner;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t o = i / inner, j = i - o * inner;
    const int64_t base = o * dim * inner + j;
    A m = -INFINITY;
    for (int64_t d = 0; d < dim; ++d) {
      const A v = sm_load<T, A>(in, base + d * inner);
      m = v > m ? v : m;
    }
    A s = 0;
    for (int64_t d = 0; d < dim; ++d) s += sm_exp(sm_load<T, A>(in, base + d * inner) - m);
    const A inv = static_cast<A>(1) / s;
    for (int64_t d = 0; d < dim; ++d)
      sm_store<T, A>(out, base + d * inner, sm_exp(sm_load<T, A>(in, base + d * inner) - m) * inv);
  }
}

template <typename T, typename A>
hipError_t launch_typed(const void* in, void* out, int64_t outer, int64_t dim, int64_t inner, hipStream_t stream) {
  const T* x = static_cast<const T*>(in);
  T* y = static_cast<T*>(out);
  if (inner == 1) {
    const int64_t blocks = (outer + 3) / 4;  // 4 waves per block
    const dim3 grid(static_cast<unsigned>(blocks < 65536 ? blocks : 65536));
    if (dim <= kWave * 4)
      hipLaunchKernelGGL((softmax_rows_cached_kernel<T, A, 4>), grid, dim3(256), 0, stream, x, y, outer, dim);
    else if (dim <= kWave * 16)
      hipLaunchKernelGGL((softmax_rows_cached_kernel<T, A, 16>), grid, dim3(256), 0, stream, x, y, outer, dim);
    else if (dim <= kWave * kCachedMaxNv)
      hipLaunchKernelGGL((softmax_rows_cached_kernel<T, A, kCachedMaxNv>), grid, dim3(256), 0, stream, x, y, outer,
                         dim);
    else
      hipLaunchKernelGGL((softmax_rows_kernel<T, A>), grid, dim3(256), 0, stream, x, y, outer, dim);
  } else {
    const int64_t n = outer * inner, blocks = (n + 255) / 256;
    hipLaunchKernelGGL((softmax_strided_kernel<T, A>), dim3(static_cast<unsigned>(blocks < 65536 ? blocks : 65536)),
                       dim3(256), 0, stream, x, y, outer, dim, inner);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_softmax(const void* in, void* out, int32_t elem_type, int64_t outer, int64_t dim, int64_t inner,
                          hipStream_t stream) {
  if (outer * dim * inner == 0) return hipSuccess;
  switch (elem_type) {
    case MOE_ELEM_FLOAT: return launch_typed<float, float>(in, out, outer, dim, inner, stream);
    case MOE_ELEM_FLOAT16: return launch_typed<_Float16, float>(in, out, outer, dim, inner, stream);
    case MOE_ELEM_BFLOAT16: return launch_typed<uint16_t, float>(in, out, outer, dim, inner, stream);
    case MOE_ELEM_DOUBLE: return launch_typed<double, double>(in, out, outer, dim, inner, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace moe
