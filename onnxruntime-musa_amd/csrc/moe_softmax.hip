// moe_softmax.hip -- the ONNX Softmax op (opset 13 semantics: one axis) for
// gfx950, the router's normalisation as a stand-alone op: y = exp(x - max) *
// (1 / sum exp(x - max)) along the axis, accumulated in fp32 (fp64 for
// double inputs), as the reference's kernel computes it
// (musa/ep/src/kernels/math/softmax_impl.mu:49-84).
//
// The input is viewed as [outer, dim, inner].  With inner == 1 one wavefront
// takes a row, or 2, 4 or 16 wavefronts of a workgroup share it.  Rows up to
// 16384 long stay in registers between the max, sum and write steps, so each
// is read once.  A longer row takes a workgroup: each thread keeps a running
// maximum and a sum of exponentials rescaled whenever its maximum rises, the
// threads' pairs merge, and a second pass writes -- two reads of the row
// instead of three (max, sum, write).  Otherwise (inner > 1) one thread takes
// an (outer, inner) position and walks dim with the same two passes, so that
// neighbouring threads read neighbouring inner elements.
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

// Values per lane of the register-held rows: the smallest of 4, 16 and 32
// that holds a row over 1, 2 or 4 waves, then 16 over 16 waves (a workgroup
// of 1024) for rows of 8193..16384: fewer registers, more waves per SIMD
// (64 per lane over 4 waves ran at 2 waves per SIMD).
// Most wavefronts sharing one register-held row (rows up to 64 * 16 * 16 =
// 16384); longer rows take softmax_rows_kernel.
constexpr int kCachedMaxWaves = 16;

// inner == 1 and dim <= 64 NV WPR: WPR wavefronts of a workgroup take one row,
// held in registers (NV elements per lane, d = lane + 64 (w + WPR i) for the
// row's wave w), so it is read once: the exponentials computed for the sum
// are the ones written.  Waves of one row combine their maxima and sums in
// LDS.
template <typename T, typename A, int NV, int WPR, int NT = 256>
__global__ void __launch_bounds__(NT) softmax_rows_cached_kernel(const T* __restrict__ in, T* __restrict__ out,
                                                                 int64_t rows, int64_t dim) {
  __shared__ A part[2][NT / kWave];  // per-wave maximum, sum
  const int lane = threadIdx.x & 63, wave = threadIdx.x / kWave;
  const int w = wave % WPR, first = wave - w;
  const int64_t rpb = blockDim.x / kWave / WPR;
  const int d = static_cast<int>(dim);
  // every wave of a workgroup runs the same iterations (uniform barriers)
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * rpb; r0 < rows; r0 += static_cast<int64_t>(gridDim.x) * rpb) {
    const int64_t r = r0 + wave / WPR;
    const bool live = r < rows;
    const T* x = in + (live ? r : 0) * dim;
    A v[NV];
    A m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int c = lane + kWave * (w + WPR * i);
      v[i] = live && c < d ? sm_load<T, A>(x, c) : static_cast<A>(-INFINITY);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) m = v[i] > m ? v[i] : m;
    m = sm_wave_max(m);
    if constexpr (WPR > 1) {
      if (lane == 0) part[0][wave] = m;
      __syncthreads();
#pragma unroll
      for (int o = 0; o < WPR; ++o) m = part[0][first + o] > m ? part[0][first + o] : m;
    }
    A s = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      if (lane + kWave * (w + WPR * i) < d) {
        v[i] = sm_exp(v[i] - m);
        s += v[i];
      }
    }
    s = sm_wave_sum(s);
    if constexpr (WPR > 1) {
      if (lane == 0) part[1][wave] = s;
      __syncthreads();  // also orders this row's reads of part[0] before the next row's writes
      s = 0;
#pragma unroll
      for (int o = 0; o < WPR; ++o) s += part[1][first + o];
    }
    const A inv = static_cast<A>(1) / s;
    if (live) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int c = lane + kWave * (w + WPR * i);
        if (c < d) sm_store<T, A>(out + r * dim, c, v[i] * inv);
      }
    }
  }
}

// Running (maximum, sum of exponentials) of one more value; exp(-inf) = 0 on
// a thread's first element, and -inf elements before any finite one add
// nothing.  A NaN makes the sum NaN wherever it arrives (it compares false
// with the maximum, so it is caught by the second test), so that its row
// comes out all NaN like the register-held kernels'.
template <typename A, typename S>
__device__ __forceinline__ void sm_online(A& m, S& s, A v) {
  if (v > m) {
    s = s * static_cast<S>(sm_exp(m - v)) + static_cast<S>(1);
    m = v;
  } else if (m != -INFINITY || v != v) {
    s += static_cast<S>(sm_exp(v - m));
  }
}

// Merges the pair (om, os) into (m, s); a side with nothing summed yet
// (s = 0, m = -inf) adds nothing.
template <typename A>
__device__ __forceinline__ void sm_merge(A& m, A& s, A om, A os) {
  const A nm = om > m ? om : m;
  s = (m == nm ? s : (s == 0 ? static_cast<A>(0) : s * sm_exp(m - nm))) +
      (om == nm ? os : (os == 0 ? static_cast<A>(0) : os * sm_exp(om - nm)));
  m = nm;
}

// inner == 1, rows longer than the register-held ones: one workgroup per
// row, the online max-and-sum pass (four loads in flight per thread), the
// threads' pairs merged in a butterfly and then across the 4 waves in LDS,
// then the write pass.
template <typename T, typename A>
__global__ void __launch_bounds__(256) softmax_rows_kernel(const T* __restrict__ in, T* __restrict__ out,
                                                           int64_t rows, int64_t dim) {
  __shared__ A part[2][256 / kWave];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid / kWave;
  const int nt = blockDim.x, nw = blockDim.x / kWave;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const T* x = in + r * dim;
    A m = -INFINITY, s = 0;
    int64_t d = tid;
    for (; d + 3 * nt < dim; d += 4 * nt) {
      A v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = sm_load<T, A>(x, d + u * nt);
#pragma unroll
      for (int u = 0; u < 4; ++u) sm_online(m, s, v[u]);
    }
    for (; d < dim; d += nt) sm_online(m, s, sm_load<T, A>(x, d));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sm_merge(m, s, __shfl_xor(m, o, kWave), __shfl_xor(s, o, kWave));
    if (lane == 0) {
      part[0][wave] = m;
      part[1][wave] = s;
    }
    __syncthreads();
    m = part[0][0];
    s = part[1][0];
    for (int w = 1; w < nw; ++w) sm_merge(m, s, part[0][w], part[1][w]);
    __syncthreads();  // every wave has read part before the next row writes it
    const A inv = static_cast<A>(1) / s;
#pragma unroll 4
    for (int64_t e = tid; e < dim; e += nt) sm_store<T, A>(out + r * dim, e, sm_exp(sm_load<T, A>(x, e) - m) * inv);
  }
}

// inner > 1: one thread per (outer, inner) position, the online max-and-sum
// pass then the write pass
template <typename T, typename A>
__global__ void __launch_bounds__(256) softmax_strided_kernel(const T* __restrict__ in, T* __restrict__ out,
                                                              int64_t outer, int64_t dim, int64_t inner) {
  const int64_t n = outer * inner;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t o = i / inner, j = i - o * inner;
    const int64_t base = o * dim * inner + j;
    // one thread sums the whole axis in sequence: the sum is kept in double
    // (the exponentials stay in A) so that its rounding does not grow with dim
    A m = -INFINITY;
    double s = 0;
    for (int64_t d = 0; d < dim; ++d) sm_online(m, s, sm_load<T, A>(in, base + d * inner));
    const A inv = static_cast<A>(1.0 / s);
    for (int64_t d = 0; d < dim; ++d)
      sm_store<T, A>(out, base + d * inner, sm_exp(sm_load<T, A>(in, base + d * inner) - m) * inv);
  }
}

template <typename T, typename A>
hipError_t launch_typed(const void* in, void* out, int64_t outer, int64_t dim, int64_t inner, hipStream_t stream) {
  const T* x = static_cast<const T*>(in);
  T* y = static_cast<T*>(out);
  if (inner == 1) {
    const dim3 block(256);
    // rows per workgroup: 4 / (waves per row)
    auto grid = [outer](int64_t rpb) {
      const int64_t blocks = (outer + rpb - 1) / rpb;
      return dim3(static_cast<unsigned>(blocks < 65536 ? blocks : 65536));
    };
    if (dim <= kWave * 4)
      hipLaunchKernelGGL((softmax_rows_cached_kernel<T, A, 4, 1>), grid(4), block, 0, stream, x, y, outer, dim);
    else if (dim <= kWave * 16)
      hipLaunchKernelGGL((softmax_rows_cached_kernel<T, A, 16, 1>), grid(4), block, 0, stream, x, y, outer, dim);
    else if (dim <= kWave * 32)
      hipLaunchKernelGGL((softmax_rows_cached_kernel<T, A, 32, 1>), grid(4), block, 0, stream, x, y, outer, dim);
    else if (dim <= kWave * 32 * 2)
      hipLaunchKernelGGL((softmax_rows_cached_kernel<T, A, 32, 2>), grid(2), block, 0, stream, x, y, outer, dim);
    else if (dim <= kWave * 32 * 4)
      hipLaunchKernelGGL((softmax_rows_cached_kernel<T, A, 32, 4>), grid(1), block, 0, stream, x, y, outer, dim);
    else if (dim <= kWave * 16 * kCachedMaxWaves)
      hipLaunchKernelGGL((softmax_rows_cached_kernel<T, A, 16, kCachedMaxWaves, 64 * kCachedMaxWaves>), grid(1),
                         dim3(64 * kCachedMaxWaves), 0, stream, x, y, outer, dim);
    else
      hipLaunchKernelGGL((softmax_rows_kernel<T, A>), grid(1), block, 0, stream, x, y, outer, dim);
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
