// moe_topk.hip -- the ONNX TopK op (opsets 10-19) for gfx950, built from the
// router's ordering rule: values by key, ties toward the lower index
// (musa/ep/src/kernels/math/topk_impl.mu:46-65).
//
// Axes up to 512 with k <= 32: lane groups of a wavefront take a slice each,
// k rounds of a group arg-max over keys held in registers
// (topk_wave_kernel).  Axes up to 8192 with k <= 64: the same rounds over a
// workgroup (topk_block_kernel).  Otherwise one workgroup per (row, inner)
// slice of the input viewed as [rows, dim, inner] sorts it: the slice's dim
// elements become order-preserving integer keys in LDS (floats:
// sign-magnitude bits flipped to two's-complement order, -0.0 folded onto
// +0.0 so that it ties with +0.0 as a value comparison does; integers: sign
// bit flipped; smallest-first negates the key; the register kernels use the
// same keys), padded to a power of two with keys that sort last, and a
// bitonic network sorts (key desc, index asc).  The first k entries are written out; values are read
// back from the input at their index, so they keep their exact bits.
//
// Axes longer than 8192 (k <= 8192) take a radix select instead
// (topk_radix_kernel): the k-th key is found digit by digit, the k winners
// are collected and only they are sorted.
//
// Every NaN (either sign, any payload) has one key, above +inf: NaNs sort as
// the largest values for largest = 1 and the smallest for largest = 0, tied
// with each other (so in index order).
#include <stdint.h>

#include <type_traits>

#include "moe_device.h"
#include "moe_launch.h"

namespace moe {
namespace {

template <typename T>
__device__ __forceinline__ uint64_t topk_key(T v);
// floats: flip all bits of negatives, set the sign bit of positives
__device__ __forceinline__ uint64_t key_f64(double d) {
  if (d == 0.0) d = 0.0;                          // -0.0 ties with +0.0
  if (d != d) return uint64_t{0xFFF8000000000000};  // every NaN: the key of +qNaN
  const uint64_t b = __builtin_bit_cast(uint64_t, d);
  return (b >> 63) ? ~b : (b | (uint64_t{1} << 63));
}
template <>
__device__ __forceinline__ uint64_t topk_key<double>(double v) { return key_f64(v); }
template <>
__device__ __forceinline__ uint64_t topk_key<float>(float v) { return key_f64(static_cast<double>(v)); }
template <>
__device__ __forceinline__ uint64_t topk_key<_Float16>(_Float16 v) { return key_f64(static_cast<double>(static_cast<float>(v))); }
template <>
__device__ __forceinline__ uint64_t topk_key<uint16_t>(uint16_t v) {  // bf16 bits
  return key_f64(static_cast<double>(bf16_to_f32(v)));
}
template <>
__device__ __forceinline__ uint64_t topk_key<int32_t>(int32_t v) {
  return static_cast<uint64_t>(static_cast<int64_t>(v)) ^ (uint64_t{1} << 63);
}
template <>
__device__ __forceinline__ uint64_t topk_key<int64_t>(int64_t v) {
  return static_cast<uint64_t>(v) ^ (uint64_t{1} << 63);
}

__device__ __forceinline__ bool entry_before(uint64_t ka, uint32_t ia, uint64_t kb, uint32_t ib) {
  return ka > kb || (ka == kb && ia < ib);
}

// Bitonic network over n (a power of two) LDS entries: segments of `size`
// alternate direction until the last merge, which leaves (key desc, index
// asc).  Every thread of the workgroup calls it; it ends on a barrier.
template <typename KT>
__device__ void bitonic_lds(KT* key, uint32_t* idx, int n, int tid, int nt) {
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int q = tid; q < (n >> 1); q += nt) {
        const int lo = 2 * stride * (q / stride) + (q % stride), hi = lo + stride;
        const bool up = (lo & size) == 0;
        const KT kl = key[lo], kh = key[hi];
        const uint32_t il = idx[lo], ih = idx[hi];
        if ((kh > kl || (kh == kl && ih < il)) == up) {
          key[lo] = kh;
          key[hi] = kl;
          idx[lo] = ih;
          idx[hi] = il;
        }
      }
      __syncthreads();
    }
  }
}

template <typename T>
__global__ void __launch_bounds__(1024) topk_kernel(const T* __restrict__ in, T* __restrict__ values,
                                                    int64_t* __restrict__ indices, TopKArgs p, int n) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint64_t* key = reinterpret_cast<uint64_t*>(smem);
  uint32_t* idx = reinterpret_cast<uint32_t*>(smem + static_cast<size_t>(n) * 8);
  const int tid = threadIdx.x, nt = blockDim.x;
  const int64_t slices = p.rows * p.inner;
  for (int64_t sl = blockIdx.x; sl < slices; sl += gridDim.x) {
    const int64_t row = sl / p.inner, in0 = sl - row * p.inner;
    const T* src = in + row * p.dim * p.inner + in0;
    for (int i = tid; i < n; i += nt) {
      if (i < p.dim) {
        const uint64_t kv = topk_key<T>(src[static_cast<int64_t>(i) * p.inner]);
        key[i] = p.largest ? kv : ~kv;
        idx[i] = static_cast<uint32_t>(i);
      } else {
        key[i] = 0;            // after every element, ties broken by index
        idx[i] = 0xFFFFFFFFu;
      }
    }
    __syncthreads();
    bitonic_lds(key, idx, n, tid, nt);
    for (int64_t j = tid; j < p.k; j += nt) {
      const uint32_t s = idx[j];
      const int64_t o = (row * p.k + j) * p.inner + in0;
      values[o] = src[static_cast<int64_t>(s) * p.inner];
      indices[o] = static_cast<int64_t>(s);
    }
    __syncthreads();  // LDS is reused by the next slice
  }
}

// Candidates of the register kernels.  Elements of 32 bits or less have
// 32-bit keys (the same order as topk_key): a candidate is then one 64-bit
// word, key above the complemented index, so that (key desc, index asc) is
// plain unsigned order and a butterfly step moves two words.  64-bit elements
// keep a (key, index) pair.  A retired or absent entry is dead(), after every
// live one.
__device__ __forceinline__ uint32_t key_f32(float f) {
  if (f == 0.0f) f = 0.0f;            // -0.0 ties with +0.0
  if (f != f) return 0xFFC00000u;     // every NaN: the key of +qNaN
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  return (b >> 31) ? ~b : (b | 0x80000000u);
}

template <typename T>
struct Packed {  // T of 32 bits or less
  using C = uint64_t;
  static __device__ __forceinline__ uint32_t key(T v);
  static __device__ __forceinline__ C make(T v, uint32_t i, bool largest) {
    const uint32_t k = largest ? key(v) : ~key(v);
    return (static_cast<uint64_t>(k) << 32) | static_cast<uint32_t>(~i);
  }
  static __device__ __forceinline__ C dead() { return 0; }
  static __device__ __forceinline__ bool before(C a, C b) { return a > b; }
  static __device__ __forceinline__ uint32_t index(C c) { return ~static_cast<uint32_t>(c); }
  static __device__ __forceinline__ C shfl(C c, int o, int width) {
    const uint32_t hi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(c >> 32), o, width));
    const uint32_t lo = static_cast<uint32_t>(__shfl_xor(static_cast<int>(c & 0xFFFFFFFFu), o, width));
    return (static_cast<uint64_t>(hi) << 32) | lo;
  }
};
template <>
__device__ __forceinline__ uint32_t Packed<float>::key(float v) { return key_f32(v); }
template <>
__device__ __forceinline__ uint32_t Packed<_Float16>::key(_Float16 v) { return key_f32(static_cast<float>(v)); }
template <>
__device__ __forceinline__ uint32_t Packed<uint16_t>::key(uint16_t v) { return key_f32(bf16_to_f32(v)); }
template <>
__device__ __forceinline__ uint32_t Packed<int32_t>::key(int32_t v) { return static_cast<uint32_t>(v) ^ 0x80000000u; }

template <typename T>
struct Pair {  // 64-bit T
  struct C {
    uint64_t k;
    uint32_t i;
  };
  static __device__ __forceinline__ C make(T v, uint32_t i, bool largest) {
    const uint64_t k = topk_key<T>(v);
    return C{largest ? k : ~k, i};
  }
  static __device__ __forceinline__ C dead() { return C{0, 0xFFFFFFFFu}; }
  static __device__ __forceinline__ bool before(C a, C b) { return entry_before(a.k, a.i, b.k, b.i); }
  static __device__ __forceinline__ uint32_t index(C c) { return c.i; }
  static __device__ __forceinline__ C shfl(C c, int o, int width) {
    const uint32_t hi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(c.k >> 32), o, width));
    const uint32_t lo = static_cast<uint32_t>(__shfl_xor(static_cast<int>(c.k & 0xFFFFFFFFu), o, width));
    const uint32_t i = static_cast<uint32_t>(__shfl_xor(static_cast<int>(c.i), o, width));
    return C{(static_cast<uint64_t>(hi) << 32) | lo, i};
  }
};

template <typename T>
using CandOps = std::conditional_t<sizeof(T) <= 4, Packed<T>, Pair<T>>;

// Short axes and small k: lane groups of G lanes take one slice each (64 / G
// slices per wavefront), every lane holding kWaveVpl candidates in
// registers; k rounds of a group arg-max (log2 G butterfly steps) under the
// same order (key desc, index asc) pick the outputs in sorted order -- no
// LDS, no barriers.  The outputs are written after the last round.
constexpr int kWaveVpl = 8;
constexpr int kWaveMaxK = 32;

template <typename T, int G>
__global__ void __launch_bounds__(256) topk_wave_kernel(const T* __restrict__ in, T* __restrict__ values,
                                                        int64_t* __restrict__ indices, TopKArgs p) {
  using O = CandOps<T>;
  using C = typename O::C;
  const int lane = threadIdx.x & 63, sub = lane % G;
  constexpr int kPerWave = kWave / G;
  const int64_t wpb = blockDim.x / kWave;
  const int64_t slices = p.rows * p.inner;
  const int dim = static_cast<int>(p.dim), k = static_cast<int>(p.k);
  const bool largest = p.largest != 0;
  for (int64_t s0 = (static_cast<int64_t>(blockIdx.x) * wpb + threadIdx.x / kWave) * kPerWave; s0 < slices;
       s0 += static_cast<int64_t>(gridDim.x) * wpb * kPerWave) {
    const int64_t sl = s0 + lane / G;
    const bool valid = sl < slices;
    const int64_t row = valid ? sl / p.inner : 0, in0 = valid ? sl - row * p.inner : 0;
    const T* src = in + row * p.dim * p.inner + in0;
    C e[kWaveVpl];
#pragma unroll
    for (int v = 0; v < kWaveVpl; ++v) {
      const int i = sub + G * v;
      e[v] = valid && i < dim ? O::make(src[static_cast<int64_t>(i) * p.inner], static_cast<uint32_t>(i), largest)
                              : O::dead();
    }
    constexpr int kWins = (kWaveMaxK + G - 1) / G;  // rounds kept per lane
    uint32_t win[kWins];
#pragma unroll
    for (int q = 0; q < kWins; ++q) win[q] = 0;
    for (int j = 0; j < k; ++j) {
      C b = e[0];
#pragma unroll
      for (int v = 1; v < kWaveVpl; ++v)
        if (O::before(e[v], b)) b = e[v];
#pragma unroll
      for (int o = G / 2; o > 0; o >>= 1) {
        const C c = O::shfl(b, o, G);
        if (O::before(c, b)) b = c;
      }
      // j < k <= dim: the winner is live; its owner retires it, and lane
      // j % G keeps round j's winner
      const uint32_t bi = O::index(b);
      if (valid && static_cast<int>(bi % G) == sub) {
#pragma unroll
        for (int v = 0; v < kWaveVpl; ++v)
          if (v == static_cast<int>(bi / G)) e[v] = O::dead();
      }
#pragma unroll
      for (int q = 0; q < kWins; ++q)
        if (q * G + sub == j) win[q] = bi;
    }
    // the k value reads go out together instead of one per round
    if (valid) {
#pragma unroll
      for (int q = 0; q < kWins; ++q) {
        const int j = q * G + sub;
        if (j < k) {
          const int64_t o = (row * p.k + j) * p.inner + in0;
          values[o] = src[static_cast<int64_t>(win[q]) * p.inner];
          indices[o] = static_cast<int64_t>(win[q]);
        }
      }
    }
  }
}

// Axes up to 8192 with k <= 64: one workgroup of 256 threads per slice, each
// thread holding VPL candidates (i = tid + 256 v) in registers; k rounds of
// a workgroup arg-max: a wave butterfly, then the 4 waves' winners compared
// in LDS (two buffers by round parity, so one barrier a round).  Each
// element is read once; the k rounds replace a full sort of the slice.
constexpr int kBlockMaxK = 64;

template <typename T, int VPL>
__global__ void __launch_bounds__(256) topk_block_kernel(const T* __restrict__ in, T* __restrict__ values,
                                                         int64_t* __restrict__ indices, TopKArgs p) {
  using O = CandOps<T>;
  using C = typename O::C;
  __shared__ C wbest[2][256 / kWave];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid / kWave;
  const int nt = blockDim.x, nw = blockDim.x / kWave;
  const int64_t slices = p.rows * p.inner;
  const int dim = static_cast<int>(p.dim), k = static_cast<int>(p.k);
  const bool largest = p.largest != 0;
  for (int64_t sl = blockIdx.x; sl < slices; sl += gridDim.x) {  // uniform per workgroup
    const int64_t row = sl / p.inner, in0 = sl - row * p.inner;
    const T* src = in + row * p.dim * p.inner + in0;
    C e[VPL];
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int i = tid + nt * v;
      e[v] = i < dim ? O::make(src[static_cast<int64_t>(i) * p.inner], static_cast<uint32_t>(i), largest)
                     : O::dead();
    }
    uint32_t mine = 0;  // the winner of round tid
    for (int j = 0; j < k; ++j) {
      C b = e[0];
#pragma unroll
      for (int v = 1; v < VPL; ++v)
        if (O::before(e[v], b)) b = e[v];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const C c = O::shfl(b, o, kWave);
        if (O::before(c, b)) b = c;
      }
      const int buf = j & 1;
      if (lane == 0) wbest[buf][wave] = b;
      // buffer buf is next written in round j + 2, after every thread has
      // passed round j + 1's barrier and so finished these reads
      __syncthreads();
      b = wbest[buf][0];
      for (int w = 1; w < nw; ++w)
        if (O::before(wbest[buf][w], b)) b = wbest[buf][w];
      // j < k <= dim, so the winner is live; its owner retires it
      const uint32_t bi = O::index(b);
      if (static_cast<int>(bi % static_cast<uint32_t>(nt)) == tid) {
#pragma unroll
        for (int v = 0; v < VPL; ++v)
          if (v == static_cast<int>(bi / static_cast<uint32_t>(nt))) e[v] = O::dead();
      }
      if (tid == j) mine = bi;
    }
    // thread j writes output j: the k value reads go out together instead of
    // one per round
    if (tid < k) {
      const int64_t o = (row * p.k + tid) * p.inner + in0;
      values[o] = src[static_cast<int64_t>(mine) * p.inner];
      indices[o] = static_cast<int64_t>(mine);
    }
    __syncthreads();  // the next slice's first rounds reuse both buffers
  }
}

// Axes longer than 8192 with k <= 8192: one workgroup of 1024 threads per
// slice.  A most-significant-digit radix select finds the k-th key: for each
// 8-bit digit, from the top, a 256-bin LDS histogram counts the keys that
// share the digits fixed so far (one read of the slice per digit) and the
// digit holding the k-th key is fixed.  The key it ends on, thr, is the k-th
// key; `need` keys equal to it belong to the output.  A collection pass then
// puts every key above thr into LDS (atomic positions: they are sorted
// afterwards) and the `need` lowest-index keys equal to thr (ranked in index
// order with wave ballots, tile by tile), and the bitonic network sorts
// those k entries.  Keys are those of the register kernels (32-bit for
// elements of 32 bits or less), so the order is the same as theirs.
template <typename T>
__device__ __forceinline__ auto radix_key(T v) {
  if constexpr (sizeof(T) <= 4) return Packed<T>::key(v);
  else return topk_key<T>(v);
}

template <typename T>
__global__ void __launch_bounds__(1024) topk_radix_kernel(const T* __restrict__ in, T* __restrict__ values,
                                                          int64_t* __restrict__ indices, TopKArgs p, int n) {
  using KT = std::conditional_t<sizeof(T) <= 4, uint32_t, uint64_t>;
  constexpr int kBits = 8 * static_cast<int>(sizeof(KT));
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  KT* lkey = reinterpret_cast<KT*>(smem);
  uint32_t* lidx = reinterpret_cast<uint32_t*>(smem + static_cast<size_t>(n) * sizeof(KT));
  __shared__ uint32_t hist[256];
  __shared__ uint32_t wcnt[1024 / kWave];
  __shared__ uint32_t s_digit, s_need, s_gt;
  const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wave = tid / kWave, nw = nt / kWave;
  const int64_t slices = p.rows * p.inner, dim = p.dim;
  const uint32_t k = static_cast<uint32_t>(p.k);
  const bool largest = p.largest != 0;
  for (int64_t sl = blockIdx.x; sl < slices; sl += gridDim.x) {  // uniform per workgroup
    const int64_t row = sl / p.inner, in0 = sl - row * p.inner;
    const T* src = in + row * p.dim * p.inner + in0;
    auto key_at = [&](int64_t i) -> KT {
      const KT kv = radix_key<T>(src[i * p.inner]);
      return largest ? kv : static_cast<KT>(~kv);
    };
    // ---- radix select: prefix holds the digits fixed so far (mask marks
    // them); need = how many of the keys matching prefix still belong to
    // the output ----
    KT prefix = 0, mask = 0;
    uint32_t need = k;
    for (int shift = kBits - 8; shift >= 0; shift -= 8) {
      for (int b = tid; b < 256; b += nt) hist[b] = 0;
      __syncthreads();
      for (int64_t i = tid; i < dim; i += nt) {
        const KT kv = key_at(i);
        if ((kv & mask) == prefix) atomicAdd(&hist[static_cast<uint32_t>(kv >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        // the largest digit d with (keys of digits above d) < need <= (keys of digits >= d)
        uint32_t above = 0;
        int d = 255;
        for (; d > 0; --d) {
          if (above + hist[d] >= need) break;
          above += hist[d];
        }
        s_digit = static_cast<uint32_t>(d);
        s_need = need - above;
      }
      __syncthreads();
      prefix |= static_cast<KT>(s_digit) << shift;
      mask |= static_cast<KT>(255) << shift;
      need = s_need;
    }
    // ---- collection: the k - need keys above thr, then the need
    // lowest-index keys equal to it ----
    const KT thr = prefix;
    const uint32_t ngt = k - need;
    if (tid == 0) s_gt = 0;
    __syncthreads();
    uint32_t taken = 0;  // keys equal to thr seen in earlier tiles (uniform)
    for (int64_t base = 0; base < dim; base += nt) {
      const int64_t i = base + tid;
      KT kv = 0;
      bool gt = false, eq = false;
      if (i < dim) {
        kv = key_at(i);
        gt = kv > thr;
        eq = kv == thr;
      }
      if (gt) {
        const uint32_t pos = atomicAdd(&s_gt, 1u);
        lkey[pos] = kv;
        lidx[pos] = static_cast<uint32_t>(i);
      }
      const uint64_t bal = __ballot(eq);
      const uint32_t before = static_cast<uint32_t>(__popcll(bal & ((uint64_t{1} << lane) - 1)));
      if (lane == 0) wcnt[wave] = static_cast<uint32_t>(__popcll(bal));
      __syncthreads();
      // between the barriers every gt position of this tile is taken and no
      // thread takes one of the next tile: the same count for all threads
      const uint32_t gt_seen = s_gt;
      uint32_t woff = 0, tot = 0;
      for (int w = 0; w < nw; ++w) {
        const uint32_t c = wcnt[w];
        woff += w < wave ? c : 0;
        tot += c;
      }
      const uint32_t r = taken + woff + before;
      if (eq && r < need) {
        lkey[ngt + r] = kv;
        lidx[ngt + r] = static_cast<uint32_t>(i);
      }
      taken += tot;
      __syncthreads();  // wcnt and s_gt are read before the next tile
      if (taken >= need && gt_seen == ngt) break;  // uniform: every winner is in LDS
    }
    // padding entries sort after every real one (key 0, the largest index)
    for (int j = static_cast<int>(k) + tid; j < n; j += nt) {
      lkey[j] = 0;
      lidx[j] = 0xFFFFFFFFu;
    }
    __syncthreads();
    bitonic_lds(lkey, lidx, n, tid, nt);
    for (int j = tid; j < static_cast<int>(k); j += nt) {
      const uint32_t s = lidx[j];
      const int64_t o = (row * p.k + j) * p.inner + in0;
      values[o] = src[static_cast<int64_t>(s) * p.inner];
      indices[o] = static_cast<int64_t>(s);
    }
    __syncthreads();  // LDS is reused by the next slice
  }
}

template <typename T>
hipError_t launch_typed(const void* in, void* values, int64_t* indices, const TopKArgs& p, hipStream_t stream) {
  const int64_t slices = p.rows * p.inner;
  if (p.dim <= kWave * kWaveVpl && p.k <= kWaveMaxK) {
    // lanes per slice: the power of two (4 .. 64) whose 8 entries per lane cover dim
    const int g = p.dim <= 4 * kWaveVpl ? 4 : (p.dim <= 8 * kWaveVpl ? 8 : (p.dim <= 16 * kWaveVpl ? 16
                : (p.dim <= 32 * kWaveVpl ? 32 : 64)));
    const int64_t per_block = 4 * (kWave / g);  // 4 waves per block
    const int64_t blocks = (slices + per_block - 1) / per_block;
    const dim3 grid(static_cast<unsigned>(blocks < (1 << 20) ? blocks : (1 << 20)));
    const T* x = static_cast<const T*>(in);
    T* v = static_cast<T*>(values);
    switch (g) {
      case 4: hipLaunchKernelGGL((topk_wave_kernel<T, 4>), grid, dim3(256), 0, stream, x, v, indices, p); break;
      case 8: hipLaunchKernelGGL((topk_wave_kernel<T, 8>), grid, dim3(256), 0, stream, x, v, indices, p); break;
      case 16: hipLaunchKernelGGL((topk_wave_kernel<T, 16>), grid, dim3(256), 0, stream, x, v, indices, p); break;
      case 32: hipLaunchKernelGGL((topk_wave_kernel<T, 32>), grid, dim3(256), 0, stream, x, v, indices, p); break;
      default: hipLaunchKernelGGL((topk_wave_kernel<T, 64>), grid, dim3(256), 0, stream, x, v, indices, p); break;
    }
    return hipGetLastError();
  }
  if (p.k <= kBlockMaxK && p.dim <= 256 * 32) {
    const dim3 grid(static_cast<unsigned>(slices < (int64_t{1} << 20) ? slices : (int64_t{1} << 20)));
    const T* x = static_cast<const T*>(in);
    T* v = static_cast<T*>(values);
    if (p.dim <= 256 * 8)
      hipLaunchKernelGGL((topk_block_kernel<T, 8>), grid, dim3(256), 0, stream, x, v, indices, p);
    else if (p.dim <= 256 * 16)
      hipLaunchKernelGGL((topk_block_kernel<T, 16>), grid, dim3(256), 0, stream, x, v, indices, p);
    else
      hipLaunchKernelGGL((topk_block_kernel<T, 32>), grid, dim3(256), 0, stream, x, v, indices, p);
    return hipGetLastError();
  }
  if (p.dim > kTopKMaxDim) {
    // radix select (the host checks k <= kTopKRadixMaxK, dim < 2^31)
    int n = 2;
    while (n < p.k) n <<= 1;
    const size_t kbytes = sizeof(T) <= 4 ? 4 : 8;
    const unsigned grid = static_cast<unsigned>(slices < (int64_t{1} << 20) ? slices : (int64_t{1} << 20));
    hipLaunchKernelGGL(topk_radix_kernel<T>, dim3(grid), dim3(1024), static_cast<size_t>(n) * (kbytes + 4), stream,
                       static_cast<const T*>(in), static_cast<T*>(values), indices, p, n);
    return hipGetLastError();
  }
  int n = 1;
  while (n < p.dim) n <<= 1;
  if (n < 2) n = 2;
  const int threads = n / 2 < 64 ? 64 : (n / 2 > 1024 ? 1024 : n / 2);
  const unsigned grid = static_cast<unsigned>(slices < (int64_t{1} << 20) ? slices : (int64_t{1} << 20));
  const size_t lds = static_cast<size_t>(n) * 12;
  hipLaunchKernelGGL(topk_kernel<T>, dim3(grid), dim3(threads), lds, stream, static_cast<const T*>(in),
                     static_cast<T*>(values), indices, p, n);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_topk(const void* in, int32_t elem_type, void* values, int64_t* indices, const TopKArgs& p,
                       hipStream_t stream) {
  if (p.rows * p.inner == 0 || p.k == 0) return hipSuccess;
  switch (elem_type) {
    case MOE_ELEM_FLOAT: return launch_typed<float>(in, values, indices, p, stream);
    case MOE_ELEM_FLOAT16: return launch_typed<_Float16>(in, values, indices, p, stream);
    case MOE_ELEM_BFLOAT16: return launch_typed<uint16_t>(in, values, indices, p, stream);
    case MOE_ELEM_DOUBLE: return launch_typed<double>(in, values, indices, p, stream);
    case MOE_ELEM_INT32: return launch_typed<int32_t>(in, values, indices, p, stream);
    case MOE_ELEM_INT64: return launch_typed<int64_t>(in, values, indices, p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace moe
