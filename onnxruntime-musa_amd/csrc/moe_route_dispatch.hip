// moe_route_dispatch.hip -- router and dispatch for gfx950.
//
// Router: one 64-lane wavefront per token.  Each lane holds up to 8 logits
// (expert e = lane + 64*i); softmax max/sum are butterfly reductions; the k
// experts are chosen by k rounds of a wave arg-max under the order
// (logit desc, expert id asc) -- the reference's TopK tie rule
// (musa/ep/src/kernels/math/topk_impl.mu:46-65: equal values -> lower index).
// Selection is on the logits; the weight of a chosen expert is its softmax
// (or sigmoid) probability, renormalised over the k chosen ones when asked.
//
// Dispatch: per-expert histogram, exclusive scan -> offsets[E+1], and a
// stable scatter that orders rows expert-major with ascending flat index
// t*k+j inside an expert (ascending token id, as the CPU EP batches tokens).
// The stable rank inside a wavefront comes from a ballot-built match mask
// (one ballot per expert-id bit) and a popcount of the lower lanes; waves are
// ordered through per-wave counts in LDS.  No unordered atomics decide a
// position, so the permutation is deterministic and bit-exact.
//
// Small T: one workgroup does all of it in one launch.  Large T: route +
// per-block histogram, a one-block scan, and a scatter pass.
#include <limits.h>

#include "moe_device.h"
#include "moe_launch.h"
#include "moe_route_device.h"

namespace moe {
namespace {

// Stable scatter of flat entries [f0, f1) by the whole workgroup.  base[e]
// (LDS) holds the next free row of expert e and is advanced here.  wcnt is an
// LDS scratch of nwaves * E ints.
__device__ void stable_scatter(const int32_t* ids, int64_t f0, int64_t f1, int E, int nbits,
                               int* base, int* wcnt, int32_t* perm, int32_t* inv_perm) {
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int nwaves = blockDim.x / kWave;
  for (int64_t s0 = f0; s0 < f1; s0 += blockDim.x) {
    for (int i = tid; i < nwaves * E; i += blockDim.x) wcnt[i] = 0;
    __syncthreads();
    const int64_t f = s0 + tid;
    const bool active = f < f1;
    const int e = active ? ids[f] : 0;
    const uint64_t mm = match_mask(e, active, nbits);
    const int r = lanes_below(mm, lane);
    if (active && r == 0) wcnt[wave * E + e] = __popcll(mm);
    __syncthreads();
    int row = 0;
    if (active) {
      int before = 0;
      for (int w = 0; w < wave; ++w) before += wcnt[w * E + e];
      row = base[e] + before + r;
    }
    __syncthreads();
    if (active) {
      perm[row] = static_cast<int32_t>(f);
      inv_perm[f] = row;
    }
    for (int x = tid; x < E; x += blockDim.x) {
      int add = 0;
      for (int w = 0; w < nwaves; ++w) add += wcnt[w * E + x];
      base[x] += add;
    }
    __syncthreads();
  }
}

// Exclusive scan of cnt[0..E) in LDS by wave 0 (E <= 512): writes
// offsets[0..E] and, if tile_offsets, the prefix of ceil(cnt / tile_m).
__device__ void scan_experts(const int* cnt, int E, int* base, int32_t* offsets,
                             int32_t* tile_offsets, int tile_m) {
  const int lane = threadIdx.x % kWave;
  if (threadIdx.x >= kWave) return;
  const int per = (E + kWave - 1) / kWave;
  const int e0 = lane * per;
  int run = 0, trun = 0;
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e < E) {
      run += cnt[e];
      if (tile_offsets) trun += (cnt[e] + tile_m - 1) / tile_m;
    }
  }
  // inclusive wave scan of run / trun
  int inc = run, tinc = trun;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int a = __shfl_up(inc, o, kWave);
    const int b = __shfl_up(tinc, o, kWave);
    if (lane >= o) {
      inc += a;
      tinc += b;
    }
  }
  int ex = inc - run, tex = tinc - trun;
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e < E) {
      offsets[e] = ex;
      base[e] = ex;
      if (tile_offsets) tile_offsets[e] = tex;
      ex += cnt[e];
      if (tile_offsets) tex += (cnt[e] + tile_m - 1) / tile_m;
    }
  }
  if (lane == kWave - 1) {
    offsets[E] = inc;
    if (tile_offsets) tile_offsets[E] = tinc;
  }
}

// ---- small T: everything in one workgroup (1024 threads) ----
template <typename LT, int VPL>
__global__ void __launch_bounds__(1024) route_dispatch_small_kernel(RouteArgs a) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int base[kMaxExperts];
  __shared__ int wcnt[16 * kMaxExperts];
  const moe_route_params& p = a.p;
  const int E = static_cast<int>(p.num_experts), k = static_cast<int>(p.k);
  const int64_t T = p.num_tokens;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int nwaves = blockDim.x / kWave;
  for (int i = tid; i < E; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  if constexpr (VPL == 1) {  // E <= 64: several tokens per wave (route_group)
    const int tpw = route_group_tokens(E);
    for (int64_t t0 = static_cast<int64_t>(wave) * tpw; t0 < T; t0 += static_cast<int64_t>(nwaves) * tpw) {
      int64_t t;
      int id;
      float w;
      if (route_group<LT>(p.logits, t0, T, E, k, p.normalize != 0, p.sigmoid != 0, lane, &t, &id, &w)) {
        const int e = lane % (kWave / tpw);
        p.topk_ids[t * k + e] = id;
        p.topk_w[t * k + e] = w;
        atomicAdd(&cnt[id], 1);  // counts only; order-independent
      }
    }
  } else {
    for (int64_t t = wave; t < T; t += nwaves) {
      int id;
      float w;
      route_token<LT, VPL>(p.logits, t, E, k, p.normalize != 0, p.sigmoid != 0, lane, &id, &w);
      if (lane < k) {
        p.topk_ids[t * k + lane] = id;
        p.topk_w[t * k + lane] = w;
        atomicAdd(&cnt[id], 1);  // counts only; order-independent
      }
    }
  }
  __syncthreads();
  scan_experts(cnt, E, base, p.offsets, a.tile_offsets, a.tile_m);
  __syncthreads();
  // make this workgroup's global writes of topk_ids visible to its own reads
  __threadfence_block();
  stable_scatter(p.topk_ids, 0, T * k, E, id_bits(E), base, wcnt, p.perm, p.inv_perm);
}

// ---- large T, pass 1: route + per-workgroup histogram ----
template <typename LT, int VPL>
__global__ void __launch_bounds__(1024) route_hist_kernel(RouteArgs a, int32_t* hist) {
  __shared__ int cnt[kMaxExperts];
  const moe_route_params& p = a.p;
  const int E = static_cast<int>(p.num_experts), k = static_cast<int>(p.k);
  const int64_t T = p.num_tokens;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int nwaves = blockDim.x / kWave;
  for (int i = tid; i < E; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kRouteTokensPerBlock;
  const int64_t t1 = t0 + kRouteTokensPerBlock < T ? t0 + kRouteTokensPerBlock : T;
  if constexpr (VPL == 1) {  // E <= 64: several tokens per wave (route_group)
    const int tpw = route_group_tokens(E);
    for (int64_t tb = t0 + static_cast<int64_t>(wave) * tpw; tb < t1; tb += static_cast<int64_t>(nwaves) * tpw) {
      int64_t t;
      int id;
      float w;
      if (route_group<LT>(p.logits, tb, t1, E, k, p.normalize != 0, p.sigmoid != 0, lane, &t, &id, &w)) {
        const int e = lane % (kWave / tpw);
        p.topk_ids[t * k + e] = id;
        p.topk_w[t * k + e] = w;
        atomicAdd(&cnt[id], 1);
      }
    }
  } else {
    for (int64_t t = t0 + wave; t < t1; t += nwaves) {
      int id;
      float w;
      route_token<LT, VPL>(p.logits, t, E, k, p.normalize != 0, p.sigmoid != 0, lane, &id, &w);
      if (lane < k) {
        p.topk_ids[t * k + lane] = id;
        p.topk_w[t * k + lane] = w;
        atomicAdd(&cnt[id], 1);
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < E; i += blockDim.x) hist[static_cast<int64_t>(blockIdx.x) * E + i] = cnt[i];
}

// ---- large T, pass 2: one workgroup scans the histograms ----
// hist[b][e] becomes the first row of expert e owned by workgroup b.  The
// 1024 threads split each expert's column of nblocks counts into parts
// (threads e + E * part); a thread reads its part in register chunks of 16
// independent loads, so the column is read at memory bandwidth rather than
// one dependent load at a time.
constexpr int kScanChunk = 16;

__global__ void __launch_bounds__(1024) dispatch_scan_kernel(RouteArgs a, int32_t* hist,
                                                             int nblocks) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int base[kMaxExperts];
  __shared__ int psum[1024];
  const int E = static_cast<int>(a.p.num_experts);
  const int parts = blockDim.x / E;  // E <= kMaxExperts <= blockDim.x
  const int tid = threadIdx.x;
  const int e = tid % E, part = tid / E;
  const bool active = part < parts;
  const int per = (nblocks + parts - 1) / parts;
  const int b0 = active ? part * per : 0;
  const int b1 = active ? min(nblocks, b0 + per) : 0;
  // column sums of each part
  int sum = 0;
  for (int c = b0; c < b1; c += kScanChunk) {
    int v[kScanChunk];
#pragma unroll
    for (int j = 0; j < kScanChunk; ++j) v[j] = c + j < b1 ? hist[static_cast<int64_t>(c + j) * E + e] : 0;
#pragma unroll
    for (int j = 0; j < kScanChunk; ++j) sum += v[j];
  }
  psum[tid] = sum;
  __syncthreads();
  if (tid < E) {
    int run = 0;
    for (int q = 0; q < parts; ++q) run += psum[q * E + tid];
    cnt[tid] = run;
  }
  __syncthreads();
  scan_experts(cnt, E, base, a.p.offsets, a.tile_offsets, a.tile_m);
  __syncthreads();
  // exclusive running sums, starting at the expert's base plus earlier parts
  if (active) {
    int run = base[e];
    for (int q = 0; q < part; ++q) run += psum[q * E + e];
    for (int c = b0; c < b1; c += kScanChunk) {
      int v[kScanChunk];
#pragma unroll
      for (int j = 0; j < kScanChunk; ++j) v[j] = c + j < b1 ? hist[static_cast<int64_t>(c + j) * E + e] : 0;
#pragma unroll
      for (int j = 0; j < kScanChunk; ++j) {
        if (c + j < b1) hist[static_cast<int64_t>(c + j) * E + e] = run;
        run += v[j];
      }
    }
  }
}

// ---- large T, pass 3: stable scatter per workgroup chunk ----
__global__ void __launch_bounds__(256) dispatch_scatter_kernel(RouteArgs a, const int32_t* hist) {
  __shared__ int base[kMaxExperts];
  __shared__ int wcnt[4 * kMaxExperts];
  const moe_route_params& p = a.p;
  const int E = static_cast<int>(p.num_experts);
  const int64_t k = p.k, T = p.num_tokens;
  for (int i = threadIdx.x; i < E; i += blockDim.x)
    base[i] = hist[static_cast<int64_t>(blockIdx.x) * E + i];
  __syncthreads();
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kRouteTokensPerBlock;
  const int64_t t1 = t0 + kRouteTokensPerBlock < T ? t0 + kRouteTokensPerBlock : T;
  stable_scatter(p.topk_ids, t0 * k, t1 * k, E, id_bits(E), base, wcnt, p.perm, p.inv_perm);
}

template <typename LT, int VPL>
hipError_t launch_typed(const RouteArgs& a, hipStream_t stream) {
  const int64_t T = a.p.num_tokens;
  if (T <= kSmallRouteTokens) {
    hipLaunchKernelGGL((route_dispatch_small_kernel<LT, VPL>), dim3(1), dim3(1024), 0, stream, a);
    return hipGetLastError();
  }
  const int nblocks = static_cast<int>((T + kRouteTokensPerBlock - 1) / kRouteTokensPerBlock);
  int32_t* hist = static_cast<int32_t*>(a.p.scratch);
  // 16 waves per workgroup: 4 tokens per wave
  hipLaunchKernelGGL((route_hist_kernel<LT, VPL>), dim3(nblocks), dim3(1024), 0, stream, a, hist);
  hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(1024), 0, stream, a, hist, nblocks);
  hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(nblocks), dim3(256), 0, stream, a,
                     static_cast<const int32_t*>(hist));
  return hipGetLastError();
}

template <typename LT>
hipError_t launch_vpl(const RouteArgs& a, hipStream_t stream) {
  const int64_t E = a.p.num_experts;
  if (E <= 64) return launch_typed<LT, 1>(a, stream);
  if (E <= 128) return launch_typed<LT, 2>(a, stream);
  if (E <= 256) return launch_typed<LT, 4>(a, stream);
  return launch_typed<LT, 8>(a, stream);
}

}  // namespace

size_t route_scratch_bytes(int64_t T, int64_t E, int64_t /*k*/) {
  if (T <= kSmallRouteTokens) return 0;
  const int64_t nblocks = (T + kRouteTokensPerBlock - 1) / kRouteTokensPerBlock;
  return static_cast<size_t>(nblocks * E) * sizeof(int32_t);
}

hipError_t launch_route_dispatch(const RouteArgs& a, hipStream_t stream) {
  // T == 0 still runs the single-workgroup kernel so offsets come out zero.
  switch (a.p.logits_type) {
    case MOE_ELEM_FLOAT: return launch_vpl<F32>(a, stream);
    case MOE_ELEM_FLOAT16: return launch_vpl<F16>(a, stream);
    case MOE_ELEM_BFLOAT16: return launch_vpl<BF16>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace moe
