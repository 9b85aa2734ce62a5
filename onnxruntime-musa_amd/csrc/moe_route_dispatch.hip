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

#include "moe_dequant.h"
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

// Router GEMM of tokens [t0, t1): logits[t][e] = sum_k x[t][k] w[e][k]
// (+ b[e]), fp32 accumulation, rounded once to the logits type, written to
// a.p.logits.  A wave takes one token at a time and up to kGateExperts
// experts; lane l accumulates k = 8 l + 512 i .. + 7 in order, then a
// butterfly adds the lanes, so every sum has a fixed order.  The x piece of
// an iteration is loaded once for all the wave's experts.  Ends on a barrier
// after which the workgroup's reads of the logits see them.
constexpr int kGateExperts = 8;

template <typename LT>
__device__ __forceinline__ void load8(const void* base, int64_t i, int64_t n, float* v) {
  using S = typename LT::storage;
  const S* p = static_cast<const S*>(base) + i;
  if (i + 8 <= n) {
    if constexpr (sizeof(S) == 2) {
      const u32x4_t q = *reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = to_f32<LT>(__builtin_bit_cast(S, static_cast<uint16_t>(q[j] & 0xFFFFu)));
        v[2 * j + 1] = to_f32<LT>(__builtin_bit_cast(S, static_cast<uint16_t>(q[j] >> 16)));
      }
    } else {
      const u32x4_t q0 = *reinterpret_cast<const u32x4_t*>(p);
      const u32x4_t q1 = *reinterpret_cast<const u32x4_t*>(p + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = __uint_as_float(q0[j]);
        v[4 + j] = __uint_as_float(q1[j]);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = i + j < n ? to_f32<LT>(p[j]) : 0.0f;
  }
}

// The same for fp16 / bf16 with MFMA (v_mfma_f32_16x16x32; tokens [t0, t0 +
// 16) are the A rows, 16 experts per B tile): the waves split (expert tile,
// K range) -- a wave's A and B fragments are 16-byte loads, so each block
// reads x and the gate weights once -- and the partial tiles of one expert
// tile are added through LDS in wave order.  Needs H % 8 == 0 (a 16-byte
// piece is then wholly inside or outside a row) and t1 - t0 <= 16.
// red: LDS of blockDim.x / 64 * 256 floats.
constexpr int kGateMfmaRows = 16;

template <typename LT>
__device__ void gate_logits_mfma(const RouteArgs& a, int64_t t0, int64_t t1, float* red) {
  using S = typename LT::storage;
  const int E = static_cast<int>(a.p.num_experts);
  const int64_t H = a.hidden;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, nwaves = blockDim.x / kWave;
  const int col = lane & 15, g = lane >> 4;
  const int ntiles = (E + 15) / 16;
  const int wpt = ntiles >= nwaves ? 1 : nwaves / ntiles;  // waves per expert tile
  const int steps = static_cast<int>((H + 31) / 32);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.gate_x, static_cast<uint32_t>(a.p.num_tokens * H * 2));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.gate_w, static_cast<uint32_t>(E * H * 2));
  const int64_t tok = t0 + col;
  // this wave's share: tiles wave / wpt (+ nwaves / wpt ...), K part wave % wpt
  for (int tile = wave / wpt; tile < ntiles; tile += nwaves / wpt) {
    const int part = wave % wpt;
    const int s0 = steps * part / wpt, s1 = steps * (part + 1) / wpt;
    const int ex = tile * 16 + col;
    floatx4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int st = s0; st < s1; ++st) {
      const int64_t k = static_cast<int64_t>(st) * 32 + 8 * g;
      const uint32_t ox = tok < t1 && k < H ? static_cast<uint32_t>((tok * H + k) * 2) : kOob;
      const uint32_t ow = ex < E && k < H ? static_cast<uint32_t>((static_cast<int64_t>(ex) * H + k) * 2) : kOob;
      const u32x4_t av = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rx, static_cast<int>(ox), 0, 0));
      const u32x4_t bv = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, static_cast<int>(ow), 0, 0));
      acc = mfma16x16x32<LT>(av, bv, acc);
    }
    if (ntiles < nwaves) {
      *reinterpret_cast<floatx4_t*>(red + (wave * 64 + lane) * 4) = acc;
    } else {
      // one wave per tile (wpt == 1): its result is final
      if (ex < E) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t t = t0 + 4 * g + r;
          if (t < t1) {
            float v = acc[r];
            if (a.gate_b) v += to_f32<LT>(static_cast<const S*>(a.gate_b)[ex]);
            static_cast<S*>(const_cast<void*>(a.p.logits))[t * E + ex] = from_f32<LT>(v);
          }
        }
      }
    }
  }
  __syncthreads();
  if (ntiles < nwaves && wave % wpt == 0 && wave / wpt < ntiles) {
    // the first wave of each tile adds the tile's partials in wave order
    const int tile = wave / wpt, ex = tile * 16 + col;
    floatx4_t acc = *reinterpret_cast<const floatx4_t*>(red + (wave * 64 + lane) * 4);
    for (int j = 1; j < wpt; ++j) acc += *reinterpret_cast<const floatx4_t*>(red + ((wave + j) * 64 + lane) * 4);
    if (ex < E) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t t = t0 + 4 * g + r;
        if (t < t1) {
          float v = acc[r];
          if (a.gate_b) v += to_f32<LT>(static_cast<const S*>(a.gate_b)[ex]);
          static_cast<S*>(const_cast<void*>(a.p.logits))[t * E + ex] = from_f32<LT>(v);
        }
      }
    }
  }
  __threadfence_block();
  __syncthreads();
}

// Router GEMM of tokens [t0, t1) (any count, fp32 or odd H): the SIMT form.
template <typename LT>
__device__ void gate_logits_simt(const RouteArgs& a, int64_t t0, int64_t t1) {
  using S = typename LT::storage;
  const int E = static_cast<int>(a.p.num_experts);
  const int64_t H = a.hidden;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, nwaves = blockDim.x / kWave;
  const int echunks = (E + kGateExperts - 1) / kGateExperts;
  S* out = static_cast<S*>(const_cast<void*>(a.p.logits));
  // work items (token, expert chunk), token-major
  const int64_t items = (t1 - t0) * echunks;
  for (int64_t it = wave; it < items; it += nwaves) {
    const int64_t t = t0 + it / echunks;
    const int e0 = static_cast<int>(it % echunks) * kGateExperts;
    const int ne = E - e0 < kGateExperts ? E - e0 : kGateExperts;
    float acc[kGateExperts];
#pragma unroll
    for (int j = 0; j < kGateExperts; ++j) acc[j] = 0.0f;
    const void* xrow = static_cast<const S*>(a.gate_x) + t * H;
    for (int64_t k = 8 * lane; k < H; k += 8 * kWave) {
      float xv[8];
      load8<LT>(xrow, k, H, xv);
#pragma unroll
      for (int j = 0; j < kGateExperts; ++j) {
        if (j < ne) {
          float wv[8];
          load8<LT>(static_cast<const S*>(a.gate_w) + static_cast<int64_t>(e0 + j) * H, k, H, wv);
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[j] = __builtin_fmaf(xv[q], wv[q], acc[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kGateExperts; ++j) {
#pragma unroll
      for (int o = kWave / 2; o > 0; o >>= 1) acc[j] += __shfl_xor(acc[j], o, kWave);
    }
    if (lane < ne) {
      float v = acc[0];
#pragma unroll
      for (int j = 1; j < kGateExperts; ++j) v = lane == j ? acc[j] : v;
      if (a.gate_b) v += to_f32<LT>(static_cast<const S*>(a.gate_b)[e0 + lane]);
      out[t * E + e0 + lane] = from_f32<LT>(v);
    }
  }
  __threadfence_block();
  __syncthreads();
}

// Router GEMM of tokens [t0, t1): MFMA blocks of 16 tokens for fp16 / bf16
// with H % 8 == 0, else the SIMT form.  red: LDS of blockDim.x / 64 * 256
// floats.
template <typename LT>
__device__ void gate_logits(const RouteArgs& a, int64_t t0, int64_t t1, float* red) {
  if constexpr (sizeof(typename LT::storage) == 2) {
    if (a.hidden % 8 == 0) {
      for (int64_t b = t0; b < t1; b += kGateMfmaRows)
        gate_logits_mfma<LT>(a, b, b + kGateMfmaRows < t1 ? b + kGateMfmaRows : t1, red);
      return;
    }
  }
  (void)red;
  gate_logits_simt<LT>(a, t0, t1);
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
  // the router GEMM's partial tiles reuse the wave-count scratch (16 waves x 256 floats)
  static_assert(16 * kMaxExperts >= 16 * 256, "router GEMM partials fit the scratch");
  if (a.gate_w) gate_logits<LT>(a, 0, T, reinterpret_cast<float*>(wcnt));
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
  __shared__ float red[16 * 256];  // router GEMM partial tiles (16 waves)
  const moe_route_params& p = a.p;
  const int E = static_cast<int>(p.num_experts), k = static_cast<int>(p.k);
  const int64_t T = p.num_tokens;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int nwaves = blockDim.x / kWave;
  for (int i = tid; i < E; i += blockDim.x) cnt[i] = 0;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kRouteTokensPerBlock;
  const int64_t t1 = t0 + kRouteTokensPerBlock < T ? t0 + kRouteTokensPerBlock : T;
  if (a.gate_w) gate_logits<LT>(a, t0, t1, red);
  __syncthreads();
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
  if (T <= kSmallRouteTokens && (!a.gate_w || T * a.p.num_experts * a.hidden <= kGateSmallMacs)) {
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

size_t route_scratch_bytes_gate(int64_t T, int64_t E) {
  if (T == 0) return 0;
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
