// moe_route_device.h -- per-token routing and stable-rank helpers shared by
// the router/dispatch kernels and the decode kernel that routes in its
// prologue.
//
// Routing: one 64-lane wavefront per token; each lane holds up to 8 logits
// (expert e = lane + 64 i); the k experts are chosen by k rounds of a wave
// arg-max under the order (logit desc, expert id asc) -- the reference's
// TopK tie rule (musa/ep/src/kernels/math/topk_impl.mu:46-65: equal values
// -> lower index).
#pragma once

#include <limits.h>

#include "moe_device.h"
#include "moe_mi355x.h"

namespace moe {

__device__ __forceinline__ bool cand_before(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

// NaN logits rank below every number (as -inf), so every arg-max round finds
// a valid expert.
template <typename LT>
__device__ __forceinline__ float load_logit(const void* p, int64_t i) {
  const float v = to_f32<LT>(static_cast<const typename LT::storage*>(p)[i]);
  return v != v ? -INFINITY : v;
}

// Routes one token with the calling wavefront.  Returns, in lanes j < k, the
// j-th chosen expert id and its weight.
template <typename LT, int VPL>
__device__ __forceinline__ void route_token(const void* logits, int64_t t, int E, int k,
                                            bool normalize, bool sigm, int lane,
                                            int* out_id, float* out_w) {
  float v[VPL];
  bool taken[VPL];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int e = lane + kWave * i;
    v[i] = e < E ? load_logit<LT>(logits, t * E + e) : -INFINITY;
    taken[i] = e >= E;
    if (e < E) m = fmaxf(m, v[i]);
  }
  float s = 0.0f;
  if (!sigm) {
    m = wave_max(m);
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (!taken[i]) s += expf(v[i] - m);
    s = wave_sum(s);
  }
  int my_id = 0;
  float my_p = 0.0f, wsum = 0.0f;
  for (int j = 0; j < k; ++j) {
    float bv = -INFINITY;
    int bid = INT_MAX;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int e = lane + kWave * i;
      if (!taken[i] && cand_before(v[i], e, bv, bid)) {
        bv = v[i];
        bid = e;
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, kWave);
      const int oid = __shfl_xor(bid, o, kWave);
      if (cand_before(ov, oid, bv, bid)) {
        bv = ov;
        bid = oid;
      }
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (lane + kWave * i == bid) taken[i] = true;
    const float p = sigm ? 1.0f / (1.0f + expf(-bv)) : expf(bv - m) / s;
    wsum += p;
    if (lane == j) {
      my_id = bid;
      my_p = p;
    }
  }
  *out_id = my_id;
  *out_w = normalize ? my_p / wsum : my_p;
}

// Ballot-built mask of the lanes (among `active`) holding the same expert id.
__device__ __forceinline__ uint64_t match_mask(int e, bool active, int nbits) {
  uint64_t mask = __ballot(active);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t bal = __ballot(active && bit);
    mask &= bit ? bal : ~bal;
  }
  return mask;
}

__device__ __forceinline__ int lanes_below(uint64_t mask, int lane) {
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  return __popcll(mask & below);
}

__device__ __forceinline__ int id_bits(int E) {
  int b = 0;
  while ((1 << b) < E) ++b;
  return b;
}

// Routing and dispatch of a small batch by one workgroup, results in LDS:
// offs[0..E] (exclusive scan of the per-expert counts) and perm[0..T k)
// (row -> flat index t k + j, expert-major, ascending flat index within an
// expert): the values the router/dispatch kernels produce.  With publish,
// the workgroup also writes topk_ids, topk_w, offsets, perm and inv_perm of
// p to global memory.  scratch: route_block_scratch_bytes() of LDS.  Needs
// E <= 128 (at most two experts per lane in the scan); every thread of the
// workgroup calls it.
//
// The logits are first copied to LDS with one load per element: when every
// workgroup of a grid routes the same batch, a load per token and wave would
// send thousands of requests for the same few cache lines to one L2 channel.
// Routes tokens t0 + lane / G (G = the power of two >= E, E <= 64: 64 / G
// tokens per wavefront) with the calling wavefront: the steps of route_token
// with log2(G) butterfly steps instead of 6.  Lanes past E hold -inf / 0,
// which the omitted steps of a full-wave butterfly would only have added or
// compared, so the sums and the chosen experts are bit-identical to
// route_token's.  Returns true in the lanes e = lane % G < k of tokens below
// T, with *t the token, *id its e-th expert and *w the weight.
template <typename LT>
__device__ __forceinline__ bool route_group(const void* logits, int64_t t0, int64_t T, int E, int k, bool normalize,
                                            bool sigm, int lane, int64_t* t, int* id, float* w) {
  const int G = E <= 8 ? 8 : (E <= 16 ? 16 : (E <= 32 ? 32 : 64));
  const int e = lane % G;
  const int64_t tok = t0 + lane / G;
  const bool valid = tok < T && e < E;
  const float v = valid ? load_logit<LT>(logits, tok * E + e) : -INFINITY;
  bool taken = !valid;
  float m = v;
  for (int o = G / 2; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, G));
  float sum = 0.0f;
  if (!sigm) {
    sum = valid ? expf(v - m) : 0.0f;
    for (int o = G / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o, G);
  }
  int my_id = 0;
  float my_p = 0.0f, wsum = 0.0f;
  for (int j = 0; j < k; ++j) {
    float bv = taken ? -INFINITY : v;
    int bid = taken ? INT_MAX : e;
    for (int o = G / 2; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o, G);
      const int oid = __shfl_xor(bid, o, G);
      if (cand_before(ov, oid, bv, bid)) {
        bv = ov;
        bid = oid;
      }
    }
    if (e == bid) taken = true;
    const float pj = sigm ? 1.0f / (1.0f + expf(-bv)) : expf(bv - m) / sum;
    wsum += pj;
    if (e == j) {
      my_id = bid;
      my_p = pj;
    }
  }
  *t = tok;
  *id = my_id;
  *w = normalize ? my_p / wsum : my_p;
  return tok < T && e < k;
}

// Tokens per wavefront of route_group.
__device__ __forceinline__ int route_group_tokens(int E) {
  return kWave / (E <= 8 ? 8 : (E <= 16 ? 16 : (E <= 32 ? 32 : 64)));
}

// LDS bytes route_dispatch_block needs as scratch.
inline size_t route_block_scratch_bytes(int64_t T, int64_t E, int64_t k, int nwaves, int logit_bytes) {
  return static_cast<size_t>((2 * E + nwaves * E + T * k) * 4 + T * E * logit_bytes);
}

// route_dispatch_block for at most 64 rows (T k) and 64 experts: the waves
// route their tokens (logits read from global, each element once per
// workgroup), then wavefront 0 alone counts, scans and ranks the rows, one
// row per lane (rank = rows with a lower flat index and the same expert,
// from a ballot-built match mask): two barriers in all, no atomics.  The
// same results as the general path.
template <typename LT>
__device__ void route_dispatch_wave(const moe_route_params& p, int* offs, int* perm, int* scratch, bool publish) {
  const int E = static_cast<int>(p.num_experts), k = static_cast<int>(p.k);
  const int T = static_cast<int>(p.num_tokens), n = T * k;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int nwaves = blockDim.x / kWave;
  int* ids = scratch;     // [n] expert of each row (flat index t k + j)
  int* cnt = ids + n;     // [E] rows per expert
  const int tpw = route_group_tokens(E);
  for (int t0 = wave * tpw; t0 < T; t0 += nwaves * tpw) {
    int64_t t;
    int id;
    float w;
    if (route_group<LT>(p.logits, t0, T, E, k, p.normalize != 0, p.sigmoid != 0, lane, &t, &id, &w)) {
      const int e = lane % (kWave / tpw);
      ids[t * k + e] = id;
      if (publish) {
        p.topk_ids[t * k + e] = id;
        p.topk_w[t * k + e] = w;
      }
    }
  }
  __syncthreads();
  if (wave == 0) {
    // a wavefront's LDS accesses complete in order, so each store below is
    // seen by the loads after it; the accesses that read other lanes'
    // stores are volatile, so that the compiler keeps them in order too
    volatile int* vcnt = cnt;
    volatile int* voffs = offs;
    const bool act = lane < n;
    const int ef = act ? ids[lane] : 0;
    const uint64_t mm = match_mask(ef, act, id_bits(E));
    const int r = lanes_below(mm, lane);
    if (lane < E) vcnt[lane] = 0;
    if (act && r == 0) vcnt[ef] = __popcll(mm);
    const int c = lane < E ? vcnt[lane] : 0;
    int inc = c;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int v = __shfl_up(inc, o, kWave);
      if (lane >= o) inc += v;
    }
    if (lane < E) {
      voffs[lane] = inc - c;
      if (publish) p.offsets[lane] = inc - c;
    }
    if (lane == kWave - 1) {
      voffs[E] = inc;
      if (publish) p.offsets[E] = inc;
    }
    if (act) {
      const int row = voffs[ef] + r;
      perm[row] = lane;
      if (publish) {
        p.perm[row] = lane;
        p.inv_perm[lane] = row;
      }
    }
  }
  __syncthreads();
}

template <typename LT>
__device__ void route_dispatch_block(const moe_route_params& p, int* offs, int* perm, int* scratch,
                                     bool publish) {
  const int E = static_cast<int>(p.num_experts), k = static_cast<int>(p.k);
  const int T = static_cast<int>(p.num_tokens), n = T * k;
  if (n <= kWave && E <= kWave) {
    route_dispatch_wave<LT>(p, offs, perm, scratch, publish);
    return;
  }
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int nwaves = blockDim.x / kWave;
  int* cnt = scratch;
  int* base = cnt + E;
  int* wcnt = base + E;
  int* ids = wcnt + nwaves * E;
  using LS = typename LT::storage;
  LS* xl = reinterpret_cast<LS*>(ids + n);  // [T][E] logits
  const LS* xg = static_cast<const LS*>(p.logits);
  for (int i = tid; i < T * E; i += blockDim.x) xl[i] = xg[i];
  for (int i = tid; i < E; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  if (E <= kWave) {
    // tokens in lane groups (route_group)
    const int tpw = route_group_tokens(E);
    for (int t0 = wave * tpw; t0 < T; t0 += nwaves * tpw) {
      int64_t t;
      int id;
      float w;
      if (route_group<LT>(xl, t0, T, E, k, p.normalize != 0, p.sigmoid != 0, lane, &t, &id, &w)) {
        const int e = lane % (kWave / tpw);
        ids[t * k + e] = id;
        atomicAdd(&cnt[id], 1);  // counts only; order-independent
        if (publish) {
          p.topk_ids[t * k + e] = id;
          p.topk_w[t * k + e] = w;
        }
      }
    }
  } else {
    // 65..128 experts: one wavefront per token, two experts per lane
    for (int t = wave; t < T; t += nwaves) {
      int id;
      float w;
      route_token<LT, 2>(xl, t, E, k, p.normalize != 0, p.sigmoid != 0, lane, &id, &w);
      if (lane < k) {
        ids[t * k + lane] = id;
        atomicAdd(&cnt[id], 1);
        if (publish) {
          p.topk_ids[t * k + lane] = id;
          p.topk_w[t * k + lane] = w;
        }
      }
    }
  }
  __syncthreads();
  if (wave == 0) {
    // experts 2 lane and 2 lane + 1 (E <= 128)
    const int e0 = 2 * lane, e1 = 2 * lane + 1;
    const int c0 = e0 < E ? cnt[e0] : 0, c1 = e1 < E ? cnt[e1] : 0;
    int inc = c0 + c1;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int v = __shfl_up(inc, o, kWave);
      if (lane >= o) inc += v;
    }
    const int ex = inc - c0 - c1;
    if (e0 < E) {
      offs[e0] = ex;
      base[e0] = ex;
      if (publish) p.offsets[e0] = ex;
    }
    if (e1 < E) {
      offs[e1] = ex + c0;
      base[e1] = ex + c0;
      if (publish) p.offsets[e1] = ex + c0;
    }
    if (lane == kWave - 1) {
      offs[E] = inc;
      if (publish) p.offsets[E] = inc;
    }
  }
  __syncthreads();
  // stable ranks: within a wave from a ballot-built match mask, across waves
  // from per-wave counts; no unordered atomic decides a position
  const int nbits = id_bits(E);
  for (int s0 = 0; s0 < n; s0 += blockDim.x) {
    for (int i = tid; i < nwaves * E; i += blockDim.x) wcnt[i] = 0;
    __syncthreads();
    const int f = s0 + tid;
    const bool active = f < n;
    const int e = active ? ids[f] : 0;
    const uint64_t mm = match_mask(e, active, nbits);
    const int r = lanes_below(mm, lane);
    if (active && r == 0) wcnt[wave * E + e] = __popcll(mm);
    __syncthreads();
    if (active) {
      int before = 0;
      for (int w = 0; w < wave; ++w) before += wcnt[w * E + e];
      const int row = base[e] + before + r;
      perm[row] = f;
      if (publish) {
        p.perm[row] = f;
        p.inv_perm[f] = row;
      }
    }
    __syncthreads();
    for (int x = tid; x < E; x += blockDim.x) {
      int add = 0;
      for (int w = 0; w < nwaves; ++w) add += wcnt[w * E + x];
      base[x] += add;
    }
    __syncthreads();
  }
}

}  // namespace moe
