// moe_expert_decode.h -- weight-streaming expert GEMV for small token counts
// (decode), where the layer is bound by reading expert weights from HBM.
//
// MFMA mapping (v_mfma_f32_16x16x32 f16/bf16): A = activations, 16 token rows
// per token group (NG groups cover up to 64 tokens); B = dequantised weights,
// 16 feature columns per weight tile.  A lane (col = lane%16, g = lane/16)
// streams 16-byte pieces of its feature's weight row: for each 128-element
// chunk of K it covers k in [32g, 32g+32) and feeds 8 of them to each of 4
// MFMA steps; the activation operand uses the same k assignment.  Each lane's
// results share one feature, so a per-block scale is one multiply per lane.
//
// What bounds this kernel is the vector-memory path (address unit and L1
// tag lookups per byte), not HBM, so the design minimises L1 accesses per
// weight byte:
//   * each wave owns WT = 2 weight tiles (16 rows each), so one activation
//     fragment is reused by 2 MFMAs (more tiles per wave cut parallelism
//     more than they save);
//   * all loads are raw buffer loads; absent tokens, features past the end
//     and the missing part of a partial last chunk use an out-of-range
//     offset, which returns zero without any memory access;
//   * per-block scales are staged once into LDS per wave and read from there.
//
// Work split: grid (feature groups, experts, K groups).  A workgroup holds 4
// wavefronts = (4/ks) feature groups x ks K-splits; partial sums of a feature
// group are combined through LDS in a fixed order.  fc2 may also split K
// across KSG workgroups (grid z); those partial rows are summed in fixed order
// by the finalize pass, so results never depend on timing.  An expert with no
// routed token exits before touching its weights.
//
// Chunks are fetched ahead into a register ring (PD slots): each wave keeps
// PD-1 chunks in flight while it dequantises and multiplies the current one.
// Everything the inner loop depends on is a template parameter and nothing
// loaded is touched before it is consumed, so the loop is straight-line code
// whose loads the compiler waits for in order.
//
// Scales: per output channel -> applied once after K; block_size a multiple of
// 128 -> applied to each chunk's partial sum (weights enter the MFMA as exact
// integers); block_size 16/32/64 -> folded into the weights before the MFMA.
#pragma once

#include <algorithm>
#include <type_traits>

#include "moe_dequant.h"
#include "moe_launch.h"

namespace moe {
namespace decode {

constexpr int kChunk = 128;             // K elements per lane-group pass

// Cache policy (the aux operand of the gfx950 buffer loads) of data a decode
// layer reads once: tile-major (pre-packed) expert weights and their block
// scales.  Bit 1 is the non-temporal hint (streaming: not kept in the
// caches).  A plain read stream of 640 MB measured ~6.95 TB/s with it and
// ~6.15 TB/s without.  Row-major weights keep the default policy: there a
// load reads 64 bytes of each 128-byte line and the next chunk's load the
// other half, which must still be in the cache.
constexpr int kStreamAux = 2;
template <int AUX>
__device__ __forceinline__ u32x4_t bload16_aux(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, AUX));
}

// kScaleStep (stream kernel, block 32 / 64): each MFMA step takes 32
// consecutive k, which lie in one scale block, so the operands stay exact
// (biased) integers and the block scale multiplies the step's fp32 result.
// kScaleMx (stream kernel, MXFP4): the same step-major k; each step's E2M1
// operands are converted with the E8M0 scale of its block folded in.
enum ScaleMode : int { kScaleNone = 0, kScaleChan = 1, kScaleBlock = 2, kScaleFold = 3, kScaleStep = 4, kScaleMx = 5 };

struct Stage {
  const void* in;  // fc1: x [T, K]; fc2: act [T*k, K]
  int64_t in_rows;
  int64_t K, nfeat;
  const uint8_t* w;  // gate / plain weight, [E, w_rows, K(/pack)]
  const void* s;
  const void* b;
  int64_t w_rows;
  const uint8_t* wl;  // linear weight (fc3 or the fused fc1)
  const void* sl;
  const void* bl;
  int64_t wl_rows;
  int32_t gate_mode, scale_type, activation, ks;
  int32_t ksg;        // K splits across workgroups (fc2 only)
  int32_t lds_scale;  // bytes of LDS per wave for staged scales
  int32_t tiled;      // weights tile-major (stream kernel only; K padded to whole chunks)
  int32_t deint;      // fc1 tile-major weights of interleaved SwiGLU stored de-interleaved:
                      // gate rows [0, nfeat), linear rows [nfeat, 2 nfeat); scales and
                      // biases keep the interleaved order
  int32_t stiled;     // step-scale block scales tile-major (stream kernel; rows as the weights')
  int64_t block_size;
  float alpha, beta, limit;
  const int32_t* offsets;
  const int32_t* perm;
  int64_t topk;
  int64_t out_rows;  // rows of one partial output plane (T*k)
  void* out;         // fc1: act [rows, nfeat] (AT); fc2: y2 [ksg][rows, nfeat] fp32
};

// Tile geometry per (weight format, token groups, gating).
template <int WF, int NG, bool GATED>
struct Geo {
  static constexpr int kVecs = WF == kInt4 ? 1 : (WF == kInt8 ? 2 : 4);  // u32x4 per tile per chunk
  static constexpr int kLaneBytes = 16 * kVecs;                           // bytes per 32 k of a row
  static constexpr int WT = 2;  // weight tiles (gate + linear of 16 features, or 2 x 16 features)
  static constexpr int FT = GATED ? WT / 2 : WT;                                       // feature tiles
  static constexpr int kChunkVgprs = WT * 4 * kVecs + 16 * NG;
  static constexpr int PD = kChunkVgprs <= 64 ? 3 : 2;
};

template <int WF, int NG, bool GATED>
struct Chunk {
  using G = Geo<WF, NG, GATED>;
  u32x4_t w[G::WT][G::kVecs];
  u32x4_t x[NG][4];
};


template <typename AT, int WF, int SM, typename ST, int NG, bool FC1, bool GATED>
__global__ void __launch_bounds__(256) gemv_kernel(Stage p) {
  using G = Geo<WF, NG, GATED>;
  constexpr int WT = G::WT, FT = G::FT, PD = G::PD, LB = G::kLaneBytes;
  constexpr bool kPerBlock = SM == kScaleBlock || SM == kScaleFold;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int e = blockIdx.y;
  const int row0 = p.offsets[e];
  const int cnt = p.offsets[e + 1] - row0;
  if (cnt == 0) return;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ks = p.ks, fgroups = 4 / ks;
  const int fg = wave / ks, kw = wave % ks;
  const int col = lane & 15, g = lane >> 4;
  const int64_t fbase = (static_cast<int64_t>(blockIdx.x) * fgroups + fg) * (16 * FT);
  const int64_t K = p.K;
  const int64_t rb = (K / 32) * LB;  // bytes of one weight row

  // ---- weight rows of the lane's tiles (tile t < FT: gate/plain, t >= FT: linear) ----
  const uint8_t* wbase_g = p.w + static_cast<int64_t>(e) * p.w_rows * rb;
  const uint8_t* wbase_l = p.wl + static_cast<int64_t>(e) * p.wl_rows * rb;
  const __amdgpu_buffer_rsrc_t rs_g = make_rsrc(wbase_g, static_cast<uint32_t>(p.w_rows * rb));
  const __amdgpu_buffer_rsrc_t rs_l = make_rsrc(wbase_l, static_cast<uint32_t>(p.wl_rows * rb));
  int64_t trow[WT];  // weight row (within the expert) of each tile for this lane
  bool tok[WT];      // feature in range
#pragma unroll
  for (int t = 0; t < WT; ++t) {
    const int64_t f = fbase + (t % FT) * 16 + col;
    tok[t] = f < p.nfeat;
    trow[t] = tile_row(tok[t] ? f : 0, GATED && t >= FT, FC1 && GATED, p.gate_mode, p.nfeat);
  }

  // ---- K range of this wave ----
  const int nchunks = static_cast<int>((K + kChunk - 1) / kChunk);
  const int nsplit = ks * p.ksg;
  const int split = static_cast<int>(blockIdx.z) * ks + kw;
  const int per = (nchunks + nsplit - 1) / nsplit;
  const int c0 = split * per < nchunks ? split * per : nchunks;
  const int c1 = c0 + per < nchunks ? c0 + per : nchunks;
  const int64_t ktail = K - static_cast<int64_t>(nchunks - 1) * kChunk;  // valid k of the last chunk

  // ---- stage this wave's block scales into LDS: sc[(t * nb + b) * 16 + col], fp32 ----
  float* sc = reinterpret_cast<float*>(smem + static_cast<size_t>(wave) * p.lds_scale);
  int64_t b0 = 0;
  int bshift = 0;
  int nb = 0;
  if constexpr (kPerBlock) {
    bshift = __builtin_ctzll(static_cast<uint64_t>(p.block_size));
    const int64_t nblk = K / p.block_size;
    b0 = (static_cast<int64_t>(c0) * kChunk) >> bshift;
    // whole chunks: the lanes of a partial last chunk that lie past K still
    // read a scale (and multiply zeros), so their blocks are staged as 0
    if (c1 > c0) nb = static_cast<int>(((static_cast<int64_t>(c1) * kChunk - 1) >> bshift) + 1 - b0);
    const typename ST::storage* sgp = static_cast<const typename ST::storage*>(p.s);
    const typename ST::storage* slp = static_cast<const typename ST::storage*>(p.sl);
    const int total = WT * 16 * nb;
    for (int i = lane; i < total; i += kWave) {
      const int b = i % nb, tc = i / nb;  // consecutive lanes read consecutive blocks of one row
      const int t = tc / 16, cc = tc % 16;
      const bool lin = GATED && t >= FT;
      const int64_t f = fbase + (t % FT) * 16 + cc;
      float v = 0.0f;
      if (f < p.nfeat && b0 + b < nblk) {
        const int64_t r = tile_row(f, lin, FC1 && GATED, p.gate_mode, p.nfeat);
        const int64_t rows = lin ? p.wl_rows : p.w_rows;
        v = to_f32<ST>((lin ? slp : sgp)[(static_cast<int64_t>(e) * rows + r) * nblk + b0 + b]);
      }
      sc[(t * nb + b) * 16 + cc] = v;
    }
  }
  __syncthreads();

  // ---- activation rows (absent tokens read nothing) ----
  const __amdgpu_buffer_rsrc_t rs_x = make_rsrc(p.in, static_cast<uint32_t>(p.in_rows * K * 2));
  uint32_t xoff[NG];
#pragma unroll
  for (int q = 0; q < NG; ++q) {
    const int m = q * 16 + col;
    if (m < cnt) {
      const int64_t src = FC1 ? p.perm[row0 + m] / p.topk : row0 + m;
      xoff[q] = static_cast<uint32_t>(src * K * 2 + g * 64);
    } else {
      xoff[q] = kOob;
    }
  }
  uint32_t woff[WT];
#pragma unroll
  for (int t = 0; t < WT; ++t) woff[t] = tok[t] ? static_cast<uint32_t>(trow[t] * rb + g * LB) : kOob;

  using CK = Chunk<WF, NG, GATED>;
  auto fetch = [&](int c, CK& d) {
    // lanes whose 32-k piece lies past K (partial last chunk) read nothing
    const bool kin = c < nchunks - 1 || 32 * g + 32 <= ktail;
    const uint32_t wc = static_cast<uint32_t>(c) * (4 * LB);
    const uint32_t xc = static_cast<uint32_t>(c) * (kChunk * 2);
#pragma unroll
    for (int t = 0; t < WT; ++t) {
      const uint32_t o = kin ? woff[t] + wc : kOob;
#pragma unroll
      for (int v = 0; v < G::kVecs; ++v) d.w[t][v] = bload16(GATED && t >= FT ? rs_l : rs_g, o + 16 * v);
    }
#pragma unroll
    for (int q = 0; q < NG; ++q) {
      const uint32_t o = kin ? xoff[q] + xc : kOob;
#pragma unroll
      for (int s = 0; s < 4; ++s) d.x[q][s] = bload16(rs_x, o + 16 * s);
    }
  };

  floatx4_t acc[WT][NG];
#pragma unroll
  for (int t = 0; t < WT; ++t)
#pragma unroll
    for (int q = 0; q < NG; ++q) acc[t][q] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int c, const CK& d) {
    floatx4_t tmp[WT][NG];
#pragma unroll
    for (int t = 0; t < WT; ++t)
#pragma unroll
      for (int q = 0; q < NG; ++q) tmp[t][q] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int t = 0; t < WT; ++t) {
        float fs = 0.0f;
        if constexpr (SM == kScaleFold) {
          const int blk = static_cast<int>(((static_cast<int64_t>(c) * kChunk + 32 * g + 8 * s) >> bshift) - b0);
          fs = sc[(t * nb + blk) * 16 + col];
        }
        const u32x4_t bw = weight_operand<AT, WF, SM == kScaleFold>(d.w[t], s, fs);
#pragma unroll
        for (int q = 0; q < NG; ++q) {
          if constexpr (SM == kScaleBlock) tmp[t][q] = mfma16x16x32<AT>(d.x[q][s], bw, tmp[t][q]);
          else acc[t][q] = mfma16x16x32<AT>(d.x[q][s], bw, acc[t][q]);
        }
      }
    }
    if constexpr (SM == kScaleBlock) {
      const int blk = static_cast<int>(((static_cast<int64_t>(c) * kChunk) >> bshift) - b0);
#pragma unroll
      for (int t = 0; t < WT; ++t) {
        const float bsc = sc[(t * nb + blk) * 16 + col];
#pragma unroll
        for (int q = 0; q < NG; ++q) acc[t][q] += tmp[t][q] * bsc;
      }
    }
  };

  // Register ring: chunk c sits in ring[(c - c0) % PD].  The main loop has no
  // conditions: each slot is consumed, then refilled with the chunk PD later,
  // clamped to the wave's last chunk (a clamped refill is never consumed).
  if (c0 < c1) {
    CK ring[PD];
    const int clast = c1 - 1;
#pragma unroll
    for (int d = 0; d < PD; ++d) fetch(min(c0 + d, clast), ring[d]);
    int c = c0;
    for (; c + PD <= c1; c += PD) {
#pragma unroll
      for (int d = 0; d < PD; ++d) {
        compute(c + d, ring[d]);
        fetch(min(c + d + PD, clast), ring[d]);
      }
    }
#pragma unroll
    for (int d = 0; d < PD - 1; ++d)
      if (c + d < c1) compute(c + d, ring[d]);
  }

  // ---- combine the ks partial sums of a feature group in wave order ----
  if (ks > 1) {
    __syncthreads();  // every wave is done with its staged scales
    floatx4_t* red = reinterpret_cast<floatx4_t*>(smem);
#pragma unroll
    for (int t = 0; t < WT; ++t)
#pragma unroll
      for (int q = 0; q < NG; ++q) red[((wave * WT + t) * NG + q) * kWave + lane] = acc[t][q];
    __syncthreads();
    if (kw != 0) return;
    for (int w = 1; w < ks; ++w)
#pragma unroll
      for (int t = 0; t < WT; ++t)
#pragma unroll
        for (int q = 0; q < NG; ++q) acc[t][q] += red[(((wave + w) * WT + t) * NG + q) * kWave + lane];
  }

  // ---- epilogue ----
  const int act_t = AT::kId;
  const bool first_split = blockIdx.z == 0;
#pragma unroll
  for (int ft = 0; ft < FT; ++ft) {
    const int tg = ft, tl = GATED ? ft + FT : ft;
    if (!tok[tg]) continue;
    const int64_t f = fbase + ft * 16 + col;
    float chg = 1.0f, chl = 1.0f;
    if constexpr (SM == kScaleChan) {
      chg = load_any(p.s, p.scale_type, static_cast<int64_t>(e) * p.w_rows + trow[tg]);
      if constexpr (GATED) chl = load_any(p.sl, p.scale_type, static_cast<int64_t>(e) * p.wl_rows + trow[tl]);
    }
    float bg = 0.0f, bl = 0.0f;
    if (p.b && first_split) bg = load_any(p.b, act_t, static_cast<int64_t>(e) * p.w_rows + trow[tg]);
    if (GATED && p.bl) bl = load_any(p.bl, act_t, static_cast<int64_t>(e) * p.wl_rows + trow[tl]);
#pragma unroll
    for (int q = 0; q < NG; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = q * 16 + 4 * g + r;
        if (m >= cnt) continue;
        const float vg = acc[tg][q][r] * chg + bg;
        const int64_t o = static_cast<int64_t>(row0 + m) * p.nfeat + f;
        if constexpr (FC1) {
          const float vl = GATED ? acc[tl][q][r] * chl + bl : 0.0f;
          const float a = apply_act<true>(vg, vl, GATED, p.activation, p.alpha, p.beta, p.limit);
          static_cast<typename AT::storage*>(p.out)[o] = from_f32<AT>(a);
        } else {
          static_cast<float*>(p.out)[static_cast<int64_t>(blockIdx.z) * p.out_rows * p.nfeat + o] = vg;
        }
      }
  }
}

template <int WF, int NG, bool GATED>
size_t lds_bytes(const Stage& st) {
  using G = Geo<WF, NG, GATED>;
  const size_t red = st.ks > 1 ? static_cast<size_t>(4) * G::WT * NG * kWave * 16 : 0;
  return std::max(static_cast<size_t>(4) * st.lds_scale, red);
}

// Token groups: one group of 16 rows up to T = 16, else 4 groups (T <= 64).
template <typename AT, int WF, int SM, typename ST, bool FC1, bool GATED>
hipError_t launch(const Stage& st, int64_t T, int64_t E, hipStream_t stream) {
  auto go = [&](auto ng_tag) -> hipError_t {
    constexpr int NG = decltype(ng_tag)::value;
    using G = Geo<WF, NG, GATED>;
    const int fgroups = 4 / st.ks;
    const int64_t fpw = 16 * G::FT;
    const int64_t waves_f = (st.nfeat + fpw - 1) / fpw;
    dim3 grid(static_cast<unsigned>((waves_f + fgroups - 1) / fgroups), static_cast<unsigned>(E),
              static_cast<unsigned>(st.ksg));
    const size_t lds = lds_bytes<WF, NG, GATED>(st);
    hipLaunchKernelGGL((gemv_kernel<AT, WF, SM, ST, NG, FC1, GATED>), grid, dim3(256), lds, stream, st);
    return hipGetLastError();
  };
  if (T <= 16) return go(std::integral_constant<int, 1>{});
  return go(std::integral_constant<int, 4>{});
}

template <typename AT, int WF, int SM, typename ST>
hipError_t launch_kinds(const Stage& st, int64_t T, int64_t E, bool fc1, bool gated, hipStream_t stream) {
  if (!fc1) return launch<AT, WF, SM, ST, false, false>(st, T, E, stream);
  if (gated) return launch<AT, WF, SM, ST, true, true>(st, T, E, stream);
  return launch<AT, WF, SM, ST, true, false>(st, T, E, stream);
}

// Per weight format translation units.
hipError_t launch_int4(const Stage& st, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream);
hipError_t launch_int8(const Stage& st, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream);
hipError_t launch_dense(const Stage& st, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream);

inline int scale_mode(const ExpertArgs& a) {
  if (a.wfmt == kDense) return kScaleNone;
  if (a.block_size == 0) return kScaleChan;
  return a.block_size % kChunk == 0 ? kScaleBlock : kScaleFold;
}

// Host mirror of Geo<>: weight tiles per wave.
inline int weight_tiles(int /*wfmt*/, int64_t /*T*/) { return 2; }

// Quantised formats: dispatch over activation type, scale mode and scale type.
template <int WF>
hipError_t launch_quant(const Stage& st, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream) {
  const bool bf = a.act_type == MOE_ELEM_BFLOAT16;
  const int sm = scale_mode(a);
  auto by_st = [&](auto at_tag, auto sm_tag) -> hipError_t {
    using AT = decltype(at_tag);
    constexpr int SM = decltype(sm_tag)::value;
    switch (a.scale_type) {
      case MOE_ELEM_FLOAT: return launch_kinds<AT, WF, SM, F32>(st, a.T, a.E, fc1, gated, stream);
      case MOE_ELEM_BFLOAT16: return launch_kinds<AT, WF, SM, BF16>(st, a.T, a.E, fc1, gated, stream);
      default: return launch_kinds<AT, WF, SM, F16>(st, a.T, a.E, fc1, gated, stream);
    }
  };
  using BLK = std::integral_constant<int, kScaleBlock>;
  using FOLD = std::integral_constant<int, kScaleFold>;
  if (sm == kScaleChan) {  // scale read once after K: the type needs no specialisation
    return bf ? launch_kinds<BF16, WF, kScaleChan, F16>(st, a.T, a.E, fc1, gated, stream)
              : launch_kinds<F16, WF, kScaleChan, F16>(st, a.T, a.E, fc1, gated, stream);
  }
  if (sm == kScaleBlock) return bf ? by_st(BF16{}, BLK{}) : by_st(F16{}, BLK{});
  return bf ? by_st(BF16{}, FOLD{}) : by_st(F16{}, FOLD{});
}

}  // namespace decode
}  // namespace moe
