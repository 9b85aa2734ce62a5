// moe_expert_decode.hip -- weight-streaming expert GEMV for small token counts
// (decode), where the layer is bound by reading expert weights from HBM.
//
// Work split: grid (feature tiles, experts).  A workgroup of 4 wavefronts owns
// 64/ks output features of one expert; each wavefront owns 16 features and a
// 1/ks share of K (ks = 1, 2 or 4; partial sums are combined through LDS in a
// fixed order, so results do not depend on timing).  An expert with no routed
// token exits before touching its weights: only the experts actually hit are
// streamed.
//
// MFMA mapping (v_mfma_f32_16x16x32 f16/bf16): A = activations, 16 token rows
// per token group (NG groups cover up to 64 tokens); B = dequantised weights,
// 16 feature columns.  A lane (col = lane%16, g = lane/16) streams 16-byte
// pieces of its feature's weight row: for each 128-element chunk of K it
// covers k in [32g, 32g+32) and feeds 8 of them to each of 4 MFMA steps;
// the activation operand uses the same k assignment.  Each lane's 4 results
// share one feature, so a per-block scale is one multiply per lane.
//
// Scales: per output channel -> applied once after K; block_size a multiple of
// 128 -> applied to each chunk's partial sum (weights enter the MFMA as exact
// integers); block_size 16/32/64 -> folded into the weights before the MFMA.
#include "moe_dequant.h"
#include "moe_launch.h"

namespace moe {
namespace {

constexpr int kChunk = 128;  // K elements per lane-group pass

struct DecodeStage {
  const void* in;  // fc1: x [T, K]; fc2: act [T*k, K]
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
  int64_t block_size;
  float alpha, beta, limit;
  const int32_t* offsets;
  const int32_t* perm;
  int64_t topk;
  void* out;  // fc1: act [rows, nfeat] (AT); fc2: y2 [rows, nfeat] fp32
};

template <int WF>
struct WVec {
  static constexpr int kVecs = WF == kInt4 ? 1 : (WF == kInt8 ? 2 : 4);  // u32x4 per lane per chunk
  static constexpr int64_t row_bytes(int64_t K) { return WF == kInt4 ? K / 2 : (WF == kInt8 ? K : 2 * K); }
};

__device__ __forceinline__ u32x4_t ld16(const uint8_t* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

// Weight operand of MFMA step s (0..3) from a lane's chunk vectors.
template <typename AT, int WF>
__device__ __forceinline__ u32x4_t weight_operand(const u32x4_t* v, int s, bool fold, float sc) {
  if constexpr (WF == kInt4) {
    return fold ? dq4_scaled<AT>(v[0][s], sc) : dq4_exact<AT>(v[0][s]);
  } else if constexpr (WF == kInt8) {
    const uint32_t a = v[s >> 1][(s & 1) * 2], b = v[s >> 1][(s & 1) * 2 + 1];
    return fold ? dq8_scaled<AT>(a, b, sc) : dq8_exact<AT>(a, b);
  } else {
    return v[s];
  }
}

template <typename AT, int WF, int NG, bool FC1>
__global__ void __launch_bounds__(256) decode_gemv_kernel(DecodeStage p) {
  __shared__ floatx4_t red[4][2 * NG][kWave];
  const int e = blockIdx.y;
  const int row0 = p.offsets[e];
  const int cnt = p.offsets[e + 1] - row0;
  if (cnt == 0) return;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ks = p.ks, ftiles = 4 / ks;
  const int ft = wave / ks, kw = wave % ks;
  const int col = lane & 15, g = lane >> 4;
  const int64_t feat = (static_cast<int64_t>(blockIdx.x) * ftiles + ft) * 16 + col;
  const bool feat_ok = feat < p.nfeat;
  const bool gated = FC1 && p.gate_mode != kGateNone;

  int64_t ng = feat, nl = feat;
  if (FC1 && p.gate_mode == kGateInterleaved) { ng = 2 * feat; nl = 2 * feat + 1; }
  else if (FC1 && p.gate_mode == kGateChunked) { nl = p.nfeat + feat; }
  const int64_t K = p.K;
  const int64_t rb = WVec<WF>::row_bytes(K);
  const uint8_t* wg_row = p.w + (static_cast<int64_t>(e) * p.w_rows + (feat_ok ? ng : 0)) * rb;
  const uint8_t* wl_row = p.wl + (static_cast<int64_t>(e) * p.wl_rows + (feat_ok ? nl : 0)) * rb;

  const bool quant = WF != kDense;
  const int64_t bs = p.block_size;
  const bool per_chan = quant && bs == 0;
  const bool blk_after = quant && bs > 0 && (bs % kChunk) == 0;
  const bool fold = quant && bs > 0 && !blk_after;
  const int64_t nblk = quant ? (bs > 0 ? K / bs : 1) : 1;
  const int64_t sg_base = (static_cast<int64_t>(e) * p.w_rows + (feat_ok ? ng : 0)) * nblk;
  const int64_t sl_base = (static_cast<int64_t>(e) * p.wl_rows + (feat_ok ? nl : 0)) * nblk;

  // activation rows for the token groups
  const uint8_t* xrow[NG];
  bool xok[NG];
#pragma unroll
  for (int q = 0; q < NG; ++q) {
    const int m = q * 16 + col;
    xok[q] = m < cnt;
    int64_t src = 0;
    if (xok[q]) src = FC1 ? p.perm[row0 + m] / p.topk : row0 + m;
    xrow[q] = static_cast<const uint8_t*>(p.in) + src * K * 2;
  }

  const int64_t nchunks = (K + kChunk - 1) / kChunk;
  const int64_t per = (nchunks + ks - 1) / ks;
  const int64_t c0 = kw * per;
  const int64_t c1 = c0 + per < nchunks ? c0 + per : nchunks;

  floatx4_t accg[NG], accl[NG];
#pragma unroll
  for (int q = 0; q < NG; ++q) {
    accg[q] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    accl[q] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  }
  constexpr int V = WVec<WF>::kVecs;
  const int64_t lane_bytes = rb / (K / 32);  // bytes per 32 k of one row

  for (int64_t c = c0; c < c1; ++c) {
    const int64_t kb = c * kChunk + 32 * g;
    const bool kok = kb + 32 <= K;
    u32x4_t wg[V], wl[V], xv[NG][4];
    const u32x4_t z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int v = 0; v < V; ++v) {
      wg[v] = (feat_ok && kok) ? ld16(wg_row + (kb / 32) * lane_bytes + 16 * v) : z;
      wl[v] = (gated && feat_ok && kok) ? ld16(wl_row + (kb / 32) * lane_bytes + 16 * v) : z;
    }
#pragma unroll
    for (int q = 0; q < NG; ++q)
#pragma unroll
      for (int s = 0; s < 4; ++s) xv[q][s] = (xok[q] && kok) ? ld16(xrow[q] + kb * 2 + 16 * s) : z;

    floatx4_t tg[NG], tl[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q) {
      tg[q] = floatx4_t{0.f, 0.f, 0.f, 0.f};
      tl[q] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float scg = 1.0f, scl = 1.0f;
      if (fold && feat_ok && kok) {
        const int64_t blk = (kb + 8 * s) / bs;
        scg = load_any(p.s, p.scale_type, sg_base + blk);
        if (gated) scl = load_any(p.sl, p.scale_type, sl_base + blk);
      }
      const u32x4_t bg = weight_operand<AT, WF>(wg, s, fold, scg);
#pragma unroll
      for (int q = 0; q < NG; ++q) tg[q] = mfma16x16x32<AT>(xv[q][s], bg, tg[q]);
      if (gated) {
        const u32x4_t bl = weight_operand<AT, WF>(wl, s, fold, scl);
#pragma unroll
        for (int q = 0; q < NG; ++q) tl[q] = mfma16x16x32<AT>(xv[q][s], bl, tl[q]);
      }
    }
    float cg = 1.0f, cl = 1.0f;
    if (blk_after && feat_ok) {
      const int64_t blk = (c * kChunk) / bs;
      cg = load_any(p.s, p.scale_type, sg_base + blk);
      if (gated) cl = load_any(p.sl, p.scale_type, sl_base + blk);
    }
#pragma unroll
    for (int q = 0; q < NG; ++q) {
      accg[q] += tg[q] * cg;
      if (gated) accl[q] += tl[q] * cl;
    }
  }

  // combine the ks partial sums of a feature tile in wave order
  if (ks > 1) {
#pragma unroll
    for (int q = 0; q < NG; ++q) {
      red[wave][q][lane] = accg[q];
      red[wave][NG + q][lane] = accl[q];
    }
    __syncthreads();
    if (kw != 0) return;
    for (int w = 1; w < ks; ++w)
#pragma unroll
      for (int q = 0; q < NG; ++q) {
        accg[q] += red[wave + w][q][lane];
        accl[q] += red[wave + w][NG + q][lane];
      }
  }
  if (!feat_ok) return;

  float chg = 1.0f, chl = 1.0f;
  if (per_chan) {
    chg = load_any(p.s, p.scale_type, sg_base);
    if (gated) chl = load_any(p.sl, p.scale_type, sl_base);
  }
  const int act_t = AT::kId;
  float bg = 0.0f, bl = 0.0f;
  if (p.b) bg = load_any(p.b, act_t, static_cast<int64_t>(e) * p.w_rows + ng);
  if (gated && p.bl) bl = load_any(p.bl, act_t, static_cast<int64_t>(e) * p.wl_rows + nl);

#pragma unroll
  for (int q = 0; q < NG; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = q * 16 + 4 * g + r;
      if (m >= cnt) continue;
      const float vg = accg[q][r] * chg + bg;
      const int64_t o = static_cast<int64_t>(row0 + m) * p.nfeat + feat;
      if constexpr (FC1) {
        const float vl = accl[q][r] * chl + bl;
        const float a = apply_act(vg, vl, gated, p.activation, p.alpha, p.beta, p.limit);
        static_cast<typename AT::storage*>(p.out)[o] = from_f32<AT>(a);
      } else {
        static_cast<float*>(p.out)[o] = vg;
      }
    }
}

template <typename AT, int WF, bool FC1>
hipError_t launch_ng(const DecodeStage& st, int64_t T, int64_t E, hipStream_t stream) {
  const int ftiles = 4 / st.ks;
  dim3 grid(static_cast<unsigned>((st.nfeat + 16 * ftiles - 1) / (16 * ftiles)),
            static_cast<unsigned>(E));
  if (T <= 16) hipLaunchKernelGGL((decode_gemv_kernel<AT, WF, 1, FC1>), grid, dim3(256), 0, stream, st);
  else if (T <= 32) hipLaunchKernelGGL((decode_gemv_kernel<AT, WF, 2, FC1>), grid, dim3(256), 0, stream, st);
  else hipLaunchKernelGGL((decode_gemv_kernel<AT, WF, 4, FC1>), grid, dim3(256), 0, stream, st);
  return hipGetLastError();
}

template <bool FC1>
hipError_t launch_stage(const DecodeStage& st, const ExpertArgs& a, hipStream_t stream) {
  const bool bf = a.act_type == MOE_ELEM_BFLOAT16;
  switch (a.wfmt) {
    case kInt4: return bf ? launch_ng<BF16, kInt4, FC1>(st, a.T, a.E, stream)
                          : launch_ng<F16, kInt4, FC1>(st, a.T, a.E, stream);
    case kInt8: return bf ? launch_ng<BF16, kInt8, FC1>(st, a.T, a.E, stream)
                          : launch_ng<F16, kInt8, FC1>(st, a.T, a.E, stream);
    default: return bf ? launch_ng<BF16, kDense, FC1>(st, a.T, a.E, stream)
                       : launch_ng<F16, kDense, FC1>(st, a.T, a.E, stream);
  }
}

// Waves per feature tile: split K inside the workgroup when the feature count
// alone gives too few workgroups to keep every CU streaming.
int pick_ks(int64_t nfeat, int64_t K, int64_t E) {
  const int64_t nchunks = (K + kChunk - 1) / kChunk;
  int ks = 1;
  while (ks < 4 && (nfeat * E) / (16 * (4 / ks)) < 4096 && nchunks >= 2 * ks) ks *= 2;
  return ks;
}

}  // namespace

bool decode_supported(const ExpertArgs& a) {
  if (a.act_type != MOE_ELEM_FLOAT16 && a.act_type != MOE_ELEM_BFLOAT16) return false;
  if (a.T > kDecodeMaxTokens) return false;
  if (a.H % 32 || a.I % 32) return false;
  if (a.wfmt != kDense && a.block_size > 0 && a.block_size < 8) return false;
  return true;
}

hipError_t launch_fc1_decode(const ExpertArgs& a, hipStream_t stream) {
  DecodeStage st{};
  st.in = a.x;
  st.K = a.H;
  st.nfeat = a.I;
  const bool fused = a.gate_mode == kGateInterleaved || a.gate_mode == kGateChunked;
  st.w = static_cast<const uint8_t*>(a.w1);
  st.s = a.s1;
  st.b = a.b1;
  st.w_rows = fused ? 2 * a.I : a.I;
  if (a.gate_mode == kGateFc3) {
    st.wl = static_cast<const uint8_t*>(a.w3);
    st.sl = a.s3;
    st.bl = a.b3;
    st.wl_rows = a.I;
  } else {
    st.wl = st.w;
    st.sl = st.s;
    st.bl = st.b;
    st.wl_rows = st.w_rows;
  }
  st.gate_mode = a.gate_mode;
  st.scale_type = a.scale_type;
  st.activation = a.activation;
  st.block_size = a.wfmt == kDense ? 0 : a.block_size;
  st.alpha = a.alpha;
  st.beta = a.beta;
  st.limit = a.limit;
  st.offsets = a.offsets;
  st.perm = a.perm;
  st.topk = a.k;
  st.out = a.act;
  st.ks = pick_ks(a.I, a.H, a.E);
  return launch_stage<true>(st, a, stream);
}

hipError_t launch_fc2_decode(const ExpertArgs& a, hipStream_t stream) {
  DecodeStage st{};
  st.in = a.act;
  st.K = a.I;
  st.nfeat = a.H;
  st.w = static_cast<const uint8_t*>(a.w2);
  st.s = a.s2;
  st.b = a.b2;
  st.w_rows = a.H;
  st.wl = st.w;
  st.sl = st.s;
  st.bl = st.b;
  st.wl_rows = a.H;
  st.gate_mode = kGateNone;
  st.scale_type = a.scale_type;
  st.activation = kIdentity;
  st.block_size = a.wfmt == kDense ? 0 : a.block_size;
  st.offsets = a.offsets;
  st.perm = a.perm;
  st.topk = a.k;
  st.out = a.y2;
  st.ks = pick_ks(a.H, a.I, a.E);
  return launch_stage<false>(st, a, stream);
}

}  // namespace moe
