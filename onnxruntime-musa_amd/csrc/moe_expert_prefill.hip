// moe_expert_prefill.hip -- grouped expert GEMM for large token counts
// (prefill), bound by MFMA throughput.
//
// Each workgroup computes a 128 (rows of one expert) x 128 (weight rows) tile
// with 4 wavefronts in a 2x2 arrangement, each wave 64x64 as 2x2
// v_mfma_f32_32x32x16 tiles with fp32 accumulation.  K advances 64 at a time
// through a double-buffered LDS stage: activations are copied as-is (fc1
// gathers token rows through the dispatch permutation, so the permuted input
// is never materialised), weights are dequantised in registers on the way
// from HBM to LDS (scale folded into the 16-bit operand).
//
// For gated activations the 128 weight rows of a tile are the gate rows and
// the linear rows of the same 64 features, so a lane holds both halves of
// each output and applies bias + activation in the epilogue.
//
// Tile order: the row tiles of one (expert, weight tile) are consecutive and
// are mapped onto one XCD (hardware workgroup ids are dealt to the 8 XCDs
// round-robin), so a weight tile is fetched from HBM once per XCD L2.
#include "moe_dequant.h"
#include "moe_launch.h"

namespace moe {
namespace {

constexpr int BM = 128, BN = 128, BK = 64, LDK = BK + 8;
constexpr int kXcds = 8;

struct PrefillStage {
  const void* in;  // fc1: x [T, K]; fc2: act [rows, K]
  int64_t K, nfeat;
  const uint8_t* w;  // gate / plain weights
  const void* s;
  const void* b;
  int64_t w_rows;
  const uint8_t* wl;
  const void* sl;
  const void* bl;
  int64_t wl_rows;
  int32_t gate_mode, scale_type, activation, E;
  int64_t block_size;
  float alpha, beta, limit;
  const int32_t* offsets;
  const int32_t* perm;
  const int32_t* tile_offsets;
  int64_t topk;
  int32_t mslots;  // row-tile slots per weight tile (upper bound)
  void* out;
};

template <int WF>
constexpr int64_t row_bytes(int64_t K) {
  return WF == kInt4 ? K / 2 : (WF == kInt8 ? K : 2 * K);
}
template <int WF>
constexpr int kBVecs = WF == kInt4 ? 1 : (WF == kInt8 ? 2 : 4);  // 16-B loads per thread per K step

__device__ __forceinline__ int remap_xcd(int b, int nb) {
  const int per = nb / kXcds, rem = nb % kXcds;
  const int x = b % kXcds, local = b / kXcds;
  return x < rem ? x * (per + 1) + local : rem * (per + 1) + (x - rem) * per + local;
}

// Scaled dequant of 8 weights held in `bits` (int4: 1 dword; int8: 2 dwords).
template <typename AT, int WF>
__device__ __forceinline__ u32x4_t dequant8(const u32x4_t* v, int d, float s, bool f16_scale,
                                            half2_t s2) {
  if constexpr (WF == kInt4) {
    const uint32_t x = v[0][d];
    if constexpr (sizeof(AT) > 0 && AT::kId == 10) {
      if (f16_scale) {
        u32x4_t r = dq4_f16_exact(x);
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = h2_bits(bits_h2(r[i]) * s2);
        return r;
      }
    }
    return dq4_scaled<AT>(x, s);
  } else {
    const uint32_t x0 = v[d >> 1][(d & 1) * 2], x1 = v[d >> 1][(d & 1) * 2 + 1];
    if constexpr (AT::kId == 10) {
      if (f16_scale) {
        u32x4_t r = dq8_f16_exact(x0, x1);
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = h2_bits(bits_h2(r[i]) * s2);
        return r;
      }
    }
    return dq8_scaled<AT>(x0, x1, s);
  }
}

template <typename AT, int WF, bool FC1>
__global__ void __launch_bounds__(256, 2) prefill_gemm_kernel(PrefillStage p) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2][BN * LDK];

  const int L = remap_xcd(blockIdx.x, gridDim.x);
  const int ntile = L / p.mslots, mslot = L % p.mslots;
  const int E = p.E;
  if (mslot >= p.tile_offsets[E]) return;
  int lo = 0, hi = E;  // last expert with tile_offsets[e] <= mslot
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (p.tile_offsets[mid] <= mslot) lo = mid;
    else hi = mid;
  }
  const int e = lo;
  const int row_begin = p.offsets[e] + (mslot - p.tile_offsets[e]) * BM;
  const int rows = min(BM, p.offsets[e + 1] - row_begin);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool gated = FC1 && p.gate_mode != kGateNone;
  const int64_t K = p.K;
  const int nk = static_cast<int>(K / BK);

  // ---- A loader: 4 rows x 16 B per thread per K step ----
  const uint8_t* asrc[4];
  const int acc16 = tid & 7;  // 16-byte column within the 128-byte row slice
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (tid >> 3) + 32 * i;
    asrc[i] = nullptr;
    if (r < rows) {
      const int64_t src = FC1 ? p.perm[row_begin + r] / p.topk : row_begin + r;
      asrc[i] = static_cast<const uint8_t*>(p.in) + src * K * 2 + acc16 * 16;
    }
  }

  // ---- B loader: one weight row, 32 k per thread per K step ----
  const int brow = tid >> 1, bhalf = tid & 1;
  int64_t feat, wrow;
  const uint8_t* wbase;
  const void* sbase;
  int64_t srows;
  if (gated) {
    feat = static_cast<int64_t>(ntile) * (BN / 2) + (brow & 63);
    const bool lin = brow >= 64;
    if (p.gate_mode == kGateFc3) {
      wrow = feat;
      wbase = lin ? p.wl : p.w;
      sbase = lin ? p.sl : p.s;
      srows = lin ? p.wl_rows : p.w_rows;
    } else {
      wrow = p.gate_mode == kGateInterleaved ? 2 * feat + (lin ? 1 : 0) : feat + (lin ? p.nfeat : 0);
      wbase = p.w;
      sbase = p.s;
      srows = p.w_rows;
    }
  } else {
    feat = static_cast<int64_t>(ntile) * BN + brow;
    wrow = feat;
    wbase = p.w;
    sbase = p.s;
    srows = p.w_rows;
  }
  const bool bok = feat < p.nfeat;
  const int64_t rb = row_bytes<WF>(K);
  const uint8_t* bsrc = wbase + (static_cast<int64_t>(e) * srows + (bok ? wrow : 0)) * rb;
  const bool quant = WF != kDense;
  const int64_t bs = p.block_size;
  const int64_t nblk = quant ? (bs > 0 ? K / bs : 1) : 1;
  const int64_t sidx = (static_cast<int64_t>(e) * srows + (bok ? wrow : 0)) * nblk;
  const bool f16_scale = p.scale_type == MOE_ELEM_FLOAT16;
  float chan_s = 1.0f;
  if (quant && bs == 0 && bok) chan_s = load_any(sbase, p.scale_type, sidx);

  constexpr int BV = kBVecs<WF>;
  const u32x4_t z = {0u, 0u, 0u, 0u};
  u32x4_t ra[4], rbv[BV];

  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ra[i] = asrc[i] ? *reinterpret_cast<const u32x4_t*>(asrc[i] + static_cast<int64_t>(kt) * BK * 2) : z;
    const int64_t boff = (static_cast<int64_t>(kt) * BK + 32 * bhalf) * rb / K;
#pragma unroll
    for (int v = 0; v < BV; ++v)
      rbv[v] = bok ? *reinterpret_cast<const u32x4_t*>(bsrc + boff + 16 * v) : z;
  };
  auto sstore = [&](int kt, int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (tid >> 3) + 32 * i;
      *reinterpret_cast<u32x4_t*>(&sA[buf][r * LDK + acc16 * 8]) = ra[i];
    }
    uint16_t* dst = &sB[buf][brow * LDK + 32 * bhalf];
    if constexpr (WF == kDense) {
#pragma unroll
      for (int v = 0; v < 4; ++v) *reinterpret_cast<u32x4_t*>(dst + 8 * v) = rbv[v];
    } else {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        float s = chan_s;
        if (bs > 0 && bok) s = load_any(sbase, p.scale_type, sidx + (static_cast<int64_t>(kt) * BK + 32 * bhalf + 8 * d) / bs);
        const _Float16 sh = static_cast<_Float16>(s);
        const half2_t s2 = {sh, sh};
        *reinterpret_cast<u32x4_t*>(dst + 8 * d) = dequant8<AT, WF>(rbv, d, s, f16_scale, s2);
      }
    }
  };

  // ---- MFMA tiles ----
  const int wm = wave >> 1, wn = wave & 1;
  // B-tile row bases of this wave's two 32-wide column blocks
  int bcol[2];
  if (gated) { bcol[0] = 32 * wn; bcol[1] = 64 + 32 * wn; }
  else { bcol[0] = 64 * wn; bcol[1] = 64 * wn + 32; }
  floatx16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int lr = lane & 31, lk = (lane >> 5) * 8;
  gload(0);
  sstore(0, 0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      u32x4_t af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const u32x4_t*>(&sA[buf][(64 * wm + 32 * i + lr) * LDK + ks * 16 + lk]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *reinterpret_cast<const u32x4_t*>(&sB[buf][(bcol[j] + lr) * LDK + ks * 16 + lk]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32x32x16<AT>(af[i], bf[j], acc[i][j]);
    }
    if (kt + 1 < nk) sstore(kt + 1, buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----
  // lane holds D[8*(r/4) + 4*(lane/32) + r%4][lane%32] of each 32x32 tile
  const int act_t = AT::kId;
  if (gated) {
    const int64_t f = static_cast<int64_t>(ntile) * (BN / 2) + 32 * wn + lr;
    if (f >= p.nfeat) return;
    int64_t ng = f, nl = f;
    if (p.gate_mode == kGateInterleaved) { ng = 2 * f; nl = 2 * f + 1; }
    else if (p.gate_mode == kGateChunked) { nl = p.nfeat + f; }
    float bg = 0.f, bl = 0.f;
    if (p.b) bg = load_any(p.b, act_t, static_cast<int64_t>(e) * p.w_rows + ng);
    if (p.bl) bl = load_any(p.bl, act_t, static_cast<int64_t>(e) * p.wl_rows + nl);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= rows) continue;
        const float a = apply_act(acc[i][0][r] + bg, acc[i][1][r] + bl, true, p.activation,
                                  p.alpha, p.beta, p.limit);
        static_cast<typename AT::storage*>(p.out)[static_cast<int64_t>(row_begin + m) * p.nfeat + f] =
            from_f32<AT>(a);
      }
  } else {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t f = static_cast<int64_t>(ntile) * BN + bcol[j] + lr;
      if (f >= p.nfeat) continue;
      float bias = 0.f;
      if (p.b) bias = load_any(p.b, act_t, static_cast<int64_t>(e) * p.w_rows + f);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = 64 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (m >= rows) continue;
          const float v = acc[i][j][r] + bias;
          const int64_t o = static_cast<int64_t>(row_begin + m) * p.nfeat + f;
          if constexpr (FC1) {
            static_cast<typename AT::storage*>(p.out)[o] = from_f32<AT>(act_single(v, p.activation));
          } else {
            static_cast<float*>(p.out)[o] = v;
          }
        }
    }
  }
}

template <typename AT, int WF, bool FC1>
hipError_t launch_typed(const PrefillStage& st, int64_t ntiles, hipStream_t stream) {
  const int64_t nb = ntiles * st.mslots;
  hipLaunchKernelGGL((prefill_gemm_kernel<AT, WF, FC1>), dim3(static_cast<unsigned>(nb)), dim3(256), 0,
                     stream, st);
  return hipGetLastError();
}

template <bool FC1>
hipError_t launch_stage(const PrefillStage& st, const ExpertArgs& a, int64_t ntiles, hipStream_t stream) {
  const bool bf = a.act_type == MOE_ELEM_BFLOAT16;
  switch (a.wfmt) {
    case kInt4: return bf ? launch_typed<BF16, kInt4, FC1>(st, ntiles, stream)
                          : launch_typed<F16, kInt4, FC1>(st, ntiles, stream);
    case kInt8: return bf ? launch_typed<BF16, kInt8, FC1>(st, ntiles, stream)
                          : launch_typed<F16, kInt8, FC1>(st, ntiles, stream);
    default: return bf ? launch_typed<BF16, kDense, FC1>(st, ntiles, stream)
                       : launch_typed<F16, kDense, FC1>(st, ntiles, stream);
  }
}

int32_t mslots_for(const ExpertArgs& a) {
  return static_cast<int32_t>((a.T * a.k + BM - 1) / BM + a.E);
}

}  // namespace

bool prefill_supported(const ExpertArgs& a) {
  if (a.act_type != MOE_ELEM_FLOAT16 && a.act_type != MOE_ELEM_BFLOAT16) return false;
  if (a.H % BK || a.I % BK) return false;
  if (a.wfmt != kDense && a.block_size > 0 && a.block_size < 8) return false;
  return true;
}

hipError_t launch_fc1_prefill(const ExpertArgs& a, hipStream_t stream) {
  PrefillStage st{};
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
  st.E = static_cast<int32_t>(a.E);
  st.block_size = a.wfmt == kDense ? 0 : a.block_size;
  st.alpha = a.alpha;
  st.beta = a.beta;
  st.limit = a.limit;
  st.offsets = a.offsets;
  st.perm = a.perm;
  st.tile_offsets = a.tile_offsets;
  st.topk = a.k;
  st.mslots = mslots_for(a);
  st.out = a.act;
  const int64_t per_tile = a.gate_mode != kGateNone ? BN / 2 : BN;
  return launch_stage<true>(st, a, (a.I + per_tile - 1) / per_tile, stream);
}

hipError_t launch_fc2_prefill(const ExpertArgs& a, hipStream_t stream) {
  PrefillStage st{};
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
  st.E = static_cast<int32_t>(a.E);
  st.block_size = a.wfmt == kDense ? 0 : a.block_size;
  st.offsets = a.offsets;
  st.perm = a.perm;
  st.tile_offsets = a.tile_offsets;
  st.topk = a.k;
  st.mslots = mslots_for(a);
  st.out = a.y2;
  return launch_stage<false>(st, a, (a.H + BN - 1) / BN, stream);
}

}  // namespace moe
