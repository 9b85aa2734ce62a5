// moe_expert_decode_lds.h -- decode expert GEMV with the activation operand
// staged in LDS (token counts up to 16 rows per expert).
//
// Why: in the v_mfma_f32_16x16x32 layout every lane needs 16 bytes of
// activations per MFMA step, which as global loads touches ~4x more L1 lines
// than the int4 weights it multiplies, and the vector-memory path, not HBM,
// becomes the limit.  Here the 4 waves of a workgroup share one K range and
// the workgroup copies the routed token rows (< 16) piece by piece into a
// double-buffered LDS slice with coalesced loads: while the waves multiply
// piece p (PC chunks of 128 k) out of one buffer, the loads of piece p+1 are
// in flight into registers and land in the other buffer before the barrier
// that closes the piece.  The vector-memory path carries weights only.
//
// Work split: grid (feature groups, experts, K groups); each wave owns FT
// features (gate + linear tiles when gated).  fc1 never splits K across
// workgroups (its activation needs the whole sum); fc2 may, writing one fp32
// plane of y2 per K group, which the finalize pass sums in order -- no
// cross-workgroup synchronisation, and results do not depend on timing.
//
// Weights: raw buffer loads through a register ring of PD chunks (see
// moe_expert_decode.h); features past the end read nothing (out-of-range
// offset).  Block scales are staged once into LDS per wave.
#pragma once

#include "moe_expert_decode.h"

namespace moe {
namespace decode {

constexpr int kLdsRows = 16;  // token rows staged (the MFMA M dimension)

struct LdsStage {
  Stage s;       // shared description (in, K, weights, scales, biases, ...)
  int32_t kr;    // K elements per K group (multiple of PC * 128)
};

template <int WF, bool GATED>
struct LGeo {
  static constexpr int kVecs = WF == kInt4 ? 1 : (WF == kInt8 ? 2 : 4);
  static constexpr int kLaneBytes = 16 * kVecs;
  static constexpr int FT = GATED ? 1 : 2;  // feature tiles per wave
  static constexpr int WT = 2;              // weight tiles per wave
  static constexpr int PC = WF == kDense ? 3 : 4;      // chunks per staged piece
  static constexpr int RD = 1;                         // pieces of weights in flight (2 measured slower:
                                                       // the deeper ring costs a wave per SIMD)
  static constexpr int PD = RD * PC;                   // register ring depth (chunks)
  static constexpr int kPitch = PC * kChunk * 2 + 16;  // LDS row pitch, bytes (16-byte skew)
  static constexpr int kBuf = kLdsRows * kPitch;       // one staged piece
};

template <int WF, bool GATED>
struct LChunk {
  u32x4_t w[LGeo<WF, GATED>::WT][LGeo<WF, GATED>::kVecs];
};

template <typename AT, int WF, int SM, typename ST, bool FC1, bool GATED>
__global__ void __launch_bounds__(256) gemv_lds_kernel(LdsStage ls) {
  using G = LGeo<WF, GATED>;
  constexpr int WT = G::WT, FT = G::FT, PD = G::PD, PC = G::PC, RD = G::RD, LB = G::kLaneBytes;
  constexpr bool kPerBlock = SM == kScaleBlock || SM == kScaleFold;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const Stage& p = ls.s;

  const int e = blockIdx.y;
  const int row0 = p.offsets[e];
  const int cnt = p.offsets[e + 1] - row0;
  if (cnt == 0) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, g = lane >> 4;
  const int64_t fbase = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * (16 * FT);
  const int64_t K = p.K;
  const int64_t rb = (K / 32) * LB;
  const int nchunks = static_cast<int>((K + kChunk - 1) / kChunk);
  const int cper = ls.kr / kChunk;
  const int c0 = static_cast<int>(blockIdx.z) * cper;
  const int c1 = c0 + cper < nchunks ? c0 + cper : nchunks;  // real chunks [c0, c1)
  const int64_t ktail = K - static_cast<int64_t>(nchunks - 1) * kChunk;

  // ---- weights: tile rows and buffer offsets ----
  const uint8_t* wbase_g = p.w + static_cast<int64_t>(e) * p.w_rows * rb;
  const uint8_t* wbase_l = p.wl + static_cast<int64_t>(e) * p.wl_rows * rb;
  const __amdgpu_buffer_rsrc_t rs_g = make_rsrc(wbase_g, static_cast<uint32_t>(p.w_rows * rb));
  const __amdgpu_buffer_rsrc_t rs_l = make_rsrc(wbase_l, static_cast<uint32_t>(p.wl_rows * rb));
  int64_t trow[WT];
  bool tok[WT];
  uint32_t woff[WT];
#pragma unroll
  for (int t = 0; t < WT; ++t) {
    const int64_t f = fbase + (t % FT) * 16 + col;
    tok[t] = f < p.nfeat;
    trow[t] = tile_row(tok[t] ? f : 0, GATED && t >= FT, FC1 && GATED, p.gate_mode, p.nfeat);
    woff[t] = tok[t] ? static_cast<uint32_t>(trow[t] * rb + g * LB) : kOob;
  }

  using CK = LChunk<WF, GATED>;
  auto fetch = [&](int c, CK& d) {
    // padding chunks past K and the missing lanes of a partial last chunk read nothing
    const bool kin = c < nchunks - 1 || (c == nchunks - 1 && 32 * g + 32 <= ktail);
    const uint32_t wc = static_cast<uint32_t>(c) * (4 * LB);
#pragma unroll
    for (int t = 0; t < WT; ++t) {
      const uint32_t o = kin ? woff[t] + wc : kOob;
#pragma unroll
      for (int v = 0; v < G::kVecs; ++v) d.w[t][v] = bload16(GATED && t >= FT ? rs_l : rs_g, o + 16 * v);
    }
  };

  // ---- activation pieces: thread slot i = tid + 256 j covers row i / 64 and
  // 16-byte piece i % 64 of the row's PC chunks; absent rows / past K read 0 ----
  constexpr int kSlots = kLdsRows * PC * kChunk * 2 / 16 / 256;  // 16-byte slots per thread
  const int nrows = cnt < kLdsRows ? cnt : kLdsRows;
  const __amdgpu_buffer_rsrc_t rs_x = make_rsrc(p.in, static_cast<uint32_t>(p.in_rows * K * 2));
  constexpr int kRowPieces = PC * kChunk * 2 / 16;
  uint32_t xsrc[kSlots];
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    const int i = tid + 256 * j;
    const int m = i / kRowPieces, pc = i % kRowPieces;
    if (m < nrows) {
      const int64_t src = FC1 ? p.perm[row0 + m] / p.topk : row0 + m;
      xsrc[j] = static_cast<uint32_t>(src * K * 2 + pc * 16);
    } else {
      xsrc[j] = kOob;
    }
  }
  u32x4_t xreg[kSlots];
  auto xload = [&](int piece) {
    const int64_t kpc = static_cast<int64_t>(c0 + piece * PC) * kChunk;  // first k of the piece
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      const int i = tid + 256 * j;
      const int64_t k = kpc + (i % kRowPieces) * 8;
      const uint32_t o = (xsrc[j] != kOob && k < K) ? xsrc[j] + static_cast<uint32_t>(kpc * 2) : kOob;
      xreg[j] = bload16(rs_x, o);
    }
  };
  auto xstore = [&](int buf) {
    uint8_t* xs = smem + buf * G::kBuf;
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
      const int i = tid + 256 * j;
      *reinterpret_cast<u32x4_t*>(xs + (i / kRowPieces) * G::kPitch + (i % kRowPieces) * 16) = xreg[j];
    }
  };

  // Start the weight stream before staging, so the first chunks are in flight
  // while the first activation piece is copied.
  // The K range is walked in whole groups of RD pieces of PC chunks; chunks
  // past c1 are padding that reads nothing and multiplies zeros (a K group
  // other than the last is a whole number of such groups).
  const int npieces = (c1 - c0 + RD * PC - 1) / (RD * PC) * RD;
  const int cend = c0 + npieces * PC;
  CK ring[PD];
#pragma unroll
  for (int d = 0; d < PD; ++d) fetch(c0 + d, ring[d]);
  xload(0);

  // ---- stage this wave's block scales: sc[(t * nb + b) * 16 + col] ----
  float* sc = reinterpret_cast<float*>(smem + 2 * G::kBuf + static_cast<size_t>(wave) * p.lds_scale);
  int64_t b0 = 0;
  int bshift = 0, nb = 0;
  if constexpr (kPerBlock) {
    bshift = __builtin_ctzll(static_cast<uint64_t>(p.block_size));
    const int64_t nblk = K / p.block_size;
    b0 = (static_cast<int64_t>(c0) * kChunk) >> bshift;
    nb = static_cast<int>(((static_cast<int64_t>(cend) * kChunk - 1) >> bshift) + 1 - b0);
    const typename ST::storage* sgp = static_cast<const typename ST::storage*>(p.s);
    const typename ST::storage* slp = static_cast<const typename ST::storage*>(p.sl);
    // lane -> (tile, row) pair; the two lane halves take alternate blocks
    const int pair = lane & 31, t = pair >> 4, cc = pair & 15;
    const bool lin = GATED && t >= FT;
    const int64_t f = fbase + (t % FT) * 16 + cc;
    const int64_t r = tile_row(f < p.nfeat ? f : 0, lin, FC1 && GATED, p.gate_mode, p.nfeat);
    const typename ST::storage* srow =
        (lin ? slp : sgp) + (static_cast<int64_t>(e) * (lin ? p.wl_rows : p.w_rows) + r) * nblk;
    for (int b = lane >> 5; b < nb; b += 2) {
      const bool ok = f < p.nfeat && b0 + b < nblk;
      sc[(t * nb + b) * 16 + cc] = ok ? to_f32<ST>(srow[b0 + b]) : 0.0f;
    }
  }
  xstore(0);
  __syncthreads();

  floatx4_t acc[WT];
#pragma unroll
  for (int t = 0; t < WT; ++t) acc[t] = floatx4_t{0.f, 0.f, 0.f, 0.f};
  // biased weights (block scales of whole chunks, or per-channel scales):
  // sx collects the activation sums that remove the bias
  constexpr bool kBiased = Biased<AT, WF>::kOk && (SM == kScaleBlock || SM == kScaleChan);
  constexpr float kOff = Biased<AT, WF>::kOffset;
  const u32x4_t ones = {Biased<AT, WF>::kOnes, Biased<AT, WF>::kOnes, Biased<AT, WF>::kOnes, Biased<AT, WF>::kOnes};
  floatx4_t sx = {0.f, 0.f, 0.f, 0.f};
  const int b0i = static_cast<int>(b0);  // K < 2^31: block indices fit 32 bits

  auto compute = [&](int c, int buf, int cin, const CK& d) {
    floatx4_t tmp[WT];
#pragma unroll
    for (int t = 0; t < WT; ++t) tmp[t] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    floatx4_t sxc = {0.f, 0.f, 0.f, 0.f};
    const uint8_t* xc = smem + buf * G::kBuf + col * G::kPitch + g * 64 + cin * (kChunk * 2);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // rows past the expert's token count were staged as zeros
      const u32x4_t a = *reinterpret_cast<const u32x4_t*>(xc + 16 * s);
      if constexpr (kBiased) {
        if constexpr (SM == kScaleBlock) sxc = mfma16x16x32<AT>(a, ones, sxc);
        else sx = mfma16x16x32<AT>(a, ones, sx);
      }
#pragma unroll
      for (int t = 0; t < WT; ++t) {
        float fs = 0.0f;
        if constexpr (SM == kScaleFold) {
          const int blk = ((c * kChunk + 32 * g + 8 * s) >> bshift) - b0i;
          fs = sc[(t * nb + blk) * 16 + col];
        }
        u32x4_t bw;
        if constexpr (kBiased) bw = weight_biased<AT, WF>(d.w[t], s);
        else bw = weight_operand<AT, WF, SM == kScaleFold>(d.w[t], s, fs);
        if constexpr (SM == kScaleBlock) tmp[t] = mfma16x16x32<AT>(a, bw, tmp[t]);
        else acc[t] = mfma16x16x32<AT>(a, bw, acc[t]);
      }
    }
    if constexpr (SM == kScaleBlock) {
      const int blk = ((c * kChunk) >> bshift) - b0i;
#pragma unroll
      for (int t = 0; t < WT; ++t) {
        floatx4_t v = tmp[t];
        if constexpr (kBiased) v -= kOff * sxc;
        acc[t] += v * sc[(t * nb + blk) * 16 + col];
      }
    }
  };

  // Pieces of PC = PD chunks: piece q uses LDS buffer q % 2 and ring slots
  // 0..PC-1; the next piece's activations are loaded during the piece and
  // stored behind it, then one barrier closes the piece.
  // With RD > 1 the ring spans RD pieces: piece q uses slots (q % RD) * PC
  // onward, so pieces are walked RD at a time to keep slot indices static.
  for (int q0 = 0; q0 < npieces; q0 += RD) {
#pragma unroll
    for (int r = 0; r < RD; ++r) {
      const int q = q0 + r;
      const int cq = c0 + q * PC;
      const bool more = q + 1 < npieces;
      if (more) xload(q + 1);
#pragma unroll
      for (int d = 0; d < PC; ++d) {
        compute(cq + d, q & 1, d, ring[r * PC + d]);
        fetch(min(cq + d + PD, cend - 1), ring[r * PC + d]);
        // keep each chunk's LDS reads and dequantisation next to its MFMAs
        __builtin_amdgcn_sched_barrier(0);
      }
      if (more) xstore((q + 1) & 1);
      __syncthreads();
    }
  }

  // ---- epilogue ----
  if constexpr (kBiased && SM == kScaleChan) {
#pragma unroll
    for (int t = 0; t < WT; ++t) acc[t] -= kOff * sx;
  }
  const int act_t = AT::kId;
  if constexpr (!FC1) {
    // fc2: this K group's plane of y2 (bias in plane 0)
#pragma unroll
    for (int t = 0; t < WT; ++t) {
      if (!tok[t]) continue;
      const int64_t f = fbase + t * 16 + col;
      float ch = 1.0f;
      if constexpr (SM == kScaleChan) ch = load_any(p.s, p.scale_type, static_cast<int64_t>(e) * p.w_rows + trow[t]);
      const float bias = (p.b && blockIdx.z == 0) ? load_any(p.b, act_t, static_cast<int64_t>(e) * p.w_rows + trow[t]) : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * g + r;
        if (m >= nrows) continue;
        static_cast<float*>(p.out)[static_cast<int64_t>(blockIdx.z) * p.out_rows * p.nfeat +
                                   static_cast<int64_t>(row0 + m) * p.nfeat + f] = acc[t][r] * ch + bias;
      }
    }
    return;
  } else {
    auto finish = [&](int ft, int m, float vg, float vl) {
      const int tg = ft, tl = GATED ? ft + FT : ft;
      float chg = 1.0f, chl = 1.0f;
      if constexpr (SM == kScaleChan) {
        chg = load_any(p.s, p.scale_type, static_cast<int64_t>(e) * p.w_rows + trow[tg]);
        if constexpr (GATED) chl = load_any(p.sl, p.scale_type, static_cast<int64_t>(e) * p.wl_rows + trow[tl]);
      }
      const float bg = p.b ? load_any(p.b, act_t, static_cast<int64_t>(e) * p.w_rows + trow[tg]) : 0.0f;
      const float bl = (GATED && p.bl) ? load_any(p.bl, act_t, static_cast<int64_t>(e) * p.wl_rows + trow[tl]) : 0.0f;
      const float a = apply_act<true>(vg * chg + bg, vl * chl + bl, GATED, p.activation, p.alpha, p.beta, p.limit);
      const int64_t f = fbase + ft * 16 + col;
      static_cast<typename AT::storage*>(p.out)[static_cast<int64_t>(row0 + m) * p.nfeat + f] = from_f32<AT>(a);
    };
#pragma unroll
    for (int ft = 0; ft < FT; ++ft) {
      if (!tok[ft]) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * g + r;
        if (m >= nrows) continue;
        finish(ft, m, acc[ft][r], GATED ? acc[GATED ? ft + FT : ft][r] : 0.0f);
      }
    }
  }
}

template <typename AT, int WF, int SM, typename ST, bool FC1, bool GATED>
hipError_t launch_lds(const LdsStage& ls, int64_t E, hipStream_t stream) {
  using G = LGeo<WF, GATED>;
  const int64_t fpw = 16 * G::FT;
  const int64_t waves_f = (ls.s.nfeat + fpw - 1) / fpw;
  dim3 grid(static_cast<unsigned>((waves_f + 3) / 4), static_cast<unsigned>(E), static_cast<unsigned>(ls.s.ksg));
  const size_t lds = static_cast<size_t>(2) * G::kBuf + static_cast<size_t>(4) * ls.s.lds_scale;
  hipLaunchKernelGGL((gemv_lds_kernel<AT, WF, SM, ST, FC1, GATED>), grid, dim3(256), lds, stream, ls);
  return hipGetLastError();
}

template <typename AT, int WF, int SM, typename ST>
hipError_t launch_lds_kinds(const LdsStage& ls, int64_t E, bool fc1, bool gated, hipStream_t stream) {
  if (!fc1) return launch_lds<AT, WF, SM, ST, false, false>(ls, E, stream);
  if (gated) return launch_lds<AT, WF, SM, ST, true, true>(ls, E, stream);
  return launch_lds<AT, WF, SM, ST, true, false>(ls, E, stream);
}

// Dispatch over activation type, scale mode and scale type for one format.
template <int WF>
hipError_t launch_lds_fmt(const LdsStage& ls, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream) {
  const bool bf = a.act_type == MOE_ELEM_BFLOAT16;
  const int sm = scale_mode(a);
  auto by_st = [&](auto at_tag, auto sm_tag) -> hipError_t {
    using AT = decltype(at_tag);
    constexpr int SM = decltype(sm_tag)::value;
    switch (a.scale_type) {
      case MOE_ELEM_FLOAT: return launch_lds_kinds<AT, WF, SM, F32>(ls, a.E, fc1, gated, stream);
      case MOE_ELEM_BFLOAT16: return launch_lds_kinds<AT, WF, SM, BF16>(ls, a.E, fc1, gated, stream);
      default: return launch_lds_kinds<AT, WF, SM, F16>(ls, a.E, fc1, gated, stream);
    }
  };
  if constexpr (WF == kDense) {
    return bf ? launch_lds_kinds<BF16, WF, kScaleNone, F16>(ls, a.E, fc1, gated, stream)
              : launch_lds_kinds<F16, WF, kScaleNone, F16>(ls, a.E, fc1, gated, stream);
  } else {
    if (sm == kScaleChan)
      return bf ? launch_lds_kinds<BF16, WF, kScaleChan, F16>(ls, a.E, fc1, gated, stream)
                : launch_lds_kinds<F16, WF, kScaleChan, F16>(ls, a.E, fc1, gated, stream);
    if (sm == kScaleBlock)
      return bf ? by_st(BF16{}, std::integral_constant<int, kScaleBlock>{})
                : by_st(F16{}, std::integral_constant<int, kScaleBlock>{});
    return bf ? by_st(BF16{}, std::integral_constant<int, kScaleFold>{})
              : by_st(F16{}, std::integral_constant<int, kScaleFold>{});
  }
}

hipError_t launch_lds_int4(const LdsStage& ls, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream);
hipError_t launch_lds_int8(const LdsStage& ls, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream);
hipError_t launch_lds_dense(const LdsStage& ls, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream);

}  // namespace decode
}  // namespace moe
