// moe_expert_prefill.hip -- grouped expert GEMM for large token counts
// (prefill), bound by MFMA throughput.
//
// A workgroup computes a tile of 128 rows (tokens of one expert, dispatch
// order) x 256 weight rows with 4 wavefronts; each wave owns 64 weight rows
// (4 tiles of 16) for all 128 rows: 8 x 4 v_mfma_f32_16x16x32 tiles, fp32
// accumulation in 128 registers.
//
//  * Weights never touch LDS.  Each lane streams 16-byte pieces of its weight
//    row straight from HBM/L2 into registers with raw buffer loads, in the
//    MFMA operand layout of the decode kernels: lane (col = lane%16,
//    g = lane/16) covers k in [KG*g, KG*g + KG) of each stage and feeds 8 of
//    them to each MFMA step.  Dequantisation (and a per-block scale) happens
//    in registers right before the MFMA.  A register ring keeps the next
//    stage's weights in flight.
//  * Activations are the shared operand: one stage (128 rows x BK) is copied
//    to LDS per workgroup (fc1 gathers token rows through the dispatch
//    permutation, so the permuted input is never materialised), double
//    buffered, one barrier per stage.  LDS traffic per MFMA is a quarter of a
//    both-operands-in-LDS tile of the same size.
//  * Gated activations: a wave's tiles 0,1 are the gate rows and tiles 2,3
//    the linear rows of the same 32 features, so each lane holds both halves
//    of its outputs and applies bias + activation in the epilogue.
//  * Scales: per output channel -> epilogue (weights enter the MFMA as exact
//    integers); per block -> folded into the 16-bit weights of each stage.
//  * Tile order: groups of 8 weight tiles are swept across all row tiles of
//    all experts, and each XCD (hardware workgroup ids are dealt to the 8
//    XCDs round-robin) receives a contiguous range of that order, so the
//    workgroups resident on one XCD share ~8 activation tiles and ~8 weight
//    tiles in its L2.
//  * fc2 may split K across workgroups; the partial sums land in separate
//    fp32 planes of y2 that finalize adds in a fixed order.
#include "moe_dequant.h"
#include "moe_launch.h"

namespace moe {
namespace {

constexpr int BM = 128;           // rows per workgroup tile
constexpr int kMT = BM / 16;      // 16-row tiles per wave (every wave covers all rows)
constexpr int kNT = 4;            // 16-wide weight tiles per wave
constexpr int BN = 4 * kNT * 16;  // weight rows per workgroup tile
constexpr int kGroupN = 8;        // weight tiles swept together over the row tiles
constexpr int kXcds = 8;

enum PScale : int { kPsNone = 0, kPsChan = 1, kPsBlock = 2, kPsHalfBlock = 3 };

template <int WF>
struct PG {
  static constexpr int BK = WF == kDense ? 64 : 128;  // k per stage
  static constexpr int KG = BK / 4;                    // k per lane group per stage
  static constexpr int NSTEP = KG / 8;                 // MFMA steps per stage
  static constexpr int BVEC = WF == kInt4 ? 1 : 2;     // 16-byte weight loads per tile per stage
  static constexpr int ROWB = BK * 2;                  // LDS bytes of one activation row per stage
  static constexpr int ABUF = BM * ROWB;               // one staged activation stage
  static constexpr int PIECES = ROWB / 16;             // 16-byte pieces per row per stage
  static constexpr int RPI = 1024 / ROWB;              // rows per 1 KB LDS-load instruction
  static constexpr int APW = BM / RPI / 4;             // LDS-load instructions per wave per stage
  static constexpr int EBITS = WF == kInt4 ? 4 : (WF == kInt8 ? 8 : 16);
  // XOR swizzle of a row's 16-byte pieces, so that the 16 rows one MFMA
  // operand read touches fall into 16 different bank groups
  static __device__ __forceinline__ int swz(int m) { return (m / (16 / PIECES)) % PIECES; }
};

struct PStage {
  const void* in;  // fc1: x [T, K]; fc2: act [rows, K]
  int64_t in_rows;
  int64_t K, nfeat;
  const uint8_t* w;  // gate / plain weights [E, w_rows, K(/pack)]
  const void* s;
  const void* b;
  int64_t w_rows;
  const uint8_t* wl;  // linear weights (fc3 or the fused fc1)
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
  int32_t mslots;   // row-tile slots (upper bound over all experts)
  int32_t ntiles;   // weight tiles of BN rows (gated: BN/2 features)
  int32_t ngroups;  // ceil(ntiles / kGroupN)
  int32_t ksplit;   // K splits (partial planes of the output)
  int32_t kstages;  // stages per K split
  int64_t out_rows;
  void* out;  // fc1: act [rows, nfeat] (AT); fc2: y2 [ksplit][rows, nfeat] fp32
};

__device__ __forceinline__ int remap_xcd(int b, int nb) {
  const int per = nb / kXcds, rem = nb % kXcds;
  const int x = b % kXcds, local = b / kXcds;
  return x < rem ? x * (per + 1) + local : rem * (per + 1) + (x - rem) * per + local;
}

template <typename AT, int WF, int SM, typename ST, bool FC1, bool GATED>
__global__ void __launch_bounds__(256, 2) prefill_kernel(PStage p) {
  using G = PG<WF>;
  constexpr int BK = G::BK, KG = G::KG, NSTEP = G::NSTEP, BVEC = G::BVEC;
  // two stage buffers as separate objects, so the compiler can tell that the
  // LDS loads filling one never alias the reads of the other
  __shared__ __attribute__((aligned(1024))) uint8_t sA0[G::ABUF];
  __shared__ __attribute__((aligned(1024))) uint8_t sA1[G::ABUF];

  // ---- tile of this workgroup ----
  const int L = remap_xcd(blockIdx.x, gridDim.x);
  const int per_split = p.ngroups * p.mslots * kGroupN;
  const int ks = L / per_split;
  const int r0 = L % per_split;
  const int nin = r0 % kGroupN;
  const int mslot = (r0 / kGroupN) % p.mslots;
  const int ntile = (r0 / kGroupN / p.mslots) * kGroupN + nin;
  if (ntile >= p.ntiles || mslot >= p.tile_offsets[p.E]) return;
  int lo = 0, hi = p.E;  // last expert with tile_offsets[e] <= mslot
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (p.tile_offsets[mid] <= mslot) lo = mid;
    else hi = mid;
  }
  const int e = lo;
  const int row_begin = p.offsets[e] + (mslot - p.tile_offsets[e]) * BM;
  const int rows = min(BM, p.offsets[e + 1] - row_begin);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS-load bases are scalar
  const int col = lane & 15, g = lane >> 4;
  const int K = static_cast<int>(p.K);  // K < 2^31 (buffer offsets are 32-bit)
  const int kbeg = ks * p.kstages * BK;
  const int nst = min(p.kstages, (K - kbeg + BK - 1) / BK);

  // ---- weight rows of this wave's tiles: tile t of lane feature fl reads
  // row row0 + drow[t] (gated: t < 2 gate, t >= 2 linear rows of the same
  // features).  drow is uniform, so one VGPR offset per lane serves all tiles
  // (the rest rides in the scalar offset).  Rows of features past nfeat are
  // read (past the buffer: zeros) but their outputs are never stored. ----
  const int64_t rb = static_cast<int64_t>(K) * G::EBITS / 8;  // bytes of one weight row
  const uint8_t* wbase_g = p.w + static_cast<int64_t>(e) * p.w_rows * rb;
  const uint8_t* wbase_l = p.wl + static_cast<int64_t>(e) * p.wl_rows * rb;
  const __amdgpu_buffer_rsrc_t rs_g = make_rsrc(wbase_g, static_cast<uint32_t>(p.w_rows * rb));
  const __amdgpu_buffer_rsrc_t rs_l = make_rsrc(wbase_l, static_cast<uint32_t>(p.wl_rows * rb));
  const int64_t fbase = GATED ? static_cast<int64_t>(ntile) * (BN / 2) + wave * 32
                              : static_cast<int64_t>(ntile) * BN + wave * 64;
  const int64_t fl = fbase + col;
  const bool interleaved = GATED && p.gate_mode == kGateInterleaved;
  const int64_t row0 = interleaved ? 2 * fl : fl;
  int64_t drow[kNT];
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    if constexpr (GATED) {
      const bool lin = t >= 2;
      if (interleaved) drow[t] = 32 * (t & 1) + (lin ? 1 : 0);
      else drow[t] = 16 * (t & 1) + ((lin && p.gate_mode == kGateChunked) ? p.nfeat : 0);
    } else {
      drow[t] = 16 * t;
    }
  }
  const uint32_t woff = static_cast<uint32_t>(row0 * rb + static_cast<int64_t>(kbeg + KG * g) * G::EBITS / 8);

  // ---- per-block scales (folded): buffer loads of each tile row's scale of
  // the lane's piece; pieces past K or of a padding stage read 0 ----
  constexpr bool kFold = SM == kPsBlock || SM == kPsHalfBlock;
  constexpr int SB = sizeof(typename ST::storage);
  const int bshift = kFold ? __builtin_ctzll(static_cast<uint64_t>(p.block_size)) : 0;
  const int64_t nblk = kFold ? (K >> bshift) : 0;
  const __amdgpu_buffer_rsrc_t rs_sg =
      make_rsrc(kFold ? static_cast<const uint8_t*>(p.s) + static_cast<int64_t>(e) * p.w_rows * nblk * SB : nullptr,
                static_cast<uint32_t>(p.w_rows * nblk * SB));
  const __amdgpu_buffer_rsrc_t rs_sl =
      make_rsrc(kFold ? static_cast<const uint8_t*>(p.sl) + static_cast<int64_t>(e) * p.wl_rows * nblk * SB : nullptr,
                static_cast<uint32_t>(p.wl_rows * nblk * SB));
  const uint32_t soff = static_cast<uint32_t>(row0 * nblk * SB);
  auto sload = [&](__amdgpu_buffer_rsrc_t r, uint32_t off, int64_t soffset) -> float {
    if constexpr (SB == 4) {
      return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off),
                                                                          static_cast<int>(soffset), 0));
    } else {
      const uint16_t h = __builtin_bit_cast(
          uint16_t, __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(off), static_cast<int>(soffset), 0));
      return to_f32<ST>(__builtin_bit_cast(typename ST::storage, h));
    }
  };

  struct Ring {
    u32x4_t w[kNT][BVEC];
    float sc[kNT][SM == kPsHalfBlock ? 2 : 1];
  };
  auto fetch = [&](int c, Ring& d) {
    const int k0 = kbeg + c * BK + KG * g;  // first k of the lane's piece
    const bool kin = (c < nst) & (k0 < K);
    const uint32_t o = kin ? woff + static_cast<uint32_t>(c * BK * G::EBITS / 8) : kOob;
    uint32_t so = kOob, so1 = kOob;
    if constexpr (kFold) {
      so = kin ? soff + static_cast<uint32_t>((k0 >> bshift) * SB) : kOob;
      if constexpr (SM == kPsHalfBlock) so1 = kin ? soff + static_cast<uint32_t>(((k0 + 16) >> bshift) * SB) : kOob;
    }
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      const __amdgpu_buffer_rsrc_t rw = GATED && t >= 2 ? rs_l : rs_g;
      const int sw = static_cast<int>(drow[t] * rb);
#pragma unroll
      for (int v = 0; v < BVEC; ++v)
        d.w[t][v] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, static_cast<int>(o + 16 * v), sw, 0));
      if constexpr (kFold) {
        const __amdgpu_buffer_rsrc_t rs = GATED && t >= 2 ? rs_sl : rs_sg;
        const int64_t ss = drow[t] * nblk * SB;
        d.sc[t][0] = sload(rs, so, ss);
        if constexpr (SM == kPsHalfBlock) d.sc[t][1] = sload(rs, so1, ss);
      }
    }
  };

  // ---- activation stages go global -> LDS directly (buffer loads with the
  // LDS bit, 1 KB per wave instruction: lane L writes bytes [16 L, 16 L + 16)
  // of the block).  Instruction j of wave w covers rows (w * APW + j) * RPI
  // + L / PIECES; lane L's LDS piece p = L % PIECES holds the row's global
  // piece p ^ swz(row).  Rows past the tile and k past K (or past the split)
  // read zeros. ----
  const __amdgpu_buffer_rsrc_t rs_x = make_rsrc(p.in, static_cast<uint32_t>(p.in_rows * K * 2));
  auto apiece = [&](int j) {  // global piece of the lane in instruction j
    const int r = (wave * G::APW + j) * G::RPI + lane / G::PIECES;
    return (lane % G::PIECES) ^ G::swz(r);
  };
  uint32_t asrc[G::APW];
#pragma unroll
  for (int j = 0; j < G::APW; ++j) {
    const int r = (wave * G::APW + j) * G::RPI + lane / G::PIECES;
    if (r < rows) {
      const int64_t src = FC1 ? p.perm[row_begin + r] / p.topk : row_begin + r;
      asrc[j] = static_cast<uint32_t>((src * K + kbeg) * 2 + apiece(j) * 16);
    } else {
      asrc[j] = kOob;
    }
  }
  auto aload = [&](int c, uint8_t* buf) {
    const int krem = K - kbeg - c * BK;  // k left in the row from this stage on
#pragma unroll
    for (int j = 0; j < G::APW; ++j) {
      const bool in = (c < nst) & (apiece(j) * 8 < krem);
      const uint32_t o = in ? asrc[j] + static_cast<uint32_t>(c * BK * 2) : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs_x, (__attribute__((address_space(3))) void*)(buf + (wave * G::APW + j) * 1024), 16,
          static_cast<int>(o), 0, 0, 0);
    }
  };

  floatx4_t acc[kMT][kNT];
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int t = 0; t < kNT; ++t) acc[i][t] = floatx4_t{0.f, 0.f, 0.f, 0.f};

  // A operand of row tile i, step s: row m = 16 i + col, global piece
  // gp0 + s; swz(m) does not depend on i
  const int gp0 = KG * 2 * g / 16;
  auto compute = [&](const uint8_t* buf, const Ring& d) {
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
      const uint8_t* xa = buf + col * G::ROWB + ((gp0 + s) ^ G::swz(col)) * 16;
      u32x4_t bw[kNT];
#pragma unroll
      for (int t = 0; t < kNT; ++t) {
        if constexpr (SM == kPsBlock && AT::kId == 10 && ST::kId == 10) {
          // fp16: exact integers, then one packed multiply by the block scale
          const u32x4_t q = weight_operand<AT, WF, false>(d.w[t], s, 0.0f);
          const _Float16 sh = static_cast<_Float16>(d.sc[t][0]);
          const half2_t s2 = {sh, sh};
#pragma unroll
          for (int r = 0; r < 4; ++r) bw[t][r] = h2_bits(bits_h2(q[r]) * s2);
        } else if constexpr (kFold) {
          const float sc = SM == kPsHalfBlock ? d.sc[t][s >> 1] : d.sc[t][0];
          bw[t] = weight_operand<AT, WF, true>(d.w[t], s, sc);
        } else {
          bw[t] = weight_operand<AT, WF, false>(d.w[t], s, 0.0f);
        }
      }
#pragma unroll
      for (int i = 0; i < kMT; ++i) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(xa + i * 16 * G::ROWB);
#pragma unroll
        for (int t = 0; t < kNT; ++t) acc[i][t] = mfma16x16x32<AT>(a, bw[t], acc[i][t]);
      }
      // keep each step's operands next to its MFMAs (bounds live registers)
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- main loop: stages in pairs (buffers / ring slots 0 and 1).  Stage
  // c + 1's activations and weights are requested before stage c is
  // multiplied; the barrier after stage c waits for the LDS loads only (the
  // weight loads issued after them stay in flight).  A padding stage past the
  // split's range reads zeros. ----
  Ring ring[2];
  aload(0, sA0);
  fetch(0, ring[0]);
  __syncthreads();
  const int npairs = (nst + 1) / 2;
  for (int q = 0; q < npairs; ++q) {
    const int c = 2 * q;
    aload(c + 1, sA1);
    fetch(c + 1, ring[1]);
    compute(sA0, ring[0]);
    __syncthreads();
    aload(c + 2, sA0);
    fetch(c + 2, ring[0]);
    compute(sA1, ring[1]);
    __syncthreads();
  }

  // ---- epilogue: lane holds D[16 i + 4 g + r][col] of tile (i, t) ----
  const int act_t = AT::kId;
  if constexpr (FC1 && GATED) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int64_t f = fl + t * 16;
      if (f >= p.nfeat) continue;
      const int64_t rg = row0 + drow[t], rl = row0 + drow[t + 2];
      float chg = 1.0f, chl = 1.0f;
      if constexpr (SM == kPsChan) {
        chg = load_any(p.s, p.scale_type, static_cast<int64_t>(e) * p.w_rows + rg);
        chl = load_any(p.sl, p.scale_type, static_cast<int64_t>(e) * p.wl_rows + rl);
      }
      const float bg = p.b ? load_any(p.b, act_t, static_cast<int64_t>(e) * p.w_rows + rg) : 0.0f;
      const float bl = p.bl ? load_any(p.bl, act_t, static_cast<int64_t>(e) * p.wl_rows + rl) : 0.0f;
#pragma unroll
      for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * i + 4 * g + r;
          if (m >= rows) continue;
          const float a = apply_act(acc[i][t][r] * chg + bg, acc[i][t + 2][r] * chl + bl, true, p.activation,
                                    p.alpha, p.beta, p.limit);
          static_cast<typename AT::storage*>(p.out)[static_cast<int64_t>(row_begin + m) * p.nfeat + f] =
              from_f32<AT>(a);
        }
    }
  } else {
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      const int64_t f = fl + t * 16;
      if (f >= p.nfeat) continue;
      float ch = 1.0f;
      if constexpr (SM == kPsChan) ch = load_any(p.s, p.scale_type, static_cast<int64_t>(e) * p.w_rows + f);
      const float bias = (p.b && ks == 0) ? load_any(p.b, act_t, static_cast<int64_t>(e) * p.w_rows + f) : 0.0f;
#pragma unroll
      for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = 16 * i + 4 * g + r;
          if (m >= rows) continue;
          const float v = acc[i][t][r] * ch + bias;
          const int64_t o = static_cast<int64_t>(row_begin + m) * p.nfeat + f;
          if constexpr (FC1) {
            static_cast<typename AT::storage*>(p.out)[o] = from_f32<AT>(act_single(v, p.activation));
          } else {
            static_cast<float*>(p.out)[static_cast<int64_t>(ks) * p.out_rows * p.nfeat + o] = v;
          }
        }
    }
  }
}

template <typename AT, int WF, int SM, typename ST, bool FC1>
hipError_t launch_kernel(const PStage& st, bool gated, hipStream_t stream) {
  const unsigned nb = static_cast<unsigned>(st.ksplit) * st.ngroups * st.mslots * kGroupN;
  if (FC1 && gated)
    hipLaunchKernelGGL((prefill_kernel<AT, WF, SM, ST, true, true>), dim3(nb), dim3(256), 0, stream, st);
  else
    hipLaunchKernelGGL((prefill_kernel<AT, WF, SM, ST, FC1, false>), dim3(nb), dim3(256), 0, stream, st);
  return hipGetLastError();
}

template <typename AT, int WF, bool FC1>
hipError_t launch_scaled(const PStage& st, const ExpertArgs& a, bool gated, hipStream_t stream) {
  if constexpr (WF == kDense) {
    return launch_kernel<AT, WF, kPsNone, F16, FC1>(st, gated, stream);
  } else {
    if (a.block_size == 0) return launch_kernel<AT, WF, kPsChan, F16, FC1>(st, gated, stream);
    const bool half = a.block_size < PG<WF>::KG;  // 16: two blocks per lane piece
    auto by_type = [&](auto st_tag) -> hipError_t {
      using ST = decltype(st_tag);
      return half ? launch_kernel<AT, WF, kPsHalfBlock, ST, FC1>(st, gated, stream)
                  : launch_kernel<AT, WF, kPsBlock, ST, FC1>(st, gated, stream);
    };
    if (a.scale_type == MOE_ELEM_FLOAT) return by_type(F32{});
    if (a.scale_type == MOE_ELEM_BFLOAT16) return by_type(BF16{});
    return by_type(F16{});
  }
}

template <bool FC1>
hipError_t launch_stage(const PStage& st, const ExpertArgs& a, bool gated, hipStream_t stream) {
  const bool bf = a.act_type == MOE_ELEM_BFLOAT16;
  switch (a.wfmt) {
    case kInt4: return bf ? launch_scaled<BF16, kInt4, FC1>(st, a, gated, stream)
                          : launch_scaled<F16, kInt4, FC1>(st, a, gated, stream);
    case kInt8: return bf ? launch_scaled<BF16, kInt8, FC1>(st, a, gated, stream)
                          : launch_scaled<F16, kInt8, FC1>(st, a, gated, stream);
    default: return bf ? launch_scaled<BF16, kDense, FC1>(st, a, gated, stream)
                       : launch_scaled<F16, kDense, FC1>(st, a, gated, stream);
  }
}

int32_t mslots_for(int64_t T, int64_t k, int64_t E) {
  return static_cast<int32_t>((T * k + BM - 1) / BM + E);
}

int bk_for(int wfmt) { return wfmt == kDense ? PG<kDense>::BK : PG<kInt4>::BK; }

void plan_grid(PStage& st, int64_t T, int64_t k, int64_t E, int wfmt, int64_t nrows_w, int32_t ksplit) {
  st.mslots = mslots_for(T, k, E);
  st.ntiles = static_cast<int32_t>((nrows_w + BN - 1) / BN);
  st.ngroups = (st.ntiles + kGroupN - 1) / kGroupN;
  const int64_t bk = bk_for(wfmt);
  const int64_t stages = (st.K + bk - 1) / bk;
  st.ksplit = ksplit;
  st.kstages = static_cast<int32_t>((stages + ksplit - 1) / ksplit);
}

}  // namespace

int32_t prefill_fc2_splits(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, int wfmt) {
  // Split K in two when the fc2 tiles would leave a partial last wave of
  // workgroups over the 256 CUs (2 resident per CU) and K is long enough.
  const int64_t tiles = ((T * k + BM - 1) / BM + std::min<int64_t>(E, T * k)) * ((H + BN - 1) / BN);
  const int64_t stages = (I + bk_for(wfmt) - 1) / bk_for(wfmt);
  return (tiles < 2048 && stages >= 32) ? 2 : 1;
}

bool prefill_supported(const ExpertArgs& a) {
  if (a.act_type != MOE_ELEM_FLOAT16 && a.act_type != MOE_ELEM_BFLOAT16) return false;
  if (a.H % 32 || a.I % 32) return false;
  if (a.wfmt != kDense && a.block_size > 0 && a.block_size < 16) return false;
  // 32-bit buffer offsets: one expert's weights and the activation rows stay below 2 GiB
  const int64_t lim = int64_t{1} << 31;
  const int64_t ebits = a.wfmt == kInt4 ? 4 : (a.wfmt == kInt8 ? 8 : 16);
  const int64_t n1 = (a.gate_mode == kGateInterleaved || a.gate_mode == kGateChunked) ? 2 * a.I : a.I;
  if (n1 * a.H * ebits / 8 >= lim || a.H * a.I * ebits / 8 >= lim) return false;
  if (a.T * a.k * std::max(a.H, a.I) * 2 >= lim) return false;
  return true;
}

hipError_t launch_fc1_prefill(const ExpertArgs& a, hipStream_t stream) {
  PStage st{};
  st.in = a.x;
  st.in_rows = a.T;
  st.K = a.H;
  st.nfeat = a.I;
  const bool fused = a.gate_mode == kGateInterleaved || a.gate_mode == kGateChunked;
  const bool gated = a.gate_mode != kGateNone;
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
  st.out_rows = a.T * a.k;
  st.out = a.act;
  // gated: a weight tile holds BN/2 features (gate + linear rows)
  plan_grid(st, a.T, a.k, a.E, a.wfmt, gated ? 2 * a.I : a.I, 1);
  return launch_stage<true>(st, a, gated, stream);
}

hipError_t launch_fc2_prefill(const ExpertArgs& a, int* y2_planes, hipStream_t stream) {
  PStage st{};
  st.in = a.act;
  st.in_rows = a.T * a.k;
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
  st.out_rows = a.T * a.k;
  st.out = a.y2;
  const int32_t splits = prefill_fc2_splits(a.T, a.H, a.I, a.E, a.k, a.wfmt);
  plan_grid(st, a.T, a.k, a.E, a.wfmt, a.H, splits);
  *y2_planes = splits;
  return launch_stage<false>(st, a, false, stream);
}

}  // namespace moe
