// moe_expert_stream.h -- decode expert GEMV (up to 64 tokens): one
// persistent workgroup per CU streams an even share of the weight tiles of
// all routed experts.  An expert's rows are taken in groups of 16 (the MFMA
// M dimension); an expert with more than 16 rows streams its weights once
// per group.
//
// Why persistent: a decode layer reads each routed expert's weights once, and
// the unit a launch grid hands out (a feature group with its whole K) is too
// coarse to spread evenly: e.g. 1568 such groups on 768 resident slots leave
// most of a third round idle, and the two experts of a single token leave
// CUs empty.  Here every workgroup takes the same number of weight tiles
// (+-1) and its waves split those tiles' K chunks evenly.
//
// Work space: tiles are (row group a, K slice s, feature tile f), f
// fastest.  A tile is 16 features (gate + linear rows when gated) or 32
// features (two 16-row weight tiles), over KSC chunks of 128 k.  Workgroup i
// takes tiles [T*i/P, T*(i+1)/P).  A run of its tiles with the same (a, s) is
// a group: the group's activation slice (<= 16 rows x KSC*128 k) is staged
// into LDS once, the group's (tile, chunk) space is cut into blocks of PD
// chunks, and the waves take equal contiguous runs of blocks.
//
// A wave's run starts and ends anywhere.  Tiles it covers completely are
// finished from registers (scales, bias, activation, store).  The partial
// tile at the start of its run goes to an LDS slot; the wave that holds the
// first chunk of a split tile adds the slots of the following waves in wave
// order and finishes it.  Every sum has an order fixed by the shapes, so
// results do not depend on timing.
//
// Weights stream through a register ring of PD chunks (one block): each
// chunk of the next block is requested as soon as the same slot of the
// current block is consumed, and a group's first block is requested while
// its activation slice is staged.
//
// Biased operands: int8/int4 weights enter the MFMA with their zero point
// and magic-exponent bias still in (1024 + q for fp16, 128 + q for bf16),
// and the bias is removed per chunk (block scales), per MFMA step (step
// scales) or once (per-channel scales) with per-row activation sums
// computed while staging.  For int4, the nibbles are placed into the 16-bit
// lanes with one and-or operation per pair (fp16) or a shift and an and-or
// (bf16, odd pairs): the odd nibbles land 4 bits up (1024 + 16 q) or 1 bit
// down (128 + 8 q), so the activations at those k are staged divided by 16
// or 8 (exact), and the k order inside each 8-k step is (0 4 1 5 2 6 3 7)
// in both operands.
//
// fc1 needs the whole K in one slice (its activation needs the full sum);
// fc2 writes one fp32 plane of y2 per K slice, which the finalize pass sums
// in order.
#pragma once

#include <type_traits>

#include "moe_expert_decode.h"
#include "moe_route_device.h"

namespace moe {
namespace decode {

constexpr int kStreamRows = 16;       // token rows staged (the MFMA M dimension)
constexpr int kStreamMaxChunks = 32;  // K chunks of one staged slice (16 x 32 x 256 B of LDS)
constexpr int kStreamFetch = 4;       // row-major weights: chunks whose loads are issued back to back
static_assert(kStreamMaxChunks * kChunk == kStreamMaxK, "host and kernel agree on the slice size");

// Chunks per block; a K slice is a whole number of blocks.
inline int stream_pd(int wfmt, bool gated) {
  (void)wfmt;
  (void)gated;
  return 4;
}

struct StreamStage {
  Stage s;
  int32_t ksc;      // chunks per K slice (multiple of the ring depth; the last slice is padded)
  int32_t nslices;  // K slices (fc2 partial planes)
  int32_t E;        // experts
  int32_t ngroups;  // bound on the row groups of all experts: E + T*k/16
  // fc1 only: with route.logits set, every workgroup routes and dispatches
  // the batch itself in its prologue (into LDS: E + 1 offsets and T k rows,
  // route_ints in all) and workgroup 0 publishes the results to route's
  // outputs; otherwise offsets and perm come from the router kernels.
  moe_route_params route;
  int32_t route_ints;
};

// Largest T * k and expert count for which the decode fc1 kernel routes in
// its prologue.
constexpr int kFusedRouteRows = 1024;
constexpr int kFusedRouteExperts = 128;

template <int WF, bool GATED>
struct SGeo {
  static constexpr int kVecs = WF == kInt4 ? 1 : (WF == kInt8 ? 2 : 4);  // u32x4 per tile per chunk
  static constexpr int kLaneBytes = 16 * kVecs;                           // bytes per 32 k of a row
  static constexpr int FT = GATED ? 1 : 2;                                // 16-feature tiles per tile
  static constexpr int WT = 2;                                            // 16-row weight tiles per tile
  static constexpr int NW = WF == kDense ? 8 : 12;                         // waves per workgroup
  static constexpr int PD = 4;                                              // chunks per block (ring depth)
};

// s_waitcnt operand that waits until at most n (< 64) vector memory
// operations are outstanding and leaves expcnt and lgkmcnt alone (gfx9
// encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int vmcnt_imm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

// Raw block scales of one lane: NSC consecutive elements in one load.
template <typename ST, int NSC>
struct ScaleRaw {
  static constexpr int kBytes = NSC * static_cast<int>(sizeof(typename ST::storage));
  using type = std::conditional_t<(kBytes > 8), u32x4_t, std::conditional_t<(kBytes > 4), u32x2_t, uint32_t>>;
  template <int AUX>
  __device__ static __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (kBytes == 1) {
      return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b8(r, static_cast<int>(off), 0, AUX));
    } else if constexpr (kBytes == 2) {
      return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(off), 0, AUX));
    } else if constexpr (kBytes == 4) {
      return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, AUX);
    } else if constexpr (kBytes == 8) {
      return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(off), 0, AUX));
    } else {
      return bload16_aux<AUX>(r, off);
    }
  }
  __device__ static __forceinline__ float elem(type v, int i) {
    if constexpr (std::is_same_v<ST, E8M0>) {
      (void)i;
      return e8m0_to_f32(v & 0xFFu);
    } else if constexpr (std::is_same_v<ST, F32>) {
      if constexpr (kBytes == 4) return __uint_as_float(v);
      else return __uint_as_float(v[i]);
    } else {
      uint32_t w;
      if constexpr (kBytes <= 4) w = v;
      else w = v[i >> 1];
      const uint16_t h = static_cast<uint16_t>(w >> (16 * (i & 1)));
      if constexpr (std::is_same_v<ST, F16>) return static_cast<float>(__builtin_bit_cast(_Float16, h));
      else return bf16_to_f32(h);
    }
  }
};

template <int WF, bool GATED, typename SR, bool RING_SCALES>
struct SChunk {
  u32x4_t w[SGeo<WF, GATED>::WT][SGeo<WF, GATED>::kVecs];
  typename SR::type sc[RING_SCALES ? SGeo<WF, GATED>::WT : 1];
};

// int4 dword (k0..k7) -> fp16 pairs (1024 + q) in k order (0 4 1 5 2 6 3 7);
// the odd-k pairs hold 1024 + 16 q.
// m_lo = 0x000F000F, m_hi = 0x00F000F0 (passed in so that they can live in VGPRs).
__device__ __forceinline__ u32x4_t dq4_f16_split(uint32_t v, uint32_t m_lo, uint32_t m_hi) {
  const uint32_t c = 0x64006400u, h = v >> 8;
  return u32x4_t{(v & m_lo) | c, (v & m_hi) | c, (h & m_lo) | c, (h & m_hi) | c};
}

// The bf16 form: 128 + q in the same k order, the odd-k pairs 128 + 8 q (a
// bf16 of magnitude 128..255 has 7 mantissa bits, so an odd nibble moves 1
// bit down, not 4 up).  m_lo = 0x000F000F, m_hi = 0x00780078.
__device__ __forceinline__ u32x4_t dq4_bf16_split(uint32_t v, uint32_t m_lo, uint32_t m_hi) {
  const uint32_t c = 0x43004300u, h = v >> 8;
  return u32x4_t{(v & m_lo) | c, ((v >> 1) & m_hi) | c, (h & m_lo) | c, ((h >> 1) & m_hi) | c};
}

// Both halves of a bf16 pair times 1/8 (exact for normal values).
__device__ __forceinline__ uint32_t bf16x2_eighth(uint32_t w) {
  const float lo = __uint_as_float(w << 16) * 0.125f, hi = __uint_as_float(w & 0xFFFF0000u) * 0.125f;
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
}

// 4 x 4 transpose of dwords across the four 16-lane rows of a wave (gfx950
// row swaps): on entry v[j] of row r holds m[r][j]; on exit v[j] of row r
// holds m[j][r].
__device__ __forceinline__ void transpose_rows4(uint32_t* v) {
  const auto a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);  // [m00 m10 m02 m12], [m20 m30 m22 m32]
  const auto b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);  // [m01 m11 m03 m13], [m21 m31 m23 m33]
  const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  v[0] = c[0];
  v[1] = c[1];
  v[2] = d[0];
  v[3] = d[1];
}

// o[r] = v of row r (same lane within the row), in every lane.
__device__ __forceinline__ void gather_rows4(uint32_t v, uint32_t* o) {
  const auto a = __builtin_amdgcn_permlane32_swap(v, v, false, false);        // [v0 v1 v0 v1], [v2 v3 v2 v3]
  const auto b = __builtin_amdgcn_permlane16_swap(a[0], a[0], false, false);  // [v0 x4], [v1 x4]
  const auto c = __builtin_amdgcn_permlane16_swap(a[1], a[1], false, false);  // [v2 x4], [v3 x4]
  o[0] = b[0];
  o[1] = b[1];
  o[2] = c[0];
  o[3] = c[1];
}

// K slices of the stream kernel: as few as fit the LDS slice, each a whole
// number of ring blocks (pd chunks).  Equal slices without padding are
// preferred (e.g. 112 chunks: 7 x 16 rather than 4 x 32 with the last half
// empty); otherwise the last slice is padded.
inline void stream_slices(int64_t K, int pd, int32_t* nsl, int32_t* ksc) {
  const int64_t nchunks = (K + kChunk - 1) / kChunk;
  const int64_t maxper = kStreamMaxChunks / pd * pd;
  const int64_t nmin = (nchunks + maxper - 1) / maxper;
  int64_t per = 0;
  for (int64_t n = nmin; n < nmin + 8 && per == 0; ++n)
    if (nchunks % n == 0 && (nchunks / n) % pd == 0) per = nchunks / n;
  if (per == 0) per = ((nchunks + nmin - 1) / nmin + pd - 1) / pd * pd;
  *nsl = static_cast<int32_t>((nchunks + per - 1) / per);
  *ksc = static_cast<int32_t>(per);
}

// Bound on the row groups (16 rows of one expert) of a call: each routed
// expert has at most one partial group.
inline int32_t stream_groups(int64_t T, int64_t E, int64_t k) {
  const int64_t rows = T * k;
  return static_cast<int32_t>(std::min(E, rows) + (rows + kStreamRows - 1) / kStreamRows);
}

// Bytes of dynamic LDS of the stream kernel (ngroups: row-group list
// entries; route_ints: routing results kept in LDS, 0 when the router
// kernels route).  The routing scratch of the prologue overlays the slice.
inline size_t stream_region_bytes(int ksc, int nw) {
  // activation slice + bias sums per (32 k, row)
  const size_t act = static_cast<size_t>(kStreamRows) * (static_cast<size_t>(ksc) * 256 + 16) +
                     static_cast<size_t>(ksc) * 4 * kStreamRows * 4;
  const size_t slots = static_cast<size_t>(nw) * 2 * 64 * 16;
  return std::max(act, slots);
}
inline size_t stream_lds_bytes(int ksc, int ngroups, int nw, int route_ints) {
  const size_t ex = (static_cast<size_t>(ngroups) * 4 + 15) / 16 * 16 + (static_cast<size_t>(route_ints) * 4 + 15) / 16 * 16;
  return ex + stream_region_bytes(ksc, nw);
}

// NSC: folded scales (block 16/32/64): elements per lane and chunk (2 for
// block 16); block scales: 4 = one load brings the scales of 4 chunks
// (block 128, K a multiple of 512), 1 = one load per chunk; step scales:
// 1 (lane group g loads the scale of step g's block).
// STREAM_NT: the weights are tile-major (pre-packed), streamed with the
// non-temporal cache policy.
//
// k assignment.  Loads are chunk-major: lane group g owns k [32 g, 32 g +
// 32) of the chunk (one 16-byte piece of int4 per row), and, in every mode
// but step, feeds 8 of them to each MFMA step, so a step's 32 k span the
// chunk's four 32-k blocks.  Step-major (kScaleStep): step st takes k
// [32 st, 32 st + 32), lane group g its 8 k at 32 st + 8 g, so a step lies
// in one block of 32; the lanes of one row exchange their dwords with a 4 x
// 4 transpose across lane groups (4 row swaps per 16 bytes), and the
// activation slice is read at 64 st + 16 g.
template <typename AT, int WF, int SM, typename ST, int NSC, bool FC1, bool GATED, bool STREAM_NT>
__global__ void __launch_bounds__((SGeo<WF, GATED>::NW * 64), 1) gemv_stream_kernel(StreamStage ss) {
  using G = SGeo<WF, GATED>;
  constexpr int kAux = STREAM_NT ? kStreamAux : 0;
  constexpr int NW = G::NW, NT = NW * 64, WT = G::WT, FT = G::FT, PD = G::PD, LB = G::kLaneBytes;
  constexpr bool kStep = SM == kScaleStep;
  constexpr bool kMx = SM == kScaleMx;  // MXFP4: step-major, E2M1 operands, E8M0 step scales
  static_assert(!kMx || (WF == kInt4 && std::is_same_v<ST, E8M0> && NSC == 1), "MXFP4: 4-bit E2M1, E8M0 scales");
  constexpr bool kBiased = Biased<AT, WF>::kOk && (SM == kScaleBlock || SM == kScaleChan || kStep);
  static_assert(!kStep || (Biased<AT, WF>::kOk && NSC == 1), "step scales: biased operands, one scale per lane");
  constexpr bool kSplit = kBiased && WF == kInt4 && AT::kId == 10;
  constexpr bool kSplitB = kBiased && WF == kInt4 && AT::kId == 16;
  constexpr bool kRingScales = SM == kScaleBlock || SM == kScaleFold || kStep || kMx;
  constexpr bool kGroupScales = SM == kScaleBlock && NSC == 4;
  // 2-byte block scales of block 128 are loaded per tile: one load per
  // lane (row col, lane group g) brings the 16 bytes that hold the scales
  // of the slice's chunks 8g .. 8g + 7 (a slice has at most 32 chunks), and
  // each block hands its 4 chunks' scales to the lanes of the row with one
  // cross-lane read per 2 chunks.  One request per row and tile, where
  // per-block loads would touch every row's cache line again for each
  // block of the tile.  The load for a tile is issued during the block
  // before it, after that block has read the previous tile's scales.
  constexpr bool kTileScales = kGroupScales && sizeof(typename ST::storage) == 2;
  static_assert(!kTileScales || kStreamMaxChunks <= 32, "a slice's scales are 4 x 16 bytes per row");
  // Chunks computed before their slots' next loads go out.  Row-major
  // weights: kStreamFetch, so that one row's consecutive 64-byte pieces
  // reach the memory controller together.  Tile-major weights (each load is
  // one 1 KB run): every chunk's next load goes out as soon as the chunk is
  // consumed, which keeps 3 of the 4 ring slots in flight while a
  // VALU-heavy chunk computes; except with grouped block scales outside the
  // tile-scale path, whose slot 0 holds the scales of the whole block.
  constexpr int kFetch = STREAM_NT && !(kGroupScales && !kTileScales) ? 1 : kStreamFetch;
  static_assert(PD % kFetch == 0, "a block is whole fetch groups");
  static_assert(!(SM == kScaleBlock && NSC == 4) || PD % 4 == 0, "grouped scales: 4 chunks of one block");
  using SR = ScaleRaw<ST, NSC>;
  using CK = SChunk<WF, GATED, SR, kRingScales>;
  constexpr int kEs = static_cast<int>(sizeof(typename ST::storage));
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int wcount[NW];
  __shared__ int loffs[kWave + 1];  // up to 64 experts: the offsets, read once
  const Stage& p = ss.s;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, g = lane >> 4;
  const int ksc = ss.ksc, nsl = ss.nslices, E = ss.E;
  const int pitch = ksc * 256 + 16;
  int* exl = reinterpret_cast<int*>(smem);  // row groups: expert | (group << 16), ascending
  int* lroute = reinterpret_cast<int*>(smem + (ss.ngroups * 4 + 15) / 16 * 16);  // [E + 1] offsets, [T k] perm
  uint8_t* region = smem + (ss.ngroups * 4 + 15) / 16 * 16 + (ss.route_ints * 4 + 15) / 16 * 16;
  uint8_t* xs = region;                                         // [16][pitch] activation slice
  // bias sums per row: [ksc][16] per chunk, step scales [ksc * 4][16] per 32 k
  float* corr = reinterpret_cast<float*>(region + 16 * pitch);
  float* slots = reinterpret_cast<float*>(region);              // [NW][WT][64] float4, after the compute

  // ---- routing (fc1 of a small batch): every workgroup computes the same
  // top-k, counts, offsets and stable permutation into LDS (the scratch
  // overlays the activation slice, not yet in use); workgroup 0 also writes
  // them out for fc2 and finalize ----
  const int32_t* offs = p.offsets;
  const int32_t* perm = p.perm;
  if constexpr (FC1) {
    if (ss.route.logits) {
      route_dispatch_block<AT>(ss.route, lroute, lroute + E + 1, reinterpret_cast<int*>(region), blockIdx.x == 0);
      offs = lroute;
      perm = lroute + E + 1;
    }
  }

  // ---- row groups: each routed expert's rows in groups of 16 (the MFMA M);
  // an expert with more rows streams its weights once per group.
  // exl[0 .. e_act) ----
  //
  // This workgroup's tiles [t_beg, t_end) follow from e_act (split below).
  // Tiles of group q (row group a = q / nsl, slice s = q % nsl) are
  // [q nft, (q + 1) nft).  Each group a workgroup touches costs a staging
  // and a split-tile reduction, about kGroupCost tiles of streaming.  With
  // fewer groups than workgroups, each group gets a whole number of
  // workgroups (group q: workgroups i with i G / P == q) when the largest
  // share that leaves is cheaper than an even split of all tiles plus the
  // second group that the workgroups on a group boundary then pay.  All
  // values are non-negative and tile counts stay far below 2^31 (row
  // groups x slices x feature tiles), so the arithmetic is 32-bit unsigned.
  // The scalar unit a CU's waves share would run it once per wave, so fc2,
  // in the one-wave case, has wave 0 alone compute it and pass it on in
  // LDS (fc1 keeps it in every wave: measured no gain there, and a loss at
  // gpt-oss int4).
  constexpr int kGroupCost = 2;
  const uint32_t P = gridDim.x, bx = blockIdx.x;
  const int nft = static_cast<int>((p.nfeat + 16 * FT - 1) / (16 * FT));
  auto split = [&](uint32_t ngq, int* tb, int* te) {
    const uint32_t nf = static_cast<uint32_t>(nft), ttot = ngq * nf;
    if (ngq == 0) {
      *tb = *te = 0;
    } else if (ngq <= P && (nf + P / ngq - 1) / (P / ngq) < kGroupCost + (ttot + P - 1) / P) {
      const uint32_t q = bx * ngq / P;
      const uint32_t w0 = (q * P + ngq - 1) / ngq, nw = ((q + 1) * P + ngq - 1) / ngq - w0;
      const uint32_t j = bx - w0;
      *tb = static_cast<int>(q * nf + nf * j / nw);
      *te = static_cast<int>(q * nf + nf * (j + 1) / nw);
    } else {
      // floor(ttot * b / P) without a 64-bit product
      const uint32_t qt = ttot / P, rt = ttot % P;
      *tb = static_cast<int>(qt * bx + rt * bx / P);
      *te = static_cast<int>(qt * (bx + 1) + rt * (bx + 1) / P);
    }
  };
  int e_act = 0, t_beg = 0, t_end = 0;
  if (E <= kWave) {
    // one wavefront: lane e's groups, then one barrier.  The offsets it
    // reads stay in LDS for the group loop (one global round trip less
    // before the first loads when they come from the router kernels).
    if (wave == 0) {
      const int lo = lane < E ? offs[lane] : 0, hi = lane < E ? offs[lane + 1] : 0;
      if (lane < E) loffs[lane] = lo;
      if (lane == E - 1) loffs[E] = hi;
      const int cnt = hi - lo;
      const int nv = (cnt + kStreamRows - 1) / kStreamRows;
      int inc = nv;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int t = __shfl_up(inc, o, kWave);
        if (lane >= o) inc += t;
      }
      for (int j = 0; j < nv; ++j) exl[inc - nv + j] = lane | (j << 16);
      int tb = 0, te = 0;
      if constexpr (!FC1) split(static_cast<uint32_t>(__builtin_amdgcn_readlane(inc, kWave - 1) * nsl), &tb, &te);
      if (lane == kWave - 1) {
        wcount[0] = inc;
        wcount[1] = tb;
        wcount[2] = te;
      }
    }
    __syncthreads();
    e_act = wcount[0];
    t_beg = wcount[1];
    t_end = wcount[2];
    offs = loffs;
  }
  for (int base = 0; base < E && E > kWave; base += NT) {
    const int e = base + tid;
    const int cnt = e < E ? offs[e + 1] - offs[e] : 0;
    const int nv = (cnt + kStreamRows - 1) / kStreamRows;
    int inc = nv;  // inclusive scan over the wave
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int t = __shfl_up(inc, o, kWave);
      if (lane >= o) inc += t;
    }
    if (lane == kWave - 1) wcount[wave] = inc;
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < NW; ++w) {
      const int c = wcount[w];
      before += w < wave ? c : 0;
      total += c;
    }
    const int x0 = e_act + before + inc - nv;
    for (int j = 0; j < nv; ++j) exl[x0 + j] = e | (j << 16);
    e_act += total;
    __syncthreads();
  }
  e_act = __builtin_amdgcn_readfirstlane(e_act);
  if (FC1 || E > kWave) split(static_cast<uint32_t>(e_act * nsl), &t_beg, &t_end);
  t_beg = __builtin_amdgcn_readfirstlane(t_beg);
  t_end = __builtin_amdgcn_readfirstlane(t_end);

  // ---- this workgroup's tiles ----
  const int64_t K = p.K;
  const int nchunks = static_cast<int>((K + kChunk - 1) / kChunk);
  const int ktail = static_cast<int>(K - static_cast<int64_t>(nchunks - 1) * kChunk);
  // Tile-major weights (pre-packed) hold whole chunks: a row's K is padded
  // with zeros to nchunks * 128 k.
  const bool tiled = STREAM_NT || p.tiled != 0;
  const uint32_t rb = tiled ? static_cast<uint32_t>(nchunks * 4 * LB)
                            : static_cast<uint32_t>((K / 32) * LB);  // bytes of one weight row
  const int per_a = nsl * nft;
  const int bpt = ksc / PD;  // blocks per tile
  int bshift = 0;
  uint32_t nblk = 0;
  if constexpr (kRingScales) {
    bshift = __builtin_ctzll(static_cast<uint64_t>(p.block_size));
    nblk = static_cast<uint32_t>(K >> bshift);
  }
  const __amdgpu_buffer_rsrc_t rs_x = make_rsrc(p.in, static_cast<uint32_t>(p.in_rows * K * 2));
  const int nfeat = static_cast<int>(p.nfeat);

  // Weight row of feature f in weight tile u: f * rmul + radd[u] (gate rows
  // 2f / linear rows 2f + 1 when interleaved; linear rows f + nfeat when
  // chunked).  Lane constants: feature offset fo[u] inside a tile, and the
  // row's byte offsets with the tile index factored out (32-bit: one
  // expert's weights are below 2 GiB).
  // Scales and biases of the interleaved layout: rows 2f / 2f + 1.  The
  // weights too, unless pre-packed de-interleaved (gate f, linear nfeat + f).
  const int rmul = (FC1 && GATED && p.gate_mode == kGateInterleaved) ? 2 : 1;
  const bool deint = FC1 && GATED && tiled && p.deint != 0;
  const int wmul = deint ? 1 : rmul;
  // Tile-major step scales (pre-packed): per (16-row tile, chunk) the 16
  // rows' nbc = 128 / block scales, 16 * nbc contiguous elements (rows as
  // the weights'); nblk_r: their elements per row, with K padded to whole
  // chunks.  One load instruction then reads 16 * nbc * 2 (or 4) bytes in
  // one run instead of one cache line per row.
  const bool stiled = (kStep || kMx) && tiled && p.stiled != 0;
  const int nbc = kChunk >> bshift;
  const uint32_t nblk_r = stiled ? static_cast<uint32_t>(nchunks * nbc) : nblk;
  // Tile-major weights (pre-packed; weight tiles start at a multiple of 16
  // rows, K is whole chunks): the 16 rows x 128 k of a weight tile and chunk
  // are one contiguous block, lane l's 16 bytes at 16 l (vector v of int8
  // one 1 KB block further), so that each load instruction reads 1 KB in
  // one run.  Row-major: row col, bytes [LB g, LB g + LB) of the chunk.
  const uint32_t cstride = tiled ? 64 * LB : 4 * LB;  // weight bytes per chunk
  const int vdelta = tiled ? 1024 - 16 : 0;           // extra offset of vector v, per v
  int fo[WT], rowb[WT];
  uint32_t wb[WT], sb[WT];
#pragma unroll
  for (int u = 0; u < WT; ++u) {
    const bool lin = GATED && u >= FT;
    const int radd = !lin ? 0 : (p.gate_mode == kGateInterleaved ? 1 : (p.gate_mode == kGateChunked ? nfeat : 0));
    fo[u] = (u % FT) * 16 + col;
    rowb[u] = fo[u] * rmul + radd;
    const int wrow = deint ? fo[u] + (lin ? nfeat : 0) : rowb[u];
    wb[u] = tiled ? static_cast<uint32_t>(wrow - col) * rb + lane * 16 : static_cast<uint32_t>(wrow) * rb + g * LB;
    // tile-major scales: lane (col, g) reads scale (32 g) / block of row col
    sb[u] = stiled ? (static_cast<uint32_t>(wrow - col) * nblk_r + static_cast<uint32_t>(col * nbc + ((32 * g) >> bshift))) * kEs
                   : static_cast<uint32_t>(rowb[u]) * nblk * kEs;
  }
  const uint32_t tws = static_cast<uint32_t>(16 * FT * wmul) * rb;          // weight bytes per tile step
  const uint32_t tss = stiled ? static_cast<uint32_t>(16 * FT * wmul) * nblk_r * kEs
                              : static_cast<uint32_t>(16 * FT * rmul) * nblk * kEs;  // scale bytes per tile step
  // masks of the int4 nibble split, kept in VGPRs so that each output pair
  // is one v_and_or_b32
  uint32_t m_lo = 0x000F000Fu, m_hi = kSplitB ? 0x00780078u : 0x00F000F0u;
  if constexpr (kSplit || kSplitB) {
    asm volatile("" : "+v"(m_lo));
    asm volatile("" : "+v"(m_hi));
  }

  for (int t = t_beg; t < t_end;) {
    const int a = static_cast<int>(static_cast<uint32_t>(t) / static_cast<uint32_t>(per_a));
    const int rem = t - a * per_a;
    const int s = static_cast<int>(static_cast<uint32_t>(rem) / static_cast<uint32_t>(nft)), f0 = rem - s * nft;
    const int ntl = t_end - t < nft - f0 ? t_end - t : nft - f0;
    const int nb = ntl * bpt;
    const int b0 = nb * wave / NW, b1 = nb * (wave + 1) / NW;
    const int ent = __builtin_amdgcn_readfirstlane(exl[a]);
    const int e = ent & 0xFFFF;
    const int row0 = __builtin_amdgcn_readfirstlane(offs[e]) + (ent >> 16) * kStreamRows;
    const int cnt = __builtin_amdgcn_readfirstlane(offs[e + 1]) - row0;
    const int nrows = cnt < kStreamRows ? cnt : kStreamRows;
    const int cs0 = s * ksc;  // first chunk of the slice

    const __amdgpu_buffer_rsrc_t rs_g = make_rsrc(p.w + static_cast<int64_t>(e) * p.w_rows * rb,
                                                  static_cast<uint32_t>(p.w_rows * rb));
    const __amdgpu_buffer_rsrc_t rs_l = make_rsrc(p.wl + static_cast<int64_t>(e) * p.wl_rows * rb,
                                                  static_cast<uint32_t>(p.wl_rows * rb));
    __amdgpu_buffer_rsrc_t ss_g = rs_g, ss_l = rs_l;
    if constexpr (kRingScales) {
      ss_g = make_rsrc(static_cast<const uint8_t*>(p.s) + static_cast<int64_t>(e) * p.w_rows * nblk_r * kEs,
                       static_cast<uint32_t>(p.w_rows * nblk_r * kEs));
      ss_l = make_rsrc(static_cast<const uint8_t*>(p.sl) + static_cast<int64_t>(e) * p.wl_rows * nblk_r * kEs,
                       static_cast<uint32_t>(p.wl_rows * nblk_r * kEs));
    }

    // weight / scale offsets of tile tl (relative to the group) for this lane
    auto tile_offs = [&](int tl, uint32_t* woff, uint32_t* soff) {
      const int ft = f0 + tl;
#pragma unroll
      for (int u = 0; u < WT; ++u) {
        // features past the end: bit 31 set (offsets are below 2 GiB), reads nothing
        const uint32_t oob = ft * (16 * FT) + fo[u] < nfeat ? 0u : kOob;
        woff[u] = (static_cast<uint32_t>(ft) * tws + wb[u]) | oob;
        soff[u] = (static_cast<uint32_t>(ft) * tss + sb[u]) | oob;
      }
    };
    CK ring[PD];
    // tile scales of the current (or, late in its last block, the next) tile
    u32x4_t tsr[WT];
    auto fetch_tsc = [&](int tl) {
      if constexpr (kTileScales) {
        uint32_t woff[WT], soff[WT];
        tile_offs(tl, woff, soff);
#pragma unroll
        for (int u = 0; u < WT; ++u)
          tsr[u] = bload16_aux<kAux>(GATED && u >= FT ? ss_l : ss_g, soff[u] + static_cast<uint32_t>(cs0) * 2 + 16 * g);
      }
    };
    // vector memory loads that fetching one block issues
    constexpr int kBlockLoads =
        PD * WT * G::kVecs + (kTileScales ? 0 : (kRingScales ? (kGroupScales ? PD / 4 : PD) * WT : 0));
    auto fetch = [&](int cl, const uint32_t* woff, const uint32_t* soff, CK& d) {
      const int cg = cs0 + cl;
      // padding chunks past K and the missing lanes of a partial last chunk
      // read nothing (branch-free: one compare against the chunk's valid k)
      const int kval = cg < nchunks - 1 ? kChunk : (cg == nchunks - 1 ? ktail : 0);
      const uint32_t wc = static_cast<uint32_t>(cg) * cstride;
      const uint32_t oob = 32 * g + 32 <= kval ? 0u : kOob;
#pragma unroll
      for (int u = 0; u < WT; ++u) {
        const uint32_t o = (woff[u] + wc) | oob;
#pragma unroll
        for (int v = 0; v < G::kVecs; ++v)
          d.w[u][v] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                      GATED && u >= FT ? rs_l : rs_g, static_cast<int>(o + 16 * v),
                                                      v * vdelta, kAux));
        if constexpr (kRingScales && !kTileScales) {
          // folded and step scales: the block of lane group g's 32 k
          constexpr bool kPerGroup = SM == kScaleFold || kStep || kMx;
          const uint32_t kk = static_cast<uint32_t>(cg) * kChunk + (kPerGroup ? 32 * g : 0);
          // a block scale multiplies the whole chunk's sum (every lane group
          // of the MFMA output), so only a chunk past K reads none
          const uint32_t so = stiled ? (soff[u] + static_cast<uint32_t>(cg * 16 * nbc * kEs)) | oob
                                     : (soff[u] + (kk >> bshift) * kEs) | (kPerGroup ? oob : (cg < nchunks ? 0u : kOob));
          // grouped: the first chunk of each group of 4 loads all 4 scales
          if (!kGroupScales || (cl & 3) == 0) d.sc[u] = SR::template load<kAux>(GATED && u >= FT ? ss_l : ss_g, so);
        }
      }
    };

    // ---- the group's activation slice goes global -> LDS directly (buffer
    // loads with the LDS bit): one 16-byte piece per lane, 1 KB per wave
    // instruction, which is 64 consecutive pieces of one row (a row of the
    // slice is ksc * 16 pieces and ksc is a multiple of 4).  Group q goes to
    // wave q % NW.  k past K reads zeros.  These loads go out before the
    // weight loads, so that staging waits for one round trip and not behind
    // the weights that every workgroup requests at the same moment. ----
    const int gpr = ksc / 4;        // 1 KB groups per row
    const int ngr = nrows * gpr;    // groups of the slice
    // source row of row m (fc1: the token of dispatched row row0 + m), lane m
    const int srcl = FC1 ? (lane < nrows ? perm[row0 + lane] / static_cast<int>(p.topk) : 0) : row0 + lane;
    for (int q = wave; q < ngr; q += NW) {
      const int m = q / gpr, r = (q - m * gpr) * 64 + lane;  // row, piece in the row
      const int64_t k = static_cast<int64_t>(cs0 + (r >> 4)) * kChunk + (r & 15) * 8;
      const int64_t src = __builtin_amdgcn_readlane(srcl, m);
      const uint32_t off = k < K ? static_cast<uint32_t>((src * K + k) * 2) : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs_x, (__attribute__((address_space(3))) void*)(xs + m * pitch + (r - lane) * 16), 16,
          static_cast<int>(off), 0, 0, 0);
    }
    // the first tile's scales (before the weights, so that waiting for them
    // does not wait for the weights)
    fetch_tsc(b0 / bpt);
    // The first block of the run.  Every wave issues its loads (with an
    // empty run they read nothing), so that the run loop is always entered
    // with the same loads in flight as at its back edge and its waits stay
    // one block deep.
    {
      uint32_t woff[WT], soff[WT];
      const int tl = b0 / bpt, cb = b0 - tl * bpt;
      tile_offs(tl, woff, soff);
      if (b0 >= b1) {
#pragma unroll
        for (int u = 0; u < WT; ++u) woff[u] = soff[u] = kOob;
      }
#pragma unroll
      for (int d = 0; d < PD; ++d) fetch(cb * PD + d, woff, soff, ring[d]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // This wave's slice pieces have landed once no more than the weight
    // loads issued after them are in flight (the compiler does not order a
    // wave's LDS reads after its own LDS-bound loads).
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(kBlockLoads));
    // Each wave finishes the pieces it loaded: the int4 split (odd k / 16
    // and the k order of the weights) in place, and the bias sums per
    // (chunk, row) of biased operands (the 16 pieces of one (row, chunk) sit
    // in 16 consecutive lanes; step-major: per (32 k, row), 4 lanes).
    if constexpr (kBiased) {
      for (int q = wave; q < ngr; q += NW) {
        const int m = q / gpr, r = (q - m * gpr) * 64 + lane;
        u32x4_t* px = reinterpret_cast<u32x4_t*>(xs + m * pitch + r * 16);
        u32x4_t y = *px;
        float cs = 0.0f;
        if constexpr (kSplit) {
          const half2_t q16 = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
          const u32x4_t x = y;
          y[0] = __builtin_amdgcn_perm(x[2], x[0], 0x05040100u);
          y[1] = h2_bits(bits_h2(__builtin_amdgcn_perm(x[2], x[0], 0x07060302u)) * q16);
          y[2] = __builtin_amdgcn_perm(x[3], x[1], 0x05040100u);
          y[3] = h2_bits(bits_h2(__builtin_amdgcn_perm(x[3], x[1], 0x07060302u)) * q16);
          float lo = 0.0f, hi = 0.0f;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const half2_t h = bits_h2(y[c]);
            const float v = static_cast<float>(h[0]) + static_cast<float>(h[1]);
            if (c & 1) hi += v;
            else lo += v;
          }
          cs = 1032.0f * lo + 1152.0f * hi;
          *px = y;
        } else if constexpr (kSplitB) {
          const u32x4_t x = y;
          y[0] = __builtin_amdgcn_perm(x[2], x[0], 0x05040100u);
          y[1] = __builtin_amdgcn_perm(x[2], x[0], 0x07060302u);
          y[2] = __builtin_amdgcn_perm(x[3], x[1], 0x05040100u);
          y[3] = __builtin_amdgcn_perm(x[3], x[1], 0x07060302u);
          float lo = 0.0f, hi = 0.0f;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float v = __uint_as_float(y[c] << 16) + __uint_as_float(y[c] & 0xFFFF0000u);
            if (c & 1) hi += v;
            else lo += v;
          }
          // even k: x (128 + q) = x (q - 8) + 136 x; odd k: (x / 8)(128 + 8 q) = x (q - 8) + 24 x
          cs = 136.0f * lo + 24.0f * hi;
          y[1] = bf16x2_eighth(y[1]);
          y[3] = bf16x2_eighth(y[3]);
          *px = y;
        } else {
          float sum = 0.0f;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            if constexpr (AT::kId == 10) {
              const half2_t h = bits_h2(y[c]);
              sum += static_cast<float>(h[0]) + static_cast<float>(h[1]);
            } else {
              sum += __uint_as_float(y[c] << 16) + __uint_as_float(y[c] & 0xFFFF0000u);
            }
          }
          cs = Biased<AT, WF>::kOffset * sum;
        }
        // per chunk (16 pieces) or, step-major, per 32 k (4 pieces)
        constexpr int kSumPieces = kStep ? 4 : 16;
#pragma unroll
        for (int o = 1; o < kSumPieces; o <<= 1) cs += __shfl_xor(cs, o, kWave);
        if ((r & (kSumPieces - 1)) == 0) corr[(r / kSumPieces) * kStreamRows + m] = cs;
      }
    }
    __syncthreads();

    // per-row bias sums of the whole slice (per-channel scales: removed once)
    floatx4_t ctot = {0.f, 0.f, 0.f, 0.f};
    if constexpr (kBiased && SM == kScaleChan) {
      for (int c = 0; c < ksc; ++c) ctot += *reinterpret_cast<const floatx4_t*>(corr + c * kStreamRows + 4 * g);
    }

    floatx4_t acc[WT], lead[WT];
#pragma unroll
    for (int u = 0; u < WT; ++u) {
      acc[u] = floatx4_t{0.f, 0.f, 0.f, 0.f};
      lead[u] = acc[u];
    }

    // tile scales of the current block's 4 chunks (chunk d: half d & 1 of
    // bsc[u][d >> 1])
    u32x2_t bsc[WT];
    auto compute = [&](int cl, int slot) {
      const CK& d = ring[slot];
      if constexpr (kMx) {
        // MXFP4: step st takes k [32 st, 32 st + 32), one E8M0 block, whose
        // power-of-two scale the FP4 conversion applies (exact for bf16, and
        // for fp16 while the scaled weight is an fp16 normal); the MFMA
        // accumulates straight into acc
        const uint8_t* xr = xs + col * pitch + cl * 256 + g * 16;
        u32x4_t wq[WT];
        float s4[WT][4];
#pragma unroll
        for (int u = 0; u < WT; ++u) {
          uint32_t v[4] = {d.w[u][0][0], d.w[u][0][1], d.w[u][0][2], d.w[u][0][3]};
          transpose_rows4(v);
          wq[u] = u32x4_t{v[0], v[1], v[2], v[3]};
          uint32_t g4[4];
          gather_rows4(__float_as_uint(SR::elem(d.sc[u], 0)), g4);
#pragma unroll
          for (int st = 0; st < 4; ++st) s4[u][st] = __uint_as_float(g4[st]);
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const u32x4_t av = *reinterpret_cast<const u32x4_t*>(xr + 64 * st);
#pragma unroll
          for (int u = 0; u < WT; ++u) acc[u] = mfma16x16x32<AT>(av, fp4_scaled<AT>(wq[u][st], s4[u][st]), acc[u]);
        }
        return;
      }
      if constexpr (kStep) {
        // Step st: k [32 st, 32 st + 32) of the chunk, one scale block.  The
        // result is sum_st s_st * (mfma_st - c_st): the products s_st * mfma_st
        // go to acc with one fma per element, and the bias sums c_st (per
        // row) times the scales (per feature) are one 16 x 16 x 4 fp32 MFMA
        // per chunk with A[row][st] = -c_st[row], B[st][feature] = s_st: lane
        // (col, g) holds A[col][g] and its own block scale B[g][col].
        const uint8_t* xr = xs + col * pitch + cl * 256 + g * 16;
        const floatx4_t zero = {0.f, 0.f, 0.f, 0.f};
        const float ncr = -corr[(cl * 4 + g) * kStreamRows + col];
        u32x4_t wq[WT][G::kVecs];
        float s4[WT][4];
#pragma unroll
        for (int u = 0; u < WT; ++u) {
          if constexpr (WF == kInt4) {
            uint32_t v[4] = {d.w[u][0][0], d.w[u][0][1], d.w[u][0][2], d.w[u][0][3]};
            transpose_rows4(v);
            wq[u][0] = u32x4_t{v[0], v[1], v[2], v[3]};
          } else {
            // 8 k = two dwords per step: transpose the even and the odd ones
            uint32_t ev[4], od[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              ev[j] = d.w[u][j >> 1][(j & 1) * 2];
              od[j] = d.w[u][j >> 1][(j & 1) * 2 + 1];
            }
            transpose_rows4(ev);
            transpose_rows4(od);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              wq[u][j >> 1][(j & 1) * 2] = ev[j];
              wq[u][j >> 1][(j & 1) * 2 + 1] = od[j];
            }
          }
          const float sg = SR::elem(d.sc[u], 0);
          acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(ncr, sg, acc[u], 0, 0, 0);
          uint32_t g4[4];
          gather_rows4(__float_as_uint(sg), g4);
#pragma unroll
          for (int st = 0; st < 4; ++st) s4[u][st] = __uint_as_float(g4[st]);
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const u32x4_t av = *reinterpret_cast<const u32x4_t*>(xr + 64 * st);
#pragma unroll
          for (int u = 0; u < WT; ++u) {
            u32x4_t bw;
            if constexpr (kSplit) bw = dq4_f16_split(wq[u][0][st], m_lo, m_hi);
            else if constexpr (kSplitB) bw = dq4_bf16_split(wq[u][0][st], m_lo, m_hi);
            else bw = weight_biased<AT, WF>(wq[u], st);
            acc[u] += mfma16x16x32<AT>(av, bw, zero) * s4[u][st];
          }
        }
        return;
      }
      floatx4_t tmp[WT];
#pragma unroll
      for (int u = 0; u < WT; ++u) tmp[u] = floatx4_t{0.f, 0.f, 0.f, 0.f};
      const uint8_t* xc = xs + col * pitch + cl * 256 + g * 64;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const u32x4_t av = *reinterpret_cast<const u32x4_t*>(xc + 16 * st);
#pragma unroll
        for (int u = 0; u < WT; ++u) {
          u32x4_t bw;
          if constexpr (kSplit) {
            bw = dq4_f16_split(d.w[u][0][st], m_lo, m_hi);
          } else if constexpr (kSplitB) {
            bw = dq4_bf16_split(d.w[u][0][st], m_lo, m_hi);
          } else if constexpr (kBiased) {
            bw = weight_biased<AT, WF>(d.w[u], st);
          } else {
            float fs = 0.0f;
            if constexpr (SM == kScaleFold) fs = SR::elem(d.sc[u], NSC == 2 ? (st >> 1) : 0);
            bw = weight_operand<AT, WF, SM == kScaleFold>(d.w[u], st, fs);
          }
          if constexpr (SM == kScaleBlock) tmp[u] = mfma16x16x32<AT>(av, bw, tmp[u]);
          else acc[u] = mfma16x16x32<AT>(av, bw, acc[u]);
        }
      }
      if constexpr (SM == kScaleBlock) {
        floatx4_t cr = {0.f, 0.f, 0.f, 0.f};
        if constexpr (kBiased) cr = *reinterpret_cast<const floatx4_t*>(corr + cl * kStreamRows + 4 * g);
#pragma unroll
        for (int u = 0; u < WT; ++u) {
          float sc;
          if constexpr (kTileScales) sc = SR::elem(bsc[u], slot & (PD - 1));
          else if constexpr (kGroupScales) sc = SR::elem(ring[slot & ~3].sc[u], slot & 3);
          else sc = SR::elem(d.sc[u], 0);
          acc[u] += (tmp[u] - cr) * sc;
        }
      }
    };

    // Raw bits of the per-channel scales and biases of tile tl (weight tile
    // u: scale ep[u] and, for fp32 scales, its upper half ep[2 WT + u]; bias
    // ep[WT + u]), requested when a tile's first block starts and converted
    // in finish.  The loads are branch-free (features past the end and
    // absent biases read nothing, as 0) and nothing uses them before the
    // tile ends, so that no wait for them sits in front of the weight stream.
    const int ses = p.scale_type == MOE_ELEM_FLOAT ? 4 : 2;
    auto load_ep = [&](int tl, uint32_t* ep) {
      const int ft = f0 + tl;
#pragma unroll
      for (int u = 0; u < WT; ++u) {
        const bool lin = GATED && u >= FT;
        const int64_t rows = lin ? p.wl_rows : p.w_rows;
        const uint32_t ri = static_cast<uint32_t>(ft * (16 * FT * rmul) + rowb[u]);  // row in the expert
        const bool in = ft * (16 * FT) + fo[u] < nfeat;
        ep[u] = ep[2 * WT + u] = 0u;
        if constexpr (SM == kScaleChan) {
          // two 16-bit halves (the upper one only for fp32 scales), so that
          // the loads do not depend on the scale type
          const __amdgpu_buffer_rsrc_t r = make_rsrc(static_cast<const uint8_t*>(lin ? p.sl : p.s) + e * rows * ses,
                                                     static_cast<uint32_t>(rows * ses));
          const uint32_t o = in ? ri * ses : kOob;
          const uint32_t oh = in && ses == 4 ? ri * ses + 2 : kOob;
          ep[u] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(o), 0, 0));
          ep[2 * WT + u] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(oh), 0, 0));
        }
        const void* bp = lin ? p.bl : p.b;
        const __amdgpu_buffer_rsrc_t rb_ = make_rsrc(bp ? static_cast<const uint8_t*>(bp) + e * rows * 2 : nullptr,
                                                     bp ? static_cast<uint32_t>(rows * 2) : 0u);
        const uint32_t ob = in && (FC1 || s == 0) ? ri * 2 : kOob;
        ep[WT + u] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(rb_, static_cast<int>(ob), 0, 0));
      }
    };
    auto ep_scale = [&](const uint32_t* ep, int u) -> float {
      if constexpr (SM != kScaleChan) {
        (void)ep;
        (void)u;
        return 1.0f;
      } else {
        const uint32_t r = ep[u];
        if (ses == 4) return __uint_as_float(r | (ep[2 * WT + u] << 16));
        if (p.scale_type == MOE_ELEM_FLOAT16) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r)));
        return bf16_to_f32(static_cast<uint16_t>(r));
      }
    };
    auto ep_bias = [&](uint32_t r) -> float {
      if constexpr (AT::kId == 10) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r)));
      else return bf16_to_f32(static_cast<uint16_t>(r));
    };

    // scales, bias and activation of tile tl; store
    auto finish = [&](int tl, const floatx4_t* v, const uint32_t* ep) {
      const int ft = f0 + tl;
      if constexpr (!FC1) {
#pragma unroll
        for (int u = 0; u < WT; ++u) {
          const int f = ft * (16 * FT) + fo[u];
          if (f >= nfeat) continue;
          float* o = static_cast<float*>(p.out) + (static_cast<int64_t>(s) * p.out_rows + row0) * nfeat + f;
          const float sc = ep_scale(ep, u), bi = ep_bias(ep[WT + u]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = 4 * g + r;
            if (m < nrows) o[m * nfeat] = (v[u][r] - ctot[r]) * sc + bi;
          }
        }
      } else {
#pragma unroll
        for (int fi = 0; fi < FT; ++fi) {
          const int ug = fi, ul = GATED ? fi + FT : fi;
          const int f = ft * (16 * FT) + fo[fi];
          if (f >= nfeat) continue;
          typename AT::storage* o = static_cast<typename AT::storage*>(p.out) + static_cast<int64_t>(row0) * nfeat + f;
          const float sg = ep_scale(ep, ug), bg = ep_bias(ep[WT + ug]);
          const float sl = ep_scale(ep, ul), bl = ep_bias(ep[WT + ul]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = 4 * g + r;
            if (m >= nrows) continue;
            const float vg = (v[ug][r] - ctot[r]) * sg + bg;
            const float vl = GATED ? (v[ul][r] - ctot[r]) * sl + bl : 0.0f;
            o[m * nfeat] = from_f32<AT>(apply_act<true>(vg, vl, GATED, p.activation, p.alpha, p.beta, p.limit));
          }
        }
      }
    };

    // ---- this wave's run of blocks ----
    int lead_tl = -1, trail_tl = -1, seg0 = 0;
    uint32_t ep[3 * WT];
    int tl = b0 / bpt, cb = b0 - tl * bpt;
    // The waves of a SIMD compete for its issue slots, which go to the
    // oldest wave among those of the highest priority.  With equal
    // priorities the oldest wave races ahead and the youngest finishes its
    // run long after, streaming alone; so each wave's priority follows the
    // share of its run still ahead of it, and a wave that lags catches up.
    const int run = b1 - b0;
    auto set_prio = [&](int bj) {
      const int rem = b1 - bj;
      const int pr = rem * 4 > run * 3 ? 3 : (rem * 2 > run ? 2 : (rem * 4 > run ? 1 : 0));
      if (pr == 3) __builtin_amdgcn_s_setprio(3);
      else if (pr == 2) __builtin_amdgcn_s_setprio(2);
      else if (pr == 1) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    };
    for (int bj = b0; bj < b1; ++bj) {
      set_prio(bj);
      if (cb == 0 || bj == b0) {
#pragma unroll
        for (int u = 0; u < WT; ++u) acc[u] = floatx4_t{0.f, 0.f, 0.f, 0.f};
        seg0 = cb;
        load_ep(tl, ep);
      }
      if constexpr (kTileScales) {
        // chunk c = 4 cb + d of the slice: lane group c / 8 = cb / 2, dword
        // (c % 8) / 2 = 2 (cb % 2) + d / 2, half d % 2
        const int src = (col + 16 * (cb >> 1)) * 4;
        const bool odd = cb & 1;
#pragma unroll
        for (int u = 0; u < WT; ++u) {
          bsc[u][0] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(odd ? tsr[u][2] : tsr[u][0])));
          bsc[u][1] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(odd ? tsr[u][3] : tsr[u][1])));
        }
      }
      // the next block (past the run's end: loads that read nothing)
      const int ntl = cb + 1 == bpt ? tl + 1 : tl, ncb = cb + 1 == bpt ? 0 : cb + 1;
      uint32_t woff[WT], soff[WT];
      tile_offs(ntl, woff, soff);
      if (bj + 1 >= b1) {
#pragma unroll
        for (int u = 0; u < WT; ++u) woff[u] = soff[u] = kOob;
      }
      // chunks in groups of kFetch: compute the group, then issue the loads
      // of the same slots back to back
#pragma unroll
      for (int h = 0; h < PD; h += kFetch) {
#pragma unroll
        for (int d = h; d < h + kFetch; ++d) {
          compute(cb * PD + d, d);
          // keep each chunk's LDS reads and dequantisation next to its MFMAs
          __builtin_amdgcn_sched_barrier(0);
        }
        // the next tile's scales, once this block (the last of its tile) has
        // read the current ones, ahead of the weights so that the next
        // block's wait for them leaves the weights in flight
        if (kTileScales && h + kFetch == PD && cb == bpt - 1 && bj + 1 < b1) fetch_tsc(tl + 1);
#pragma unroll
        for (int d = h; d < h + kFetch; ++d) fetch(ncb * PD + d, woff, soff, ring[d]);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (cb == bpt - 1 || bj == b1 - 1) {
        if (seg0 == 0 && cb == bpt - 1) {
          finish(tl, acc, ep);
        } else if (seg0 != 0) {
#pragma unroll
          for (int u = 0; u < WT; ++u) lead[u] = acc[u];
          lead_tl = tl;
        } else {
          trail_tl = tl;
        }
      }
      tl = ntl;
      cb = ncb;
    }

    __builtin_amdgcn_s_setprio(0);
    // ---- split tiles: lead partials to LDS, owners add them in wave order ----
    __syncthreads();  // every wave is done with the activation slice
    if (lead_tl >= 0) {
#pragma unroll
      for (int u = 0; u < WT; ++u)
        *reinterpret_cast<floatx4_t*>(slots + ((wave * WT + u) * 64 + lane) * 4) = lead[u];
    }
    __syncthreads();
    if (trail_tl >= 0) {
      const int tile_end = (trail_tl + 1) * bpt;
      for (int w = wave + 1; w < NW; ++w) {
        const int wb0 = nb * w / NW, wb1 = nb * (w + 1) / NW;
        if (wb0 >= tile_end) break;
        if (wb1 > wb0) {
#pragma unroll
          for (int u = 0; u < WT; ++u) acc[u] += *reinterpret_cast<const floatx4_t*>(slots + ((w * WT + u) * 64 + lane) * 4);
        }
      }
      finish(trail_tl, acc, ep);
    }
    __syncthreads();  // slots read before the next group stages
    t += ntl;
  }
}

int stream_grid(int nw);

template <typename AT, int WF, int SM, typename ST, int NSC, bool FC1, bool GATED>
hipError_t launch_stream(const StreamStage& ss, hipStream_t stream) {
  using G = SGeo<WF, GATED>;
  auto kern = ss.s.tiled ? gemv_stream_kernel<AT, WF, SM, ST, NSC, FC1, GATED, true>
                         : gemv_stream_kernel<AT, WF, SM, ST, NSC, FC1, GATED, false>;
  const size_t lds = stream_lds_bytes(ss.ksc, ss.ngroups, G::NW, ss.route_ints);  // <= 157 KB
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(stream_grid(G::NW))), dim3(G::NW * 64), lds, stream, ss);
  return hipGetLastError();
}

template <typename AT, int WF, int SM, typename ST, int NSC>
hipError_t launch_stream_kinds(const StreamStage& ss, bool fc1, bool gated, hipStream_t stream) {
  if (!fc1) return launch_stream<AT, WF, SM, ST, NSC, false, false>(ss, stream);
  if (gated) return launch_stream<AT, WF, SM, ST, NSC, true, true>(ss, stream);
  return launch_stream<AT, WF, SM, ST, NSC, true, false>(ss, stream);
}

// Dispatch over activation type, scale mode, scale type and scales per lane.
template <int WF>
hipError_t launch_stream_fmt(const StreamStage& ss, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream) {
  const bool bf = a.act_type == MOE_ELEM_BFLOAT16;
  if constexpr (WF == kDense) {
    return bf ? launch_stream_kinds<BF16, WF, kScaleNone, F16, 1>(ss, fc1, gated, stream)
              : launch_stream_kinds<F16, WF, kScaleNone, F16, 1>(ss, fc1, gated, stream);
  } else {
    const int sm = scale_mode(a);
    if (sm == kScaleChan)
      return bf ? launch_stream_kinds<BF16, WF, kScaleChan, F16, 1>(ss, fc1, gated, stream)
                : launch_stream_kinds<F16, WF, kScaleChan, F16, 1>(ss, fc1, gated, stream);
    auto by_st = [&](auto at_tag, auto sm_tag, auto nsc_tag) -> hipError_t {
      using AT = decltype(at_tag);
      constexpr int SM = decltype(sm_tag)::value, NSC = decltype(nsc_tag)::value;
      switch (a.scale_type) {
        case MOE_ELEM_FLOAT: return launch_stream_kinds<AT, WF, SM, F32, NSC>(ss, fc1, gated, stream);
        case MOE_ELEM_BFLOAT16: return launch_stream_kinds<AT, WF, SM, BF16, NSC>(ss, fc1, gated, stream);
        default: return launch_stream_kinds<AT, WF, SM, F16, NSC>(ss, fc1, gated, stream);
      }
    };
    using BLK = std::integral_constant<int, kScaleBlock>;
    using FOLD = std::integral_constant<int, kScaleFold>;
    using ONE = std::integral_constant<int, 1>;
    using TWO = std::integral_constant<int, 2>;
    using FOUR = std::integral_constant<int, 4>;
    if (sm == kScaleBlock) {
      // block 128 and K a multiple of 512: 4 chunks' scales are one aligned load
      if (a.block_size == 128 && ss.s.K % 512 == 0) return bf ? by_st(BF16{}, BLK{}, FOUR{}) : by_st(F16{}, BLK{}, FOUR{});
      return bf ? by_st(BF16{}, BLK{}, ONE{}) : by_st(F16{}, BLK{}, ONE{});
    }
    if constexpr (WF == kInt4) {
      if (a.mx) {  // MXFP4: E8M0 scales of block 32
        return bf ? launch_stream_kinds<BF16, WF, kScaleMx, E8M0, 1>(ss, fc1, gated, stream)
                  : launch_stream_kinds<F16, WF, kScaleMx, E8M0, 1>(ss, fc1, gated, stream);
      }
    }
    // blocks of 32 / 64 with a biased operand form: step scales
    using STEP = std::integral_constant<int, kScaleStep>;
    if (a.block_size == 32 || a.block_size == 64) {
      if constexpr (WF == kInt4) {
        return bf ? by_st(BF16{}, STEP{}, ONE{}) : by_st(F16{}, STEP{}, ONE{});
      } else {
        // int8: biased operands with fp16 activations only
        if (!bf) return by_st(F16{}, STEP{}, ONE{});
      }
    }
    // folded block scales: a lane's 32 k span two blocks of 16
    if (a.block_size == 16) return bf ? by_st(BF16{}, FOLD{}, TWO{}) : by_st(F16{}, FOLD{}, TWO{});
    return bf ? by_st(BF16{}, FOLD{}, ONE{}) : by_st(F16{}, FOLD{}, ONE{});
  }
}

hipError_t launch_stream_int4(const StreamStage& ss, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream);
hipError_t launch_stream_int8(const StreamStage& ss, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream);
hipError_t launch_stream_dense(const StreamStage& ss, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream);

}  // namespace decode
}  // namespace moe
