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
// current block is consumed, and a group's first block is requested before
// its activation slice is staged.  Block scales travel in the ring beside
// the weights.
//
// Biased operands: int8/int4 weights enter the MFMA with their zero point
// and magic-exponent bias still in (1024 + q for fp16, 128 + q for bf16),
// and the bias is removed per chunk (block scales) or once (per-channel
// scales) with per-row activation sums computed while staging.  For int4
// with fp16 activations, the nibbles are placed into the 16-bit lanes with
// two and-or operations per pair: the odd nibbles land 4 bits up (1024 +
// 16 q), so the activations at those k are staged divided by 16 (exact),
// and the k order inside each 8-k step is (0 4 1 5 2 6 3 7) in both
// operands.
//
// fc1 needs the whole K in one slice (its activation needs the full sum);
// fc2 writes one fp32 plane of y2 per K slice, which the finalize pass sums
// in order.
#pragma once

#include <type_traits>

#include "moe_expert_decode.h"

namespace moe {
namespace decode {

constexpr int kStreamRows = 16;       // token rows staged (the MFMA M dimension)
constexpr int kStreamMaxChunks = 36;  // K chunks of one staged slice (16 x 36 x 256 B of LDS)
constexpr int kStreamFetch = 4;       // chunks whose loads are issued back to back

// Chunks per block (= register ring depth); a K slice is a whole number of
// blocks.  8 only for gated int4 (fc1 + fc3): fc2's 7 KB rows measured 6%
// faster with 4.
inline int stream_pd(int wfmt, bool gated) { return wfmt == kInt4 && gated ? 8 : 4; }

struct StreamStage {
  Stage s;
  int32_t ksc;      // chunks per K slice (multiple of the ring depth; the last slice is padded)
  int32_t nslices;  // K slices (fc2 partial planes)
  int32_t E;        // experts
  int32_t ngroups;  // bound on the row groups of all experts: E + T*k/16
};

template <int WF, bool GATED>
struct SGeo {
  static constexpr int kVecs = WF == kInt4 ? 1 : (WF == kInt8 ? 2 : 4);  // u32x4 per tile per chunk
  static constexpr int kLaneBytes = 16 * kVecs;                           // bytes per 32 k of a row
  static constexpr int FT = GATED ? 1 : 2;                                // 16-feature tiles per tile
  static constexpr int WT = 2;                                            // 16-row weight tiles per tile
  static constexpr int NW = WF == kDense ? 8 : 12;                         // waves per workgroup
  static constexpr int PD = WF == kInt4 && GATED ? 8 : 4;                         // ring depth (chunks)
};

// Raw block scales of one lane: NSC consecutive elements in one load.
template <typename ST, int NSC>
struct ScaleRaw {
  static constexpr int kBytes = NSC * static_cast<int>(sizeof(typename ST::storage));
  using type = std::conditional_t<(kBytes > 8), u32x4_t, std::conditional_t<(kBytes > 4), u32x2_t, uint32_t>>;
  __device__ static __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (kBytes == 2) {
      return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(off), 0, 0));
    } else if constexpr (kBytes == 4) {
      return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, 0);
    } else if constexpr (kBytes == 8) {
      return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(off), 0, 0));
    } else {
      return bload16(r, off);
    }
  }
  __device__ static __forceinline__ float elem(type v, int i) {
    if constexpr (std::is_same_v<ST, F32>) {
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

// Bytes of dynamic LDS of the stream kernel (ngroups: row-group list entries).
inline size_t stream_lds_bytes(int ksc, int ngroups, int nw) {
  const size_t ex = (static_cast<size_t>(ngroups) * 4 + 15) / 16 * 16;
  const size_t act = static_cast<size_t>(kStreamRows) * (static_cast<size_t>(ksc) * 256 + 16) +
                     static_cast<size_t>(ksc) * kStreamRows * 4;
  const size_t slots = static_cast<size_t>(nw) * 2 * 64 * 16;
  return ex + std::max(act, slots);
}

// NSC: folded scales (block 16/32/64): elements per lane and chunk (2 for
// block 16); block scales: 4 = one load brings the scales of 4 chunks
// (block 128, K a multiple of 512), 1 = one load per chunk.
template <typename AT, int WF, int SM, typename ST, int NSC, bool FC1, bool GATED>
__global__ void __launch_bounds__((SGeo<WF, GATED>::NW * 64), 1) gemv_stream_kernel(StreamStage ss) {
  using G = SGeo<WF, GATED>;
  constexpr int NW = G::NW, NT = NW * 64, WT = G::WT, FT = G::FT, PD = G::PD, LB = G::kLaneBytes;
  constexpr bool kBiased = Biased<AT, WF>::kOk && (SM == kScaleBlock || SM == kScaleChan);
  constexpr bool kSplit = kBiased && WF == kInt4 && AT::kId == 10;
  constexpr bool kRingScales = SM == kScaleBlock || SM == kScaleFold;
  constexpr bool kGroupScales = SM == kScaleBlock && NSC == 4;
  static_assert(PD % kStreamFetch == 0, "a block is whole fetch groups");
  using SR = ScaleRaw<ST, NSC>;
  using CK = SChunk<WF, GATED, SR, kRingScales>;
  constexpr int kEs = static_cast<int>(sizeof(typename ST::storage));
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int wcount[NW];
  const Stage& p = ss.s;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, g = lane >> 4;
  const int ksc = ss.ksc, nsl = ss.nslices, E = ss.E;
  const int pitch = ksc * 256 + 16;
  int* exl = reinterpret_cast<int*>(smem);  // row groups: expert | (group << 16), ascending
  uint8_t* region = smem + (ss.ngroups * 4 + 15) / 16 * 16;
  uint8_t* xs = region;                                         // [16][pitch] activation slice
  float* corr = reinterpret_cast<float*>(region + 16 * pitch);  // [ksc][16] bias sums per chunk and row
  float* slots = reinterpret_cast<float*>(region);              // [NW][WT][64] float4, after the compute

  // ---- row groups: each routed expert's rows in groups of 16 (the MFMA M);
  // an expert with more rows streams its weights once per group.
  // exl[0 .. e_act) ----
  int e_act = 0;
  for (int base = 0; base < E; base += NT) {
    const int e = base + tid;
    const int cnt = e < E ? p.offsets[e + 1] - p.offsets[e] : 0;
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

  // ---- this workgroup's tiles ----
  const int64_t K = p.K;
  const int nchunks = static_cast<int>((K + kChunk - 1) / kChunk);
  const int ktail = static_cast<int>(K - static_cast<int64_t>(nchunks - 1) * kChunk);
  const uint32_t rb = static_cast<uint32_t>((K / 32) * LB);  // bytes of one weight row
  const int nft = static_cast<int>((p.nfeat + 16 * FT - 1) / (16 * FT));
  const int64_t per_a = static_cast<int64_t>(nsl) * nft;
  const int64_t ttot = e_act * per_a;
  const int64_t t_beg = ttot * blockIdx.x / gridDim.x;
  const int64_t t_end = ttot * (blockIdx.x + 1) / gridDim.x;
  const int bpt = ksc / PD;  // blocks per tile
  int bshift = 0;
  uint32_t nblk = 0;
  if constexpr (kRingScales) {
    bshift = __builtin_ctzll(static_cast<uint64_t>(p.block_size));
    nblk = static_cast<uint32_t>(K >> bshift);
  }
  const __amdgpu_buffer_rsrc_t rs_x = make_rsrc(p.in, static_cast<uint32_t>(p.in_rows * K * 2));
  const int act_t = AT::kId;
  const int nfeat = static_cast<int>(p.nfeat);

  // Weight row of feature f in weight tile u: f * rmul + radd[u] (gate rows
  // 2f / linear rows 2f + 1 when interleaved; linear rows f + nfeat when
  // chunked).  Lane constants: feature offset fo[u] inside a tile, and the
  // row's byte offsets with the tile index factored out (32-bit: one
  // expert's weights are below 2 GiB).
  const int rmul = (FC1 && GATED && p.gate_mode == kGateInterleaved) ? 2 : 1;
  int fo[WT], rowb[WT];
  uint32_t wb[WT], sb[WT];
#pragma unroll
  for (int u = 0; u < WT; ++u) {
    const bool lin = GATED && u >= FT;
    const int radd = !lin ? 0 : (p.gate_mode == kGateInterleaved ? 1 : (p.gate_mode == kGateChunked ? nfeat : 0));
    fo[u] = (u % FT) * 16 + col;
    rowb[u] = fo[u] * rmul + radd;
    wb[u] = static_cast<uint32_t>(rowb[u]) * rb + g * LB;
    sb[u] = static_cast<uint32_t>(rowb[u]) * nblk * kEs;
  }
  const uint32_t tws = static_cast<uint32_t>(16 * FT * rmul) * rb;          // weight bytes per tile step
  const uint32_t tss = static_cast<uint32_t>(16 * FT * rmul) * nblk * kEs;  // scale bytes per tile step
  // masks of the int4 nibble split, kept in VGPRs so that each output pair
  // is one v_and_or_b32
  uint32_t m_lo = 0x000F000Fu, m_hi = 0x00F000F0u;
  if constexpr (kSplit) {
    asm volatile("" : "+v"(m_lo));
    asm volatile("" : "+v"(m_hi));
  }

  for (int64_t t = t_beg; t < t_end;) {
    const int a = static_cast<int>(t / per_a);
    const int rem = static_cast<int>(t - a * per_a);
    const int s = rem / nft, f0 = rem - s * nft;
    const int ntl = static_cast<int>(t_end - t < nft - f0 ? t_end - t : nft - f0);
    const int nb = ntl * bpt;
    const int b0 = nb * wave / NW, b1 = nb * (wave + 1) / NW;
    const int ent = __builtin_amdgcn_readfirstlane(exl[a]);
    const int e = ent & 0xFFFF;
    const int row0 = __builtin_amdgcn_readfirstlane(p.offsets[e]) + (ent >> 16) * kStreamRows;
    const int cnt = __builtin_amdgcn_readfirstlane(p.offsets[e + 1]) - row0;
    const int nrows = cnt < kStreamRows ? cnt : kStreamRows;
    const int cs0 = s * ksc;  // first chunk of the slice

    const __amdgpu_buffer_rsrc_t rs_g = make_rsrc(p.w + static_cast<int64_t>(e) * p.w_rows * rb,
                                                  static_cast<uint32_t>(p.w_rows * rb));
    const __amdgpu_buffer_rsrc_t rs_l = make_rsrc(p.wl + static_cast<int64_t>(e) * p.wl_rows * rb,
                                                  static_cast<uint32_t>(p.wl_rows * rb));
    __amdgpu_buffer_rsrc_t ss_g = rs_g, ss_l = rs_l;
    if constexpr (kRingScales) {
      ss_g = make_rsrc(static_cast<const uint8_t*>(p.s) + static_cast<int64_t>(e) * p.w_rows * nblk * kEs,
                       static_cast<uint32_t>(p.w_rows * nblk * kEs));
      ss_l = make_rsrc(static_cast<const uint8_t*>(p.sl) + static_cast<int64_t>(e) * p.wl_rows * nblk * kEs,
                       static_cast<uint32_t>(p.wl_rows * nblk * kEs));
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
    auto fetch = [&](int cl, const uint32_t* woff, const uint32_t* soff, CK& d) {
      const int cg = cs0 + cl;
      // padding chunks past K and the missing lanes of a partial last chunk
      // read nothing (branch-free: one compare against the chunk's valid k)
      const int kval = cg < nchunks - 1 ? kChunk : (cg == nchunks - 1 ? ktail : 0);
      const uint32_t oob = 32 * g + 32 <= kval ? 0u : kOob;
      const uint32_t wc = static_cast<uint32_t>(cg) * (4 * LB);
#pragma unroll
      for (int u = 0; u < WT; ++u) {
        const uint32_t o = (woff[u] + wc) | oob;
#pragma unroll
        for (int v = 0; v < G::kVecs; ++v) d.w[u][v] = bload16(GATED && u >= FT ? rs_l : rs_g, o + 16 * v);
        if constexpr (kRingScales) {
          const uint32_t kk = static_cast<uint32_t>(cg) * kChunk + (SM == kScaleFold ? 32 * g : 0);
          // a block scale multiplies the whole chunk's sum (every lane group
          // of the MFMA output), so only a chunk past K reads none
          const uint32_t so = (soff[u] + (kk >> bshift) * kEs) | (SM == kScaleFold ? oob : (cg < nchunks ? 0u : kOob));
          // grouped: the first chunk of each group of 4 loads all 4 scales
          if (!kGroupScales || (cl & 3) == 0) d.sc[u] = SR::load(GATED && u >= FT ? ss_l : ss_g, so);
        }
      }
    };

    // ---- first block of this wave's run, then the activation slice ----
    if (b0 < b1) {
      uint32_t woff[WT], soff[WT];
      const int tl = b0 / bpt, cb = b0 - tl * bpt;
      tile_offs(tl, woff, soff);
#pragma unroll
      for (int d = 0; d < PD; ++d) fetch(cb * PD + d, woff, soff, ring[d]);
    }
    {
      // rounds of kJ 16-byte pieces per thread: loads first, then transform and store
      constexpr int kJ = 3;
      const int per_row = ksc * 16;  // 16-byte pieces per row
      const int npc = nrows * per_row;
      for (int i0 = 0; i0 < npc; i0 += NT * kJ) {
        u32x4_t xv[kJ];
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
          const int i = i0 + tid + NT * j;
          uint32_t off = kOob;
          if (i < npc) {
            const int m = i / per_row, r = i - m * per_row;
            const int64_t k = static_cast<int64_t>(cs0 + (r >> 4)) * kChunk + (r & 15) * 8;
            const int64_t src = FC1 ? p.perm[row0 + m] / p.topk : row0 + m;
            if (k < K) off = static_cast<uint32_t>((src * K + k) * 2);
          }
          xv[j] = bload16(rs_x, off);
        }
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
          const int i = i0 + tid + NT * j;
          u32x4_t y = xv[j];
          float cs = 0.0f;
          if constexpr (kSplit) {
            const half2_t q16 = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
            const u32x4_t x = xv[j];
            y[0] = __builtin_amdgcn_perm(x[2], x[0], 0x05040100u);
            y[1] = h2_bits(bits_h2(__builtin_amdgcn_perm(x[2], x[0], 0x07060302u)) * q16);
            y[2] = __builtin_amdgcn_perm(x[3], x[1], 0x05040100u);
            y[3] = h2_bits(bits_h2(__builtin_amdgcn_perm(x[3], x[1], 0x07060302u)) * q16);
            float lo = 0.0f, hi = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const half2_t h = bits_h2(y[q]);
              const float v = static_cast<float>(h[0]) + static_cast<float>(h[1]);
              if (q & 1) hi += v;
              else lo += v;
            }
            cs = 1032.0f * lo + 1152.0f * hi;
          } else if constexpr (kBiased) {
            float sum = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              if constexpr (AT::kId == 10) {
                const half2_t h = bits_h2(y[q]);
                sum += static_cast<float>(h[0]) + static_cast<float>(h[1]);
              } else {
                sum += __uint_as_float(y[q] << 16) + __uint_as_float(y[q] & 0xFFFF0000u);
              }
            }
            cs = Biased<AT, WF>::kOffset * sum;
          }
          if constexpr (kBiased) {
            // the 16 pieces of one (row, chunk) sit in 16 consecutive lanes
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) cs += __shfl_xor(cs, o, kWave);
          }
          if (i < npc) {
            const int m = i / per_row, r = i - m * per_row;
            *reinterpret_cast<u32x4_t*>(xs + m * pitch + r * 16) = y;
            if (kBiased && (r & 15) == 0) corr[(r >> 4) * kStreamRows + m] = cs;
          }
        }
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

    auto compute = [&](int cl, int slot) {
      const CK& d = ring[slot];
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
          const float sc = kGroupScales ? SR::elem(ring[slot & ~3].sc[u], slot & 3) : SR::elem(d.sc[u], 0);
          acc[u] += (tmp[u] - cr) * sc;
        }
      }
    };

    // Per-channel scales and biases of tile tl (ep[u], ep[WT + u] for weight
    // tile u), requested when a tile's first block starts so that finishing
    // it never waits behind the weight stream.
    auto load_ep = [&](int tl, float* ep) {
      const int ft = f0 + tl;
#pragma unroll
      for (int u = 0; u < WT; ++u) {
        const bool lin = GATED && u >= FT;
        ep[u] = 1.0f;
        ep[WT + u] = 0.0f;
        if (ft * (16 * FT) + fo[u] < nfeat) {
          const int64_t ri = static_cast<int64_t>(e) * (lin ? p.wl_rows : p.w_rows) + ft * (16 * FT * rmul) + rowb[u];
          if constexpr (SM == kScaleChan) ep[u] = load_any(lin ? p.sl : p.s, p.scale_type, ri);
          const void* bp = lin ? p.bl : p.b;
          if (bp && (FC1 || s == 0)) ep[WT + u] = load_any(bp, act_t, ri);
        }
      }
    };

    // scales, bias and activation of tile tl; store
    auto finish = [&](int tl, const floatx4_t* v, const float* ep) {
      const int ft = f0 + tl;
      if constexpr (!FC1) {
#pragma unroll
        for (int u = 0; u < WT; ++u) {
          const int f = ft * (16 * FT) + fo[u];
          if (f >= nfeat) continue;
          float* o = static_cast<float*>(p.out) + (static_cast<int64_t>(s) * p.out_rows + row0) * nfeat + f;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = 4 * g + r;
            if (m < nrows) o[m * nfeat] = (v[u][r] - ctot[r]) * ep[u] + ep[WT + u];
          }
        }
      } else {
#pragma unroll
        for (int fi = 0; fi < FT; ++fi) {
          const int ug = fi, ul = GATED ? fi + FT : fi;
          const int f = ft * (16 * FT) + fo[fi];
          if (f >= nfeat) continue;
          typename AT::storage* o = static_cast<typename AT::storage*>(p.out) + static_cast<int64_t>(row0) * nfeat + f;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = 4 * g + r;
            if (m >= nrows) continue;
            const float vg = (v[ug][r] - ctot[r]) * ep[ug] + ep[WT + ug];
            const float vl = GATED ? (v[ul][r] - ctot[r]) * ep[ul] + ep[WT + ul] : 0.0f;
            o[m * nfeat] = from_f32<AT>(apply_act<true>(vg, vl, GATED, p.activation, p.alpha, p.beta, p.limit));
          }
        }
      }
    };

    // ---- this wave's run of blocks ----
    int lead_tl = -1, trail_tl = -1, seg0 = 0;
    float ep[2 * WT];
    int tl = b0 / bpt, cb = b0 - tl * bpt;
    for (int b = b0; b < b1; ++b) {
      if (cb == 0 || b == b0) {
#pragma unroll
        for (int u = 0; u < WT; ++u) acc[u] = floatx4_t{0.f, 0.f, 0.f, 0.f};
        seg0 = cb;
        load_ep(tl, ep);
      }
      // next block of the run (past its end: loads that read nothing)
      const int ntl = cb + 1 == bpt ? tl + 1 : tl, ncb = cb + 1 == bpt ? 0 : cb + 1;
      uint32_t woff[WT], soff[WT];
      tile_offs(ntl, woff, soff);
      if (b + 1 >= b1) {
#pragma unroll
        for (int u = 0; u < WT; ++u) woff[u] = soff[u] = kOob;
      }
      // chunks in groups of kStreamFetch: compute the group, then issue the
      // loads of the same slots of the next block back to back (one row's
      // consecutive 64-byte pieces reach the memory controller together)
#pragma unroll
      for (int h = 0; h < PD; h += kStreamFetch) {
#pragma unroll
        for (int d = h; d < h + kStreamFetch; ++d) {
          compute(cb * PD + d, d);
          // keep each chunk's LDS reads and dequantisation next to its MFMAs
          __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int d = h; d < h + kStreamFetch; ++d) fetch(ncb * PD + d, woff, soff, ring[d]);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (cb == bpt - 1 || b == b1 - 1) {
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
  auto kern = gemv_stream_kernel<AT, WF, SM, ST, NSC, FC1, GATED>;
  const size_t lds = stream_lds_bytes(ss.ksc, ss.ngroups, G::NW);  // <= 152 KB + the group list
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
