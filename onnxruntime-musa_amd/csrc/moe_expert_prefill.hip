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
//  * Tile order: groups of 2-4 weight tiles (plan_grid) are swept across all
//    row tiles of all experts, and each XCD (hardware workgroup ids are
//    dealt to the 8 XCDs round-robin) receives a contiguous range of that
//    order, so the workgroups resident on one XCD share a few weight tiles
//    and their row tiles' activations in its L2.
//  * fc2 may split K across workgroups; the partial sums land in separate
//    fp32 planes of y2 that finalize adds in a fixed order.
#include <algorithm>
#include <climits>
#include <type_traits>

#include "moe_dequant.h"
#include "moe_launch.h"

namespace moe {
namespace {

constexpr int BM = 128;           // rows per workgroup tile
constexpr int kMT = BM / 32;      // 32-row blocks per wave (every wave covers all rows)
constexpr int kNT = 2;            // 32-wide weight blocks per wave
constexpr int BN = 4 * kNT * 32;  // weight rows per workgroup tile
constexpr int kXcds = 8;

enum PScale : int { kPsNone = 0, kPsChan = 1, kPsBlock = 2 };

template <int WF>
struct PG {
  static constexpr int BK = WF == kDense ? 64 : 128;  // k per stage
  static constexpr int KH = BK / 2;                    // k per lane half per stage
  static constexpr int NSTEP = KH / 8;                 // MFMA steps per stage
  static constexpr int EBITS = WF == kInt4 ? 4 : (WF == kInt8 ? 8 : 16);
  static constexpr int BVEC = KH * EBITS / 8 / 16;     // 16-byte weight loads per block per stage
  static constexpr int ROWB = BK * 2;                  // LDS bytes of one activation row per stage
  static constexpr int ABUF = BM * ROWB;               // one staged activation stage
  static constexpr int PIECES = ROWB / 16;             // 16-byte pieces per row per stage
  static constexpr int RPI = 1024 / ROWB;              // rows per 1 KB LDS-load instruction
  static constexpr int APW = BM / RPI / 4;             // LDS-load instructions per wave per stage
  // XOR swizzle of a row's 16-byte pieces: the 8 rows one 128-byte LDS
  // cycle of an operand read touches fall into different bank groups
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
  int32_t gn;       // weight tiles swept together over the row tiles
  int32_t ngroups;  // ceil(ntiles / gn)
  int32_t ksplit;   // K splits (partial planes of the output)
  int32_t out_half; // fc2 with one plane: y2 stored in the activation type
  int32_t kstages;  // stages per K split
  int32_t tiled;    // weights tile-major (int4 / int8 / 16-bit), K padded to whole chunks of 128
  int32_t deint;    // fused interleaved fc1 stored de-interleaved (gate rows, then linear rows)
  int32_t stiled;   // block scales (block 32 / 64) tile-major, rows as the weights
  int64_t out_rows;
  void* out;  // fc1: act [rows, nfeat] (AT); fc2: y2 [ksplit][rows, nfeat] fp32
};

// Place in the tile order of hardware workgroup b when n of the grid's
// workgroups have a tile: XCD x (= b mod 8) takes the x-th contiguous eighth
// of [0, n) with its first workgroups; -1 for the rest, which exit.
__device__ __forceinline__ int remap_xcd(int b, int n) {
  const int per = n / kXcds, rem = n % kXcds;
  const int x = b % kXcds, local = b / kXcds;
  if (local >= per + (x < rem ? 1 : 0)) return -1;
  return x < rem ? x * (per + 1) + local : rem * (per + 1) + (x - rem) * per + local;
}

// MFMA layout (v_mfma_f32_32x32x16): lane l = 32 h + r holds A row r / B
// column r for k group h (8 k); D element (row 8 (q / 4) + 4 h + q % 4,
// column r) in accumulator register q.  Within a stage, lane half h covers
// k in [KH h, KH h + KH) and feeds k = KH h + 8 s .. + 7 to MFMA step s; the
// activation operand is read with the same assignment.
//
// NSC: block scales per lane half and stage (KH / block_size, at least 1).
template <typename AT, int WF, int SM, typename ST, int NSC, bool FC1, bool GATED>
__global__ void __launch_bounds__(256, 2) prefill_kernel(PStage p) {
  using G = PG<WF>;
  constexpr int BK = G::BK, KH = G::KH, NSTEP = G::NSTEP, BVEC = G::BVEC;
  constexpr bool kFold = SM == kPsBlock;
  // two stage buffers as separate objects, so the compiler can tell that the
  // LDS loads filling one never alias the reads of the other
  __shared__ __attribute__((aligned(1024))) uint8_t sA0[G::ABUF];
  __shared__ __attribute__((aligned(1024))) uint8_t sA1[G::ABUF];

  // ---- tile of this workgroup ----
  // The grid is sized for the most row tiles a routing can give (mslots);
  // the order runs over the row tiles this routing gave (tile_offsets[E]),
  // so that every XCD's share is a full eighth of the real work and the
  // surplus workgroups exit at once on every XCD alike (with the bound, the
  // empty row slots sat at the end of each group, unevenly over the XCDs).
  // Measured per layer: Qwen3 fp16 T=8192 -3.7%, gpt-oss int4 T=8192
  // -2.6%, MXFP4 -1.6%, Mixtral int4 T=512 -3.6%; Mixtral int4/int8
  // T=4096 +1%.
  // Up to 255 experts, each wave holds tile_offsets[0..E] in its lanes (one
  // round of independent loads); the expert of a row tile is then a ballot
  // count, not a chain of dependent loads.
  constexpr int kTc = 4;  // 64-entry chunks held
  const int tl64 = threadIdx.x & 63;
  int tov[kTc];
  const bool held = p.E < kTc * 64;
#pragma unroll
  for (int c = 0; c < kTc; ++c) {
    const int i = c * 64 + tl64;
    tov[c] = held && i <= p.E ? p.tile_offsets[i] : INT_MAX;
  }
  int mt;
  if (held) {
    const int ce = p.E >> 6;
    const int v = ce == 0 ? tov[0] : (ce == 1 ? tov[1] : (ce == 2 ? tov[2] : tov[3]));
    mt = __builtin_amdgcn_readlane(v, p.E & 63);
  } else {
    mt = p.tile_offsets[p.E];
  }
  const int per_split = p.ngroups * mt * p.gn;
  const int L = remap_xcd(static_cast<int>(blockIdx.x), p.ksplit * per_split);
  if (L < 0) return;
  const int ks = L / per_split;
  const int r0 = L % per_split;
  const int nin = r0 % p.gn;
  const int mslot = (r0 / p.gn) % mt;
  const int ntile = (r0 / p.gn / mt) * p.gn + nin;
  if (ntile >= p.ntiles) return;
  int e;  // last expert with tile_offsets[e] <= mslot (the entries are non-decreasing)
  if (held) {
    int n = 0;
#pragma unroll
    for (int c = 0; c < kTc; ++c) n += __popcll(__ballot(tov[c] <= mslot));
    e = n - 1;
  } else {
    int lo = 0, hi = p.E;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (p.tile_offsets[mid] <= mslot) lo = mid;
      else hi = mid;
    }
    e = lo;
  }
  const int row_begin = p.offsets[e] + (mslot - p.tile_offsets[e]) * BM;
  const int rows = min(BM, p.offsets[e + 1] - row_begin);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS-load bases are scalar
  const int lr = lane & 31, h = lane >> 5;
  const int K = static_cast<int>(p.K);  // K < 2^31 (buffer offsets are 32-bit)
  const int kbeg = ks * p.kstages * BK;
  const int nst = min(p.kstages, (K - kbeg + BK - 1) / BK);

  // ---- weight rows: block j of lane feature fl reads row row0 + drow[j]
  // (gated: j = 0 gate, j = 1 linear row of the same feature).  drow is
  // uniform, so one VGPR offset per lane serves both blocks (the rest rides in
  // the scalar offset).  Rows of features past nfeat are read (past the
  // buffer: zeros) but their outputs are never stored. ----
  // bytes of one weight row (tile-major: K padded to whole stages of BK)
  const bool tiled = p.tiled != 0;
  const int64_t rb = tiled ? static_cast<int64_t>((K + 127) / 128) * 128 * G::EBITS / 8  // whole chunks of 128 k
                           : static_cast<int64_t>(K) * G::EBITS / 8;
  const uint8_t* wbase_g = p.w + static_cast<int64_t>(e) * p.w_rows * rb;
  const uint8_t* wbase_l = p.wl + static_cast<int64_t>(e) * p.wl_rows * rb;
  const __amdgpu_buffer_rsrc_t rs_g = make_rsrc(wbase_g, static_cast<uint32_t>(p.w_rows * rb));
  const __amdgpu_buffer_rsrc_t rs_l = make_rsrc(wbase_l, static_cast<uint32_t>(p.wl_rows * rb));
  const int64_t fl = GATED ? static_cast<int64_t>(ntile) * (BN / 2) + wave * 32 + lr
                           : static_cast<int64_t>(ntile) * BN + wave * 64 + lr;
  // row0 / drow: rows of the scales and biases; wrow0 / wdrow: weight rows
  // (the same, unless a fused interleaved fc1 is stored de-interleaved)
  const bool interleaved = GATED && p.gate_mode == kGateInterleaved;
  const int64_t row0 = interleaved ? 2 * fl : fl;
  int64_t drow[kNT];
  if constexpr (GATED) {
    drow[0] = 0;
    drow[1] = interleaved ? 1 : (p.gate_mode == kGateChunked ? p.nfeat : 0);
  } else {
    drow[0] = 0;
    drow[1] = 32;
  }
  const bool deint = interleaved && tiled && p.deint != 0;
  const int64_t wrow0 = deint ? fl : row0;
  int64_t wdrow[kNT];
#pragma unroll
  for (int j = 0; j < kNT; ++j) wdrow[j] = deint ? (j == 0 ? 0 : p.nfeat) : drow[j];
  // Tile-major weights (pre-packed): the 16 rows x 128 k of a weight tile
  // and chunk are one block of CB bytes in which piece q (16 bytes) of row r
  // sits at ((q % kv) * 64 + (q / kv) * 16 + r) * 16, kv = 16-byte vectors
  // per 32 k (1 int4, 2 int8, 4 16-bit).  A stage is one chunk (int4, int8)
  // or half of one (16-bit, 64 k); lane half h reads the stage's 32-k groups
  // from KH h / 32 on, BVEC pieces of its row.  wdrow steps (0, 32, nfeat)
  // are whole tiles, so they stay row offsets.
  constexpr int kKv = WF == kInt8 ? 2 : (WF == kDense ? 4 : 1);
  constexpr int CB = 1024 * kKv;
  const uint32_t woff =
      tiled ? static_cast<uint32_t>((wrow0 / 16) * 16 * rb + (wrow0 % 16) * 16 + (KH / 32) * 256 * h)
            : static_cast<uint32_t>(wrow0 * rb + static_cast<int64_t>(kbeg + KH * h) * G::EBITS / 8);
  // bytes from woff to the lane's first piece of stage c
  auto wstage = [&](int c) -> uint32_t {
    if (!tiled) return static_cast<uint32_t>(c * BK * G::EBITS / 8);
    const int k = kbeg + c * BK;  // a multiple of 64
    return static_cast<uint32_t>((k / 128) * CB + ((k / 32) % 4) * 256);
  };
  // offset of vector v beyond 16 v (tiled: piece BVEC h + v)
  int vdelta[BVEC];
#pragma unroll
  for (int v = 0; v < BVEC; ++v) vdelta[v] = tiled ? (v % kKv) * 1024 + (v / kKv) * 256 - 16 * v : 0;

  // ---- per-block scales (folded).  Loading a 2-byte scale per lane and
  // stage touches one cache line per row, as much address work as a weight
  // load; so each wave instead loads windows of WB consecutive block scales
  // of its 64 rows (block j = lane / 32, row lr: 16 bytes per lane), one
  // window ahead, into a wave-private LDS area, and reads the scale of each
  // stage from there.  Blocks past K (and padding stages) weigh 0. ----
  constexpr int SB = sizeof(typename ST::storage);
  constexpr int WB = 16 / SB;  // blocks per window
  const int bshift = kFold ? __builtin_ctzll(static_cast<uint64_t>(p.block_size)) : 0;
  const int nblk = kFold ? (K >> bshift) : 0;
  // Tile-major scales (pre-packed for the decode kernels, block 32 / 64):
  // per (16-row tile, chunk of 128 k) the 16 rows' nbc = 128 / block scales;
  // nblk_r elements per row with K padded to whole chunks.  A window of WB
  // blocks is then WB / nbc pieces of nbc * SB bytes, one per chunk.
  const bool stiled = kFold && p.stiled != 0;
  const int nbc = 128 >> bshift;
  const int nblk_r = stiled ? (K + 127) / 128 * nbc : nblk;
  const __amdgpu_buffer_rsrc_t rs_sg =
      make_rsrc(kFold ? static_cast<const uint8_t*>(p.s) + static_cast<int64_t>(e) * p.w_rows * nblk_r * SB : nullptr,
                static_cast<uint32_t>(p.w_rows * nblk_r * SB));
  const __amdgpu_buffer_rsrc_t rs_sl =
      make_rsrc(kFold ? static_cast<const uint8_t*>(p.sl) + static_cast<int64_t>(e) * p.wl_rows * nblk_r * SB : nullptr,
                static_cast<uint32_t>(p.wl_rows * nblk_r * SB));
  // this lane loads the scale row of block j = h, row lr
  const int64_t srow = stiled ? wrow0 + wdrow[h] : row0 + drow[h];
  const uint32_t srow_off = stiled ? static_cast<uint32_t>(((srow / 16) * 16 * nblk_r + (srow % 16) * nbc) * SB)
                                   : static_cast<uint32_t>(srow * nblk * SB);
  const bool s_aligned = (nblk * SB) % 16 == 0;
  // tile-major: dwords per chunk piece (log2: 0, 1 or 2) and bytes per chunk
  const int s_per_log = stiled ? __builtin_ctz(static_cast<unsigned>(nbc * SB / 4)) : 0;
  const uint32_t s_cstride = static_cast<uint32_t>(16 * nbc * SB);
  u32x4_t swin = {0u, 0u, 0u, 0u};  // window in flight (registers)
  auto sfetch = [&](int m) {        // window m: blocks [WB m, WB m + WB)
    if constexpr (kFold) {
      if (stiled) {
        // dword q of the window: piece q >> s_per_log (chunk WB m / nbc + that), dword q % per in it
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t o = srow_off + static_cast<uint32_t>(WB * m / nbc + (q >> s_per_log)) * s_cstride +
                             4u * static_cast<uint32_t>(q & ((1 << s_per_log) - 1));
          const uint32_t og = h == 0 ? o : kOob, ol = h == 1 ? o : kOob;
          swin[q] = __builtin_amdgcn_raw_buffer_load_b32(rs_sg, static_cast<int>(og), 0, 0) |
                    __builtin_amdgcn_raw_buffer_load_b32(rs_sl, static_cast<int>(ol), 0, 0);
        }
        return;
      }
      const uint32_t o = srow_off + static_cast<uint32_t>(m * 16);
      const uint32_t og = h == 0 ? o : kOob, ol = h == 1 ? o : kOob;
      if (s_aligned) {
        swin = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs_sg, static_cast<int>(og), 0, 0)) |
               __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs_sl, static_cast<int>(ol), 0, 0));
      } else if constexpr (SB == 1) {
        // 1-byte (E8M0) scales: rows start at any byte
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t w = 0;
#pragma unroll
          for (int b = 0; b < 4; ++b)
            w |= static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b8(rs_sg, static_cast<int>(og + 4 * q + b), 0, 0) |
                                       __builtin_amdgcn_raw_buffer_load_b8(rs_sl, static_cast<int>(ol + 4 * q + b), 0, 0))
                 << (8 * b);
          swin[q] = w;
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(rs_sg, static_cast<int>(og + 4 * q), 0, 0) |
                              __builtin_amdgcn_raw_buffer_load_b16(rs_sl, static_cast<int>(ol + 4 * q), 0, 0);
          const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(rs_sg, static_cast<int>(og + 4 * q + 2), 0, 0) |
                              __builtin_amdgcn_raw_buffer_load_b16(rs_sl, static_cast<int>(ol + 4 * q + 2), 0, 0);
          swin[q] = lo | (hi << 16);
        }
      }
    }
  };
  // wave-private window buffers: [2][64 lanes][16 bytes], lanes 20 bytes
  // apart: the 32 lanes that read one 2-byte scale each (lane lr reads lane
  // j * 32 + lr's window) then fall on distinct banks (a 16-byte stride put
  // 2 to 4 of them on one bank)
  constexpr int kWin = 20;
  __shared__ __attribute__((aligned(16))) uint8_t sS[kFold ? 4 * 2 * 64 * kWin : 16];
  uint8_t* const swave = sS + (kFold ? wave * 2 * 64 * kWin : 0);
  auto sstore = [&](int m) {
    if constexpr (kFold) {
      uint32_t* d = reinterpret_cast<uint32_t*>(swave + ((m & 1) * 64 + lane) * kWin);
#pragma unroll
      for (int q = 0; q < 4; ++q) d[q] = swin[q];
    }
  };
  auto win_of = [&](int c) { return ((kbeg + c * BK) >> bshift) / WB; };  // window of stage c
  // scale of block j for block index b (this lane's row), 0 past K
  auto sread = [&](int j, int b) -> float {
    const typename ST::storage* ent =
        reinterpret_cast<const typename ST::storage*>(swave + (((b / WB) & 1) * 64 + j * 32 + lr) * kWin);
    const float v = to_f32<ST>(ent[b % WB]);
    return b < nblk ? v : 0.0f;
  };

  struct Ring {
    u32x4_t w[kNT][BVEC];
  };
  auto fetch = [&](int c, Ring& d) {
    const int k0 = kbeg + c * BK + KH * h;  // first k of the lane's range
    const bool kin = (c < nst) & (k0 < K);
    const uint32_t o = kin ? woff + wstage(c) : kOob;
#pragma unroll
    for (int j = 0; j < kNT; ++j) {
      const __amdgpu_buffer_rsrc_t rw = GATED && j == 1 ? rs_l : rs_g;
      const int sw = static_cast<int>(wdrow[j] * rb);
#pragma unroll
      for (int v = 0; v < BVEC; ++v)
        d.w[j][v] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rw, static_cast<int>(o + 16 * v), sw + vdelta[v], 0));
    }
  };

  // Weight operand of block j, step s: 8 k as 16-bit values; sc: the block
  // scale of the step.
  auto bop = [&](const Ring& d, int j, int s, float sc) -> u32x4_t {
    if constexpr (std::is_same_v<ST, E8M0>) {
      // MXFP4: E2M1 pairs times the power-of-two block scale in one
      // conversion each (exact within the 16-bit type's range)
      return fp4_scaled<AT>(d.w[j][s >> 2][s & 3], sc);
    }
    u32x4_t q;
    if constexpr (WF == kInt4) q = dq4_exact<AT>(d.w[j][s >> 2][s & 3]);
    else if constexpr (WF == kInt8) q = dq8_exact<AT>(d.w[j][s >> 1][(s & 1) * 2], d.w[j][s >> 1][(s & 1) * 2 + 1]);
    else q = d.w[j][s];
    if constexpr (kFold) {
      if constexpr (AT::kId == 10 && ST::kId == 10) {
        // fp16 scales: one packed multiply of the exact integers
        const _Float16 sh = static_cast<_Float16>(sc);
        const half2_t s2 = {sh, sh};
#pragma unroll
        for (int r = 0; r < 4; ++r) q[r] = h2_bits(bits_h2(q[r]) * s2);
      } else {
        if constexpr (WF == kInt4) q = dq4_scaled<AT>(d.w[j][s >> 2][s & 3], sc);
        else q = dq8_scaled<AT>(d.w[j][s >> 1][(s & 1) * 2], d.w[j][s >> 1][(s & 1) * 2 + 1], sc);
      }
    }
    return q;
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

  floatx16_t acc[kMT][kNT];
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int j = 0; j < kNT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // A operand of row block i, step s: row 32 i + lr, global piece
  // (2 KH h + 16 s) / 16; swz(row) does not depend on i.
  const uint8_t* arow0 = sA0 + lr * G::ROWB;
  const uint8_t* arow1 = sA1 + lr * G::ROWB;
  const int sw = G::swz(lr);
  auto aread = [&](const uint8_t* arow, int s, int i) -> u32x4_t {
    const int piece = ((KH * 2 * h + 16 * s) / 16) ^ sw;
    return *reinterpret_cast<const u32x4_t*>(arow + i * 32 * G::ROWB + piece * 16);
  };

  // One stage, software pipelined over its steps: the activation reads and
  // the dequantisation of step s + 1 are issued among the MFMAs of step s.
  auto compute = [&](int c, const uint8_t* arow, const Ring& d) {
    // block scales of this stage: NSC per lane half and block j
    float sc[kNT][NSC];
#pragma unroll
    for (int j = 0; j < kNT; ++j)
#pragma unroll
      for (int q = 0; q < NSC; ++q)
        sc[j][q] = kFold ? sread(j, (kbeg + c * BK + KH * h + q * (KH / NSC)) >> bshift) : 1.0f;
    u32x4_t a[kMT], b[kNT];
#pragma unroll
    for (int i = 0; i < kMT; ++i) a[i] = aread(arow, 0, i);
#pragma unroll
    for (int j = 0; j < kNT; ++j) b[j] = bop(d, j, 0, sc[j][0]);
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
      u32x4_t an[kMT], bn[kNT];
      if (s + 1 < NSTEP) {
#pragma unroll
        for (int i = 0; i < kMT; ++i) an[i] = aread(arow, s + 1, i);
#pragma unroll
        for (int j = 0; j < kNT; ++j) bn[j] = bop(d, j, s + 1, sc[j][(s + 1) * NSC / NSTEP]);
      }
#pragma unroll
      for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int j = 0; j < kNT; ++j) acc[i][j] = mfma32x32x16<AT>(a[i], b[j], acc[i][j]);
      // (the compiler's own interleave of these MFMAs, reads and dequant
      // measured 2-5% faster than a fixed 1 MFMA : 4 VALU : 1/2 DS pattern)
      if (s + 1 < NSTEP) {
#pragma unroll
        for (int i = 0; i < kMT; ++i) a[i] = an[i];
#pragma unroll
        for (int j = 0; j < kNT; ++j) b[j] = bn[j];
      }
    }
  };

  // ---- main loop: stages in pairs (buffers / ring slots 0 and 1).  Stage
  // c + 1's activations and weights are requested before stage c is
  // multiplied; the barrier after stage c waits for the LDS loads only (the
  // weight loads issued after them stay in flight).  A padding stage past the
  // split's range reads zeros. ----
  // Scale windows: the first is stored before the loop, the next one is in
  // flight; when stage c + 1 enters a new window, the in-flight one is stored
  // (its buffer held the window before the current one) and the one after
  // is requested.
  auto swindow = [&](int c) {
    if constexpr (kFold) {
      if (win_of(c + 1) != win_of(c)) {
        sstore(win_of(c + 1));
        sfetch(win_of(c + 1) + 1);
      }
    }
  };
  Ring ring[2];
  if constexpr (kFold) {
    sfetch(win_of(0));
    sstore(win_of(0));
    sfetch(win_of(0) + 1);
  }
  aload(0, sA0);
  fetch(0, ring[0]);
  __syncthreads();
  const int npairs = (nst + 1) / 2;
  // The scheduling barriers keep the next stage's loads at the top of the
  // stage (left alone, the scheduler sinks them next to the barrier, which
  // then waits for their full latency).
  for (int q = 0; q < npairs; ++q) {
    const int c = 2 * q;
    aload(c + 1, sA1);
    fetch(c + 1, ring[1]);
    __builtin_amdgcn_sched_barrier(0);
    compute(c, arow0, ring[0]);
    swindow(c);
    __syncthreads();
    aload(c + 2, sA0);
    fetch(c + 2, ring[0]);
    __builtin_amdgcn_sched_barrier(0);
    compute(c + 1, arow1, ring[1]);
    swindow(c + 1);
    __syncthreads();
  }

  // ---- epilogue: acc[i][j][q] is D[32 i + 8 (q / 4) + 4 h + q % 4][lr].
  // Element offsets are 32-bit from the tile's first row; a full tile (the
  // common case) stores without per-row checks. ----
  const int act_t = AT::kId;
  const int nf = static_cast<int>(p.nfeat);  // nfeat * 128 < 2^31 (checked on the host)
  auto for_rows = [&](auto&& emit) {
    if (rows == BM) {
#pragma unroll
      for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int q = 0; q < 16; ++q) emit(i, q, 32 * i + 8 * (q >> 2) + 4 * h + (q & 3));
    } else {
#pragma unroll
      for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int m = 32 * i + 8 * (q >> 2) + 4 * h + (q & 3);
          if (m < rows) emit(i, q, m);
        }
    }
  };
  if constexpr (FC1 && GATED) {
    if (fl < p.nfeat) {
      const int64_t rg = row0 + drow[0], rl = row0 + drow[1];
      float chg = 1.0f, chl = 1.0f;
      if constexpr (SM == kPsChan) {
        chg = load_any(p.s, p.scale_type, static_cast<int64_t>(e) * p.w_rows + rg);
        chl = load_any(p.sl, p.scale_type, static_cast<int64_t>(e) * p.wl_rows + rl);
      }
      const float bg = p.b ? load_any(p.b, act_t, static_cast<int64_t>(e) * p.w_rows + rg) : 0.0f;
      const float bl = p.bl ? load_any(p.bl, act_t, static_cast<int64_t>(e) * p.wl_rows + rl) : 0.0f;
      typename AT::storage* const op =
          static_cast<typename AT::storage*>(p.out) + static_cast<int64_t>(row_begin) * p.nfeat + fl;
      if (p.activation == kSwiglu) {
        for_rows([&](int i, int q, int m) {
          op[m * nf] = from_f32<AT>(swiglu_f<true>(acc[i][0][q] * chg + bg, acc[i][1][q] * chl + bl, p.alpha,
                                                   p.beta, p.limit));
        });
      } else {
        for_rows([&](int i, int q, int m) {
          op[m * nf] = from_f32<AT>(apply_act<true>(acc[i][0][q] * chg + bg, acc[i][1][q] * chl + bl, true,
                                                    p.activation, p.alpha, p.beta, p.limit));
        });
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < kNT; ++j) {
      const int64_t f = fl + 32 * j;
      if (f >= p.nfeat) continue;
      float ch = 1.0f;
      if constexpr (SM == kPsChan) ch = load_any(p.s, p.scale_type, static_cast<int64_t>(e) * p.w_rows + f);
      const float bias = (p.b && ks == 0) ? load_any(p.b, act_t, static_cast<int64_t>(e) * p.w_rows + f) : 0.0f;
      if constexpr (FC1) {
        typename AT::storage* const op =
            static_cast<typename AT::storage*>(p.out) + static_cast<int64_t>(row_begin) * p.nfeat + f;
        for_rows([&](int i, int q, int m) {
          op[m * nf] = from_f32<AT>(act_single<true>(acc[i][j][q] * ch + bias, p.activation));
        });
      } else if (p.out_half) {
        typename AT::storage* const op =
            static_cast<typename AT::storage*>(p.out) + static_cast<int64_t>(row_begin) * p.nfeat + f;
        for_rows([&](int i, int q, int m) { op[m * nf] = from_f32<AT>(acc[i][j][q] * ch + bias); });
      } else {
        float* const op = static_cast<float*>(p.out) + static_cast<int64_t>(ks) * p.out_rows * p.nfeat +
                          static_cast<int64_t>(row_begin) * p.nfeat + f;
        for_rows([&](int i, int q, int m) { op[m * nf] = acc[i][j][q] * ch + bias; });
      }
    }
  }
}

template <typename AT, int WF, int SM, typename ST, int NSC, bool FC1>
hipError_t launch_kernel(const PStage& st, bool gated, hipStream_t stream) {
  const unsigned nb = static_cast<unsigned>(st.ksplit) * st.ngroups * st.mslots * st.gn;
  if (FC1 && gated)
    hipLaunchKernelGGL((prefill_kernel<AT, WF, SM, ST, NSC, true, true>), dim3(nb), dim3(256), 0, stream, st);
  else
    hipLaunchKernelGGL((prefill_kernel<AT, WF, SM, ST, NSC, FC1, false>), dim3(nb), dim3(256), 0, stream, st);
  return hipGetLastError();
}

template <typename AT, int WF, bool FC1>
hipError_t launch_scaled(const PStage& st, const ExpertArgs& a, bool gated, hipStream_t stream) {
  if constexpr (WF == kDense) {
    return launch_kernel<AT, WF, kPsNone, F16, 1, FC1>(st, gated, stream);
  } else {
    if (a.block_size == 0) return launch_kernel<AT, WF, kPsChan, F16, 1, FC1>(st, gated, stream);
    // scales per lane half and stage: KH / block_size (block_size >= 16)
    const int64_t nsc = std::max<int64_t>(1, PG<WF>::KH / a.block_size);
    auto by_type = [&](auto st_tag) -> hipError_t {
      using ST = decltype(st_tag);
      if (nsc == 4) return launch_kernel<AT, WF, kPsBlock, ST, 4, FC1>(st, gated, stream);
      if (nsc == 2) return launch_kernel<AT, WF, kPsBlock, ST, 2, FC1>(st, gated, stream);
      return launch_kernel<AT, WF, kPsBlock, ST, 1, FC1>(st, gated, stream);
    };
    if constexpr (WF == kInt4) {
      if (a.mx) return launch_kernel<AT, WF, kPsBlock, E8M0, 2, FC1>(st, gated, stream);  // block 32
    }
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
  // Weight tiles per sweep group: 4, 3 or 2, whichever pads ntiles least
  // (ties: the larger).  Padding slots are workgroups that exit at once but
  // still take their place in each XCD's range; measured per group size
  // (layer time, T = 8192 unless noted): gpt-oss int4 fc2 (12 tiles) 0.93
  // ms at 8 -> 0.765 at 4, Qwen3 fp16 fc1 (6 tiles) 0.566 at 8 -> 0.48 at
  // 2 or 3, Mixtral int8 T=4096 (112 and 16 tiles) 0.5% faster at 4 than
  // at 8; 16 was 5% slower there.
  st.gn = 4;
  for (int g = 4, best = 1 << 30; g >= 2; --g) {
    const int pad = (st.ntiles + g - 1) / g * g - st.ntiles;
    if (pad < best) {
      best = pad;
      st.gn = g;
    }
  }
  if (st.ntiles == 1) st.gn = 1;  // one weight tile (N <= 256): no padding slots
  st.ngroups = (st.ntiles + st.gn - 1) / st.gn;
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
  if (std::max(a.H, a.I) * BM >= lim) return false;  // 32-bit in-tile offsets of the epilogue
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
  st.tiled = a.tiled1;
  st.deint = a.deint1;
  st.stiled = a.stiled1;
  // gated: a weight tile holds BN/2 features (gate + linear rows)
  plan_grid(st, a.T, a.k, a.E, a.wfmt, gated ? 2 * a.I : a.I, 1);
  return launch_stage<true>(st, a, gated, stream);
}

hipError_t launch_fc2_prefill(const ExpertArgs& a, int* y2_planes, int* y2_half, hipStream_t stream) {
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
  st.tiled = a.tiled2;
  st.stiled = a.stiled2;
  const int32_t splits = prefill_fc2_splits(a.T, a.H, a.I, a.E, a.k, a.wfmt);
  plan_grid(st, a.T, a.k, a.E, a.wfmt, a.H, splits);
  // 16-bit activations and one plane: y2 goes out in the activation type
  // (one rounding of the expert output before the fp32 weighted sum; half
  // the bytes written and read)
  st.out_half = splits == 1 && (a.act_type == MOE_ELEM_FLOAT16 || a.act_type == MOE_ELEM_BFLOAT16) ? 1 : 0;
  *y2_planes = splits;
  *y2_half = st.out_half;
  return launch_stage<false>(st, a, false, stream);
}

}  // namespace moe
