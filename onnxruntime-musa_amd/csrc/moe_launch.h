// moe_launch.h -- internal launcher interface between the host op and the
// gfx950 kernels.  POD argument structs + stream, returning hipError_t, the
// reference's device-launcher convention (musa/ep/src/kernels/math/topk_impl.h:10-33).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_mi355x.h"

namespace moe {

enum WeightFormat : int { kDense = 0, kInt4 = 4, kInt8 = 8 };

// How the activation input pairs are laid out in the fc1 output.
enum GateMode : int {
  kGateNone = 0,         // a = act(fc1)
  kGateFc3 = 1,          // gate = fc1 row i, linear = fc3 row i
  kGateInterleaved = 2,  // fused fc1 [2I]: gate = row 2i, linear = row 2i+1
  kGateChunked = 3       // fused fc1 [2I]: gate = row i, linear = row I+i
};

enum ExpertPath : int { kPathSimt = 0, kPathDecode = 1, kPathPrefill = 2 };

// Maximum router width handled by the wave-per-token router (8 values per lane).
constexpr int64_t kMaxExperts = 512;
constexpr int64_t kMaxTopK = 64;
// Token count up to which routing + dispatch runs as one single-workgroup kernel.
constexpr int64_t kSmallRouteTokens = 256;
// Tokens routed per workgroup in the multi-workgroup router: one token per
// wave of its 16 when experts take two per lane (E > 64), and enough
// workgroups to cover the CUs (8192 tokens: 512 workgroups).
constexpr int kRouteTokensPerBlock = 16;

struct RouteArgs {
  moe_route_params p;
  int32_t* tile_offsets;  // optional [E+1]: prefix of ceil(count_e / tile_m)
  int32_t tile_m;
  // Router GEMM fused into the routing kernels (gate_w non-null): the
  // logits [T, E] = x [T, H] * gate_w [E, H]^T (+ gate_b [E]) are computed
  // with fp32 accumulation, rounded to the logits type and written to
  // p.logits (a workspace buffer) by the workgroup that routes those tokens.
  const void* gate_x;
  const void* gate_w;
  const void* gate_b;
  int64_t hidden;
};
// Largest T * E * H routed by the single-workgroup router with the router
// GEMM fused (larger products take the multi-workgroup router).
constexpr int64_t kGateSmallMacs = int64_t{1} << 22;

size_t route_scratch_bytes(int64_t T, int64_t E, int64_t k);
// Scratch of the routing kernels with the router GEMM fused (every T > 0 may
// take the multi-workgroup router).
size_t route_scratch_bytes_gate(int64_t T, int64_t E);
hipError_t launch_route_dispatch(const RouteArgs& a, hipStream_t stream);

struct ExpertArgs {
  int64_t T, H, I, E, k;
  int32_t act_type;    // moe_elem_type of input/output/bias
  int32_t wfmt;        // WeightFormat
  int32_t scale_type;  // moe_elem_type of scales (quantized only)
  int64_t block_size;  // 0 = one scale per output channel
  int32_t activation;  // moe_activation
  int32_t gate_mode;   // GateMode
  float alpha, beta, limit;
  // routing (device)
  const int32_t* offsets;       // [E+1]
  const int32_t* perm;          // [T*k]
  const int32_t* inv_perm;      // [T*k]
  const int32_t* topk_ids;      // [T*k]
  const float* topk_w;          // [T*k]
  const int32_t* tile_offsets;  // [E+1], prefill path
  // fc1 / fc3
  const void* x;  // [T, H]
  const void *w1, *s1, *b1;
  const void *w3, *s3, *b3;
  // fc2
  const void *w2, *s2, *b2;
  // 1: the stage's weights are in the tile-major layout of moe_prepack.hip
  // (fc1 and fc3 together; fc2), else in the op's row-major layout
  int32_t tiled1, tiled2;
  // 1: the tile-major fused fc1 of interleaved SwiGLU is de-interleaved
  int32_t deint1;
  // 1: the stage's block scales (block 32 / 64) are tile-major too
  int32_t stiled1, stiled2;
  // 1: MXFP4 experts (OCP MX v1.0): wfmt kInt4's packing (two elements per
  // byte, even k low) of FP4 E2M1 values, scale_type uint8 E8M0 block
  // scales of block_size 32
  int32_t mx;
  // intermediates
  void* act;   // [T*k, I] in act_type
  float* y2;   // [y2_planes][T*k, H] fp32 (partial sums when split over K)
  int32_t y2_planes;
  int32_t y2_half;  // 1: y2 is one plane in the activation type (16-bit prefill without a K split)
  void* out;   // [T, H] act_type
};

hipError_t launch_fc1_simt(const ExpertArgs& a, hipStream_t stream);
hipError_t launch_fc2_simt(const ExpertArgs& a, hipStream_t stream);
// route: when non-null, the fc1 kernel routes and dispatches the batch in its
// prologue and writes route's outputs (decode_routes_in_fc1 says when it can).
hipError_t launch_fc1_decode(const ExpertArgs& a, const moe_route_params* route, hipStream_t stream);
bool decode_routes_in_fc1(const ExpertArgs& a);
hipError_t launch_fc2_decode(const ExpertArgs& a, int* y2_planes, hipStream_t stream);
hipError_t launch_fc1_prefill(const ExpertArgs& a, hipStream_t stream);
hipError_t launch_fc2_prefill(const ExpertArgs& a, int* y2_planes, int* y2_half, hipStream_t stream);
hipError_t launch_finalize(const ExpertArgs& a, hipStream_t stream);

// ONNX TopK over the middle axis of [rows, dim, inner] (moe_topk.hip).
struct TopKArgs {
  int64_t rows, dim, inner, k;
  int32_t largest, sorted;
};
constexpr int64_t kTopKMaxDim = 8192;  // one workgroup sorts a slice in LDS
// Longer axes: radix select, then a sort of the k winners in LDS.
constexpr int64_t kTopKRadixMaxK = 8192;
constexpr int64_t kTopKRadixMaxDim = (int64_t{1} << 31) - 1;  // 32-bit indices in LDS
hipError_t launch_topk(const void* in, int32_t elem_type, void* values, int64_t* indices, const TopKArgs& p,
                       hipStream_t stream);

// ONNX Softmax along the middle axis of [outer, dim, inner] (moe_softmax.hip).
hipError_t launch_softmax(const void* in, void* out, int32_t elem_type, int64_t outer, int64_t dim, int64_t inner,
                          hipStream_t stream);

// Reorders row-major quantized weights [rows, row_bytes] (rows a multiple of
// 16 and of expert_rows, row_bytes a multiple of 16) into the tile-major
// layout read by the decode and prefill kernels (moe_prepack.hip): rows of
// ceil(row_bytes / cbytes) * cbytes bytes (cbytes = 64 for int4, 128 for
// int8; the padding is zeros), with each expert's interleaved row pairs
// split into halves when deint (expert_rows a multiple of 32).
hipError_t launch_prepack(const uint8_t* src, uint8_t* dst, int64_t rows, int64_t row_bytes, int cbytes,
                          int64_t expert_rows, bool deint, hipStream_t stream);
// Reorders block scales [rows, nblk] of block 32 or 64 (elem_bytes 1, 2 or 4)
// into the tile-major layout of the step-scale decode kernels: per (16-row
// tile, chunk of 128 k) the 16 rows' 128 / block scales, blocks past K zero,
// rows de-interleaved like their weights when deint (moe_prepack.hip).
hipError_t launch_prepack_scales(const void* src, void* dst, int elem_bytes, int64_t rows, int64_t nblk, int block,
                                 int64_t expert_rows, bool deint, hipStream_t stream);
// Bytes of one packed weight row: K padded to whole chunks of 128.
inline int64_t packed_row_bytes(int64_t K, int wfmt) { return (K + 127) / 128 * (wfmt == kInt4 ? 64 : 128); }

// Whether the MFMA paths accept this problem (fp16/bf16 activations, K a
// multiple of 32, block sizes the dequant loaders handle).
bool decode_supported(const ExpertArgs& a);
bool prefill_supported(const ExpertArgs& a);
// K splits (partial planes of y2) the prefill fc2 kernel uses for a problem.
int32_t prefill_fc2_splits(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, int wfmt);

// Row tile of the prefill grouped GEMM (rows of one expert per workgroup).
constexpr int kPrefillTileM = 128;
// Largest token count served by the decode (weight-streaming) path.
constexpr int64_t kDecodeMaxTokens = 64;
// Token count up to which decode stages the activation rows in LDS (in
// groups of 16 rows per expert).
constexpr int64_t kLdsMaxTokens = 64;
// Largest K of one LDS activation slice of the decode stream kernel (32
// chunks of 128 k); fc1 streams only when its K fits one slice.
constexpr int64_t kStreamMaxK = 32 * 128;
// Most K splits across workgroups of the decode fc2 kernel (partial planes of y2).
constexpr int kMaxDecodeKsplit = 8;

// Launch plan of the decode kernels, shared by the workspace planner and the
// launchers so both agree on the partial-plane sizes.
struct DecodePlan {
  bool stream1 = false;  // fc1: persistent kernel, activation slice staged in LDS
  bool stream2 = false;  // fc2: persistent kernel
  int32_t nsl1 = 1, ksc1 = 0;  // fc1 K slices, chunks of 128 k per slice
  int32_t nsl2 = 1, ksc2 = 0;  // fc2 K slices (partial planes of y2), chunks per slice
  int32_t y2_planes_max = 1;
};
DecodePlan plan_decode(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, int wfmt, int gate_mode);

}  // namespace moe
