// moe_expert_decode.hip -- host launchers of the decode (weight-streaming)
// expert kernels.  Up to kLdsMaxTokens tokens, persistent workgroups stage
// the activation rows in LDS (moe_expert_stream.h); up to kDecodeMaxTokens
// the rows are read from global memory (moe_expert_decode.h).  The quantised
// instantiations live in moe_expert_decode_int4.hip / _int8.hip.
#include <atomic>

#include "moe_expert_stream.h"

namespace moe {
namespace decode {

hipError_t launch_dense(const Stage& st, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream) {
  if (a.act_type == MOE_ELEM_BFLOAT16)
    return launch_kinds<BF16, kDense, kScaleNone, F16>(st, a.T, a.E, fc1, gated, stream);
  return launch_kinds<F16, kDense, kScaleNone, F16>(st, a.T, a.E, fc1, gated, stream);
}

hipError_t launch_stream_dense(const StreamStage& ss, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream) {
  return launch_stream_fmt<kDense>(ss, a, fc1, gated, stream);
}

// One persistent workgroup per CU of the current device (cached per device).
int stream_grid(int /*nw*/) {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

namespace {

// Splits of K for the global-activation kernel: ks waves inside a workgroup
// and, for fc2, ksg workgroups (partial output planes summed by finalize).
void pick_splits(Stage& st, const ExpertArgs& a, bool gated, bool allow_ksg) {
  const int wt = weight_tiles(a.wfmt, a.T);
  const int ft = gated ? wt / 2 : wt;
  const int64_t waves_f = (st.nfeat + 16 * ft - 1) / (16 * ft);
  const int64_t e_act = std::min<int64_t>(a.E, a.T * a.k);
  const int64_t nchunks = (st.K + kChunk - 1) / kChunk;
  const int pd = 3;
  int ks = 1, ksg = 1;
  auto lds_per_wave = [&](int splits) -> int64_t {
    if (st.block_size == 0) return 0;
    const int64_t per = (nchunks + splits - 1) / splits;
    const int64_t nb = (per * kChunk + st.block_size - 1) / st.block_size + 1;
    return static_cast<int64_t>(wt) * 16 * nb * 4;
  };
  for (;;) {
    const int64_t waves = e_act * waves_f * ks * ksg;
    const bool need_more = waves < 2048 || lds_per_wave(ks * ksg) > 24576;
    if (!need_more || nchunks < static_cast<int64_t>(2) * pd * ks * ksg) break;
    if (ks < 4) ks *= 2;
    else if (allow_ksg && ksg < kMaxDecodeKsplit) ksg *= 2;
    else break;
  }
  st.ks = ks;
  st.ksg = ksg;
  st.lds_scale = static_cast<int32_t>((lds_per_wave(ks * ksg) + 15) / 16 * 16);
}

hipError_t dispatch(const Stage& st, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream) {
  switch (a.wfmt) {
    case kInt4: return launch_int4(st, a, fc1, gated, stream);
    case kInt8: return launch_int8(st, a, fc1, gated, stream);
    default: return launch_dense(st, a, fc1, gated, stream);
  }
}

hipError_t dispatch_stream(const StreamStage& ss, const ExpertArgs& a, bool fc1, bool gated, hipStream_t stream) {
  switch (a.wfmt) {
    case kInt4: return launch_stream_int4(ss, a, fc1, gated, stream);
    case kInt8: return launch_stream_int8(ss, a, fc1, gated, stream);
    default: return launch_stream_dense(ss, a, fc1, gated, stream);
  }
}

}  // namespace
}  // namespace decode

DecodePlan plan_decode(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, int wfmt, int gate_mode) {
  DecodePlan pl;
  if (T > kDecodeMaxTokens) return pl;
  pl.y2_planes_max = kMaxDecodeKsplit;
  if (T > kLdsMaxTokens) return pl;
  // fc1 streams only when its whole K fits one LDS slice; fc2 always streams
  decode::stream_slices(H, decode::stream_pd(wfmt, gate_mode != kGateNone), &pl.nsl1, &pl.ksc1);
  decode::stream_slices(I, decode::stream_pd(wfmt, false), &pl.nsl2, &pl.ksc2);
  // the stream kernel indexes its tiles (row groups x slices x feature
  // tiles) with 32-bit arithmetic
  const int64_t ng = decode::stream_groups(T, E, k);
  const bool fits = ng * pl.nsl1 * ((I + 15) / 16) <= (int64_t{1} << 24) && ng * pl.nsl2 * ((H + 31) / 32) <= (int64_t{1} << 24);
  pl.stream1 = pl.nsl1 == 1 && fits;
  pl.stream2 = fits;
  pl.y2_planes_max = std::max<int32_t>(pl.nsl2, kMaxDecodeKsplit);
  return pl;
}

bool decode_supported(const ExpertArgs& a) {
  if (a.act_type != MOE_ELEM_FLOAT16 && a.act_type != MOE_ELEM_BFLOAT16) return false;
  if (a.T > kDecodeMaxTokens) return false;
  if (a.H % 32 || a.I % 32) return false;
  if (a.wfmt != kDense && a.block_size > 0 && a.block_size < 8) return false;
  // 32-bit buffer offsets: one expert's weights and the activations stay below 2 GiB
  const int64_t wb = a.wfmt == kInt4 ? 1 : (a.wfmt == kInt8 ? 2 : 4);  // bytes per 2 k
  const int64_t n1 = (a.gate_mode == kGateInterleaved || a.gate_mode == kGateChunked) ? 2 * a.I : a.I;
  const int64_t lim = int64_t{1} << 31;
  if (n1 * a.H / 2 * wb >= lim || a.H * a.I / 2 * wb >= lim) return false;
  if (a.T * a.k * std::max(a.H, a.I) * 2 >= lim) return false;
  // MXFP4: the stream kernels only (both stages)
  if (a.mx) {
    const DecodePlan pl = plan_decode(a.T, a.H, a.I, a.E, a.k, a.wfmt, a.gate_mode);
    if (!pl.stream1 || !pl.stream2) return false;
  }
  return true;
}

namespace {

decode::Stage fc1_stage(const ExpertArgs& a) {
  decode::Stage st{};
  st.in = a.x;
  st.in_rows = a.T;
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
  st.out_rows = a.T * a.k;
  st.tiled = a.tiled1;
  st.deint = a.deint1;
  st.stiled = a.stiled1;
  return st;
}

decode::Stage fc2_stage(const ExpertArgs& a) {
  decode::Stage st{};
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
  st.block_size = a.wfmt == kDense ? 0 : a.block_size;
  st.offsets = a.offsets;
  st.perm = a.perm;
  st.topk = a.k;
  st.out = a.y2;
  st.out_rows = a.T * a.k;
  st.tiled = a.tiled2;
  st.stiled = a.stiled2;
  return st;
}

}  // namespace

bool decode_routes_in_fc1(const ExpertArgs& a) {
  if (a.T * a.k > decode::kFusedRouteRows || a.E > decode::kFusedRouteExperts) return false;
  const DecodePlan pl = plan_decode(a.T, a.H, a.I, a.E, a.k, a.wfmt, a.gate_mode);
  // the routing scratch overlays the activation-slice region (bounds over
  // both wave counts of the stream kernel: 8 and 12 waves)
  return pl.stream1 && route_block_scratch_bytes(a.T, a.E, a.k, 12, 2) <= decode::stream_region_bytes(pl.ksc1, 8);
}

hipError_t launch_fc1_decode(const ExpertArgs& a, const moe_route_params* route, hipStream_t stream) {
  const bool gated = a.gate_mode != kGateNone;
  decode::Stage st = fc1_stage(a);
  const DecodePlan pl = plan_decode(a.T, a.H, a.I, a.E, a.k, a.wfmt, a.gate_mode);
  if (pl.stream1) {
    decode::StreamStage ss{};
    ss.s = st;
    ss.ksc = pl.ksc1;
    ss.nslices = 1;
    ss.E = static_cast<int32_t>(a.E);
    ss.ngroups = decode::stream_groups(a.T, a.E, a.k);
    if (route) {
      if (!decode_routes_in_fc1(a)) return hipErrorInvalidValue;
      ss.route = *route;
      ss.route_ints = static_cast<int32_t>(a.E + 1 + a.T * a.k);
    }
    return decode::dispatch_stream(ss, a, true, gated, stream);
  }
  if (route) return hipErrorInvalidValue;
  decode::pick_splits(st, a, gated, false);
  return decode::dispatch(st, a, true, gated, stream);
}

hipError_t launch_fc2_decode(const ExpertArgs& a, int* y2_planes, hipStream_t stream) {
  decode::Stage st = fc2_stage(a);
  const DecodePlan pl = plan_decode(a.T, a.H, a.I, a.E, a.k, a.wfmt, a.gate_mode);
  if (pl.stream2) {
    decode::StreamStage ss{};
    ss.s = st;
    ss.ksc = pl.ksc2;
    ss.nslices = pl.nsl2;
    ss.E = static_cast<int32_t>(a.E);
    ss.ngroups = decode::stream_groups(a.T, a.E, a.k);
    *y2_planes = pl.nsl2;
    return decode::dispatch_stream(ss, a, false, false, stream);
  }
  decode::pick_splits(st, a, false, true);
  *y2_planes = st.ksg;
  return decode::dispatch(st, a, false, false, stream);
}

}  // namespace moe
