// moe_op.cc -- host side of the com.microsoft MoE / QMoE kernels (C++20).
//
// Mirrors the reference's op-kernel structure: attributes are read once at
// creation and the kernel is immutable afterwards (ctor pattern
// musa/ep/src/kernels/llm/attention.cc:63-72); Compute validates inputs,
// plans scratch and enqueues device launches on the caller's stream with no
// host synchronisation (attention.cc:100-256, scratch pattern :29-61).
// Errors never cross the ABI as exceptions: every entry point returns a
// status (the reference wraps entries in EXCEPTION_TO_RETURNED_STATUS_*,
// musa/ep/src/plugin_ep_utils.h:92-106).
//
// Input contract (op schemas of ONNX Runtime 1.26, com.microsoft, since 1):
//   MoE : input, router_probs, fc1_experts_weights, fc1_experts_bias?,
//         fc2_experts_weights, fc2_experts_bias?, fc3_experts_weights?,
//         fc3_experts_bias?
//   QMoE: input, router_probs, fc1_experts_weights, fc1_scales,
//         fc1_experts_bias?, fc2_experts_weights, fc2_scales,
//         fc2_experts_bias?, fc3_experts_weights?, fc3_scales?,
//         fc3_experts_bias?
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <limits>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <utility>

#include "moe_launch.h"
#include "moe_mi355x.h"

namespace {

thread_local std::string g_last_error;

moe_status fail(moe_status code, std::string msg) {
  g_last_error = std::move(msg);
  return code;
}

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

bool is_float_type(int32_t t) {
  return t == MOE_ELEM_FLOAT || t == MOE_ELEM_FLOAT16 || t == MOE_ELEM_BFLOAT16;
}
size_t elem_size(int32_t t) { return t == MOE_ELEM_FLOAT ? 4 : (t == MOE_ELEM_UINT8 ? 1 : 2); }

std::string dims_str(const moe_tensor& t) {
  std::string s = "[";
  for (int i = 0; i < t.rank; ++i) s += (i ? "," : "") + std::to_string(t.dims[i]);
  return s + "]";
}

// Shapes and pointers of one call, validated.
struct Problem {
  int64_t T = 0, H = 0, I = 0, E = 0, k = 0, N1 = 0;
  int32_t act_type = 0, scale_type = MOE_ELEM_FLOAT16, wfmt = moe::kDense, gate_mode = moe::kGateNone;
  int32_t mx = 0;  // MXFP4 experts: uint8 (E8M0) scales with 4-bit weights, block 32
  int64_t block_size = 0;
  const moe_tensor* in[11] = {};
};

// Workspace sections, byte offsets from the workspace base.
struct Layout {
  size_t topk_ids, topk_w, offsets, tile_offsets, perm, inv_perm, route_scratch, logits, act, y2, total;
  int32_t y2_planes;
  size_t route_scratch_bytes;
  moe::DecodePlan decode;
};

Layout plan_layout(const Problem& p) {
  Layout l{};
  const size_t rows = static_cast<size_t>(p.T * p.k);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += align_up(bytes);
    return at;
  };
  l.topk_ids = take(rows * 4);
  l.topk_w = take(rows * 4);
  l.offsets = take(static_cast<size_t>(p.E + 1) * 4);
  l.tile_offsets = take(static_cast<size_t>(p.E + 1) * 4);
  l.perm = take(rows * 4);
  l.inv_perm = take(rows * 4);
  // routing scratch for either router (logits given, or the router GEMM
  // fused), and the logits the fused router writes
  l.route_scratch_bytes = std::max(moe::route_scratch_bytes(p.T, p.E, p.k), moe::route_scratch_bytes_gate(p.T, p.E));
  l.route_scratch = take(l.route_scratch_bytes);
  l.logits = take(static_cast<size_t>(p.T * p.E) * elem_size(p.act_type));
  l.act = take(rows * static_cast<size_t>(p.I) * elem_size(p.act_type));
  l.decode = moe::plan_decode(p.T, p.H, p.I, p.E, p.k, p.wfmt, p.gate_mode);
  l.y2_planes = std::max<int32_t>({1, l.decode.y2_planes_max,
                                    moe::prefill_fc2_splits(p.T, p.H, p.I, p.E, p.k, p.wfmt)});
  l.y2 = take(rows * static_cast<size_t>(p.H) * 4 * static_cast<size_t>(l.y2_planes));
  l.total = o;
  return l;
}

}  // namespace

struct moe_kernel {
  bool quantized = false;
  moe_attributes attrs{};
  int32_t forced_path = -1;
  std::mutex mu;
  std::map<std::pair<int, void*>, std::pair<void*, size_t>> ws_cache;  // (device, stream) -> buffer
  // stage profiling
  bool profiling = false;
  hipEvent_t ev[5] = {};
  bool ev_recorded = false;
  int32_t last_path = -1;
  // debug switches, read from the environment at creation (the role of the
  // reference's MUSA_EP_TRACE_KERNELS / MUSA_EP_TRACE_SYNC,
  // musa/ep/src/kernels/shared_inc/kernel_base.h:48-80): trace prints a
  // begin and an end line per call to stderr; debug_sync waits for the
  // stream after each stage and turns a failure into MOE_EP_FAIL naming it
  bool trace = false, debug_sync = false;
  // Pre-packed (tile-major) expert weights by input index (QMoE: 2 fc1, 5
  // fc2, 8 fc3 and 3, 6, 9 their block scales; MoE: 2 fc1, 4 fc2, 6 fc3):
  // the caller-owned device copy and the tensor it was packed from (shape,
  // type and data pointer).
  struct Packed {
    const void* data = nullptr;
    moe_tensor src{};
    bool deint = false;  // fused interleaved fc1 stored de-interleaved
  };
  Packed packed[11];

  ~moe_kernel() {
    for (auto& kv : ws_cache)
      if (kv.second.first) (void)hipFree(kv.second.first);
    for (auto& e : ev)
      if (e) (void)hipEventDestroy(e);
  }
};

namespace {

moe_status validate(const moe_kernel* kr, const moe_tensor* inputs, int32_t n, Problem* out) {
  Problem p;
  const bool q = kr->quantized;
  const int32_t need = q ? 7 : 5;
  const int32_t max_in = q ? 11 : 8;
  if (!inputs || n < need)
    return fail(MOE_INVALID_ARGUMENT, std::string(q ? "QMoE" : "MoE") + " expects at least " +
                                          std::to_string(need) + " inputs, got " + std::to_string(n));
  if (n > max_in) {
    for (int32_t i = max_in; i < n; ++i)
      if (inputs[i].data)
        return fail(MOE_NOT_IMPLEMENTED,
                    "input " + std::to_string(i) + " (zero points) is not supported");
    n = max_in;
  }
  for (int32_t i = 0; i < n; ++i) p.in[i] = inputs[i].data ? &inputs[i] : nullptr;
  const moe_tensor *x = p.in[0], *router = p.in[1], *w1 = p.in[2];
  const moe_tensor *s1 = q ? p.in[3] : nullptr, *b1 = q ? p.in[4] : p.in[3];
  const moe_tensor *w2 = q ? p.in[5] : p.in[4], *s2 = q ? p.in[6] : nullptr;
  const moe_tensor *b2 = q ? p.in[7] : p.in[5];
  const moe_tensor *w3 = q ? (n > 8 ? p.in[8] : nullptr) : (n > 6 ? p.in[6] : nullptr);
  const moe_tensor *s3 = q ? (n > 9 ? p.in[9] : nullptr) : nullptr;
  const moe_tensor *b3 = q ? (n > 10 ? p.in[10] : nullptr) : (n > 7 ? p.in[7] : nullptr);
  if (!x || !router || !w1 || !w2) return fail(MOE_INVALID_ARGUMENT, "missing required input");
  if (q && (!s1 || !s2)) return fail(MOE_INVALID_ARGUMENT, "QMoE requires fc1_scales and fc2_scales");

  // input [T, H] or [B, S, H]
  if (x->rank != 2 && x->rank != 3)
    return fail(MOE_INVALID_ARGUMENT, "input must be 2D or 3D, got " + dims_str(*x));
  p.H = x->dims[x->rank - 1];
  p.T = x->dims[0] * (x->rank == 3 ? x->dims[1] : 1);
  p.act_type = x->elem_type;
  if (!is_float_type(p.act_type))
    return fail(MOE_NOT_IMPLEMENTED, "input type must be float, float16 or bfloat16");
  if (router->elem_type != p.act_type)
    return fail(MOE_INVALID_ARGUMENT, "router_probs must have the input's type");
  if (router->rank != 2 || router->dims[0] != p.T)
    return fail(MOE_INVALID_ARGUMENT, "router_probs must be [num_tokens, num_experts], got " + dims_str(*router));
  p.E = router->dims[1];
  if (p.E <= 0) return fail(MOE_INVALID_ARGUMENT, "num_experts must be positive");
  if (p.E > moe::kMaxExperts)
    return fail(MOE_NOT_IMPLEMENTED, "num_experts > " + std::to_string(moe::kMaxExperts));

  const moe_attributes& at = kr->attrs;
  p.k = at.k;
  if (p.k < 1 || p.k > p.E)
    return fail(MOE_INVALID_ARGUMENT, "k must be in [1, num_experts], got " + std::to_string(p.k));
  if (p.k > moe::kMaxTopK) return fail(MOE_NOT_IMPLEMENTED, "k > 64 is not supported");

  int64_t pack = 1;
  if (q) {
    pack = at.expert_weight_bits == 4 ? 2 : 1;
    p.wfmt = at.expert_weight_bits == 4 ? moe::kInt4 : moe::kInt8;
    if (w1->elem_type != MOE_ELEM_UINT8 || w2->elem_type != MOE_ELEM_UINT8 ||
        (w3 && w3->elem_type != MOE_ELEM_UINT8))
      return fail(MOE_INVALID_ARGUMENT, "QMoE expert weights must be uint8");
    p.scale_type = s1->elem_type;
    // uint8 scales: MXFP4 experts (OCP MX v1.0 FP4 E2M1 elements, E8M0
    // scales per 32 k), a library extension beyond the 1.26 QMoE schema,
    // whose scale type T2 is a float type
    p.mx = p.scale_type == MOE_ELEM_UINT8 ? 1 : 0;
    if ((!is_float_type(p.scale_type) && !p.mx) || s2->elem_type != p.scale_type ||
        (s3 && s3->elem_type != p.scale_type))
      return fail(MOE_INVALID_ARGUMENT, "QMoE scales must share one float type (or uint8 E8M0 for MXFP4)");
    if (p.mx && (at.expert_weight_bits != 4 || at.block_size != 32))
      return fail(MOE_INVALID_ARGUMENT, "MXFP4 experts (uint8 E8M0 scales) need expert_weight_bits 4 and "
                                        "block_size 32");
    p.block_size = at.block_size;
  } else {
    if (w1->elem_type != p.act_type || w2->elem_type != p.act_type ||
        (w3 && w3->elem_type != p.act_type))
      return fail(MOE_INVALID_ARGUMENT, "MoE expert weights must have the input's type");
  }
  if (w1->rank != 3 || w2->rank != 3)
    return fail(MOE_INVALID_ARGUMENT, "expert weights must be 3D");
  if (w1->dims[0] != p.E || w2->dims[0] != p.E)
    return fail(MOE_INVALID_ARGUMENT, "expert weight dim 0 must equal num_experts");
  if (w1->dims[2] * pack != p.H)
    return fail(MOE_INVALID_ARGUMENT, "fc1_experts_weights " + dims_str(*w1) + " does not match hidden_size " +
                                          std::to_string(p.H));
  if (w2->dims[1] != p.H)
    return fail(MOE_INVALID_ARGUMENT, "fc2_experts_weights " + dims_str(*w2) + " does not match hidden_size");
  p.I = w2->dims[2] * pack;
  if (p.I <= 0 || p.H <= 0) return fail(MOE_INVALID_ARGUMENT, "hidden and inter sizes must be positive");

  const bool swiglu = at.activation_type == MOE_ACT_SWIGLU;
  if (w3) {
    if (swiglu && at.swiglu_fusion != 0)
      return fail(MOE_INVALID_ARGUMENT, "fc3 weights require swiglu_fusion = 0");
    p.gate_mode = moe::kGateFc3;
    p.N1 = p.I;
    if (w3->rank != 3 || w3->dims[0] != p.E || w3->dims[1] != p.I || w3->dims[2] * pack != p.H)
      return fail(MOE_INVALID_ARGUMENT, "fc3_experts_weights must be [E, inter, hidden/pack], got " + dims_str(*w3));
    if (q && !s3) return fail(MOE_INVALID_ARGUMENT, "fc3_scales required with fc3_experts_weights");
  } else if (swiglu) {
    if (at.swiglu_fusion == 1) p.gate_mode = moe::kGateInterleaved;
    else if (at.swiglu_fusion == 2) p.gate_mode = moe::kGateChunked;
    else
      return fail(MOE_NOT_IMPLEMENTED,
                  "swiglu without fc3 needs fused fc1 weights (swiglu_fusion 1 or 2)");
    p.N1 = 2 * p.I;
  } else {
    p.N1 = p.I;
  }
  if (w1->dims[1] != p.N1)
    return fail(MOE_INVALID_ARGUMENT, "fc1_experts_weights dim 1 must be " + std::to_string(p.N1) + ", got " +
                                          dims_str(*w1));
  auto check_bias = [&](const moe_tensor* b, int64_t N, const char* name) -> moe_status {
    if (!b) return MOE_OK;
    if (b->elem_type != p.act_type || b->rank != 2 || b->dims[0] != p.E || b->dims[1] != N)
      return fail(MOE_INVALID_ARGUMENT, std::string(name) + " must be [" + std::to_string(p.E) + ", " +
                                            std::to_string(N) + "] of the input's type, got " + dims_str(*b));
    return MOE_OK;
  };
  moe_status st;
  if ((st = check_bias(b1, p.N1, "fc1_experts_bias")) != MOE_OK) return st;
  if ((st = check_bias(b2, p.H, "fc2_experts_bias")) != MOE_OK) return st;
  if ((st = check_bias(b3, p.I, "fc3_experts_bias")) != MOE_OK) return st;

  if (q) {
    const int64_t bs = p.block_size;
    if (bs > 0) {
      if (bs < 16 || (bs & (bs - 1)))
        return fail(MOE_INVALID_ARGUMENT, "block_size must be a power of two >= 16, got " + std::to_string(bs));
      if (p.H % bs || p.I % bs)
        return fail(MOE_INVALID_ARGUMENT, "block_size must divide hidden_size and inter_size");
    }
    auto check_scale = [&](const moe_tensor* s, int64_t N, int64_t K, const char* name) -> moe_status {
      const bool ok = bs > 0 ? (s->rank == 3 && s->dims[0] == p.E && s->dims[1] == N && s->dims[2] == K / bs)
                             : (s->rank == 2 && s->dims[0] == p.E && s->dims[1] == N);
      if (!ok)
        return fail(MOE_INVALID_ARGUMENT, std::string(name) + " has shape " + dims_str(*s) +
                                              (bs > 0 ? ", expected [E, N, K/block_size]" : ", expected [E, N]"));
      return MOE_OK;
    };
    if ((st = check_scale(s1, p.N1, p.H, "fc1_scales")) != MOE_OK) return st;
    if ((st = check_scale(s2, p.H, p.I, "fc2_scales")) != MOE_OK) return st;
    if (w3 && (st = check_scale(s3, p.I, p.H, "fc3_scales")) != MOE_OK) return st;
  }
  if (p.T * p.k > std::numeric_limits<int32_t>::max() / 2)
    return fail(MOE_NOT_IMPLEMENTED, "num_tokens * k exceeds the int32 row index range");
  *out = p;
  return MOE_OK;
}

// Inputs of one call with pre-packed weights in place of theirs: a packed
// input may come with data == NULL (shape taken from the packed tensor), or
// as the tensor that was packed (same data pointer, shape and type) or the
// packed copy itself.  Any other tensor is an error: the kernel would compute
// with the weights it packed, not with the ones given.
moe_status with_packed(const moe_kernel* kr, const moe_tensor* inputs, int32_t n, moe_tensor* local) {
  for (int32_t i = 0; i < n; ++i) local[i] = inputs[i];
  for (int32_t i = 0; i < n && i < 11; ++i) {
    const auto& pk = kr->packed[i];
    if (!pk.data) continue;
    if (inputs[i].data && inputs[i].data != pk.data) {
      bool same = inputs[i].elem_type == pk.src.elem_type && inputs[i].rank == pk.src.rank;
      for (int d = 0; same && d < pk.src.rank; ++d) same = inputs[i].dims[d] == pk.src.dims[d];
      if (!same)
        return fail(MOE_INVALID_ARGUMENT, "input " + std::to_string(i) + " " + dims_str(inputs[i]) +
                                              " differs from the pre-packed weights " + dims_str(pk.src));
      if (inputs[i].data != pk.src.data)
        return fail(MOE_INVALID_ARGUMENT, "input " + std::to_string(i) +
                                              " is not the tensor that was pre-packed (another data pointer); "
                                              "pass that tensor, its packed copy or NULL");
    }
    // the packed copy (whatever its descriptor) or NULL: the packed tensor's shape
    local[i] = pk.src;
    local[i].data = pk.data;
  }
  return MOE_OK;
}

bool env_set(const char* name) {
  const char* v = std::getenv(name);
  return v && *v && std::strcmp(v, "0") != 0;
}

// Input indices of the fc1 / fc2 / fc3 expert weights: QMoE 2, 5, 8; MoE
// 2, 4, 6.
int fc2_input(const moe_kernel* kr) { return kr->quantized ? 5 : 4; }
int fc3_input(const moe_kernel* kr) { return kr->quantized ? 8 : 6; }

// Bytes of one row's chunk of 128 k: int4 64, int8 128, 16-bit (MoE) 256.
int64_t chunk_bytes(const moe_kernel* kr) {
  if (!kr->quantized) return 256;
  return kr->attrs.expert_weight_bits == 4 ? 64 : 128;
}

// Bytes of the tile-major copy of expert-weight input idx, or 0 when the
// kernels read that input in the op's layout (see moe_prepack.hip).  A
// weight is packed when each expert's rows are whole 16-row tiles (the
// gate and linear halves of a fused fc1 each), rows are whole 16-byte
// pieces (K is padded to whole chunks of 128 in the copy), and the kernels
// that read it take tile-major weights: fp16/bf16 activations (MFMA paths,
// MoE weights of the activations' type); fc1/fc3 with K within one decode
// activation slice.
// Bytes of the tile-major copy of QMoE block-scale input idx (3 fc1, 6
// fc2, 9 fc3), or 0: scales are packed for the step-scale decode kernels
// (block 32 or 64; int4, or int8 with fp16 activations) when their weights
// are packed too (same row and K rules).
size_t prepack_scale_bytes(const moe_kernel* kr, int32_t idx, const moe_tensor* s, int32_t act_type) {
  const moe_attributes& at = kr->attrs;
  const int64_t bs = at.block_size;
  const bool mx = s->elem_type == MOE_ELEM_UINT8;  // MXFP4 E8M0 scales (block 32)
  if (bs != 32 && bs != 64) return 0;
  if (mx && (bs != 32 || at.expert_weight_bits != 4)) return 0;
  if (act_type != MOE_ELEM_FLOAT16 && act_type != MOE_ELEM_BFLOAT16) return 0;
  if (!mx && at.expert_weight_bits == 8 && act_type != MOE_ELEM_FLOAT16) return 0;
  const int64_t E = s->dims[0], N = s->dims[1], nblk = s->dims[2];
  const int64_t es = s->elem_type == MOE_ELEM_FLOAT ? 4 : (mx ? 1 : 2);
  if (N <= 0 || N % 16 || nblk <= 0) return 0;
  const int64_t nchunks = (nblk * bs + 127) / 128;
  const int64_t cbytes = at.expert_weight_bits == 4 ? 64 : 128;
  if (N * nchunks * cbytes >= (int64_t{1} << 31)) return 0;  // the weights' packing rule
  const bool swiglu = at.activation_type == MOE_ACT_SWIGLU;
  if (idx != 6) {
    if (nchunks * 128 > moe::kStreamMaxK) return 0;
    if (swiglu && (at.swiglu_fusion == 1 || at.swiglu_fusion == 2) && N % 32) return 0;
  }
  return static_cast<size_t>(E * N * nchunks * (128 / bs) * es);
}

moe_status prepack_bytes(const moe_kernel* kr, int32_t idx, const moe_tensor* w, int32_t act_type,
                         size_t* bytes) {
  *bytes = 0;
  const bool q = kr->quantized;
  const bool scales = q && (idx == 3 || idx == 6 || idx == 9);
  const bool weights = idx == 2 || idx == fc2_input(kr) || idx == fc3_input(kr);
  if (!weights && !scales)
    return fail(MOE_INVALID_ARGUMENT, q ? "input_index must be 2, 5 or 8 (QMoE expert weights) or 3, 6 or 9 "
                                          "(their scales), got " + std::to_string(idx)
                                        : "input_index must be 2, 4 or 6 (MoE expert weights), got " +
                                              std::to_string(idx));
  if (!w || !w->data) return fail(MOE_INVALID_ARGUMENT, "null weights");
  if (!is_float_type(act_type)) return fail(MOE_INVALID_ARGUMENT, "act_type must be a float type");
  if (scales) {
    // per output channel [E, N] (kept as given) or per block [E, N, K / block]
    if ((w->rank != 2 && w->rank != 3) || (!is_float_type(w->elem_type) && w->elem_type != MOE_ELEM_UINT8) ||
        w->dims[0] <= 0)
      return fail(MOE_INVALID_ARGUMENT, "QMoE scales must be 2D or 3D float (or uint8 E8M0), got " + dims_str(*w));
    if (w->rank == 3) *bytes = prepack_scale_bytes(kr, idx, w, act_type);
    return MOE_OK;
  }
  if (q && (w->elem_type != MOE_ELEM_UINT8 || w->rank != 3 || w->dims[0] <= 0))
    return fail(MOE_INVALID_ARGUMENT, "QMoE expert weights must be 3D uint8, got " + dims_str(*w));
  if (!q && (!is_float_type(w->elem_type) || w->rank != 3 || w->dims[0] <= 0))
    return fail(MOE_INVALID_ARGUMENT, "MoE expert weights must be 3D float, got " + dims_str(*w));
  if (act_type == MOE_ELEM_FLOAT) return MOE_OK;
  if (!q && w->elem_type != act_type) return MOE_OK;  // the op rejects the call: nothing to pack for
  const moe_attributes& at = kr->attrs;
  const int64_t cbytes = chunk_bytes(kr);
  const int64_t E = w->dims[0], N = w->dims[1], rb = w->dims[2] * (q ? 1 : 2);  // bytes of a row
  const bool swiglu = at.activation_type == MOE_ACT_SWIGLU;
  if (N <= 0 || N % 16 || rb <= 0 || rb % 16) return MOE_OK;
  const int64_t rbp = (rb + cbytes - 1) / cbytes * cbytes;  // padded to whole chunks
  if (N * rbp >= (int64_t{1} << 31)) return MOE_OK;        // 32-bit buffer offsets per expert
  if (idx != fc2_input(kr)) {
    if (rbp / cbytes * 128 > moe::kStreamMaxK) return MOE_OK;
    if (swiglu && (at.swiglu_fusion == 1 || at.swiglu_fusion == 2) && N % 32) return MOE_OK;
  }
  *bytes = static_cast<size_t>(E * N * rbp);
  return MOE_OK;
}

// Whether input idx is packed de-interleaved: the fused fc1 of interleaved
// SwiGLU (weights and scales).
bool prepack_deint(const moe_kernel* kr, int32_t idx) {
  return (idx == 2 || idx == 3) && kr->attrs.activation_type == MOE_ACT_SWIGLU && kr->attrs.swiglu_fusion == 1;
}

moe::ExpertArgs expert_args(const moe_kernel* kr, const Problem& p, const Layout& l, uint8_t* ws,
                            void* output) {
  const bool q = kr->quantized;
  moe::ExpertArgs a{};
  a.T = p.T; a.H = p.H; a.I = p.I; a.E = p.E; a.k = p.k;
  a.act_type = p.act_type;
  a.wfmt = p.wfmt;
  a.scale_type = p.scale_type;
  a.block_size = p.block_size;
  a.activation = kr->attrs.activation_type;
  a.gate_mode = p.gate_mode;
  a.alpha = kr->attrs.activation_alpha;
  a.beta = kr->attrs.activation_beta;
  a.limit = kr->attrs.has_swiglu_limit ? kr->attrs.swiglu_limit : std::numeric_limits<float>::infinity();
  a.offsets = reinterpret_cast<const int32_t*>(ws + l.offsets);
  a.perm = reinterpret_cast<const int32_t*>(ws + l.perm);
  a.inv_perm = reinterpret_cast<const int32_t*>(ws + l.inv_perm);
  a.topk_ids = reinterpret_cast<const int32_t*>(ws + l.topk_ids);
  a.topk_w = reinterpret_cast<const float*>(ws + l.topk_w);
  a.tile_offsets = reinterpret_cast<const int32_t*>(ws + l.tile_offsets);
  auto d = [&](int i) -> const void* { return p.in[i] ? p.in[i]->data : nullptr; };
  a.x = d(0);
  a.w1 = d(2);
  if (q) {
    a.s1 = d(3); a.b1 = d(4); a.w2 = d(5); a.s2 = d(6); a.b2 = d(7);
    a.w3 = d(8); a.s3 = d(9); a.b3 = d(10);
  } else {
    a.b1 = d(3); a.w2 = d(4); a.b2 = d(5); a.w3 = d(6); a.b3 = d(7);
  }
  a.tiled1 = kr->packed[2].data ? 1 : 0;
  a.tiled2 = kr->packed[fc2_input(kr)].data ? 1 : 0;
  a.deint1 = a.tiled1 && kr->packed[2].deint ? 1 : 0;
  a.stiled1 = q && kr->packed[3].data ? 1 : 0;
  a.stiled2 = q && kr->packed[6].data ? 1 : 0;
  a.mx = p.mx;
  a.act = ws + l.act;
  a.y2 = reinterpret_cast<float*>(ws + l.y2);
  a.y2_planes = 1;
  a.y2_half = 0;
  a.out = output;
  return a;
}

// Expert-kernel family of a call, -1 when none takes it.  Tile-major
// weights are read by the decode stream kernels and the prefill kernels only.
int choose_path(const moe_kernel* kr, const moe::ExpertArgs& a) {
  const int forced = kr->forced_path;
  const bool tiled = a.tiled1 || a.tiled2;
  bool decode = moe::decode_supported(a);
  if (decode && tiled) {
    const moe::DecodePlan pl = moe::plan_decode(a.T, a.H, a.I, a.E, a.k, a.wfmt, a.gate_mode);
    decode = (!a.tiled1 || pl.stream1) && (!a.tiled2 || pl.stream2);
  }
  const bool prefill = moe::prefill_supported(a);
  if (forced == moe::kPathSimt) return tiled ? -1 : moe::kPathSimt;
  if (forced == moe::kPathDecode) return decode ? moe::kPathDecode : -1;
  if (forced == moe::kPathPrefill) return prefill ? moe::kPathPrefill : -1;
  if (decode) return moe::kPathDecode;
  if (prefill) return moe::kPathPrefill;
  return tiled ? -1 : moe::kPathSimt;
}

moe_status hip_fail(hipError_t e, const char* what) {
  return fail(MOE_EP_FAIL, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace

extern "C" {

moe_status moe_attributes_init(moe_attributes* a, const char* op_type) {
  if (!a || !op_type) return fail(MOE_INVALID_ARGUMENT, "null argument");
  const bool q = std::strcmp(op_type, "QMoE") == 0;
  if (!q && std::strcmp(op_type, "MoE") != 0)
    return fail(MOE_INVALID_ARGUMENT, std::string("unknown op type ") + op_type);
  *a = moe_attributes{};
  a->k = 1;
  a->activation_type = MOE_ACT_RELU;
  a->normalize_routing_weights = 0;
  a->use_sparse_mixer = 0;
  a->swiglu_fusion = 0;
  a->has_swiglu_limit = 0;
  a->swiglu_limit = std::numeric_limits<float>::infinity();
  a->activation_alpha = 1.0f;
  a->activation_beta = 0.0f;
  a->expert_weight_bits = q ? 4 : 0;
  a->block_size = 0;
  a->router_sigmoid = 0;
  return MOE_OK;
}

moe_status moe_parse_activation(const char* name, int32_t* act) {
  if (!name || !act) return fail(MOE_INVALID_ARGUMENT, "null argument");
  static const std::pair<const char*, int32_t> kNames[] = {
      {"relu", MOE_ACT_RELU}, {"gelu", MOE_ACT_GELU}, {"silu", MOE_ACT_SILU},
      {"identity", MOE_ACT_IDENTITY}, {"swiglu", MOE_ACT_SWIGLU}};
  for (const auto& kv : kNames)
    if (std::strcmp(kv.first, name) == 0) {
      *act = kv.second;
      return MOE_OK;
    }
  return fail(MOE_INVALID_ARGUMENT, std::string("unsupported activation_type ") + name);
}

moe_status moe_kernel_create(const char* op_type, const moe_attributes* attrs, moe_kernel** out) {
  try {
    if (!op_type || !attrs || !out) return fail(MOE_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    const bool q = std::strcmp(op_type, "QMoE") == 0;
    if (!q && std::strcmp(op_type, "MoE") != 0)
      return fail(MOE_INVALID_ARGUMENT, std::string("unknown op type ") + op_type);
    const moe_attributes& a = *attrs;
    if (a.activation_type < MOE_ACT_RELU || a.activation_type > MOE_ACT_SWIGLU)
      return fail(MOE_INVALID_ARGUMENT, "invalid activation_type");
    if (a.use_sparse_mixer) return fail(MOE_NOT_IMPLEMENTED, "use_sparse_mixer is not supported");
    if (a.swiglu_fusion < 0 || a.swiglu_fusion > 2)
      return fail(MOE_INVALID_ARGUMENT, "swiglu_fusion must be 0, 1 or 2");
    if (a.k < 1) return fail(MOE_INVALID_ARGUMENT, "k must be >= 1");
    if (q && a.expert_weight_bits != 4 && a.expert_weight_bits != 8)
      return fail(MOE_INVALID_ARGUMENT, "expert_weight_bits must be 4 or 8, got " +
                                            std::to_string(a.expert_weight_bits));
    if (a.block_size < 0) return fail(MOE_INVALID_ARGUMENT, "block_size must be >= 0");
    if (a.block_size > 0 && (a.block_size < 16 || (a.block_size & (a.block_size - 1))))
      return fail(MOE_INVALID_ARGUMENT, "block_size must be a power of two >= 16");
    auto* k = new moe_kernel();
    k->quantized = q;
    k->attrs = a;
    k->trace = env_set("MOE_TRACE_KERNELS");
    k->debug_sync = env_set("MOE_DEBUG_SYNC");
    *out = k;
    return MOE_OK;
  } catch (const std::exception& e) {
    return fail(MOE_FAIL, e.what());
  }
}

moe_status moe_kernel_set_expert_path(moe_kernel* kernel, int32_t path) {
  if (!kernel) return fail(MOE_INVALID_ARGUMENT, "null kernel");
  if (path < -1 || path > moe::kPathPrefill) return fail(MOE_INVALID_ARGUMENT, "path must be -1..2");
  kernel->forced_path = path;
  return MOE_OK;
}

moe_status moe_kernel_prepack_size(const moe_kernel* kernel, int32_t input_index, const moe_tensor* weights,
                                   int32_t act_type, size_t* bytes) {
  try {
    if (!kernel || !bytes) return fail(MOE_INVALID_ARGUMENT, "null argument");
    return prepack_bytes(kernel, input_index, weights, act_type, bytes);
  } catch (const std::exception& e) {
    return fail(MOE_FAIL, e.what());
  }
}

moe_status moe_kernel_prepack(moe_kernel* kernel, int32_t input_index, const moe_tensor* weights, int32_t act_type,
                              void* dst, size_t dst_bytes, void* stream, int32_t* is_packed) {
  try {
    if (!kernel || !is_packed) return fail(MOE_INVALID_ARGUMENT, "null argument");
    *is_packed = 0;
    size_t need = 0;
    const moe_status st = prepack_bytes(kernel, input_index, weights, act_type, &need);
    if (st != MOE_OK) return st;
    if (need == 0) return MOE_OK;
    if (!dst || dst_bytes < need)
      return fail(MOE_INVALID_ARGUMENT, "pre-pack buffer too small: need " + std::to_string(need) + " bytes");
    if (reinterpret_cast<uintptr_t>(dst) % 16 || reinterpret_cast<uintptr_t>(weights->data) % 16)
      return fail(MOE_INVALID_ARGUMENT, "weights and pre-pack buffer must be 16-byte aligned");
    const int cbytes = static_cast<int>(chunk_bytes(kernel));
    const bool deint = prepack_deint(kernel, input_index);
    const bool scales = kernel->quantized && (input_index == 3 || input_index == 6 || input_index == 9);
    const hipError_t e =
        scales ? moe::launch_prepack_scales(weights->data, dst,
                                            weights->elem_type == MOE_ELEM_FLOAT ? 4
                                                : (weights->elem_type == MOE_ELEM_UINT8 ? 1 : 2),
                                            weights->dims[0] * weights->dims[1], weights->dims[2],
                                            static_cast<int>(kernel->attrs.block_size), weights->dims[1], deint,
                                            static_cast<hipStream_t>(stream))
               : moe::launch_prepack(static_cast<const uint8_t*>(weights->data), static_cast<uint8_t*>(dst),
                                     weights->dims[0] * weights->dims[1],
                                     weights->dims[2] * (kernel->quantized ? 1 : 2), cbytes, weights->dims[1],
                                     deint, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "pre-pack launch");
    kernel->packed[input_index].data = dst;
    kernel->packed[input_index].src = *weights;
    kernel->packed[input_index].deint = deint;
    *is_packed = 1;
    return MOE_OK;
  } catch (const std::exception& e) {
    return fail(MOE_FAIL, e.what());
  }
}

moe_status moe_kernel_workspace_size(const moe_kernel* kernel, const moe_tensor* inputs, int32_t n,
                                     size_t* bytes) {
  try {
    if (!kernel || !bytes) return fail(MOE_INVALID_ARGUMENT, "null argument");
    if (!inputs || n < 0 || n > 64) return fail(MOE_INVALID_ARGUMENT, "bad inputs");
    moe_tensor local[64];
    moe_status st = with_packed(kernel, inputs, n, local);
    if (st != MOE_OK) return st;
    Problem p;
    st = validate(kernel, local, n, &p);
    if (st != MOE_OK) return st;
    *bytes = plan_layout(p).total;
    return MOE_OK;
  } catch (const std::exception& e) {
    return fail(MOE_FAIL, e.what());
  }
}

moe_status moe_kernel_workspace_layout(const moe_kernel* kernel, const moe_tensor* inputs, int32_t n,
                                       moe_workspace_layout* out) {
  try {
    if (!kernel || !out) return fail(MOE_INVALID_ARGUMENT, "null argument");
    if (!inputs || n < 0 || n > 64) return fail(MOE_INVALID_ARGUMENT, "bad inputs");
    moe_tensor local[64];
    moe_status st = with_packed(kernel, inputs, n, local);
    if (st != MOE_OK) return st;
    Problem p;
    st = validate(kernel, local, n, &p);
    if (st != MOE_OK) return st;
    const Layout l = plan_layout(p);
    out->topk_ids = l.topk_ids;
    out->topk_w = l.topk_w;
    out->offsets = l.offsets;
    out->perm = l.perm;
    out->inv_perm = l.inv_perm;
    out->total = l.total;
    out->act = l.act;
    out->y2 = l.y2;
    out->y2_planes_max = static_cast<size_t>(l.y2_planes);
    out->logits = l.logits;
    return MOE_OK;
  } catch (const std::exception& e) {
    return fail(MOE_FAIL, e.what());
  }
}

}  // extern "C"

namespace {

// The router GEMM's operands: gate_w [E, H] of the input's type (the
// transposed B operand of the graph's MatMul(x, W[H, E])), gate_b [E] or
// NULL.  Fills the router_probs descriptor of `local` (shape [T, E]; its data
// is the workspace's logits buffer, set once the workspace is known).
moe_status gate_router_input(const moe_tensor* gate_w, const moe_tensor* gate_b, moe_tensor* local, int32_t n) {
  if (!gate_w || !gate_w->data) return fail(MOE_INVALID_ARGUMENT, "router_weight is required");
  if (n < 2) return fail(MOE_INVALID_ARGUMENT, "too few inputs");
  const moe_tensor& x = local[0];
  if (!x.data || (x.rank != 2 && x.rank != 3)) return fail(MOE_INVALID_ARGUMENT, "input must be 2D or 3D");
  const int64_t H = x.dims[x.rank - 1], T = x.dims[0] * (x.rank == 3 ? x.dims[1] : 1);
  if (gate_w->rank != 2 || gate_w->dims[1] != H || gate_w->dims[0] <= 0)
    return fail(MOE_INVALID_ARGUMENT, "router_weight must be [num_experts, hidden_size], got " + dims_str(*gate_w));
  if (gate_w->elem_type != x.elem_type) return fail(MOE_INVALID_ARGUMENT, "router_weight must have the input's type");
  const int64_t es = elem_size(x.elem_type);
  if (T * H * es >= (int64_t{1} << 31) || gate_w->dims[0] * H * es >= (int64_t{1} << 31))
    return fail(MOE_NOT_IMPLEMENTED, "the fused router reads input and router_weight with 32-bit offsets (< 2 GiB each)");
  if (gate_b && gate_b->data &&
      (gate_b->rank != 1 || gate_b->dims[0] != gate_w->dims[0] || gate_b->elem_type != x.elem_type))
    return fail(MOE_INVALID_ARGUMENT, "router_bias must be [num_experts] of the input's type, got " + dims_str(*gate_b));
  moe_tensor r{};
  r.data = gate_w->data;  // placeholder for validation; replaced by the logits buffer
  r.elem_type = x.elem_type;
  r.rank = 2;
  r.dims[0] = T;
  r.dims[1] = gate_w->dims[0];
  local[1] = r;
  return MOE_OK;
}

moe_status compute_impl(const moe_kernel* kernel, const moe_tensor* inputs, int32_t n, void* output,
                        void* workspace, size_t workspace_bytes, void* stream_ptr,
                        const moe_tensor* gate_w = nullptr, const moe_tensor* gate_b = nullptr) {
  try {
    if (!inputs || n < 0 || n > 64) return fail(MOE_INVALID_ARGUMENT, "bad inputs");
    moe_tensor local[64];
    moe_status st = with_packed(kernel, inputs, n, local);
    if (st != MOE_OK) return st;
    if (gate_w && (st = gate_router_input(gate_w, gate_b, local, n)) != MOE_OK) return st;
    Problem p;
    st = validate(kernel, local, n, &p);
    if (st != MOE_OK) return st;
    if (p.T == 0) return MOE_OK;
    if (!output) return fail(MOE_INVALID_ARGUMENT, "null output");
    const Layout l = plan_layout(p);
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    if (ws) {
      if (workspace_bytes < l.total)
        return fail(MOE_INVALID_ARGUMENT, "workspace too small: need " + std::to_string(l.total) + " bytes");
    } else {
      int dev = 0;
      hipError_t e = hipGetDevice(&dev);
      if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
      auto* mk = const_cast<moe_kernel*>(kernel);
      std::lock_guard<std::mutex> lock(mk->mu);
      auto& slot = mk->ws_cache[{dev, stream_ptr}];
      if (slot.second < l.total) {
        if (slot.first) {
          // the previous buffer may still be in use by work queued on this stream
          e = hipStreamSynchronize(stream);
          if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
          (void)hipFree(slot.first);
          slot = {nullptr, 0};
        }
        void* buf = nullptr;
        e = hipMalloc(&buf, l.total);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc(workspace)");
        slot = {buf, l.total};
      }
      ws = static_cast<uint8_t*>(slot.first);
    }

    moe::RouteArgs ra{};
    ra.p.logits = p.in[1]->data;
    ra.p.logits_type = p.act_type;
    ra.p.normalize = kernel->attrs.normalize_routing_weights;
    ra.p.sigmoid = kernel->attrs.router_sigmoid;
    ra.p.num_tokens = p.T;
    ra.p.num_experts = p.E;
    ra.p.k = p.k;
    ra.p.topk_ids = reinterpret_cast<int32_t*>(ws + l.topk_ids);
    ra.p.topk_w = reinterpret_cast<float*>(ws + l.topk_w);
    ra.p.offsets = reinterpret_cast<int32_t*>(ws + l.offsets);
    ra.p.perm = reinterpret_cast<int32_t*>(ws + l.perm);
    ra.p.inv_perm = reinterpret_cast<int32_t*>(ws + l.inv_perm);
    ra.p.scratch = ws + l.route_scratch;
    ra.p.scratch_bytes = l.route_scratch_bytes;
    ra.tile_offsets = reinterpret_cast<int32_t*>(ws + l.tile_offsets);
    ra.tile_m = moe::kPrefillTileM;
    if (gate_w) {
      ra.p.logits = ws + l.logits;
      ra.gate_x = p.in[0]->data;
      ra.gate_w = gate_w->data;
      ra.gate_b = gate_b ? gate_b->data : nullptr;
      ra.hidden = p.H;
    }
    moe::ExpertArgs a = expert_args(kernel, p, l, ws, output);
    auto packed = [&](int i) { return kernel->packed[i].data != nullptr; };
    const bool q = kernel->quantized;
    if (p.gate_mode == moe::kGateFc3 &&
        (packed(2) != packed(fc3_input(kernel)) || (q && packed(3) != packed(9))))
      return fail(MOE_NOT_IMPLEMENTED, "fc1 and fc3 weights (and scales) must both be pre-packed or neither");
    if (q && ((packed(3) && !packed(2)) || (packed(6) && !packed(5)) || (packed(9) && !packed(8))))
      return fail(MOE_NOT_IMPLEMENTED, "pre-packed scales need their weights pre-packed");
    const int path = choose_path(kernel, a);
    if (path < 0)
      return fail(MOE_NOT_IMPLEMENTED, kernel->forced_path >= 0
                                           ? "forced expert path does not support this problem"
                                           : "pre-packed weights need fp16/bf16 activations (MFMA kernels)");

    auto* mk = const_cast<moe_kernel*>(kernel);
    const bool prof = mk->profiling;
    hipError_t e = hipSuccess;
    auto mark = [&](int i) {
      if (prof && e == hipSuccess) e = hipEventRecord(mk->ev[i], stream);
    };
    // MOE_DEBUG_SYNC: wait for each stage and report the first that fails
    const char* failed_stage = nullptr;
    auto stage_done = [&](const char* name) {
      if (!kernel->debug_sync || e != hipSuccess) return;
      e = hipStreamSynchronize(stream);
      if (e == hipSuccess) e = hipGetLastError();
      if (e != hipSuccess) failed_stage = name;
    };
    // small decode batches are routed inside the fc1 kernel (one launch less)
    const bool route_in_fc1 = !gate_w && path == moe::kPathDecode && moe::decode_routes_in_fc1(a);
    mark(0);
    if (!route_in_fc1) {
      e = e == hipSuccess ? moe::launch_route_dispatch(ra, stream) : e;
      if (e != hipSuccess) return hip_fail(e, "router/dispatch launch");
      stage_done("router/dispatch");
    }
    mark(1);
    switch (path) {
      case moe::kPathDecode:
        e = e == hipSuccess ? moe::launch_fc1_decode(a, route_in_fc1 ? &ra.p : nullptr, stream) : e;
        stage_done("fc1 (decode)");
        mark(2);
        if (e == hipSuccess) e = moe::launch_fc2_decode(a, &a.y2_planes, stream);
        stage_done("fc2 (decode)");
        break;
      case moe::kPathPrefill:
        e = e == hipSuccess ? moe::launch_fc1_prefill(a, stream) : e;
        stage_done("fc1 (prefill)");
        mark(2);
        if (e == hipSuccess) e = moe::launch_fc2_prefill(a, &a.y2_planes, &a.y2_half, stream);
        stage_done("fc2 (prefill)");
        break;
      default:
        e = e == hipSuccess ? moe::launch_fc1_simt(a, stream) : e;
        stage_done("fc1 (simt)");
        mark(2);
        if (e == hipSuccess) e = moe::launch_fc2_simt(a, stream);
        stage_done("fc2 (simt)");
        break;
    }
    if (e != hipSuccess)
      return hip_fail(e, failed_stage ? (std::string("stage ") + failed_stage + " (MOE_DEBUG_SYNC)").c_str()
                                      : "expert launch");
    mark(3);
    e = moe::launch_finalize(a, stream);
    if (e != hipSuccess) return hip_fail(e, "finalize launch");
    stage_done("finalize");
    if (e != hipSuccess) return hip_fail(e, "stage finalize (MOE_DEBUG_SYNC)");
    mark(4);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
    mk->last_path = path;
    mk->ev_recorded = prof;
    return MOE_OK;
  } catch (const std::bad_alloc&) {
    return fail(MOE_FAIL, "out of host memory");
  } catch (const std::exception& e) {
    return fail(MOE_FAIL, e.what());
  }
}

}  // namespace

// Scratch of moe_kernel_compute_noalloc: the workspace of callers that
// cannot allocate device memory.  The host-side name is only a stand-in for
// the array: host code uses the device address that scratch_address() looks
// up once per device (each GPU holds its own copy, from the library's first
// use on it until the process ends).
static __device__ __align__(256) uint8_t scratch[MOE_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kScratchDevices = 64;
std::atomic<void*> g_scratch_ptr[kScratchDevices];
std::mutex g_scratch_mu;

// Device address of the current device's scratch array.
moe_status scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kScratchDevices)
    return fail(MOE_EP_FAIL, "device " + std::to_string(dev) + " is beyond the scratch table");
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
      if (!p) return fail(MOE_EP_FAIL, "hipGetSymbolAddress(scratch) returned NULL");
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return MOE_OK;
}

}  // namespace

extern "C" {

moe_status moe_kernel_compute(const moe_kernel* kernel, const moe_tensor* inputs, int32_t n, void* output,
                              void* workspace, size_t workspace_bytes, void* stream_ptr) {
  if (!kernel) return fail(MOE_INVALID_ARGUMENT, "null kernel");
  if (kernel->trace) {
    std::fprintf(stderr, "MOE_KERNEL_BEGIN %s kernel=%p\n", kernel->quantized ? "QMoE" : "MoE",
                 static_cast<const void*>(kernel));
    std::fflush(stderr);
  }
  const moe_status st = compute_impl(kernel, inputs, n, output, workspace, workspace_bytes, stream_ptr);
  if (kernel->trace) {
    std::fprintf(stderr, "MOE_KERNEL_END %s kernel=%p path=%d status=%d%s%s\n", kernel->quantized ? "QMoE" : "MoE",
                 static_cast<const void*>(kernel), kernel->last_path, static_cast<int>(st),
                 st == MOE_OK ? "" : " ", st == MOE_OK ? "" : g_last_error.c_str());
    std::fflush(stderr);
  }
  return st;
}

moe_status moe_kernel_compute_fused_router(const moe_kernel* kernel, const moe_tensor* inputs, int32_t n,
                                          const moe_tensor* router_weight, const moe_tensor* router_bias,
                                          void* output, void* workspace, size_t workspace_bytes, void* stream) {
  if (!kernel) return fail(MOE_INVALID_ARGUMENT, "null kernel");
  if (!router_weight) return fail(MOE_INVALID_ARGUMENT, "router_weight is required");
  if (kernel->trace) {
    std::fprintf(stderr, "MOE_KERNEL_BEGIN %s+router kernel=%p\n", kernel->quantized ? "QMoE" : "MoE",
                 static_cast<const void*>(kernel));
    std::fflush(stderr);
  }
  const moe_status st = compute_impl(kernel, inputs, n, output, workspace, workspace_bytes, stream, router_weight,
                                     router_bias && router_bias->data ? router_bias : nullptr);
  if (kernel->trace) {
    std::fprintf(stderr, "MOE_KERNEL_END %s+router kernel=%p path=%d status=%d%s%s\n",
                 kernel->quantized ? "QMoE" : "MoE", static_cast<const void*>(kernel), kernel->last_path,
                 static_cast<int>(st), st == MOE_OK ? "" : " ", st == MOE_OK ? "" : g_last_error.c_str());
    std::fflush(stderr);
  }
  return st;
}

moe_status moe_kernel_compute_noalloc(const moe_kernel* kernel, const moe_tensor* inputs, int32_t n, void* output,
                                      void* stream) {
  try {
    if (!kernel) return fail(MOE_INVALID_ARGUMENT, "null kernel");
    size_t need = 0;
    moe_status st = moe_kernel_workspace_size(kernel, inputs, n, &need);
    if (st != MOE_OK) return st;
    if (need > MOE_NOALLOC_SCRATCH_BYTES)
      return fail(MOE_INVALID_ARGUMENT, "moe_kernel_compute_noalloc: this call needs " + std::to_string(need) +
                                            " bytes of workspace, more than the library's scratch (" +
                                            std::to_string(static_cast<size_t>(MOE_NOALLOC_SCRATCH_BYTES)) +
                                            " bytes); pass a workspace to moe_kernel_compute instead");
    void* ws = nullptr;
    st = scratch_address(&ws);
    if (st != MOE_OK) return st;
    return moe_kernel_compute(kernel, inputs, n, output, ws, MOE_NOALLOC_SCRATCH_BYTES, stream);
  } catch (const std::exception& e) {
    return fail(MOE_FAIL, e.what());
  }
}

void moe_kernel_release(moe_kernel* kernel) { delete kernel; }

moe_status moe_kernel_set_profiling(moe_kernel* kernel, int32_t enable) {
  if (!kernel) return fail(MOE_INVALID_ARGUMENT, "null kernel");
  if (enable && !kernel->ev[0]) {
    for (auto& ev : kernel->ev) {
      const hipError_t e = hipEventCreate(&ev);
      if (e != hipSuccess) return hip_fail(e, "hipEventCreate");
    }
  }
  kernel->profiling = enable != 0;
  kernel->ev_recorded = false;
  return MOE_OK;
}

moe_status moe_kernel_stage_times(moe_kernel* kernel, float* ms, int32_t* path) {
  if (!kernel || !ms) return fail(MOE_INVALID_ARGUMENT, "null argument");
  if (!kernel->ev_recorded) return fail(MOE_INVALID_ARGUMENT, "no profiled call recorded");
  hipError_t e = hipEventSynchronize(kernel->ev[4]);
  if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
  for (int i = 0; i < 4; ++i) {
    e = hipEventElapsedTime(&ms[i], kernel->ev[i], kernel->ev[i + 1]);
    if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
  }
  if (path) *path = kernel->last_path;
  return MOE_OK;
}

const char* moe_last_error(void) { return g_last_error.c_str(); }

size_t moe_route_dispatch_scratch_size(int64_t num_tokens, int64_t num_experts, int64_t k) {
  return moe::route_scratch_bytes(num_tokens, num_experts, k);
}

moe_status moe_topk_launch(const moe_topk_params* p, void* stream) {
  try {
    if (!p) return fail(MOE_INVALID_ARGUMENT, "null params");
    if (p->rows < 0 || p->dim < 0 || p->inner < 0) return fail(MOE_INVALID_ARGUMENT, "negative shape");
    if (p->largest != 0 && p->largest != 1) return fail(MOE_INVALID_ARGUMENT, "TopK largest must be 0 or 1");
    if (p->sorted != 0 && p->sorted != 1) return fail(MOE_INVALID_ARGUMENT, "TopK sorted must be 0 or 1");
    if (p->k < 0 || p->k > p->dim) return fail(MOE_INVALID_ARGUMENT, "TopK K value is outside axis range");
    switch (p->elem_type) {
      case MOE_ELEM_FLOAT: case MOE_ELEM_FLOAT16: case MOE_ELEM_BFLOAT16:
      case MOE_ELEM_DOUBLE: case MOE_ELEM_INT32: case MOE_ELEM_INT64: break;
      default: return fail(MOE_NOT_IMPLEMENTED, "TopK unsupported dtype");
    }
    if (p->rows * p->inner == 0 || p->k == 0) return MOE_OK;
    if (p->dim > moe::kTopKMaxDim && (p->k > moe::kTopKRadixMaxK || p->dim > moe::kTopKRadixMaxDim))
      return fail(MOE_NOT_IMPLEMENTED, "TopK with k > " + std::to_string(moe::kTopKRadixMaxK) +
                                           " on an axis longer than " + std::to_string(moe::kTopKMaxDim) +
                                           " (or an axis of 2^31 or more)");
    if (!p->input || !p->values || !p->indices) return fail(MOE_INVALID_ARGUMENT, "null tensor");
    const moe::TopKArgs a{p->rows, p->dim, p->inner, p->k, p->largest, p->sorted};
    const hipError_t e = moe::launch_topk(p->input, p->elem_type, p->values, p->indices, a,
                                          static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "TopK launch");
    return MOE_OK;
  } catch (const std::exception& e) {
    return fail(MOE_FAIL, e.what());
  }
}

moe_status moe_softmax_launch(const moe_softmax_params* p, void* stream) {
  try {
    if (!p) return fail(MOE_INVALID_ARGUMENT, "null params");
    if (p->outer < 0 || p->dim < 0 || p->inner < 0) return fail(MOE_INVALID_ARGUMENT, "negative shape");
    switch (p->elem_type) {
      case MOE_ELEM_FLOAT: case MOE_ELEM_FLOAT16: case MOE_ELEM_BFLOAT16: case MOE_ELEM_DOUBLE: break;
      default: return fail(MOE_NOT_IMPLEMENTED, "Softmax unsupported dtype");
    }
    if (p->outer * p->dim * p->inner == 0) return MOE_OK;
    if (!p->input || !p->output) return fail(MOE_INVALID_ARGUMENT, "null tensor");
    const hipError_t e = moe::launch_softmax(p->input, p->output, p->elem_type, p->outer, p->dim, p->inner,
                                             static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "Softmax launch");
    return MOE_OK;
  } catch (const std::exception& e) {
    return fail(MOE_FAIL, e.what());
  }
}

moe_status moe_route_dispatch_launch(const moe_route_params* params, void* stream) {
  if (!params) return fail(MOE_INVALID_ARGUMENT, "null params");
  const moe_route_params& p = *params;
  if (p.num_tokens < 0 || p.num_experts <= 0 || p.k < 1 || p.k > p.num_experts)
    return fail(MOE_INVALID_ARGUMENT, "bad routing shape");
  if (p.num_experts > moe::kMaxExperts || p.k > moe::kMaxTopK)
    return fail(MOE_NOT_IMPLEMENTED, "routing shape beyond supported limits");
  if (!is_float_type(p.logits_type)) return fail(MOE_INVALID_ARGUMENT, "bad logits type");
  if (p.num_tokens > 0 && (!p.logits || !p.topk_ids || !p.topk_w || !p.offsets || !p.perm || !p.inv_perm))
    return fail(MOE_INVALID_ARGUMENT, "null routing buffer");
  const size_t need = moe::route_scratch_bytes(p.num_tokens, p.num_experts, p.k);
  if (need > 0 && (!p.scratch || p.scratch_bytes < need))
    return fail(MOE_INVALID_ARGUMENT, "routing scratch too small: need " + std::to_string(need));
  moe::RouteArgs ra{};
  ra.p = p;
  ra.tile_offsets = nullptr;
  ra.tile_m = moe::kPrefillTileM;
  const hipError_t e = moe::launch_route_dispatch(ra, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "router/dispatch launch");
  return MOE_OK;
}

const char* moe_version(void) { return "moe-mi355x 0.1.0 (gfx950)"; }

}  // extern "C"
