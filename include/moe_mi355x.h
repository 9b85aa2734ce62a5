/*
 * moe_mi355x.h -- C ABI of the MI355X (gfx950) MoE / QMoE library.
 *
 * The library implements the com.microsoft MoE and QMoE contrib ops (ONNX
 * Runtime 1.26 op schemas, since-version 1) as hand-written HIP kernels.
 * Everything here is plain C: pointers, sizes, enums and POD structs.  A HIP
 * stream is passed as `void*` (hipStream_t), as ORT hands it to a plugin
 * kernel through KernelContext::GetGPUComputeStream().
 *
 * Two layers are exported:
 *
 *   1. The op kernel (moe_kernel_*): what a Plugin-EP kernel registration
 *      binds.  It replaces, one for one, the reference's kernel object:
 *        moe_kernel_create   <- OpKernelBase<Derived>::CreateKernelImpl and the
 *                               attribute-reading constructor
 *                               (musa/ep/src/kernels/shared_inc/kernel_base.h:36-43,
 *                                pattern musa/ep/src/kernels/llm/attention.cc:63-72,
 *                                AttrOrDefault kernel_attributes.h:21-28)
 *        moe_kernel_compute  <- OpKernelBase<Derived>::ComputeImpl -> Derived::Compute
 *                               (kernel_base.h:45-84; attention.cc:100-256)
 *        moe_kernel_release  <- OpKernelBase<Derived>::ReleaseImpl (kernel_base.h:86-89)
 *      Inputs are given in the op's schema order (MoE: 8 inputs, QMoE: 11).
 *
 *      Extension beyond the 1.26 schema (whose QMoE scales T2 are float
 *      types): QMoE with uint8 scales reads MXFP4 experts (OCP Microscaling
 *      Formats v1.0, the format gpt-oss ships): expert weights are FP4 E2M1
 *      values two per byte, even k in the low nibble (the int4 packing),
 *      scales are E8M0 bytes (2^(e - 127), 0xFF = NaN) per block of 32 along
 *      K; expert_weight_bits must be 4 and block_size 32, and the three
 *      scale inputs must all be uint8.
 *
 *   2. Stage launchers (moe_route_dispatch_launch): the device-launcher layer
 *      below a kernel, following the reference convention of POD params +
 *      device pointers + stream returning a runtime status
 *      (musa/ep/src/kernels/math/topk_impl.h:10-33,
 *       shared_inc/device_kernel_types.h:258-266).
 *
 * Status codes use OrtErrorCode numbering so a Plugin-EP shim can pass them to
 * OrtApi::CreateStatus unchanged (the reference maps failures the same way:
 * ORT_INVALID_ARGUMENT for bad attributes/shapes, ORT_NOT_IMPLEMENTED for an
 * unsupported dtype/feature, ORT_EP_FAIL for runtime errors; e.g.
 * musa/ep/src/kernels/math/topk.cc:143-187, attention.cc:101-158).
 *
 * Threading: a moe_kernel is immutable after creation; moe_kernel_compute may
 * be called concurrently from several threads on different streams when each
 * call passes its own workspace.  With workspace == NULL the kernel uses a
 * workspace it caches per (device, stream), guarded by a mutex.
 *
 * Debugging (read from the environment when a kernel is created, the role of
 * the reference's MUSA_EP_TRACE_KERNELS / MUSA_EP_TRACE_SYNC,
 * musa/ep/src/kernels/shared_inc/kernel_base.h:48-80):
 *   MOE_TRACE_KERNELS=1  one MOE_KERNEL_BEGIN and one MOE_KERNEL_END line per
 *                        moe_kernel_compute call on stderr (the end line
 *                        carries the path and the status);
 *   MOE_DEBUG_SYNC=1     moe_kernel_compute waits for its stream after each
 *                        stage and returns MOE_EP_FAIL naming the first stage
 *                        that failed (this breaks the no-synchronisation
 *                        promise below on purpose).
 */
#ifndef MOE_MI355X_H_
#define MOE_MI355X_H_

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define MOE_API __attribute__((visibility("default")))
#else
#define MOE_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* OrtErrorCode numbering. */
typedef enum moe_status {
  MOE_OK = 0,
  MOE_FAIL = 1,
  MOE_INVALID_ARGUMENT = 2,
  MOE_NOT_IMPLEMENTED = 9,
  MOE_EP_FAIL = 11
} moe_status;

/* ONNX TensorProto element types, as the reference's MusaElementType
 * (musa/ep/src/kernels/shared_inc/device_kernel_types.h:47-62). */
typedef enum moe_elem_type {
  MOE_ELEM_FLOAT = 1,
  MOE_ELEM_UINT8 = 2,
  MOE_ELEM_INT32 = 6,   /* TopK only */
  MOE_ELEM_INT64 = 7,   /* TopK only */
  MOE_ELEM_FLOAT16 = 10,
  MOE_ELEM_DOUBLE = 11, /* TopK only */
  MOE_ELEM_BFLOAT16 = 16
} moe_elem_type;

typedef enum moe_activation {
  MOE_ACT_RELU = 0,
  MOE_ACT_GELU = 1,
  MOE_ACT_SILU = 2,
  MOE_ACT_IDENTITY = 3,
  MOE_ACT_SWIGLU = 4
} moe_activation;

/* Node attributes of com.microsoft MoE / QMoE.  moe_attributes_init() fills
 * the schema defaults; a shim sets each field it finds on the node. */
typedef struct moe_attributes {
  int64_t k;                         /* "k", default 1 */
  int32_t activation_type;           /* "activation_type", moe_activation, default relu */
  int32_t normalize_routing_weights; /* default 0 */
  int32_t use_sparse_mixer;          /* default 0; nonzero -> MOE_NOT_IMPLEMENTED */
  int32_t swiglu_fusion;             /* 0 unfused, 1 interleaved, 2 chunked; default 0 */
  int32_t has_swiglu_limit;          /* "swiglu_limit" present? */
  float swiglu_limit;
  float activation_alpha;            /* default 1.0 */
  float activation_beta;             /* default 0.0 */
  int64_t expert_weight_bits;        /* QMoE only, default 4 */
  int64_t block_size;                /* QMoE only, 0 = absent (per output channel) */
  int32_t router_sigmoid;            /* library extension: sigmoid instead of softmax, default 0 */
} moe_attributes;

/* A tensor handed to the kernel.  data == NULL marks an absent optional
 * input.  Device pointers (HBM); dims are row-major. */
typedef struct moe_tensor {
  const void *data;
  int32_t elem_type; /* moe_elem_type */
  int32_t rank;
  int64_t dims[4];
} moe_tensor;

typedef struct moe_kernel moe_kernel;

/* Fills `attrs` with the schema defaults of op_type ("MoE" or "QMoE"). */
MOE_API moe_status moe_attributes_init(moe_attributes *attrs, const char *op_type);

/* Parses the activation_type attribute string ("relu", "gelu", "silu",
 * "identity", "swiglu"). */
MOE_API moe_status moe_parse_activation(const char *name, int32_t *activation);

/* Creates an immutable kernel for one node.  Validates the attributes. */
MOE_API moe_status moe_kernel_create(const char *op_type, const moe_attributes *attrs,
                             moe_kernel **out);

/* Workspace bytes moe_kernel_compute needs for these inputs (shapes only are
 * read).  Validates shapes and types. */
MOE_API moe_status moe_kernel_workspace_size(const moe_kernel *kernel, const moe_tensor *inputs,
                                     int32_t num_inputs, size_t *bytes);

/* Runs the op: output is a device buffer of the input's shape and type.
 * All work is enqueued on `stream`; no device->host reads.  With a caller
 * workspace (at least moe_kernel_workspace_size bytes) the call allocates
 * nothing and does not synchronise.  workspace may be NULL: the kernel then
 * uses a workspace it caches per (device, stream).  The first call on a
 * (device, stream) allocates it (hipMalloc), and a later call that needs a
 * larger one waits for the stream (hipStreamSynchronize), frees the old
 * buffer and allocates a new one; calls that fit the cached size neither
 * allocate nor synchronise.  A caller that must not block passes a workspace
 * sized for its largest batch. */
MOE_API moe_status moe_kernel_compute(const moe_kernel *kernel, const moe_tensor *inputs,
                              int32_t num_inputs, void *output, void *workspace,
                              size_t workspace_bytes, void *stream);

MOE_API void moe_kernel_release(moe_kernel *kernel);

/* Router-GEMM fusion: the op with its router logits computed in the routing
 * kernels instead of taken as an input.  router_probs (inputs[1]) may be
 * absent (data == NULL; the other inputs as for moe_kernel_compute):
 *   logits[t, e] = sum_h input[t, h] * router_weight[e, h] (+ router_bias[e])
 * with fp32 accumulation, rounded once to the input's type (as the graph's
 * separate MatMul would store them), then routed as router_probs would be.
 * router_weight is [num_experts, hidden_size] of the input's type: the
 * transposed B operand of the MatMul(x, W[hidden, experts]) that feeds the
 * MoE node (a plugin EP transposes that initializer once, at set-up);
 * router_bias is [num_experts] or NULL.  The routing kernels compute each
 * token's logits and route it in the same launch.  This replaces the
 * MatMul -> MoE node pair that the reference's fusion machinery matches and
 * compiles into one node (musa/ep/src/fusion/fusion_matcher.h:26-34,
 * musa/ep/src/fusion/fusion_node_compute.cc:201-300).  The workspace is the
 * same as moe_kernel_compute's (moe_kernel_workspace_size with router_probs
 * described as [T, num_experts]; only shapes are read); the logits it
 * leaves there are at moe_workspace_layout.logits. */
MOE_API moe_status moe_kernel_compute_fused_router(const moe_kernel *kernel, const moe_tensor *inputs,
                                                   int32_t num_inputs, const moe_tensor *router_weight,
                                                   const moe_tensor *router_bias, void *output,
                                                   void *workspace, size_t workspace_bytes, void *stream);

/* Runs the op like moe_kernel_compute, allocating nothing: the workspace is
 * a static device array of the library, MOE_NOALLOC_SCRATCH_BYTES (64 MiB)
 * on each GPU it runs on, held from the library's first use of that GPU
 * until the process ends.  No counterpart in the reference: this is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops and harnesses that forbid hipMalloc).  It calls no
 * hipMalloc/hipFree and does not synchronise.  A problem whose workspace
 * (moe_kernel_workspace_size) exceeds the array returns
 * MOE_INVALID_ARGUMENT; decode batches fit (Mixtral-shaped QMoE at 64
 * tokens needs 19.5 MiB, gpt-oss-shaped at 512 tokens 34 MiB), large
 * prefill batches do not.  Every call on
 * one GPU uses the same array, so calls that overlap on one GPU (several
 * streams or threads) race: serialise them on one stream, or give each its
 * own workspace through moe_kernel_compute.  No part of the array needs
 * clearing between calls (each call writes every byte it reads). */
#define MOE_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
MOE_API moe_status moe_kernel_compute_noalloc(const moe_kernel *kernel, const moe_tensor *inputs,
                                              int32_t num_inputs, void *output, void *stream);

/* Byte offsets, inside a caller-provided workspace, of the routing results a
 * moe_kernel_compute call leaves there (int32 topk_ids[T*k], float
 * topk_w[T*k], int32 offsets[E+1], int32 perm[T*k], int32 inv_perm[T*k]) and
 * of the stage intermediates: act[T*k, I] (fc1/fc3 + activation output, input
 * type, rows in dispatch order) and y2[y2_planes_max][T*k, H] (fp32 fc2
 * partial sums over K ranges, bias in plane 0, rows in dispatch order; planes
 * a call does not use are left untouched; a 16-bit prefill call without a K
 * split writes one plane of the input type there instead).
 * Library extension for parity tests; no reference counterpart. */
typedef struct moe_workspace_layout {
  size_t topk_ids, topk_w, offsets, perm, inv_perm, total;
  size_t act, y2, y2_planes_max;
  size_t logits; /* [T, E] of the input's type: the fused router's logits */
} moe_workspace_layout;
MOE_API moe_status moe_kernel_workspace_layout(const moe_kernel *kernel, const moe_tensor *inputs,
                                       int32_t num_inputs, moe_workspace_layout *out);

/* Selects the expert-FFN kernel family: -1 automatic (default), 0 generic
 * SIMT, 1 weight-streaming decode, 2 MFMA prefill.  A forced family that does
 * not support a problem makes moe_kernel_compute return MOE_NOT_IMPLEMENTED.
 * Library extension for tests and benchmarks; no reference counterpart.
 * Call before the kernel is shared between threads. */
MOE_API moe_status moe_kernel_set_expert_path(moe_kernel *kernel, int32_t path);

/* Weight pre-pack at session initialisation: the role of ONNX Runtime's
 * OpKernel::PrePack(tensor, input_idx, alloc, is_packed, prepacked_weights)
 * (onnxruntime/core/framework/op_kernel.h of ORT 1.26, not vendored in the
 * reference; the reference carries the session option that shares pre-packed
 * weights, "ep.musa.enable_prepack_weight_sharing",
 * musa/ep/src/ep_factory.cc:472-478, musa/ep/src/ep.h:35).
 *
 * Expert weights (QMoE input_index 2 fc1, 5 fc2, 8 fc3; MoE 2 fc1, 4 fc2, 6
 * fc3, fp16 / bf16 weights of the activations' type; `weights` is the
 * constant initializer on the device) are reordered once into a tile-major
 * layout: each 16 rows x 128 k of an expert's [N, K/pack] matrix become one
 * contiguous block (1 KB int4, 2 KB int8, 4 KB 16-bit), so that every
 * weight load instruction of the decode and prefill kernels reads 1 KB
 * runs rather than one cache line per row; K is padded with zeros to whole
 * chunks of 128, and the fused fc1 of interleaved SwiGLU is stored with its
 * gate rows first and its linear rows after.  Block scales of block size 32
 * or 64 (input_index 3 fc1, 6 fc2, 9 fc3; int4, or int8 with fp16
 * activations) are packed the same way, the 16 rows' scales of each chunk
 * contiguous; they need their weights packed too.  act_type is the op's
 * input element type T (known from the node at kernel creation).
 *
 * moe_kernel_prepack_size: bytes of the packed copy, or 0 when the kernel
 *   reads that input in the op's layout (fp32 activations, MoE weights not
 *   of the activations' type, N not a multiple of 16 (32 for a fused fc1),
 *   rows not whole 16-byte pieces, fc1/fc3 K above 4096, scales of other
 *   block sizes).
 * moe_kernel_prepack: writes the packed copy into dst (device, at least that
 *   many bytes, 16-byte aligned) on stream, records dst and sets *is_packed.
 *   Every later compute (and workspace query) reads that input from dst; the
 *   caller may then pass data == NULL for it (its shape is taken from the
 *   packed tensor) or the same tensor (shape checked).  dst must stay valid
 *   while the kernel lives; the source may be freed once the stream has run
 *   the pack.  A later call that passes a tensor for a packed input must
 *   pass the one that was packed (same data pointer) or dst itself;
 *   another tensor, even of the same shape, is MOE_INVALID_ARGUMENT.  fc1
 *   and fc3 are packed together or not at all, and packed scales need
 *   packed weights (else compute returns MOE_NOT_IMPLEMENTED).  Call before
 *   the kernel is shared between threads. */
MOE_API moe_status moe_kernel_prepack_size(const moe_kernel *kernel, int32_t input_index,
                                           const moe_tensor *weights, int32_t act_type, size_t *bytes);
MOE_API moe_status moe_kernel_prepack(moe_kernel *kernel, int32_t input_index, const moe_tensor *weights,
                                      int32_t act_type, void *dst, size_t dst_bytes, void *stream,
                                      int32_t *is_packed);
/* Stage profiling (the role of the reference's EP profiler hooks,
 * musa/ep/src/ep_profiling.cc:141-288, with real producers): when enabled,
 * moe_kernel_compute records HIP events on its stream around each stage.
 * moe_kernel_stage_times waits for the last call's events and returns the
 * stage durations in milliseconds: ms[0] router+dispatch, ms[1] fc1 (+fc3,
 * activation), ms[2] fc2, ms[3] finalize; *path receives the expert-kernel
 * family used (0 SIMT, 1 decode, 2 prefill).  Single-threaded use only. */
MOE_API moe_status moe_kernel_set_profiling(moe_kernel *kernel, int32_t enable);
MOE_API moe_status moe_kernel_stage_times(moe_kernel *kernel, float *ms, int32_t *path);

/* Message of the last non-OK status returned on this thread. */
MOE_API const char *moe_last_error(void);

/* ------------------------------------------------------------------ */
/* Stage launcher: router (softmax/sigmoid + top-k, ties -> lower expert id)
 * and dispatch (per-expert histogram, exclusive scan, stable scatter).
 * Device outputs:
 *   topk_ids  [T*k] int32   expert of token t's j-th choice (j by descending logit)
 *   topk_w    [T*k] float   routing weight
 *   offsets   [E+1] int32   exclusive scan of per-expert counts (offsets[E] = T*k)
 *   perm      [T*k] int32   row -> flat index t*k+j, expert-major, tokens ascending
 *   inv_perm  [T*k] int32   flat index -> row
 * scratch: moe_route_dispatch_scratch_size() bytes of device memory. */
typedef struct moe_route_params {
  const void *logits;
  int32_t logits_type; /* moe_elem_type */
  int32_t normalize;
  int32_t sigmoid;
  int32_t pad_;
  int64_t num_tokens, num_experts, k;
  int32_t *topk_ids;
  float *topk_w;
  int32_t *offsets;
  int32_t *perm;
  int32_t *inv_perm;
  void *scratch;
  size_t scratch_bytes;
} moe_route_params;

MOE_API size_t moe_route_dispatch_scratch_size(int64_t num_tokens, int64_t num_experts, int64_t k);
MOE_API moe_status moe_route_dispatch_launch(const moe_route_params *params, void *stream);

/* ------------------------------------------------------------------ */
/* ONNX TopK (opsets 10-19) on the router's ordering rule: the k largest
 * (largest = 1) or smallest (largest = 0) elements along one axis, ties
 * toward the lower index, always in sorted order (sorted = 0 admits any
 * order).  The input is viewed as [rows, dim, inner] with the axis in the
 * middle; values [rows, k, inner] keep the input's type, indices are int64.
 * Types: float, float16, bfloat16, double, int32, int64.  -0.0 ties with
 * +0.0; every NaN (either sign, any payload) sorts above +inf, NaNs tied
 * with each other.  Any axis length; k up to 8192 on axes longer than 8192
 * (radix select), any k on shorter ones.  Replaces the reference's TopK kernel launchers
 * LaunchMusaTopK{PairReduce,BlockSort,...}Kernel(input, values, indices,
 * MusaTopKParams{rows, dim, inner, k, largest, sorted}, elem_type, stream)
 * (musa/ep/src/kernels/math/topk_impl.h:10-33,
 * shared_inc/device_kernel_types.h:258-266) and their validation
 * (musa/ep/src/kernels/math/topk.cc:133-200): k outside [0, dim] ->
 * MOE_INVALID_ARGUMENT, an unsupported type, or k > 8192 on an axis
 * longer than 8192 -> MOE_NOT_IMPLEMENTED. */
typedef struct moe_topk_params {
  const void *input;
  int32_t elem_type; /* moe_elem_type */
  int32_t largest;
  int32_t sorted;
  int32_t pad_;
  int64_t rows, dim, inner, k;
  void *values;
  int64_t *indices;
} moe_topk_params;
MOE_API moe_status moe_topk_launch(const moe_topk_params *params, void *stream);

/* ONNX Softmax (opset 13 semantics: one axis), the router's normalisation
 * as a stand-alone op: y = exp(x - max) / sum exp(x - max) along the axis of
 * the input viewed as [outer, dim, inner], accumulated in fp32 (fp64 for
 * double).  Types: float, float16, bfloat16, double.  Replaces the
 * reference's LaunchMusaSoftmaxKernel(input, output, outer, dim, inner,
 * elem_type, stream) (musa/ep/src/kernels/math/softmax_impl.h:5-8); an
 * unsupported type -> MOE_NOT_IMPLEMENTED, a negative size ->
 * MOE_INVALID_ARGUMENT. */
typedef struct moe_softmax_params {
  const void *input;
  void *output;
  int32_t elem_type; /* moe_elem_type */
  int32_t pad_;
  int64_t outer, dim, inner;
} moe_softmax_params;
MOE_API moe_status moe_softmax_launch(const moe_softmax_params *params, void *stream);

/* Library version string. */
MOE_API const char *moe_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MOE_MI355X_H_ */
