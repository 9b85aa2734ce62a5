"""Host-side mirror of the com.microsoft MoE / QMoE op kernels.

One object per graph node, like the reference's kernel object: attributes are
fixed at construction (musa/ep/src/kernels/llm/attention.cc:63-72 reads them
in the constructor through AttrOrDefault, kernel_attributes.h:21-28), and each
call validates inputs and enqueues the HIP kernels on the current torch stream
(the role of Compute, attention.cc:100-256).  Inputs follow the op schema
order; pass None for an absent optional input.  Tensors must be contiguous
and resident on the GPU: torch provides device memory and streams only, all
arithmetic runs in lib/libmoe_mi355x.so.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import torch

from ._capi import (ACTIVATIONS, ELEM_BFLOAT16, ELEM_DOUBLE, ELEM_FLOAT, ELEM_FLOAT16, ELEM_INT32, ELEM_INT64,
                    ELEM_UINT8, PATHS, MoeAttributes, MoeError, MoeRouteParams, MoeSoftmaxParams, MoeTensor,
                    MoeTopKParams, MoeWorkspaceLayout, check, load_library)

_ELEM = {torch.float32: ELEM_FLOAT, torch.float16: ELEM_FLOAT16, torch.bfloat16: ELEM_BFLOAT16,
         torch.uint8: ELEM_UINT8}

MOE_INPUTS = ("input", "router_probs", "fc1_experts_weights", "fc1_experts_bias", "fc2_experts_weights",
              "fc2_experts_bias", "fc3_experts_weights", "fc3_experts_bias")
QMOE_INPUTS = ("input", "router_probs", "fc1_experts_weights", "fc1_scales", "fc1_experts_bias",
               "fc2_experts_weights", "fc2_scales", "fc2_experts_bias", "fc3_experts_weights", "fc3_scales",
               "fc3_experts_bias")


def _tensor_desc(t: Optional[torch.Tensor]) -> MoeTensor:
    d = MoeTensor()
    if t is None:
        d.data = None
        return d
    if not t.is_cuda:
        raise ValueError("MoE inputs must be GPU tensors")
    if not t.is_contiguous():
        raise ValueError("MoE inputs must be contiguous")
    if t.dim() > 4:
        raise ValueError("rank > 4")
    if t.dtype not in _ELEM:
        raise ValueError(f"unsupported dtype {t.dtype}")
    d.data = t.data_ptr() if t.numel() else 1  # non-null marker for empty tensors
    d.elem_type = _ELEM[t.dtype]
    d.rank = t.dim()
    for i, s in enumerate(t.shape):
        d.dims[i] = s
    return d


class _MoEOp:
    op_type = "MoE"
    input_names: Sequence[str] = MOE_INPUTS

    def __init__(self, *, k: int = 1, activation_type: str = "relu", normalize_routing_weights: int = 0,
                 use_sparse_mixer: int = 0, swiglu_fusion: int = 0, swiglu_limit: Optional[float] = None,
                 activation_alpha: float = 1.0, activation_beta: float = 0.0, expert_weight_bits: int = 4,
                 block_size: int = 0, router_sigmoid: int = 0, expert_path: str = "auto"):
        self._lib = load_library()
        lib = self._lib
        a = MoeAttributes()
        check(lib.moe_attributes_init(ctypes.byref(a), self.op_type.encode()))
        act = ctypes.c_int32()
        check(lib.moe_parse_activation(activation_type.encode(), ctypes.byref(act)))
        a.k = int(k)
        a.activation_type = act.value
        a.normalize_routing_weights = int(normalize_routing_weights)
        a.use_sparse_mixer = int(use_sparse_mixer)
        a.swiglu_fusion = int(swiglu_fusion)
        if swiglu_limit is not None:
            a.has_swiglu_limit = 1
            a.swiglu_limit = float(swiglu_limit)
        a.activation_alpha = float(activation_alpha)
        a.activation_beta = float(activation_beta)
        if self.op_type == "QMoE":
            a.expert_weight_bits = int(expert_weight_bits)
            a.block_size = int(block_size or 0)
        a.router_sigmoid = int(router_sigmoid)
        h = ctypes.c_void_p()
        check(lib.moe_kernel_create(self.op_type.encode(), ctypes.byref(a), ctypes.byref(h)))
        self._h = h
        self.attributes = a
        self._packed = {}
        if expert_path != "auto":
            check(lib.moe_kernel_set_expert_path(h, PATHS[expert_path]))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.moe_kernel_release(h)
            self._h = None

    WEIGHT_INPUTS = ()

    def prepack(self, input_index: int, weights: torch.Tensor, act_dtype: torch.dtype,
                stream: Optional[torch.cuda.Stream] = None) -> Optional[torch.Tensor]:
        """Pre-packs one expert-weight input at session set-up: the role of
        ONNX Runtime's OpKernel::PrePack for a constant initializer.  Returns
        the tile-major device copy, which every later call reads in place of
        that input (the op keeps it alive), or None when the kernel reads that
        input in the op's layout."""
        d = _tensor_desc(weights)
        nb = ctypes.c_size_t()
        check(self._lib.moe_kernel_prepack_size(self._h, int(input_index), ctypes.byref(d), _ELEM[act_dtype],
                                                ctypes.byref(nb)))
        if nb.value == 0:
            return None
        s = stream if stream is not None else torch.cuda.current_stream(weights.device)
        with torch.cuda.stream(s):
            dst = torch.empty((nb.value,), dtype=torch.uint8, device=weights.device)
        packed = ctypes.c_int32()
        check(self._lib.moe_kernel_prepack(self._h, int(input_index), ctypes.byref(d), _ELEM[act_dtype],
                                           ctypes.c_void_p(dst.data_ptr()), nb.value, ctypes.c_void_p(s.cuda_stream),
                                           ctypes.byref(packed)))
        if not packed.value:
            return None
        self._packed[int(input_index)] = dst
        return dst

    def prepack_all(self, *inputs) -> list:
        """Pre-packs every expert-weight input present in a schema-ordered
        input list; returns the input indices that were packed."""
        done = []
        act = inputs[0].dtype
        for i in self.WEIGHT_INPUTS:
            if i < len(inputs) and inputs[i] is not None and self.prepack(i, inputs[i], act) is not None:
                done.append(i)
        return done

    def _descs(self, inputs):
        if len(inputs) > len(self.input_names):
            raise ValueError(f"{self.op_type} takes at most {len(self.input_names)} inputs")
        arr = (MoeTensor * len(inputs))(*[_tensor_desc(t) for t in inputs])
        return arr, len(inputs)

    def set_profiling(self, enable: bool = True) -> None:
        check(self._lib.moe_kernel_set_profiling(self._h, int(enable)))

    STAGES = ("route_dispatch", "fc1", "fc2", "finalize")
    PATH_NAMES = ("simt", "decode", "prefill")

    def stage_times(self) -> dict:
        """Stage durations (ms) of the last profiled call, from HIP events
        recorded on the call's stream; waits for that call to finish."""
        ms = (ctypes.c_float * 4)()
        path = ctypes.c_int32()
        check(self._lib.moe_kernel_stage_times(self._h, ms, ctypes.byref(path)))
        out = {n: float(ms[i]) for i, n in enumerate(self.STAGES)}
        out["path"] = self.PATH_NAMES[path.value]
        return out

    def workspace_size(self, *inputs) -> int:
        arr, n = self._descs(inputs)
        out = ctypes.c_size_t()
        check(self._lib.moe_kernel_workspace_size(self._h, arr, n, ctypes.byref(out)))
        return out.value

    def workspace_layout(self, *inputs) -> dict:
        arr, n = self._descs(inputs)
        lay = MoeWorkspaceLayout()
        check(self._lib.moe_kernel_workspace_layout(self._h, arr, n, ctypes.byref(lay)))
        return {name: getattr(lay, name) for name, _ in MoeWorkspaceLayout._fields_}

    def __call__(self, *inputs, out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
                 stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        arr, n = self._descs(inputs)
        x = inputs[0]
        s = stream if stream is not None else torch.cuda.current_stream(x.device)
        if out is None:
            with torch.cuda.stream(s):  # the caching allocator ties the block to the launch stream
                out = torch.empty_like(x)
        elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
            raise ValueError("out must match the input's shape and dtype")
        ws_ptr, ws_bytes = None, 0
        if workspace is not None:
            ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        check(self._lib.moe_kernel_compute(self._h, arr, n, out.data_ptr() if out.numel() else None, ws_ptr,
                                           ws_bytes, ctypes.c_void_p(s.cuda_stream)))
        return out

    def fused_router(self, *inputs, router_weight: torch.Tensor, router_bias: Optional[torch.Tensor] = None,
                     out: Optional[torch.Tensor] = None, workspace: Optional[torch.Tensor] = None,
                     stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        """The op with the router GEMM fused (moe_kernel_compute_fused_router):
        inputs in schema order with router_probs None; router_weight [E, H]
        (the transposed MatMul operand), router_bias [E] or None."""
        x = inputs[0]
        if inputs[1] is not None:
            raise ValueError("router_probs must be None: the fused router computes the logits")
        arr, n = self._descs(inputs)
        s = stream if stream is not None else torch.cuda.current_stream(x.device)
        if out is None:
            with torch.cuda.stream(s):
                out = torch.empty_like(x)
        elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
            raise ValueError("out must match the input's shape and dtype")
        wd = _tensor_desc(router_weight)
        bd = _tensor_desc(router_bias)
        ws_ptr, ws_bytes = None, 0
        if workspace is not None:
            ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        check(self._lib.moe_kernel_compute_fused_router(self._h, arr, n, ctypes.byref(wd), ctypes.byref(bd),
                                                        out.data_ptr() if out.numel() else None, ws_ptr, ws_bytes,
                                                        ctypes.c_void_p(s.cuda_stream)))
        return out

    def bind_fused_router(self, *inputs, router_weight: torch.Tensor, router_bias: Optional[torch.Tensor] = None,
                          out: torch.Tensor, workspace: torch.Tensor, stream: Optional[torch.cuda.Stream] = None):
        """bind() for the fused router: a zero-argument callable that enqueues
        one moe_kernel_compute_fused_router on fixed buffers."""
        arr, n = self._descs(inputs)
        s = stream if stream is not None else torch.cuda.current_stream(inputs[0].device)
        wd, bd = _tensor_desc(router_weight), _tensor_desc(router_bias)
        fn = self._lib.moe_kernel_compute_fused_router
        args = (self._h, arr, n, ctypes.byref(wd), ctypes.byref(bd), ctypes.c_void_p(out.data_ptr()),
                ctypes.c_void_p(workspace.data_ptr()), workspace.numel() * workspace.element_size(),
                ctypes.c_void_p(s.cuda_stream))
        keep = (inputs, router_weight, router_bias, out, workspace, wd, bd)

        def call():
            check(fn(*args))
            return keep[3]
        return call

    def compute_noalloc(self, *inputs, out: torch.Tensor, stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        """The op on the library's static scratch (moe_kernel_compute_noalloc):
        no device allocation, for callers that cannot allocate.  `out` is
        given by the caller.  Calls that overlap on one GPU race."""
        arr, n = self._descs(inputs)
        x = inputs[0]
        if out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
            raise ValueError("out must match the input's shape and dtype")
        s = stream if stream is not None else torch.cuda.current_stream(x.device)
        check(self._lib.moe_kernel_compute_noalloc(self._h, arr, n, out.data_ptr() if out.numel() else None,
                                                   ctypes.c_void_p(s.cuda_stream)))
        return out

    def bind(self, *inputs, out: torch.Tensor, workspace: torch.Tensor,
             stream: Optional[torch.cuda.Stream] = None):
        """Pre-builds the C arguments for repeated calls on fixed buffers (a
        serving loop); returns a zero-argument callable that enqueues one
        invocation.  The tensors must stay alive while the callable is used."""
        arr, n = self._descs(inputs)
        s = stream if stream is not None else torch.cuda.current_stream(inputs[0].device)
        fn = self._lib.moe_kernel_compute
        args = (self._h, arr, n, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(workspace.data_ptr()),
                workspace.numel() * workspace.element_size(), ctypes.c_void_p(s.cuda_stream))
        keep = (inputs, out, workspace)

        def call():
            check(fn(*args))
            return keep[1]
        return call


class MoE(_MoEOp):
    """com.microsoft MoE (float expert weights)."""
    op_type = "MoE"
    input_names = MOE_INPUTS
    # fc1, fc2, fc3 expert weights (packed when fp16 / bf16, like the activations)
    WEIGHT_INPUTS = (2, 4, 6)


class QMoE(_MoEOp):
    """com.microsoft QMoE (int8 / int4 expert weights with scales)."""
    op_type = "QMoE"
    input_names = QMOE_INPUTS
    # fc1, fc2, fc3 expert weights and their block scales (packed for the
    # step-scale decode kernels: block 32 / 64)
    WEIGHT_INPUTS = (2, 3, 5, 6, 8, 9)


def route_dispatch(logits: torch.Tensor, k: int, normalize: bool = False, sigmoid: bool = False,
                   stream: Optional[torch.cuda.Stream] = None) -> dict:
    """Runs the router + dispatch stage alone.  Returns device tensors
    topk_ids [T, k], topk_w [T, k], offsets [E+1], perm [T*k], inv_perm [T*k]."""
    lib = load_library()
    if logits.dim() != 2:
        raise ValueError("logits must be [T, E]")
    T, E = logits.shape
    dev = logits.device
    s = stream if stream is not None else torch.cuda.current_stream(dev)
    nscratch = lib.moe_route_dispatch_scratch_size(T, E, k)
    # results and scratch are allocated on the launch stream: the caching
    # allocator then reuses the scratch block (freed on return) only for work
    # ordered after this launch on that stream
    with torch.cuda.stream(s):
        res = {
            "topk_ids": torch.empty((T, k), dtype=torch.int32, device=dev),
            "topk_w": torch.empty((T, k), dtype=torch.float32, device=dev),
            "offsets": torch.empty((E + 1,), dtype=torch.int32, device=dev),
            "perm": torch.empty((T * k,), dtype=torch.int32, device=dev),
            "inv_perm": torch.empty((T * k,), dtype=torch.int32, device=dev),
        }
        scratch = torch.empty((max(nscratch, 1),), dtype=torch.uint8, device=dev)
    p = MoeRouteParams()
    p.logits = logits.data_ptr() if logits.numel() else None
    p.logits_type = _ELEM[logits.dtype]
    p.normalize = int(normalize)
    p.sigmoid = int(sigmoid)
    p.num_tokens, p.num_experts, p.k = T, E, k
    for name in ("topk_ids", "topk_w", "offsets", "perm", "inv_perm"):
        setattr(p, name, res[name].data_ptr() if res[name].numel() else None)
    p.scratch = scratch.data_ptr()
    p.scratch_bytes = nscratch
    check(lib.moe_route_dispatch_launch(ctypes.byref(p), ctypes.c_void_p(s.cuda_stream)))
    return res


_TOPK_ELEM = {torch.float32: ELEM_FLOAT, torch.float16: ELEM_FLOAT16, torch.bfloat16: ELEM_BFLOAT16,
              torch.float64: ELEM_DOUBLE, torch.int32: ELEM_INT32, torch.int64: ELEM_INT64}


def topk(x: torch.Tensor, k: int, axis: int = -1, largest: int = 1, sorted: int = 1,
         stream: Optional[torch.cuda.Stream] = None):
    """ONNX TopK (attributes axis, largest, sorted; K as a host integer, as
    the reference binds it to CPU memory, musa/ep/src/kernels/math/topk.cc:163-177).
    Returns (values, int64 indices) of shape x.shape with the axis cut to k."""
    lib = load_library()
    if x.dim() < 1:
        raise ValueError("TopK input rank must be at least 1")
    if not x.is_cuda or not x.is_contiguous():
        raise ValueError("TopK input must be a contiguous GPU tensor")
    ax = axis + x.dim() if axis < 0 else axis
    if not 0 <= ax < x.dim():
        raise ValueError("TopK axis out of range")
    shape = list(x.shape)
    rows = 1
    for d in shape[:ax]:
        rows *= d
    inner = 1
    for d in shape[ax + 1:]:
        inner *= d
    out_shape = shape[:ax] + [max(int(k), 0)] + shape[ax + 1:]
    s = stream if stream is not None else torch.cuda.current_stream(x.device)
    with torch.cuda.stream(s):
        values = torch.empty(out_shape, dtype=x.dtype, device=x.device)
        indices = torch.empty(out_shape, dtype=torch.int64, device=x.device)
    p = MoeTopKParams()
    p.input = x.data_ptr() if x.numel() else None
    p.elem_type = _TOPK_ELEM.get(x.dtype, 0)
    p.largest, p.sorted = int(largest), int(sorted)
    p.rows, p.dim, p.inner, p.k = rows, shape[ax], inner, int(k)
    p.values = values.data_ptr() if values.numel() else None
    p.indices = indices.data_ptr() if indices.numel() else None
    check(lib.moe_topk_launch(ctypes.byref(p), ctypes.c_void_p(s.cuda_stream)))
    return values, indices


def softmax(x: torch.Tensor, axis: int = -1, stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """ONNX Softmax (opset 13: along one axis, default -1) for float,
    float16, bfloat16 and double."""
    lib = load_library()
    if not x.is_cuda or not x.is_contiguous():
        raise ValueError("Softmax input must be a contiguous GPU tensor")
    if x.dim() == 0:
        raise ValueError("Softmax input rank must be at least 1")
    ax = axis + x.dim() if axis < 0 else axis
    if not 0 <= ax < x.dim():
        raise ValueError("Softmax axis out of range")
    outer = 1
    for d in x.shape[:ax]:
        outer *= d
    inner = 1
    for d in x.shape[ax + 1:]:
        inner *= d
    s = stream if stream is not None else torch.cuda.current_stream(x.device)
    with torch.cuda.stream(s):
        y = torch.empty_like(x)
    p = MoeSoftmaxParams()
    p.input = x.data_ptr() if x.numel() else None
    p.output = y.data_ptr() if y.numel() else None
    p.elem_type = _TOPK_ELEM.get(x.dtype, 0) if x.dtype.is_floating_point else 0
    p.outer, p.dim, p.inner = outer, x.shape[ax], inner
    check(lib.moe_softmax_launch(ctypes.byref(p), ctypes.c_void_p(s.cuda_stream)))
    return y


__all__ = ["MoE", "QMoE", "route_dispatch", "topk", "softmax", "MoeError", "MOE_INPUTS", "QMOE_INPUTS"]
