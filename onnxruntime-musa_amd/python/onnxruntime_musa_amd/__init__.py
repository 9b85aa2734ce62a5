"""MI355X (gfx950) MoE / QMoE kernels for ONNX Runtime.

Mirrors the reference's Python package surface
(musa/ep/python/onnxruntime_musa/__init__.py:18-40: get_library_path(),
get_ep_name()) and adds the host-side op mirror used by tests and benchmarks:

    from onnxruntime_musa_amd import MoE, QMoE
    op = QMoE(k=2, activation_type="swiglu", expert_weight_bits=4, block_size=128)
    y = op(x, router_logits, fc1_w, fc1_s, None, fc2_w, fc2_s, None, fc3_w, fc3_s)

Every call runs the hand-written HIP kernels of lib/libmoe_mi355x.so; there is
no CPU or PyTorch fallback.  A missing library raises at import of the op.
"""
from ._capi import get_library_path, load_library, MoeError  # noqa: F401
from .ops import MoE, QMoE, route_dispatch, softmax, topk  # noqa: F401

EP_NAME = "MI355XExecutionProvider"


def get_ep_name() -> str:
    """Name under which the plugin registers its execution provider."""
    return EP_NAME


__all__ = ["get_library_path", "get_ep_name", "load_library", "MoeError", "MoE", "QMoE",
           "route_dispatch", "EP_NAME"]
