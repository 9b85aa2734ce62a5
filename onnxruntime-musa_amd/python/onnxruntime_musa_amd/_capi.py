"""ctypes binding of include/moe_mi355x.h (the library's C ABI)."""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

_PKG_ROOT = Path(__file__).resolve().parents[2]  # onnxruntime-musa_amd/
LIB_NAME = "libmoe_mi355x.so"

MOE_OK, MOE_FAIL, MOE_INVALID_ARGUMENT, MOE_NOT_IMPLEMENTED, MOE_EP_FAIL = 0, 1, 2, 9, 11
STATUS_NAMES = {0: "OK", 1: "FAIL", 2: "INVALID_ARGUMENT", 9: "NOT_IMPLEMENTED", 11: "EP_FAIL"}

ELEM_FLOAT, ELEM_UINT8, ELEM_FLOAT16, ELEM_BFLOAT16 = 1, 2, 10, 16
ELEM_INT32, ELEM_INT64, ELEM_DOUBLE = 6, 7, 11
ACTIVATIONS = {"relu": 0, "gelu": 1, "silu": 2, "identity": 3, "swiglu": 4}
PATHS = {"auto": -1, "simt": 0, "decode": 1, "prefill": 2}


class MoeError(RuntimeError):
    """A non-OK moe_status; .code is the OrtErrorCode-numbered status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {message}")
        self.code = code


class MoeAttributes(ctypes.Structure):
    _fields_ = [
        ("k", ctypes.c_int64),
        ("activation_type", ctypes.c_int32),
        ("normalize_routing_weights", ctypes.c_int32),
        ("use_sparse_mixer", ctypes.c_int32),
        ("swiglu_fusion", ctypes.c_int32),
        ("has_swiglu_limit", ctypes.c_int32),
        ("swiglu_limit", ctypes.c_float),
        ("activation_alpha", ctypes.c_float),
        ("activation_beta", ctypes.c_float),
        ("expert_weight_bits", ctypes.c_int64),
        ("block_size", ctypes.c_int64),
        ("router_sigmoid", ctypes.c_int32),
    ]


class MoeTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("elem_type", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("dims", ctypes.c_int64 * 4),
    ]


class MoeWorkspaceLayout(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in ("topk_ids", "topk_w", "offsets", "perm", "inv_perm", "total",
                                               "act", "y2", "y2_planes_max", "logits")]


class MoeRouteParams(ctypes.Structure):
    _fields_ = [
        ("logits", ctypes.c_void_p),
        ("logits_type", ctypes.c_int32),
        ("normalize", ctypes.c_int32),
        ("sigmoid", ctypes.c_int32),
        ("pad_", ctypes.c_int32),
        ("num_tokens", ctypes.c_int64),
        ("num_experts", ctypes.c_int64),
        ("k", ctypes.c_int64),
        ("topk_ids", ctypes.c_void_p),
        ("topk_w", ctypes.c_void_p),
        ("offsets", ctypes.c_void_p),
        ("perm", ctypes.c_void_p),
        ("inv_perm", ctypes.c_void_p),
        ("scratch", ctypes.c_void_p),
        ("scratch_bytes", ctypes.c_size_t),
    ]


class MoeTopKParams(ctypes.Structure):
    _fields_ = [
        ("input", ctypes.c_void_p),
        ("elem_type", ctypes.c_int32),
        ("largest", ctypes.c_int32),
        ("sorted", ctypes.c_int32),
        ("pad_", ctypes.c_int32),
        ("rows", ctypes.c_int64),
        ("dim", ctypes.c_int64),
        ("inner", ctypes.c_int64),
        ("k", ctypes.c_int64),
        ("values", ctypes.c_void_p),
        ("indices", ctypes.c_void_p),
    ]


class MoeSoftmaxParams(ctypes.Structure):
    _fields_ = [
        ("input", ctypes.c_void_p),
        ("output", ctypes.c_void_p),
        ("elem_type", ctypes.c_int32),
        ("pad_", ctypes.c_int32),
        ("outer", ctypes.c_int64),
        ("dim", ctypes.c_int64),
        ("inner", ctypes.c_int64),
    ]


# (name, restype, argtypes) of every function the header declares.
EXPORTS = [
    ("moe_attributes_init", ctypes.c_int, [ctypes.POINTER(MoeAttributes), ctypes.c_char_p]),
    ("moe_parse_activation", ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int32)]),
    ("moe_kernel_create", ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(MoeAttributes),
                                         ctypes.POINTER(ctypes.c_void_p)]),
    ("moe_kernel_workspace_size", ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(MoeTensor), ctypes.c_int32,
                                                 ctypes.POINTER(ctypes.c_size_t)]),
    ("moe_kernel_compute", ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(MoeTensor), ctypes.c_int32,
                                          ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    ("moe_kernel_release", None, [ctypes.c_void_p]),
    ("moe_kernel_compute_fused_router", ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(MoeTensor), ctypes.c_int32,
                                                       ctypes.POINTER(MoeTensor), ctypes.POINTER(MoeTensor),
                                                       ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                                       ctypes.c_void_p]),
    ("moe_kernel_compute_noalloc", ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(MoeTensor), ctypes.c_int32,
                                                  ctypes.c_void_p, ctypes.c_void_p]),
    ("moe_kernel_workspace_layout", ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(MoeTensor), ctypes.c_int32,
                                                   ctypes.POINTER(MoeWorkspaceLayout)]),
    ("moe_kernel_set_expert_path", ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32]),
    ("moe_kernel_prepack_size", ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(MoeTensor),
                                               ctypes.c_int32, ctypes.POINTER(ctypes.c_size_t)]),
    ("moe_kernel_prepack", ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(MoeTensor), ctypes.c_int32,
                                          ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                          ctypes.POINTER(ctypes.c_int32)]),
    ("moe_kernel_set_profiling", ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32]),
    ("moe_kernel_stage_times", ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_float),
                                              ctypes.POINTER(ctypes.c_int32)]),
    ("moe_last_error", ctypes.c_char_p, []),
    ("moe_route_dispatch_scratch_size", ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]),
    ("moe_route_dispatch_launch", ctypes.c_int, [ctypes.POINTER(MoeRouteParams), ctypes.c_void_p]),
    ("moe_topk_launch", ctypes.c_int, [ctypes.POINTER(MoeTopKParams), ctypes.c_void_p]),
    ("moe_softmax_launch", ctypes.c_int, [ctypes.POINTER(MoeSoftmaxParams), ctypes.c_void_p]),
    ("moe_version", ctypes.c_char_p, []),
]

_lib = None


def get_library_path() -> str:
    """Absolute path of the in-tree built library (MOE_MI355X_LIBRARY overrides)."""
    env = os.environ.get("MOE_MI355X_LIBRARY")
    if env:
        return str(Path(env).resolve())
    return str(_PKG_ROOT / "lib" / LIB_NAME)


def load_library():
    """Loads the HIP library once.  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = get_library_path()
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} not found: build it first (python -c 'import __graft_entry__ as g; g.build()' "
            "or make -C onnxruntime-musa_amd)")
    lib = ctypes.CDLL(path)
    for name, res, args in EXPORTS:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status: int) -> None:
    if status != MOE_OK:
        msg = load_library().moe_last_error()
        raise MoeError(status, msg.decode() if msg else "")
