"""ctypes wrapper of the C restatement (oracle/libmoe_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, and only as the checker.  The product library
never loads it.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
# MOE_ORACLE_LIB selects another build of the same source (the sanitizer
# build of oracle/Makefile's sanitize-test target)
LIB = Path(os.environ.get("MOE_ORACLE_LIB") or HERE / "libmoe_oracle.so")

ORC_F32, ORC_U8, ORC_F16, ORC_BF16 = 1, 2, 10, 16
ACT = {"relu": 0, "gelu": 1, "silu": 2, "identity": 3, "swiglu": 4}
_DT = {"f32": ORC_F32, "f16": ORC_F16, "bf16": ORC_BF16}


class OrcArgs(ctypes.Structure):
    _fields_ = [
        ("num_tokens", ctypes.c_int64), ("hidden", ctypes.c_int64), ("inter", ctypes.c_int64),
        ("num_experts", ctypes.c_int64), ("k", ctypes.c_int64),
        ("activation", ctypes.c_int32), ("normalize", ctypes.c_int32), ("swiglu_fusion", ctypes.c_int32),
        ("swiglu_limit", ctypes.c_float), ("alpha", ctypes.c_float), ("beta", ctypes.c_float),
        ("router_sigmoid", ctypes.c_int32), ("quant_bits", ctypes.c_int32), ("block_size", ctypes.c_int64),
        ("act_dtype", ctypes.c_int32), ("scale_dtype", ctypes.c_int32),
        ("x", ctypes.c_void_p), ("logits", ctypes.c_void_p),
        ("w1", ctypes.c_void_p), ("s1", ctypes.c_void_p), ("b1", ctypes.c_void_p),
        ("w2", ctypes.c_void_p), ("s2", ctypes.c_void_p), ("b2", ctypes.c_void_p),
        ("w3", ctypes.c_void_p), ("s3", ctypes.c_void_p), ("b3", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("topk_ids", ctypes.c_void_p), ("topk_w", ctypes.c_void_p), ("expert_offsets", ctypes.c_void_p),
        ("perm", ctypes.c_void_p), ("out_f32", ctypes.c_void_p), ("token_mask", ctypes.c_void_p),
        ("num_threads", ctypes.c_int32), ("weight_format", ctypes.c_int32),
    ]


_lib = None


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise FileNotFoundError(f"{LIB} missing: run make -C oracle")
        lib = ctypes.CDLL(str(LIB))
        lib.orc_moe_forward.argtypes = [ctypes.POINTER(OrcArgs)]
        lib.orc_moe_forward.restype = ctypes.c_int
        lib.orc_route.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                  ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
        lib.orc_route.restype = ctypes.c_int
        lib.orc_dispatch.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                     ctypes.c_void_p, ctypes.c_void_p]
        lib.orc_dispatch.restype = ctypes.c_int
        lib.orc_dequant.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                    ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
        lib.orc_dequant.restype = ctypes.c_int
        lib.orc_dequant_mxfp4.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                          ctypes.c_void_p]
        lib.orc_dequant_mxfp4.restype = ctypes.c_int
        lib.orc_e2m1_to_f32.argtypes = [ctypes.c_uint32]
        lib.orc_e2m1_to_f32.restype = ctypes.c_float
        lib.orc_e8m0_to_f32.argtypes = [ctypes.c_uint32]
        lib.orc_e8m0_to_f32.restype = ctypes.c_float
        lib.orc_activation.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                       ctypes.c_int32, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                       ctypes.c_void_p]
        lib.orc_activation.restype = None
        for n in ("orc_f16_to_f32", "orc_bf16_to_f32"):
            getattr(lib, n).argtypes = [ctypes.c_uint16]
            getattr(lib, n).restype = ctypes.c_float
        for n in ("orc_f32_to_f16", "orc_f32_to_bf16"):
            getattr(lib, n).argtypes = [ctypes.c_float]
            getattr(lib, n).restype = ctypes.c_uint16
        _lib = lib
    return _lib


def _ptr(a: Optional[np.ndarray]):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def route(logits: np.ndarray, k: int, normalize: bool = False, sigmoid: bool = False):
    """fp32 logits [T, E] -> (ids [T,k] int32, w [T,k] float32)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = lg.shape
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    rc = load().orc_route(_ptr(lg), T, E, k, int(normalize), int(sigmoid), _ptr(ids), _ptr(w))
    if rc:
        raise ValueError(f"orc_route rc={rc}")
    return ids, w


def topk(x: np.ndarray, k: int, axis: int = -1, largest: int = 1):
    """ONNX TopK restated: along `axis`, the k largest (or smallest) values
    in sorted order, ties toward the lower index -- the reference's pair order
    (musa/ep/src/kernels/math/topk_impl.mu:46-65: by value, then by index).
    -0.0 and +0.0 compare equal.  Integers are compared exactly (no float
    conversion).  Returns (values, int64 indices)."""
    a = np.moveaxis(np.asarray(x), axis, -1)
    lead = a.shape[:-1]
    flat = a.reshape(-1, a.shape[-1])
    d = flat.shape[1]
    vals = np.empty((flat.shape[0], k), dtype=a.dtype)
    idx = np.empty((flat.shape[0], k), dtype=np.int64)
    for r in range(flat.shape[0]):
        row = flat[r]
        if np.issubdtype(row.dtype, np.integer):
            key = [int(v) for v in row]
        else:
            key = [float(v) + 0.0 for v in row]  # -0.0 -> +0.0
        order = sorted(range(d), key=(lambda i: (-key[i], i)) if largest else (lambda i: (key[i], i)))[:k]
        idx[r] = order
        vals[r] = row[order]
    out_shape = lead + (k,)
    return (np.moveaxis(vals.reshape(out_shape), -1, axis), np.moveaxis(idx.reshape(out_shape), -1, axis))


def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """ONNX Softmax restated in float64: exp(x - max) * (1 / sum exp(x - max))
    along `axis` (musa/ep/src/kernels/math/softmax_impl.mu:49-84 computes
    the same steps in fp32, or fp64 for double)."""
    a = np.asarray(x, dtype=np.float64)
    m = np.max(a, axis=axis, keepdims=True)
    e = np.exp(a - m)
    return e * (1.0 / np.sum(e, axis=axis, keepdims=True))


def gate_logits(x: np.ndarray, w: np.ndarray, b: Optional[np.ndarray], dtype: str) -> np.ndarray:
    """Router GEMM restated: logits[t, e] = sum_h x[t, h] w[e, h] (+ b[e]),
    evaluated in float64 and rounded once to the activation type -- what the
    graph's MatMul(x, W[H, E]) (+ Add) feeding the MoE node stores.  Arrays
    are in their storage types (bf16 as uint16); returns the same type."""
    xf = to_f32(x, dtype).astype(np.float64)
    wf = to_f32(w, dtype).astype(np.float64)
    lg = xf @ wf.T
    if b is not None:
        lg = lg + to_f32(b, dtype).astype(np.float64)
    if dtype == "bf16":
        # RNE of the float64 value: via float32 is exact here only when the
        # float32 rounding is not itself a tie; a direct RNE avoids that
        return f64_to_bf16_bits(lg)
    if dtype == "f16":
        return lg.astype(np.float16)
    return lg.astype(np.float32)


def f64_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    """float64 -> bf16 bits, round to nearest even (one rounding)."""
    v = np.asarray(v, np.float64)
    f = v.astype(np.float32)  # nearest float32 (RNE)
    bits = f.view(np.uint32).astype(np.uint64)
    up = (bits + np.uint64(0x10000)) & np.uint64(0xFFFF0000)
    down = bits & np.uint64(0xFFFF0000)
    vu = up.astype(np.uint32).view(np.float32).astype(np.float64)
    vd = down.astype(np.uint32).view(np.float32).astype(np.float64)
    du, dd = np.abs(vu - v), np.abs(vd - v)
    pick_up = (du < dd) | ((du == dd) & (((down >> np.uint64(16)) & np.uint64(1)) == 1))
    out = np.where(pick_up, up, down) >> np.uint64(16)
    return out.astype(np.uint16)


def dispatch(ids: np.ndarray, E: int):
    """ids [T, k] -> (offsets [E+1], perm [T*k])."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, k = ids.shape
    offs = np.zeros(E + 1, np.int32)
    perm = np.zeros(T * k, np.int32)
    rc = load().orc_dispatch(_ptr(ids), T, k, E, _ptr(offs), _ptr(perm))
    if rc:
        raise ValueError(f"orc_dispatch rc={rc}")
    return offs, perm


def dequant(q: np.ndarray, scales: np.ndarray, scale_dtype: str, bits: int, block: int, N: int, K: int):
    out = np.zeros((N, K), np.float32)
    rc = load().orc_dequant(_ptr(np.ascontiguousarray(q)), _ptr(np.ascontiguousarray(scales)), _DT[scale_dtype],
                            bits, block, N, K, _ptr(out))
    if rc:
        raise ValueError(f"orc_dequant rc={rc}")
    return out


def dequant_mxfp4(q: np.ndarray, scales: np.ndarray, N: int, K: int) -> np.ndarray:
    """MXFP4 [N, K/2] bytes + [N, K/32] E8M0 scale bytes -> fp32 [N, K]."""
    out = np.zeros((N, K), np.float32)
    rc = load().orc_dequant_mxfp4(_ptr(np.ascontiguousarray(q, np.uint8)), _ptr(np.ascontiguousarray(scales, np.uint8)),
                                  N, K, _ptr(out))
    if rc:
        raise ValueError(f"orc_dequant_mxfp4 rc={rc}")
    return out


def activation(h1: np.ndarray, h3: Optional[np.ndarray], inter: int, act: str, fusion: int = 0,
               alpha: float = 1.0, beta: float = 0.0, limit: float = float("inf")) -> np.ndarray:
    h1 = np.ascontiguousarray(h1, dtype=np.float32)
    h3 = None if h3 is None else np.ascontiguousarray(h3, dtype=np.float32)
    out = np.zeros(inter, np.float32)
    load().orc_activation(_ptr(h1), _ptr(h3), inter, ACT[act], fusion, alpha, beta, limit, _ptr(out))
    return out


def moe_forward(*, x, logits, w1, w2, k, hidden, inter, experts, act_dtype="f32", activation="relu",
                normalize=0, swiglu_fusion=0, swiglu_limit=None, alpha=1.0, beta=0.0, router_sigmoid=0,
                bits=0, block_size=0, scale_dtype="f16", s1=None, b1=None, s2=None, b2=None, w3=None,
                s3=None, b3=None, token_mask=None, threads=0, weight_format=0):
    """Runs the restated op.  Arrays are numpy in their storage types (bf16 as
    uint16).  Returns dict(out, out_f32, topk_ids, topk_w, offsets, perm)."""
    T = x.shape[0]
    a = OrcArgs()
    a.num_tokens, a.hidden, a.inter, a.num_experts, a.k = T, hidden, inter, experts, k
    a.activation = ACT[activation]
    a.normalize = int(normalize)
    a.swiglu_fusion = int(swiglu_fusion)
    a.swiglu_limit = float("inf") if swiglu_limit is None else float(swiglu_limit)
    a.alpha, a.beta = alpha, beta
    a.router_sigmoid = int(router_sigmoid)
    a.quant_bits = int(bits)
    a.block_size = int(block_size or 0)
    a.act_dtype = _DT[act_dtype]
    a.scale_dtype = _DT[scale_dtype]
    keep = []

    def c(arr):
        if arr is None:
            return None
        arr = np.ascontiguousarray(arr)
        keep.append(arr)
        return arr.ctypes.data

    a.x, a.logits = c(x), c(logits)
    a.w1, a.s1, a.b1 = c(w1), c(s1), c(b1)
    a.w2, a.s2, a.b2 = c(w2), c(s2), c(b2)
    a.w3, a.s3, a.b3 = c(w3), c(s3), c(b3)
    out = np.zeros(x.shape, dtype=x.dtype)
    out_f32 = np.zeros((T, hidden), np.float32)
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    offs = np.zeros(experts + 1, np.int32)
    perm = np.zeros(T * k, np.int32)
    a.out, a.out_f32 = out.ctypes.data, out_f32.ctypes.data
    a.topk_ids, a.topk_w, a.expert_offsets, a.perm = ids.ctypes.data, w.ctypes.data, offs.ctypes.data, perm.ctypes.data
    if token_mask is not None:
        a.token_mask = c(np.asarray(token_mask, dtype=np.uint8))
    a.num_threads = int(threads)
    a.weight_format = int(weight_format)
    rc = load().orc_moe_forward(ctypes.byref(a))
    if rc:
        raise ValueError(f"orc_moe_forward rc={rc}")
    return dict(out=out, out_f32=out_f32, topk_ids=ids, topk_w=w, offsets=offs, perm=perm)


def forward_problem(cfg, host: dict, token_mask=None, threads=0):
    """Runs the oracle on a workloads.Problem's inputs copied to the host
    (dict name -> numpy array, names as in the op schema)."""
    return moe_forward(
        x=host["input"], logits=host["router_probs"], w1=host["fc1_experts_weights"],
        w2=host["fc2_experts_weights"], k=cfg.k, hidden=cfg.hidden, inter=cfg.inter, experts=cfg.experts,
        act_dtype=cfg.dtype, activation=cfg.activation, normalize=cfg.normalize, swiglu_fusion=cfg.swiglu_fusion,
        swiglu_limit=cfg.swiglu_limit, alpha=cfg.alpha, beta=cfg.beta,
        router_sigmoid=getattr(cfg, "router_sigmoid", 0), bits=cfg.bits, block_size=cfg.block_size,
        # (MXFP4 E8M0 scale bytes are read per weight_format; the type is unused)
        scale_dtype=cfg.scale_dtype if cfg.scale_dtype in _DT else "f32",
        s1=host.get("fc1_scales"), b1=host.get("fc1_experts_bias"),
        s2=host.get("fc2_scales"), b2=host.get("fc2_experts_bias"), w3=host.get("fc3_experts_weights"),
        s3=host.get("fc3_scales"), b3=host.get("fc3_experts_bias"), token_mask=token_mask, threads=threads,
        weight_format=1 if getattr(cfg, "weight_format", "int") == "mxfp4" else 0)


def f16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    return np.asarray(u16, np.uint16).view(np.float16).astype(np.float32)


def bf16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """RNE, as the reference's float32_to_bfloat16_bits (test/ops/op_test_utils.py:235-245)."""
    bits = np.asarray(x, np.float32).view(np.uint32)
    return ((bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def to_f32(arr: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_bits_to_f32(arr)
    return np.asarray(arr).astype(np.float32)


os.environ.setdefault("OMP_WAIT_POLICY", "PASSIVE")
