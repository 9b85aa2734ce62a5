"""CPU tests of the C ABI (include/moe_mi355x.h): the built library loads,
exports exactly the declared symbols, and its host-side logic (attribute
defaults, activation parsing, node validation, workspace sizing) behaves as
the op contract says.  No call here launches a kernel or touches a GPU.

The validation cases follow the reference's error mapping: bad attributes or
shapes -> ORT_INVALID_ARGUMENT, unsupported type/feature ->
ORT_NOT_IMPLEMENTED (musa/ep/src/kernels/math/topk.cc:143-187,
musa/ep/src/kernels/llm/attention.cc:101-158).
"""
from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from onnxruntime_musa_amd import _capi as C

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "moe_mi355x.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"MOE_API\s+[^;(]*?\b(moe_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    path = Path(C.get_library_path())
    if not path.exists():
        pytest.fail(f"{path} is not built; run __graft_entry__.build()")
    return C.load_library()


def test_header_declares_every_binding():
    assert declared_functions() == sorted(n for n, _, _ in C.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_library_exports_nothing_else(lib):
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--defined-only", C.get_library_path()], capture_output=True, text=True,
                         check=True).stdout
    syms = {ln.split()[-1].split("@")[0] for ln in out.splitlines() if ln.strip() and ln.split()[-2] in "TtWD"}
    syms = {s for s in syms if not s.startswith("MOE_MI355X")}
    assert syms == set(declared_functions())


def test_version(lib):
    v = lib.moe_version().decode()
    assert re.search(r"\d+\.\d+\.\d+", v) and "gfx950" in v


def attrs(lib, op="MoE", **kw):
    a = C.MoeAttributes()
    assert lib.moe_attributes_init(ctypes.byref(a), op.encode()) == C.MOE_OK
    for key, val in kw.items():
        setattr(a, key, val)
    return a


def test_attribute_defaults(lib):
    a = attrs(lib, "MoE")
    assert (a.k, a.activation_type, a.normalize_routing_weights, a.use_sparse_mixer, a.swiglu_fusion) == (1, 0, 0, 0, 0)
    assert a.has_swiglu_limit == 0 and a.activation_alpha == 1.0 and a.activation_beta == 0.0
    assert a.router_sigmoid == 0
    q = attrs(lib, "QMoE")
    assert q.expert_weight_bits == 4 and q.block_size == 0


def test_attribute_init_rejects_unknown_op(lib):
    a = C.MoeAttributes()
    assert lib.moe_attributes_init(ctypes.byref(a), b"Gemm") == C.MOE_INVALID_ARGUMENT
    assert lib.moe_last_error()


@pytest.mark.parametrize("name,code", list(C.ACTIVATIONS.items()))
def test_parse_activation(lib, name, code):
    v = ctypes.c_int32(-1)
    assert lib.moe_parse_activation(name.encode(), ctypes.byref(v)) == C.MOE_OK
    assert v.value == code


def test_parse_activation_rejects_unknown(lib):
    v = ctypes.c_int32(-1)
    assert lib.moe_parse_activation(b"tanh", ctypes.byref(v)) == C.MOE_INVALID_ARGUMENT


def create(lib, op="MoE", **kw):
    a = attrs(lib, op, **kw)
    h = ctypes.c_void_p()
    st = lib.moe_kernel_create(op.encode(), ctypes.byref(a), ctypes.byref(h))
    return st, h


@pytest.mark.parametrize("op,kw,code", [
    ("MoE", dict(k=0), C.MOE_INVALID_ARGUMENT),
    ("MoE", dict(use_sparse_mixer=1), C.MOE_NOT_IMPLEMENTED),
    ("MoE", dict(swiglu_fusion=3, activation_type=4), C.MOE_INVALID_ARGUMENT),
    ("QMoE", dict(expert_weight_bits=3), C.MOE_INVALID_ARGUMENT),
    ("MoE", dict(activation_type=7), C.MOE_INVALID_ARGUMENT),
])
def test_create_rejects_bad_attributes(lib, op, kw, code):
    st, h = create(lib, op, **kw)
    assert st == code
    assert not h.value


FAKE = 0x1000  # shapes only are read by workspace_size; no pointer is dereferenced


def tensor(dims, et=C.ELEM_FLOAT16, data=FAKE):
    t = C.MoeTensor()
    t.data = data
    t.elem_type = et
    t.rank = len(dims)
    for i, d in enumerate(dims):
        t.dims[i] = d
    return t


def qmoe_inputs(T=16, H=256, I=512, E=8, bits=4, bs=128, fc3=True, bias=False):
    p = 2 if bits == 4 else 1
    sc = (lambda N, K: [E, N, K // bs]) if bs else (lambda N, K: [E, N])
    ins = [tensor([T, H]), tensor([T, E]), tensor([E, I, H // p], C.ELEM_UINT8), tensor(sc(I, H)),
           tensor([E, I]) if bias else tensor([0], data=None),
           tensor([E, H, I // p], C.ELEM_UINT8), tensor(sc(H, I)),
           tensor([E, H]) if bias else tensor([0], data=None)]
    if fc3:
        ins += [tensor([E, I, H // p], C.ELEM_UINT8), tensor(sc(I, H)), tensor([0], data=None)]
    return ins


def ws_size(lib, h, ins):
    arr = (C.MoeTensor * len(ins))(*ins)
    n = ctypes.c_size_t(0)
    st = lib.moe_kernel_workspace_size(h, arr, len(ins), ctypes.byref(n))
    return st, n.value


@pytest.fixture
def qkernel(lib):
    st, h = create(lib, "QMoE", k=2, activation_type=4, block_size=128)
    assert st == C.MOE_OK
    yield h
    lib.moe_kernel_release(h)


def test_workspace_size_valid_qmoe(lib, qkernel):
    st, n = ws_size(lib, qkernel, qmoe_inputs())
    assert st == C.MOE_OK, lib.moe_last_error()
    # at least routing results + fc1 activations (T*k*I fp16) + fc2 partials (T*k*H fp32)
    assert n >= 16 * 2 * (512 * 2 + 256 * 4)


def test_workspace_size_grows_with_tokens(lib, qkernel):
    small = ws_size(lib, qkernel, qmoe_inputs(T=16))[1]
    big = ws_size(lib, qkernel, qmoe_inputs(T=4096))[1]
    assert big > small


def test_workspace_layout_is_inside_workspace(lib, qkernel):
    ins = qmoe_inputs(T=64)
    arr = (C.MoeTensor * len(ins))(*ins)
    lay = C.MoeWorkspaceLayout()
    assert lib.moe_kernel_workspace_layout(qkernel, arr, len(ins), ctypes.byref(lay)) == C.MOE_OK
    T, k, E = 64, 2, 8
    spans = sorted([(lay.topk_ids, 4 * T * k), (lay.topk_w, 4 * T * k), (lay.offsets, 4 * (E + 1)),
                    (lay.perm, 4 * T * k), (lay.inv_perm, 4 * T * k)])
    for (a, n), (b, _) in zip(spans, spans[1:]):
        assert a + n <= b, "routing arrays overlap"
    assert spans[-1][0] + spans[-1][1] <= lay.total
    assert all(off % 16 == 0 for off, _ in spans)


def mutate(ins, i, **kw):
    ins = list(ins)
    t = ins[i]
    dims = kw.get("dims", [t.dims[j] for j in range(t.rank)])
    ins[i] = tensor(dims, kw.get("et", t.elem_type), kw.get("data", t.data))
    return ins


@pytest.mark.parametrize("case,code", [
    (lambda b: b[:5], C.MOE_INVALID_ARGUMENT),                                   # too few inputs
    (lambda b: mutate(b, 0, dims=[16]), C.MOE_INVALID_ARGUMENT),                 # input rank 1
    (lambda b: mutate(b, 0, et=C.ELEM_UINT8), C.MOE_NOT_IMPLEMENTED),            # integer activations
    (lambda b: mutate(b, 1, et=C.ELEM_FLOAT), C.MOE_INVALID_ARGUMENT),           # router type mismatch
    (lambda b: mutate(b, 1, dims=[15, 8]), C.MOE_INVALID_ARGUMENT),              # router rows != tokens
    (lambda b: mutate(b, 2, et=C.ELEM_FLOAT16), C.MOE_INVALID_ARGUMENT),         # QMoE weights not uint8
    (lambda b: mutate(b, 2, dims=[8, 512, 256]), C.MOE_INVALID_ARGUMENT),        # fc1 K not packed
    (lambda b: mutate(b, 3, dims=[8, 512, 4]), C.MOE_INVALID_ARGUMENT),          # fc1 scale blocks wrong
    (lambda b: mutate(mutate(mutate(b, 3, et=C.ELEM_UINT8), 6, et=C.ELEM_UINT8), 9, et=C.ELEM_UINT8),
     C.MOE_INVALID_ARGUMENT),                                                    # E8M0 (MXFP4) with block 128
    (lambda b: mutate(b, 6, et=C.ELEM_FLOAT), C.MOE_INVALID_ARGUMENT),           # scale types differ
    (lambda b: mutate(b, 8, dims=[8, 256, 128]), C.MOE_INVALID_ARGUMENT),        # fc3 shape
    (lambda b: mutate(b, 9, data=None), C.MOE_INVALID_ARGUMENT),                 # fc3 without scales
    (lambda b: mutate(b, 4, dims=[8, 511], data=FAKE), C.MOE_INVALID_ARGUMENT),  # fc1 bias shape
    (lambda b: b + [tensor([8, 512], C.ELEM_UINT8)], C.MOE_NOT_IMPLEMENTED),     # zero points given
    (lambda b: mutate(b, 1, dims=[16, 16]), C.MOE_INVALID_ARGUMENT),             # E mismatch vs weights
    (lambda b: mutate(b, 1, dims=[16, 600]), C.MOE_NOT_IMPLEMENTED),            # more than 512 experts
])
def test_workspace_size_rejects_bad_inputs(lib, qkernel, case, code):
    st, _ = ws_size(lib, qkernel, case(qmoe_inputs()))
    assert st == code, lib.moe_last_error()
    assert lib.moe_last_error()


def test_absent_zero_point_inputs_are_accepted(lib, qkernel):
    ins = qmoe_inputs() + [tensor([0], data=None)] * 3
    assert ws_size(lib, qkernel, ins)[0] == C.MOE_OK


def test_block_size_rules(lib):
    for bs, code in [(8, C.MOE_INVALID_ARGUMENT), (48, C.MOE_INVALID_ARGUMENT), (1024, C.MOE_INVALID_ARGUMENT),
                     (16, C.MOE_OK), (256, C.MOE_OK)]:
        st, h = create(lib, "QMoE", k=2, activation_type=4, block_size=bs)
        if st != C.MOE_OK:
            assert st == code
            continue
        got = ws_size(lib, h, qmoe_inputs(bs=bs))[0]
        lib.moe_kernel_release(h)
        assert got == code, (bs, lib.moe_last_error())


def test_swiglu_without_fc3_needs_fusion(lib):
    st, h = create(lib, "QMoE", k=2, activation_type=4, block_size=128, swiglu_fusion=0)
    assert st == C.MOE_OK
    ins = qmoe_inputs(fc3=False)
    assert ws_size(lib, h, ins)[0] == C.MOE_NOT_IMPLEMENTED
    lib.moe_kernel_release(h)
    st, h = create(lib, "QMoE", k=2, activation_type=4, block_size=128, swiglu_fusion=1)
    ins = mutate(mutate(qmoe_inputs(fc3=False), 2, dims=[8, 1024, 128]), 3, dims=[8, 1024, 2])
    assert ws_size(lib, h, ins)[0] == C.MOE_OK, lib.moe_last_error()
    # fc3 given together with a fused layout is contradictory
    assert ws_size(lib, h, qmoe_inputs(fc3=True))[0] == C.MOE_INVALID_ARGUMENT
    lib.moe_kernel_release(h)


def test_k_range(lib):
    for k, code in [(8, C.MOE_OK), (9, C.MOE_INVALID_ARGUMENT)]:
        st, h = create(lib, "QMoE", k=k, activation_type=4, block_size=128)
        assert st == C.MOE_OK
        assert ws_size(lib, h, qmoe_inputs())[0] == code
        lib.moe_kernel_release(h)


def test_route_scratch_size_monotone(lib):
    # small batches run in one workgroup and need no scratch; large ones keep
    # per-block histograms
    a = lib.moe_route_dispatch_scratch_size(16, 8, 2)
    b = lib.moe_route_dispatch_scratch_size(65536, 128, 8)
    assert 0 <= a < b


def test_set_expert_path_validates(lib, qkernel):
    assert lib.moe_kernel_set_expert_path(qkernel, 1) == C.MOE_OK
    assert lib.moe_kernel_set_expert_path(qkernel, 7) == C.MOE_INVALID_ARGUMENT
    assert lib.moe_kernel_set_expert_path(qkernel, -1) == C.MOE_OK


# ---- weight pre-pack (the OpKernel::PrePack role): which inputs a kernel
# packs, and how many bytes the tile-major copy takes.  prepack_size reads
# the shape and type only. ----
def prepack_size(lib, h, idx, dims, act=C.ELEM_FLOAT16, et=C.ELEM_UINT8):
    t = tensor(dims, et)
    n = ctypes.c_size_t(123)
    st = lib.moe_kernel_prepack_size(h, idx, ctypes.byref(t), act, ctypes.byref(n))
    return st, n.value


# packed row bytes: K padded to whole chunks of 128 (64 bytes int4, 128 int8)
@pytest.mark.parametrize("bits,idx,dims,packed_rb", [
    (4, 2, [8, 512, 128], 128),      # fc1 int4: H = 256 -> whole chunks, 16-row tiles
    (4, 5, [8, 256, 256], 256),      # fc2 int4, I = 512
    (4, 8, [8, 512, 128], 128),      # fc3
    (8, 2, [8, 512, 256], 256),      # int8
    (4, 2, [8, 520, 128], 0),        # N not a multiple of 16
    (4, 2, [8, 512, 96], 128),       # K = 192: padded to 2 chunks
    (8, 5, [8, 256, 192], 256),      # int8 K = 192
    (4, 5, [8, 2880, 1440], 1472),   # gpt-oss fc2 K = 2880: 22.5 chunks -> 23
    (4, 2, [8, 512, 100], 0),        # rows not whole 16-byte pieces
    (4, 2, [8, 512, 4096], 0),       # fc1 K = 8192: above one decode activation slice
    (4, 5, [8, 512, 4096], 4096),    # fc2 K = 8192 streams in slices
])
def test_prepack_size_rules(lib, bits, idx, dims, packed_rb):
    st, h = create(lib, "QMoE", k=2, activation_type=4, block_size=128, expert_weight_bits=bits)
    assert st == C.MOE_OK
    try:
        st, n = prepack_size(lib, h, idx, dims)
        assert st == C.MOE_OK, lib.moe_last_error()
        assert n == dims[0] * dims[1] * packed_rb
    finally:
        lib.moe_kernel_release(h)


@pytest.mark.parametrize("bits,block,act,idx,dims,elem,packed", [
    (4, 32, C.ELEM_BFLOAT16, 3, [8, 5760, 90], C.ELEM_BFLOAT16, 8 * 5760 * 23 * 4 * 2),  # gpt-oss fc1
    (4, 32, C.ELEM_BFLOAT16, 6, [8, 2880, 90], C.ELEM_BFLOAT16, 8 * 2880 * 23 * 4 * 2),
    (4, 64, C.ELEM_FLOAT16, 6, [8, 256, 5], C.ELEM_FLOAT, 8 * 256 * 3 * 2 * 4),          # K = 320: 3 chunks
    (8, 32, C.ELEM_FLOAT16, 9, [8, 512, 8], C.ELEM_FLOAT16, 8 * 512 * 2 * 4 * 2),
    (8, 32, C.ELEM_BFLOAT16, 3, [8, 512, 8], C.ELEM_BFLOAT16, 0),  # int8 + bf16: folded scales
    (4, 128, C.ELEM_FLOAT16, 3, [8, 512, 2], C.ELEM_FLOAT16, 0),   # block 128: per-chunk scales
    (4, 16, C.ELEM_FLOAT16, 3, [8, 512, 16], C.ELEM_FLOAT16, 0),   # block 16: folded
    (4, 32, C.ELEM_FLOAT16, 3, [8, 520, 8], C.ELEM_FLOAT16, 0),    # N not a multiple of 16
    (4, 32, C.ELEM_FLOAT16, 6, [8, 512], C.ELEM_FLOAT16, 0),       # per-channel scales stay as given
    (4, 32, C.ELEM_BFLOAT16, 3, [8, 5760, 90], C.ELEM_UINT8, 8 * 5760 * 23 * 4),  # MXFP4 E8M0 bytes
    (4, 64, C.ELEM_BFLOAT16, 3, [8, 512, 4], C.ELEM_UINT8, 0),     # E8M0 needs block 32
])
def test_prepack_size_scales(lib, bits, block, act, idx, dims, elem, packed):
    st, h = create(lib, "QMoE", k=2, activation_type=4, swiglu_fusion=1, block_size=block,
                   expert_weight_bits=bits)
    assert st == C.MOE_OK
    try:
        assert prepack_size(lib, h, idx, dims, act=act, et=elem) == (C.MOE_OK, packed)
    finally:
        lib.moe_kernel_release(h)


def test_prepack_size_interleaved_fc1(lib):
    # the fused fc1 of interleaved SwiGLU is packed de-interleaved: each
    # half (gate rows, linear rows) must be whole 16-row tiles
    st, h = create(lib, "QMoE", k=2, activation_type=4, swiglu_fusion=1, block_size=32)
    assert st == C.MOE_OK
    try:
        assert prepack_size(lib, h, 2, [8, 1024, 128]) == (C.MOE_OK, 8 * 1024 * 128)
        assert prepack_size(lib, h, 2, [8, 5760, 1440]) == (C.MOE_OK, 8 * 5760 * 1472)
        assert prepack_size(lib, h, 2, [8, 1040, 128]) == (C.MOE_OK, 0)
        assert prepack_size(lib, h, 5, [8, 256, 256])[1] == 8 * 256 * 256
    finally:
        lib.moe_kernel_release(h)


def test_prepack_size_chunked_fc1_needs_whole_tiles_per_half(lib):
    st, h = create(lib, "QMoE", k=2, activation_type=4, swiglu_fusion=2, block_size=0)
    assert st == C.MOE_OK
    try:
        assert prepack_size(lib, h, 2, [8, 1024, 128])[1] == 8 * 1024 * 128
        assert prepack_size(lib, h, 2, [8, 48, 128]) == (C.MOE_OK, 0)  # I = 24: the linear half starts mid-tile
    finally:
        lib.moe_kernel_release(h)


def test_prepack_size_fp32_activations_stay_row_major(lib, qkernel):
    assert prepack_size(lib, qkernel, 2, [8, 512, 128], act=C.ELEM_FLOAT) == (C.MOE_OK, 0)
    st, h = create(lib, "MoE", k=2, activation_type=2)
    assert st == C.MOE_OK
    try:
        assert prepack_size(lib, h, 2, [8, 512, 256], act=C.ELEM_FLOAT, et=C.ELEM_FLOAT) == (C.MOE_OK, 0)
    finally:
        lib.moe_kernel_release(h)


# MoE (16-bit weights of the activations' type): fc1 2, fc2 4, fc3 6; a
# row's K padded to whole chunks of 128 k (256 bytes)
@pytest.mark.parametrize("idx,dims,et,act,packed_rb", [
    (2, [8, 512, 256], C.ELEM_FLOAT16, C.ELEM_FLOAT16, 512),
    (4, [8, 256, 768], C.ELEM_BFLOAT16, C.ELEM_BFLOAT16, 1536),
    (6, [8, 512, 256], C.ELEM_FLOAT16, C.ELEM_FLOAT16, 512),
    (2, [8, 512, 320], C.ELEM_FLOAT16, C.ELEM_FLOAT16, 768),     # K = 320: 2.5 chunks -> 3
    (4, [8, 256, 8192], C.ELEM_FLOAT16, C.ELEM_FLOAT16, 16384),  # fc2 K = 8192 streams in slices
    (2, [8, 512, 8192], C.ELEM_FLOAT16, C.ELEM_FLOAT16, 0),      # fc1 K above one decode slice
    (2, [8, 520, 256], C.ELEM_FLOAT16, C.ELEM_FLOAT16, 0),       # N not a multiple of 16
    (2, [8, 512, 100], C.ELEM_FLOAT16, C.ELEM_FLOAT16, 0),       # rows not whole 16-byte pieces
    (2, [8, 512, 256], C.ELEM_BFLOAT16, C.ELEM_FLOAT16, 0),      # not the activations' type
])
def test_prepack_size_moe(lib, idx, dims, et, act, packed_rb):
    st, h = create(lib, "MoE", k=2, activation_type=4)
    assert st == C.MOE_OK
    try:
        st, n = prepack_size(lib, h, idx, dims, act=act, et=et)
        assert st == C.MOE_OK, lib.moe_last_error()
        assert n == dims[0] * dims[1] * packed_rb
    finally:
        lib.moe_kernel_release(h)


@pytest.mark.parametrize("idx,dims,et", [
    (3, [8, 512], C.ELEM_FLOAT16),          # fc1 bias
    (5, [8, 256, 512], C.ELEM_FLOAT16),     # fc2 bias index (QMoE's fc2 weights)
    (8, [8, 256, 512], C.ELEM_FLOAT16),
    (2, [8, 512, 256], C.ELEM_UINT8),       # not a float type
    (2, [512, 256], C.ELEM_FLOAT16),        # not 3D
])
def test_prepack_moe_rejects_bad_arguments(lib, idx, dims, et):
    st, h = create(lib, "MoE", k=2, activation_type=4)
    assert st == C.MOE_OK
    try:
        assert prepack_size(lib, h, idx, dims, et=et)[0] == C.MOE_INVALID_ARGUMENT
    finally:
        lib.moe_kernel_release(h)


@pytest.mark.parametrize("idx,dims,et,act", [
    (3, [8, 512, 128], C.ELEM_INT32, C.ELEM_FLOAT16),   # scales neither float nor uint8 (E8M0)
    (6, [8, 512, 4, 1], C.ELEM_FLOAT16, C.ELEM_FLOAT16),  # scales neither 2D nor 3D
    (4, [8, 512], C.ELEM_FLOAT16, C.ELEM_FLOAT16),       # a bias input
    (0, [16, 256], C.ELEM_FLOAT16, C.ELEM_FLOAT16),
    (2, [512, 128], C.ELEM_UINT8, C.ELEM_FLOAT16),      # not 3D
    (2, [8, 512, 128], C.ELEM_FLOAT16, C.ELEM_FLOAT16),  # not uint8
    (2, [8, 512, 128], C.ELEM_UINT8, C.ELEM_UINT8),      # act_type not a float type
])
def test_prepack_rejects_bad_arguments(lib, qkernel, idx, dims, et, act):
    st, _ = prepack_size(lib, qkernel, idx, dims, act=act, et=et)
    assert st == C.MOE_INVALID_ARGUMENT


def test_prepack_not_packed_writes_nothing(lib, qkernel):
    # an input the kernel keeps row-major: OK, *is_packed = 0, no device work
    t = tensor([8, 520, 128], C.ELEM_UINT8)
    flag = ctypes.c_int32(7)
    st = lib.moe_kernel_prepack(qkernel, 2, ctypes.byref(t), C.ELEM_FLOAT16, None, 0, None, ctypes.byref(flag))
    assert st == C.MOE_OK and flag.value == 0


def test_prepack_rejects_small_buffer(lib, qkernel):
    t = tensor([8, 512, 128], C.ELEM_UINT8)
    flag = ctypes.c_int32(7)
    st = lib.moe_kernel_prepack(qkernel, 2, ctypes.byref(t), C.ELEM_FLOAT16, ctypes.c_void_p(FAKE), 100, None,
                                ctypes.byref(flag))
    assert st == C.MOE_INVALID_ARGUMENT and flag.value == 0
    assert b"too small" in lib.moe_last_error()


# ---- moe_topk_launch validation (returns before any launch) ----
def topk_status(lib, **kw):
    p = C.MoeTopKParams()
    p.input, p.values, p.indices = FAKE, FAKE, FAKE
    p.elem_type, p.largest, p.sorted = C.ELEM_FLOAT, 1, 1
    p.rows, p.dim, p.inner, p.k = 2, 16, 1, 4
    for key, val in kw.items():
        setattr(p, key, val)
    return lib.moe_topk_launch(ctypes.byref(p), None)


@pytest.mark.parametrize("kw,code", [
    (dict(k=17), C.MOE_INVALID_ARGUMENT),          # k > dim (musa/ep/src/kernels/math/topk.cc:174-177)
    (dict(k=-1), C.MOE_INVALID_ARGUMENT),
    (dict(largest=2), C.MOE_INVALID_ARGUMENT),     # topk.cc:143-150
    (dict(sorted=3), C.MOE_INVALID_ARGUMENT),
    (dict(elem_type=C.ELEM_UINT8), C.MOE_NOT_IMPLEMENTED),  # topk.cc:179-183
    (dict(dim=9000, k=8193), C.MOE_NOT_IMPLEMENTED),  # long axis: the k winners are sorted in LDS
    (dict(dim=1 << 31, k=3), C.MOE_NOT_IMPLEMENTED),     # 32-bit indices in LDS
    (dict(k=0), C.MOE_OK),                         # empty output: nothing to launch
    (dict(rows=0), C.MOE_OK),
])
def test_topk_validation(lib, kw, code):
    assert topk_status(lib, **kw) == code


@pytest.mark.parametrize("kw,code", [
    (dict(elem_type=C.ELEM_INT32), C.MOE_NOT_IMPLEMENTED),
    (dict(dim=-1), C.MOE_INVALID_ARGUMENT),
    (dict(outer=0), C.MOE_OK),
])
def test_softmax_validation(lib, kw, code):
    p = C.MoeSoftmaxParams()
    p.input, p.output, p.elem_type = FAKE, FAKE, C.ELEM_FLOAT
    p.outer, p.dim, p.inner = 4, 8, 1
    for key, val in kw.items():
        setattr(p, key, val)
    assert lib.moe_softmax_launch(ctypes.byref(p), None) == code


def test_trace_lines_on_an_error_path(lib, capfd, monkeypatch):
    # MOE_TRACE_KERNELS is read at creation; a call rejected by validation
    # (no launch) still prints its begin and end lines, with the status
    monkeypatch.setenv("MOE_TRACE_KERNELS", "1")
    st, h = create(lib, "QMoE", k=2, activation_type=4, block_size=128)
    assert st == C.MOE_OK
    try:
        ins = mutate(qmoe_inputs(), 1, dims=[15, 8])
        arr = (C.MoeTensor * len(ins))(*ins)
        assert lib.moe_kernel_compute(h, arr, len(ins), FAKE, None, 0, None) == C.MOE_INVALID_ARGUMENT
    finally:
        lib.moe_kernel_release(h)
    err = capfd.readouterr().err
    assert "MOE_KERNEL_BEGIN QMoE" in err and "MOE_KERNEL_END QMoE" in err
    assert f"status={C.MOE_INVALID_ARGUMENT} router_probs" in err
