"""Pre-packed (tile-major) expert weights on the GPU: QMoE int4 / int8 and
MoE fp16 / bf16.

The pack kernel's output is compared byte for byte with a numpy statement of
the layout (onnxruntime-musa_amd/csrc/moe_prepack.hip).  The op reading
pre-packed weights is compared with the same op reading the row-major
weights: the kernels add the same products in the same order and only the
load addresses differ, so the outputs must be bit-identical.  Full-size
configurations are also checked against the oracle with pre-packed weights.
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

from moe_testutil import check_problem
from onnxruntime_musa_amd import MoeError
from onnxruntime_musa_amd.workloads import CONFIGS, make_problem, to_host

pytestmark = pytest.mark.gpu

C2, C3, C4 = CONFIGS["c2_qmoe_int8_mixtral"], CONFIGS["c3_qmoe_int4_mixtral"], CONFIGS["c4_qmoe_int4_gptoss"]
C5 = CONFIGS["c5_moe_f16_qwen3"]


def pack_reference(w: np.ndarray, bits: int, deint: bool = False) -> np.ndarray:
    """Tile-major layout: one block of 16 * cb bytes per (16-row tile, chunk
    of 128 k), cb = 64 (int4), 128 (int8) or 256 (16-bit) bytes of a row per
    chunk; the 16-byte piece q of row r of the tile sits at slot (q % kv) *
    64 + (q // kv) * 16 + r of the block, kv = cb / 64.  Rows are padded with
    zeros to whole chunks; deint: each expert's rows 0, 2, 4, .. then 1, 3,
    5, .."""
    w = np.ascontiguousarray(w)
    if w.dtype != np.uint8:  # 16-bit weights: their bytes
        w = w.view(np.uint8)
    E, N, rb = w.shape
    cb = {4: 64, 8: 128, 16: 256}[bits]
    kv, cp, nch = cb // 64, cb // 16, -(-rb // cb)
    if deint:
        w = np.concatenate([w[:, 0::2], w[:, 1::2]], axis=1)
    w = np.concatenate([w, np.zeros((E, N, nch * cb - rb), np.uint8)], axis=2)
    pieces = w.reshape(E * N // 16, 16, nch, cp, 16)  # tile, row, chunk, piece, byte
    out = np.empty((E * N // 16, nch, cb, 16), np.uint8)  # tile, chunk, slot, byte
    for q in range(cp):
        for r in range(16):
            out[:, :, (q % kv) * 64 + (q // kv) * 16 + r, :] = pieces[:, r, :, q, :]
    return out.reshape(-1)


@pytest.mark.parametrize("cfg", [C2, C3], ids=["int8", "int4"])
@pytest.mark.parametrize("idx", [2, 5, 8])
def test_pack_layout(cuda, cfg, idx):
    p = make_problem(cfg, 4, seed=11, device=cuda, gen="numpy", hidden=256, inter=384)
    op = p.make_op()
    w = p.schema_inputs()[idx]
    packed = op.prepack(idx, w, torch.float16)
    torch.cuda.synchronize()
    assert packed is not None
    np.testing.assert_array_equal(packed.cpu().numpy(), pack_reference(to_host(w), cfg.bits))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("idx", [2, 5])
def test_pack_layout_padded_and_deinterleaved(cuda, bits, idx):
    # gpt-oss-shaped: K not whole chunks (320 = 2.5 chunks for fc1, 160 =
    # 1.25 for fc2) and the fused fc1 of interleaved SwiGLU
    p = make_problem(replace(C4, bits=bits), 4, seed=12, device=cuda, gen="numpy", hidden=320, inter=160, experts=4)
    op = p.make_op()
    w = p.schema_inputs()[idx]
    packed = op.prepack(idx, w, torch.bfloat16)
    torch.cuda.synchronize()
    assert packed is not None
    np.testing.assert_array_equal(packed.cpu().numpy(), pack_reference(to_host(w), bits, deint=idx == 2))


@pytest.mark.parametrize("dtype,over", [("f16", dict(hidden=256, inter=384)),
                                        ("bf16", dict(hidden=320, inter=160, use_fc3=False, swiglu_fusion=1))],
                         ids=["f16-fc3", "bf16-interleaved-k320"])
@pytest.mark.parametrize("which", ["fc1", "fc2", "fc3"])
def test_pack_layout_moe(cuda, dtype, over, which):
    p = make_problem(replace(C5, dtype=dtype, experts=4, k=2, router="normal", **over), 4, seed=14, device=cuda,
                     gen="numpy")
    idx = {"fc1": 2, "fc2": 4, "fc3": 6}[which]
    ins = p.schema_inputs()
    w = ins[idx] if idx < len(ins) else None
    if w is None:
        pytest.skip("no fc3 weights (fused fc1)")
    op = p.make_op()
    packed = op.prepack(idx, w, w.dtype)
    torch.cuda.synchronize()
    assert packed is not None
    deint = idx == 2 and p.cfg.swiglu_fusion == 1
    np.testing.assert_array_equal(packed.cpu().numpy(), pack_reference(to_host(w), 16, deint=deint))


def pack_scales_reference(s: np.ndarray, block: int, deint: bool = False) -> np.ndarray:
    """Tile-major block scales: per (16-row tile, chunk of 128 k) the 16 rows'
    128 / block scales contiguous, blocks past K zero; rows de-interleaved
    like the weights of a fused interleaved fc1."""
    E, N, nblk = s.shape
    nb = 128 // block
    nch = -(-nblk * block // 128)
    if deint:
        s = np.concatenate([s[:, 0::2], s[:, 1::2]], axis=1)
    s = np.concatenate([s, np.zeros((E, N, nch * nb - nblk), s.dtype)], axis=2)
    return np.ascontiguousarray(s.reshape(E, N // 16, 16, nch, nb).transpose(0, 1, 3, 2, 4)).reshape(-1)


@pytest.mark.parametrize("block,sdt", [(32, "bf16"), (64, "f32"), (32, "f16")])
@pytest.mark.parametrize("idx", [3, 6])
def test_pack_scales_layout(cuda, block, sdt, idx):
    dtype = "f16" if sdt == "f16" else "bf16"
    p = make_problem(replace(C4, block_size=block, scale_dtype=sdt, dtype=dtype), 4, seed=13, device=cuda,
                     gen="numpy", hidden=320, inter=192, experts=4)
    op = p.make_op()
    sc = p.schema_inputs()[idx]
    packed = op.prepack(idx, sc, p.schema_inputs()[0].dtype)
    torch.cuda.synchronize()
    assert packed is not None
    host = to_host(sc)
    got = packed.cpu().numpy().view(host.dtype)
    np.testing.assert_array_equal(got, pack_scales_reference(host, block, deint=idx == 3))


VARIANTS = {
    "int8-chan-fc3": (C2, dict(hidden=256, inter=512)),
    "int4-b128-fc3": (C3, dict(hidden=256, inter=512)),
    "int4-b64-f32-bf16": (C3, dict(hidden=384, inter=256, block_size=64, scale_dtype="f32", dtype="bf16")),
    "int8-b32-bf16": (C2, dict(hidden=256, inter=384, block_size=32, scale_dtype="bf16", dtype="bf16")),
    "int4-b16": (C3, dict(hidden=256, inter=256, block_size=16)),
    "int4-chunked-bias": (C3, dict(hidden=256, inter=512, use_fc3=False, swiglu_fusion=2, bias=True)),
    "int8-silu": (C2, dict(hidden=256, inter=384, use_fc3=False, activation="silu", bias=True)),
    "int4-fc2-slices": (C3, dict(hidden=512, inter=8192, experts=4)),
    # gpt-oss-shaped: step scales (block 32), K padded to whole chunks,
    # fused fc1 stored de-interleaved, clamp and biases
    "int4-b32-gptoss": (C4, dict(hidden=320, inter=160, experts=8)),
    "int4-b32-gptoss-wide": (C4, dict(hidden=2880, inter=480, experts=6)),
    "int4-b32-f16": (C3, dict(hidden=256, inter=384, block_size=32)),
    "int8-b32-f16-deint": (C4, dict(hidden=320, inter=160, experts=8, bits=8, dtype="f16", scale_dtype="f16")),
    "int4-b64-bf16-odd-blocks": (C4, dict(hidden=320, inter=192, experts=8, block_size=64)),
    # MoE fp16 / bf16 weights: 256-byte chunks, prefill stages of half a chunk
    "f16-moe-fc3": (C5, dict(hidden=256, inter=384, experts=8, k=2, router="normal")),
    "bf16-moe-interleaved-k320": (C5, dict(hidden=320, inter=160, experts=8, k=2, router="normal", dtype="bf16",
                                           use_fc3=False, swiglu_fusion=1, bias=True)),
    "f16-moe-silu-fc2-slices": (C5, dict(hidden=512, inter=8192, experts=4, k=2, router="normal", use_fc3=False,
                                         activation="silu")),
}


def run_pair(p, path):
    inputs = p.schema_inputs()
    plain, packed = p.make_op(expert_path=path), p.make_op(expert_path=path)
    done = packed.prepack_all(*inputs)
    y0, y1 = plain(*inputs), packed(*inputs)
    torch.cuda.synchronize()
    return done, y0, y1


@pytest.mark.parametrize("name", list(VARIANTS))
@pytest.mark.parametrize("path,T", [("decode", 1), ("decode", 16), ("decode", 40), ("decode", 64),
                                    ("prefill", 17), ("prefill", 300), ("auto", 130)])
def test_packed_equals_row_major(cuda, name, path, T):
    cfg, over = VARIANTS[name]
    p = make_problem(replace(cfg, **over), T, seed=T + 5, device=cuda, gen="numpy")
    done, y0, y1 = run_pair(p, path)
    assert done, "nothing was packed"
    assert torch.equal(y0, y1), f"{name} T={T} {path}: max diff {(y0.float() - y1.float()).abs().max().item()}"


@pytest.mark.parametrize("path,T", [("decode", 16), ("decode", 64), ("prefill", 40)])
def test_packed_weights_with_row_major_scales(cuda, path, T):
    # step scales read row-major scales when only the weights are packed
    p = make_problem(replace(C4, hidden=320, inter=160, experts=8), T, seed=T + 6, device=cuda, gen="numpy")
    inputs = p.schema_inputs()
    plain, packed = p.make_op(expert_path=path), p.make_op(expert_path=path)
    assert [i for i in (2, 5) if packed.prepack(i, inputs[i], inputs[0].dtype) is not None] == [2, 5]
    y0, y1 = plain(*inputs), packed(*inputs)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)


def test_packed_scales_need_packed_weights(cuda):
    p = make_problem(replace(C4, hidden=320, inter=160, experts=8), 8, seed=3, device=cuda, gen="numpy")
    inputs = p.schema_inputs()
    op = p.make_op()
    assert op.prepack(6, inputs[6], inputs[0].dtype) is not None
    with pytest.raises(MoeError) as ei:
        op(*inputs)
    assert ei.value.code == 9


def test_packed_inputs_may_be_absent(cuda):
    p = make_problem(replace(C3, hidden=256, inter=512), 16, seed=3, device=cuda, gen="numpy")
    inputs = p.schema_inputs()
    op = p.make_op()
    y0 = op(*inputs).clone()
    assert op.prepack_all(*inputs) == [2, 5, 8]
    y1 = op(*inputs).clone()
    none = [None if i in (2, 5, 8) else t for i, t in enumerate(inputs)]
    y2 = op(*none)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1) and torch.equal(y0, y2)


def test_packed_rejects_other_shape(cuda):
    p = make_problem(replace(C3, hidden=256, inter=512), 16, seed=3, device=cuda, gen="numpy")
    inputs = p.schema_inputs()
    op = p.make_op()
    op.prepack_all(*inputs)
    other = make_problem(replace(C3, hidden=256, inter=256), 16, seed=3, device=cuda, gen="numpy").schema_inputs()
    with pytest.raises(MoeError) as ei:
        op(*inputs[:5], other[5], *inputs[6:])
    assert ei.value.code == 2


def test_packed_rejects_another_tensor_of_the_same_shape(cuda):
    # a copy of the packed weights (same shape and type, another pointer)
    # would silently compute with the old packed copy: it is an error; the
    # packed tensor itself and its packed copy are accepted
    p = make_problem(replace(C3, hidden=256, inter=512), 16, seed=3, device=cuda, gen="numpy")
    inputs = p.schema_inputs()
    op = p.make_op()
    y0 = op(*inputs).clone()
    op.prepack_all(*inputs)
    with pytest.raises(MoeError) as ei:
        op(*inputs[:5], inputs[5].clone(), *inputs[6:])
    assert ei.value.code == 2 and "pre-packed" in str(ei.value)
    y1 = op(*inputs[:5], op._packed[5], *inputs[6:])
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)


def test_packed_needs_an_mfma_path(cuda):
    p = make_problem(replace(C3, hidden=256, inter=512), 8, seed=3, device=cuda, gen="numpy")
    inputs = p.schema_inputs()
    op = p.make_op(expert_path="simt")
    op.prepack_all(*inputs)
    with pytest.raises(MoeError) as ei:
        op(*inputs)
    assert ei.value.code == 9


def test_fc1_and_fc3_pack_together(cuda):
    p = make_problem(replace(C3, hidden=256, inter=512), 8, seed=3, device=cuda, gen="numpy")
    inputs = p.schema_inputs()
    op = p.make_op()
    assert op.prepack(2, inputs[2], torch.float16) is not None
    with pytest.raises(MoeError) as ei:
        op(*inputs)
    assert ei.value.code == 9


@pytest.mark.parametrize("name,T", [("c3_qmoe_int4_mixtral", 16), ("c3_qmoe_int4_mixtral", 1),
                                    ("c2_qmoe_int8_mixtral", 16), ("c2_qmoe_int8_mixtral", 1)])
def test_full_decode_prepacked(cuda, name, T):
    p = make_problem(CONFIGS[name], T, seed=300 + T, device=cuda)
    check_problem(p, threads=16, prepack=True)


@pytest.mark.parametrize("T", [16, 8192])
def test_full_c5_prepacked(cuda, T):
    p = make_problem(C5, T, seed=500 + T, device=cuda)
    check_problem(p, sample_tokens=48 if T > 64 else None, threads=16, prepack=True, report=True)


@pytest.mark.parametrize("name", ["c2_qmoe_int8_mixtral", "c3_qmoe_int4_mixtral"])
def test_full_prefill_prepacked(cuda, name):
    p = make_problem(CONFIGS[name], 4096, seed=4097, device=cuda)
    check_problem(p, sample_tokens=48, threads=16, prepack=True)


@pytest.mark.parametrize("T", [1, 16, 64])
def test_full_c4_decode_prepacked(cuda, T):
    p = make_problem(C4, T, seed=400 + T, device=cuda)
    check_problem(p, threads=16, prepack=True, report=True)


def test_full_c4_prefill_prepacked(cuda):
    p = make_problem(C4, 8192, seed=8193, device=cuda)
    check_problem(p, sample_tokens=48, threads=16, prepack=True, report=True)
