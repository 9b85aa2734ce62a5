"""MXFP4 experts (OCP MX v1.0: FP4 E2M1 elements, E8M0 scales per block of 32
along K) on the GPU: the QMoE op with uint8 scales, against the oracle
(weight_format 1, pinned by the known-answer and quantizer tests in
tests/test_oracle.py) on the decode, prefill and SIMT paths, with and without
pre-packing.

Decode and prefill fold each block's power-of-two scale into the FP4
conversion of its elements (exact for bf16, and for fp16 while the scaled
weight is an fp16 normal); SIMT decodes in fp32.
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

from moe_testutil import check_problem
from onnxruntime_musa_amd import MoeError
from onnxruntime_musa_amd.workloads import CONFIGS, make_problem

pytestmark = pytest.mark.gpu

X1 = CONFIGS["x1_mxfp4_gptoss"]

SMALL = {
    # gpt-oss shape scaled down: interleaved SwiGLU with clamp, biases, K
    # not whole chunks of 128 (320 = 2.5, 160 = 1.25)
    "gptoss-bf16": dict(hidden=320, inter=160, experts=8),
    "gptoss-f16": dict(hidden=320, inter=160, experts=8, dtype="f16"),
    "fc3-f16": dict(hidden=256, inter=384, experts=6, k=2, dtype="f16", use_fc3=True, swiglu_fusion=0,
                    swiglu_limit=None, alpha=1.0, beta=0.0, bias=False),
    "silu-bf16": dict(hidden=256, inter=256, experts=8, activation="silu", use_fc3=False, swiglu_fusion=0,
                      swiglu_limit=None, alpha=1.0, beta=0.0),
}


@pytest.mark.parametrize("name", list(SMALL))
@pytest.mark.parametrize("path,T", [("decode", 1), ("decode", 16), ("decode", 64), ("prefill", 17),
                                    ("prefill", 300), ("auto", 130)])
@pytest.mark.parametrize("prepack", [False, True], ids=["rowmajor", "packed"])
def test_mxfp4_matches_oracle(cuda, name, path, T, prepack):
    p = make_problem(replace(X1, **SMALL[name]), T, seed=T + 31, device=cuda, gen="numpy")
    check_problem(p, path=path, prepack=prepack)


@pytest.mark.parametrize("T", [1, 8, 64])
def test_mxfp4_simt_f32(cuda, T):
    p = make_problem(replace(X1, dtype="f32"), T, seed=T + 41, device=cuda, gen="numpy", hidden=256, inter=128,
                     experts=8)
    check_problem(p, path="simt")


@pytest.mark.parametrize("path,T", [("decode", 16), ("decode", 64), ("prefill", 40)])
def test_mxfp4_packed_equals_row_major(cuda, path, T):
    p = make_problem(X1, T, seed=T + 7, device=cuda, gen="numpy", hidden=320, inter=160, experts=8)
    inputs = p.schema_inputs()
    plain, packed = p.make_op(expert_path=path), p.make_op(expert_path=path)
    assert packed.prepack_all(*inputs) == [2, 3, 5, 6]
    y0, y1 = plain(*inputs), packed(*inputs)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)


def test_mxfp4_wide_scale_range(cuda):
    # E8M0 scales far below 1 (down to 2^-30 of the encoder's): the bf16
    # operand of an E2M1 value times any power of two in range is exact, so
    # decode (scale folded into the conversion) still matches the oracle
    p = make_problem(X1, 16, seed=5, device=cuda, gen="numpy", hidden=320, inter=160, experts=8)
    s1 = p.inputs["fc1_scales"]
    rng = np.random.default_rng(3)
    shift = torch.from_numpy(rng.integers(-30, 5, size=tuple(s1.shape)).astype(np.int64)).to(s1.device)
    p.inputs["fc1_scales"] = (s1.to(torch.int64) + shift).clamp(1, 254).to(torch.uint8)
    p.inputs["fc1_experts_bias"] = None
    p.inputs["fc2_experts_bias"] = None
    cfg = replace(p.cfg, bias=False, swiglu_limit=None)
    p.cfg = cfg
    check_problem(p, path="decode")


def test_mxfp4_full_decode_prepacked(cuda):
    p = make_problem(X1, 16, seed=216, device=cuda)
    check_problem(p, threads=16, prepack=True, report=True)


def test_mxfp4_full_prefill_prepacked(cuda):
    p = make_problem(X1, 8192, seed=8216, device=cuda)
    check_problem(p, sample_tokens=48, threads=16, prepack=True, report=True)


@pytest.mark.parametrize("over", [dict(block_size=64), dict(bits=8)])
def test_mxfp4_needs_4_bits_and_block_32(cuda, over):
    p = make_problem(X1, 4, seed=1, device=cuda, gen="numpy", hidden=256, inter=128, experts=4)
    ins = p.schema_inputs()
    kw = p.cfg.op_kwargs()
    kw.update(expert_weight_bits=over.get("bits", 4), block_size=over.get("block_size", 32))
    op = type(p.make_op())(**kw)
    with pytest.raises(MoeError) as ei:
        op(*ins)
    assert ei.value.code == 2
