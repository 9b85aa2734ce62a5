"""MoE / QMoE op on the GPU against the oracle, per expert-kernel family.

Every case checks routing ids, offsets and the dispatch permutation
bit-exactly (read back from the op's workspace) and the output against the
oracle with the build's tolerances (fp32 max-abs 1e-4, fp16/bf16
rtol = atol = 2e-2), following the reference's CPU-vs-device pattern
(test/ops/op_test_utils.py:274-308).
"""
import pytest
import torch

from moe_testutil import check_problem
from onnxruntime_musa_amd.workloads import CONFIGS, make_problem

pytestmark = pytest.mark.gpu

C1, C2, C3, C4, C5 = (CONFIGS[n] for n in ("c1_moe_f32", "c2_qmoe_int8_mixtral", "c3_qmoe_int4_mixtral",
                                           "c4_qmoe_int4_gptoss", "c5_moe_f16_qwen3"))


def test_c1_full_config(cuda):
    """configs[0] as specified: fp32 MoE, 64 tokens, H=128, I=256, E=8, top-2, SiLU, normalised, biases."""
    p = make_problem(C1, 64, seed=0, device=cuda)
    err = check_problem(p)
    assert err <= 1e-4


# Scaled-down shapes of each config; every expert-kernel family at decode and prefill token counts.
SMALL = {
    "c2": (C2, dict(hidden=256, inter=512)),
    "c3": (C3, dict(hidden=256, inter=512)),
    "c4": (C4, dict(hidden=192, inter=320, experts=8)),
    "c5": (C5, dict(hidden=256, inter=192, experts=32, k=4)),
    "c1f16": (C1, dict(dtype="f16")),
    "c1bf16": (C1, dict(dtype="bf16")),
}


@pytest.mark.parametrize("name", list(SMALL))
@pytest.mark.parametrize("path,T", [("simt", 5), ("decode", 1), ("decode", 16), ("decode", 40), ("decode", 64),
                                    ("prefill", 17), ("prefill", 300), ("auto", 7), ("auto", 520)])
def test_small_configs_all_paths(cuda, name, path, T):
    cfg, over = SMALL[name]
    p = make_problem(cfg, T, seed=T + 3, device=cuda, gen="numpy", **over)
    check_problem(p, path)


QUANT_VARIANTS = [
    dict(bits=8, block_size=0, scale_dtype="f16"),
    dict(bits=8, block_size=128, scale_dtype="f32"),
    dict(bits=8, block_size=32, scale_dtype="bf16"),
    dict(bits=4, block_size=0, scale_dtype="f16"),
    dict(bits=4, block_size=16, scale_dtype="f16"),
    dict(bits=4, block_size=32, scale_dtype="f16"),
    dict(bits=4, block_size=32, scale_dtype="bf16"),
    dict(bits=4, block_size=32, scale_dtype="f32"),
    dict(bits=8, block_size=32, scale_dtype="f16"),
    dict(bits=4, block_size=64, scale_dtype="f32"),
    dict(bits=4, block_size=256, scale_dtype="f16"),
]


@pytest.mark.parametrize("q", QUANT_VARIANTS, ids=lambda q: f"int{q['bits']}-bs{q['block_size']}-{q['scale_dtype']}")
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("path,T", [("decode", 9), ("decode", 48), ("prefill", 200)])
def test_quant_formats(cuda, q, dtype, path, T):
    p = make_problem(C3, T, seed=2, device=cuda, gen="numpy", hidden=256, inter=512, dtype=dtype, **q)
    check_problem(p, path)


@pytest.mark.parametrize("base,over", [
    (C5, dict(hidden=256, inter=3072, experts=8, k=2)),
    (C3, dict(hidden=256, inter=4096)),
    (C2, dict(hidden=256, inter=4096)),
    (C4, dict(hidden=256, inter=2880, experts=8)),
    (C4, dict(hidden=2880, inter=256, experts=8)),
], ids=["dense", "int4", "int8", "int4-bs32-bf16", "int4-bs32-bf16-k2880-fc1"])
@pytest.mark.parametrize("T", [1, 4, 16])
def test_decode_long_k_groups(cuda, base, over, T):
    """Few experts and a long fc2 K: the decode path splits K across
    workgroups into partial planes (K groups are whole multiples of the
    kernel's chunk walk; the last one is padded past K)."""
    p = make_problem(base, T, seed=11 + T, device=cuda, gen="numpy", **over)
    check_problem(p, "decode")


ACTS = [
    dict(activation="relu", use_fc3=False),
    dict(activation="gelu", use_fc3=False),
    dict(activation="silu", use_fc3=False),
    dict(activation="identity", use_fc3=False),
    dict(activation="silu", use_fc3=True),
    dict(activation="swiglu", use_fc3=True),
    dict(activation="swiglu", use_fc3=False, swiglu_fusion=1),
    dict(activation="swiglu", use_fc3=False, swiglu_fusion=2),
    dict(activation="swiglu", use_fc3=False, swiglu_fusion=1, swiglu_limit=0.5, alpha=1.702, beta=1.0),
]


@pytest.mark.parametrize("act", ACTS, ids=lambda a: "-".join(f"{v}" for v in a.values()))
@pytest.mark.parametrize("path,T", [("simt", 6), ("decode", 6), ("prefill", 150)])
def test_activations_and_gating(cuda, act, path, T):
    p = make_problem(C3, T, seed=5, device=cuda, gen="numpy", hidden=128, inter=256, bias=True, **act)
    check_problem(p, path)


def test_three_d_input_and_no_bias_k_equals_e(cuda):
    p = make_problem(C2, 24, seed=9, device=cuda, gen="numpy", hidden=128, inter=128, experts=4, k=4)
    p.inputs["input"] = p.inputs["input"].reshape(4, 6, 128).contiguous()
    p.inputs["router_probs"] = p.inputs["router_probs"]
    op = p.make_op()
    y = op(*p.schema_inputs())
    assert y.shape == (4, 6, 128)
    p.inputs["input"] = p.inputs["input"].reshape(24, 128)
    check_problem(p)


def test_single_expert_is_dense_ffn(cuda):
    p = make_problem(C2, 33, seed=4, device=cuda, gen="numpy", hidden=128, inter=256, experts=1, k=1)
    check_problem(p)


def test_empty_tokens(cuda):
    p = make_problem(C3, 0, seed=1, device=cuda, gen="numpy", hidden=128, inter=256)
    op = p.make_op()
    y = op(*p.schema_inputs())
    assert y.shape == (0, 128)


def test_odd_shapes_fall_back_to_simt(cuda):
    """H, I not multiples of 32: the MFMA families decline, the generic kernels run."""
    p = make_problem(C2, 10, seed=6, device=cuda, gen="numpy", hidden=72, inter=100, dtype="f16")
    check_problem(p)
