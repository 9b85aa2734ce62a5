"""The benchmark configurations at full size against the oracle.

Decode token counts are checked on every token; prefill token counts check
routing for every token and the expert output on a seeded sample of tokens
(tokens are independent once routed, so a sample is an exact spot check).
Each case prints its largest error and the share of the tolerance the worst
element uses (pytest -rP shows the lines of passed tests).
"""
import pytest

from moe_testutil import check_problem
from onnxruntime_musa_amd.workloads import CONFIGS, make_problem

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["c2_qmoe_int8_mixtral", "c3_qmoe_int4_mixtral"])
@pytest.mark.parametrize("T", [1, 16])
def test_mixtral_decode(cuda, name, T):
    p = make_problem(CONFIGS[name], T, seed=100 + T, device=cuda)
    check_problem(p, threads=16, report=True)


@pytest.mark.parametrize("name", ["c2_qmoe_int8_mixtral", "c3_qmoe_int4_mixtral"])
def test_mixtral_prefill_4096(cuda, name):
    p = make_problem(CONFIGS[name], 4096, seed=4096, device=cuda)
    check_problem(p, sample_tokens=128, threads=16, report=True)


@pytest.mark.parametrize("T", [1, 16, 64, 512])
def test_gptoss_tokens(cuda, T):
    p = make_problem(CONFIGS["c4_qmoe_int4_gptoss"], T, seed=200 + T, device=cuda)
    check_problem(p, sample_tokens=128, threads=16, report=True)


def test_gptoss_8192(cuda):
    p = make_problem(CONFIGS["c4_qmoe_int4_gptoss"], 8192, seed=8192, device=cuda)
    check_problem(p, sample_tokens=128, threads=16, report=True)


def test_qwen3_zipf_8192(cuda):
    p = make_problem(CONFIGS["c5_moe_f16_qwen3"], 8192, seed=5, device=cuda)
    check_problem(p, sample_tokens=128, threads=16, report=True)
