"""moe_kernel_compute_noalloc against moe_kernel_compute with a caller
workspace: the same kernels on the library's static scratch, so outputs are
bit-identical.  Two calls in a row, the second with a smaller input (the
scratch keeps the first call's contents), on the decode and prefill paths;
a problem larger than the scratch is rejected with INVALID_ARGUMENT."""
from dataclasses import replace

import pytest
import torch

from onnxruntime_musa_amd import MoeError
from onnxruntime_musa_amd.workloads import CONFIGS, make_problem

pytestmark = pytest.mark.gpu

C3, C4 = CONFIGS["c3_qmoe_int4_mixtral"], CONFIGS["c4_qmoe_int4_gptoss"]


def _pair(cuda, cfg, T, seed, path="auto"):
    p = make_problem(cfg, T, seed=seed, device=cuda, gen="numpy")
    inputs = p.schema_inputs()
    op = p.make_op(expert_path=path)
    ws = torch.empty((op.workspace_size(*inputs),), dtype=torch.uint8, device=cuda)
    ref = op(*inputs, workspace=ws)
    got = op.compute_noalloc(*inputs, out=torch.empty_like(inputs[0]))
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.parametrize("cfg,over,path,sizes", [
    (C3, dict(hidden=512, inter=1024), "decode", (16, 3)),
    (C3, dict(hidden=512, inter=1024), "prefill", (300, 70)),
    (C4, dict(hidden=256, inter=256, experts=16), "auto", (64, 1)),
])
def test_noalloc_matches_workspace_entry_point(cuda, cfg, over, path, sizes):
    for T in sizes:  # the second call is smaller
        ref, got = _pair(cuda, replace(cfg, **over), T, seed=T, path=path)
        assert torch.equal(ref, got), f"T={T}: max diff {(ref.float() - got.float()).abs().max().item()}"


def test_noalloc_full_decode_size(cuda):
    # Mixtral-shaped int4 at 16 tokens: the headline decode shape
    ref, got = _pair(cuda, C3, 16, seed=16)
    assert torch.equal(ref, got)


def test_noalloc_rejects_a_workspace_above_the_scratch(cuda):
    p = make_problem(replace(C3, hidden=512, inter=4096), 4096, seed=1, device=cuda, gen="numpy")
    inputs = p.schema_inputs()
    op = p.make_op()
    assert op.workspace_size(*inputs) > 64 << 20
    with pytest.raises(MoeError) as ei:
        op.compute_noalloc(*inputs, out=torch.empty_like(inputs[0]))
    assert ei.value.code == 2 and "scratch" in str(ei.value)
