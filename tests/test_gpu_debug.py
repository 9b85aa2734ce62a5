"""The debugging switches on the GPU: MOE_DEBUG_SYNC (wait for the stream
after each stage, report the failing stage) and MOE_TRACE_KERNELS (a begin
and an end line per call), the role of the reference's MUSA_EP_TRACE_SYNC /
MUSA_EP_TRACE_KERNELS (musa/ep/src/kernels/shared_inc/kernel_base.h:48-80).
Outputs with the switches on equal those without, bit for bit, on each
expert path."""
from dataclasses import replace

import pytest
import torch

from onnxruntime_musa_amd.workloads import CONFIGS, make_problem

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,path,T,over", [
    ("c3_qmoe_int4_mixtral", "decode", 16, dict(hidden=256, inter=512)),
    ("c3_qmoe_int4_mixtral", "prefill", 300, dict(hidden=256, inter=512)),
    ("c1_moe_f32", "simt", 64, {}),
])
def test_debug_sync_and_trace(cuda, capfd, monkeypatch, name, path, T, over):
    p = make_problem(replace(CONFIGS[name], **over), T, seed=4, device=cuda, gen="numpy")
    inputs = p.schema_inputs()
    monkeypatch.delenv("MOE_DEBUG_SYNC", raising=False)
    monkeypatch.delenv("MOE_TRACE_KERNELS", raising=False)
    plain = p.make_op(expert_path=path)
    monkeypatch.setenv("MOE_DEBUG_SYNC", "1")
    monkeypatch.setenv("MOE_TRACE_KERNELS", "1")
    dbg = p.make_op(expert_path=path)  # the switches are read when a kernel is created
    y0, y1 = plain(*inputs), dbg(*inputs)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    err = capfd.readouterr().err
    op = "QMoE" if p.cfg.bits else "MoE"
    assert err.count(f"MOE_KERNEL_BEGIN {op}") == 1 and err.count(f"MOE_KERNEL_END {op}") == 1
    assert "status=0" in err
