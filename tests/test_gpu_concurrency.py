"""One kernel object shared by several threads, each on its own stream.

The reference runs one session from several threads and streams
(test/multi_stream/test_allocator_cache_shared_session.py:62-79); the C ABI
promises that concurrent moe_kernel_compute calls are safe when each passes
its own workspace, or share one cached workspace per (device, stream) when
they pass none.  Every output must be bit-identical to a serial call (the
kernels' sums have a fixed order).  Streams keep the default priority.
"""
import threading
from dataclasses import replace

import pytest
import torch

from onnxruntime_musa_amd.workloads import CONFIGS, make_problem

pytestmark = pytest.mark.gpu

C3 = CONFIGS["c3_qmoe_int4_mixtral"]


@pytest.mark.parametrize("T", [16, 300])  # decode (routing inside fc1) and prefill
@pytest.mark.parametrize("own_workspace", [True, False])
def test_shared_kernel_threads_and_streams(cuda, T, own_workspace):
    p = make_problem(replace(C3, hidden=256, inter=512), T, seed=T, device=cuda, gen="numpy")
    inputs = p.schema_inputs()
    op = p.make_op()
    op.prepack_all(*inputs)
    ref = op(*inputs).clone()
    torch.cuda.synchronize()
    results, errors = {}, []

    def worker(i):
        try:
            s = torch.cuda.Stream(device=cuda)
            outs = []
            with torch.cuda.stream(s):
                ws = torch.empty((op.workspace_size(*inputs),), dtype=torch.uint8, device=cuda) if own_workspace else None
                for _ in range(12):
                    outs.append(op(*inputs, workspace=ws, stream=s))
            s.synchronize()
            results[i] = outs
        except Exception as e:  # reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    assert len(results) == 4
    for outs in results.values():
        for y in outs:
            assert torch.equal(y, ref)
