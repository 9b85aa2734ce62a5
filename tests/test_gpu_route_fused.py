"""Routing inside the decode fc1 kernel.

Small decode batches (T * k <= 1024, E <= 128) are routed and dispatched by
every workgroup of the fc1 kernel in its prologue, and workgroup 0 writes the
results out for fc2 and finalize.  These cases check those results (ids,
offsets, permutation bit-exact; weights to fp32 rounding) and the layer
output against the oracle at the limits of that path and just past them
(where the router kernels run instead), including the reference's TopK tie
cases (test/ops/test_topk.py:230-246 ties -> lower index, :307-323 all-equal
-> arange(k)).
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

from moe_testutil import check_problem
from onnxruntime_musa_amd.workloads import CONFIGS, make_problem

pytestmark = pytest.mark.gpu

C3, C5 = CONFIGS["c3_qmoe_int4_mixtral"], CONFIGS["c5_moe_f16_qwen3"]
SMALL5 = dict(hidden=256, inter=192)


@pytest.mark.parametrize("E,k,T", [
    (8, 2, 1), (8, 8, 64),       # every expert taken by every token
    (64, 16, 64),                # T k = 1024: the largest batch routed in fc1
    (64, 17, 61),                # T k = 1037: router kernels
    (65, 2, 16),                 # two experts per lane from here on
    (128, 8, 16), (128, 8, 64),  # E = 128: the most experts routed in fc1
    (128, 64, 16),               # k = 64 (the op's limit), T k = 1024
    (129, 4, 16),                # E = 129: router kernels
    (33, 5, 7),
])
def test_decode_routing_limits(cuda, E, k, T):
    p = make_problem(replace(C5, experts=E, k=k, **SMALL5), T, seed=E * 100 + T, device=cuda, gen="numpy")
    check_problem(p, path="decode")


def _with_logits(p, logits):
    dt = p.inputs["router_probs"].dtype
    p.inputs["router_probs"] = torch.from_numpy(logits.astype(np.float32)).to(dt).to(p.inputs["input"].device)
    return p


@pytest.mark.parametrize("normalize", [0, 1])
def test_decode_routing_all_equal(cuda, normalize):
    p = make_problem(replace(C3, hidden=256, inter=512, normalize=normalize), 16, seed=1, device=cuda,
                     gen="numpy")
    check_problem(_with_logits(p, np.zeros((16, 8))), path="decode")


def test_decode_routing_ties_at_k_boundary(cuda):
    # three experts share the second-largest logit: the lower ids win
    rng = np.random.default_rng(5)
    lg = rng.standard_normal((40, 8)) - 4.0
    for t in range(40):
        top = rng.integers(8)
        tie = rng.choice([e for e in range(8) if e != top], size=3, replace=False)
        lg[t, top] = 2.0
        lg[t, tie] = 1.0
    p = make_problem(replace(C3, hidden=256, inter=512), 40, seed=2, device=cuda, gen="numpy")
    check_problem(_with_logits(p, lg), path="decode")


@pytest.mark.parametrize("normalize,T,path", [(1, 24, "decode"), (0, 24, "decode"), (1, 300, "prefill")])
def test_routing_sigmoid(cuda, normalize, T, path):
    # routing inside fc1 (decode) and by the router kernels (T > 256), both
    # against the oracle's sigmoid router: ids, offsets, permutation exact
    p = make_problem(replace(C5, experts=32, k=4, router_sigmoid=1, normalize=normalize, **SMALL5), T, seed=9,
                     device=cuda, gen="numpy")
    check_problem(p, path=path)
