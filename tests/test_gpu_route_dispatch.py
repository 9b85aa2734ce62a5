"""Router + dispatch stage on the GPU against the oracle: ids, offsets and the
permutation bit-exact; weights to fp32 rounding.  Includes the reference's
TopK tie known-answer cases (test/ops/test_topk.py:230-246 ties -> lower
index, :307-323 all-equal -> arange(k), :212-227 adjacent floats are not ties).
"""
import numpy as np
import pytest
import torch

from onnxruntime_musa_amd import route_dispatch
from oracle import oracle

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _run(cuda, logits_f32, k, dt="f32", normalize=False, sigmoid=False):
    lt = torch.from_numpy(np.ascontiguousarray(logits_f32, dtype=np.float32)).to(DT[dt]).to(cuda)
    r = route_dispatch(lt, k, normalize, sigmoid)
    torch.cuda.synchronize()
    got = {n: v.cpu().numpy() for n, v in r.items()}
    rounded = lt.float().cpu().numpy()
    T, E = rounded.shape
    ids, w = oracle.route(rounded, k, normalize, sigmoid)
    offs, perm = oracle.dispatch(ids, E)
    np.testing.assert_array_equal(got["topk_ids"], ids)
    np.testing.assert_array_equal(got["offsets"], offs)
    np.testing.assert_array_equal(got["perm"], perm)
    if T:
        np.testing.assert_array_equal(got["inv_perm"][got["perm"]], np.arange(T * k))
    np.testing.assert_allclose(got["topk_w"], w, rtol=2e-6, atol=1e-7)
    return got


@pytest.mark.parametrize("T", [0, 1, 3, 16, 64, 255, 256, 257, 1000, 4096, 8192])
@pytest.mark.parametrize("E,k", [(8, 2), (32, 4), (128, 8)])
def test_route_dispatch_random(cuda, T, E, k):
    rng = np.random.default_rng(T * 7919 + E)
    _run(cuda, rng.standard_normal((T, E)), k, "f16", normalize=True)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("normalize,sigmoid", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_route_dispatch_dtypes_modes(cuda, dt, normalize, sigmoid):
    rng = np.random.default_rng(11)
    _run(cuda, rng.standard_normal((300, 16)), 3, dt, bool(normalize), bool(sigmoid))


@pytest.mark.parametrize("E,k", [(1, 1), (5, 5), (64, 64), (65, 3), (129, 7), (256, 16), (512, 8)])
@pytest.mark.parametrize("T", [7, 700])
def test_route_dispatch_odd_widths(cuda, E, k, T):
    rng = np.random.default_rng(E * 31 + k)
    _run(cuda, rng.standard_normal((T, E)), k, "f32", normalize=True)


@pytest.mark.parametrize("T", [50, 3000])
def test_route_dispatch_heavy_ties(cuda, T):
    """Logits on a coarse grid: ties everywhere, including at the k boundary."""
    rng = np.random.default_rng(5)
    logits = np.round(rng.standard_normal((T, 16)) * 2) / 2
    _run(cuda, logits, 4, "f32")


@pytest.mark.parametrize("E,k", [(8, 2), (4000 // 32, 16)])
def test_all_equal_logits_pick_lowest_ids(cuda, E, k):
    got = _run(cuda, np.full((5, E), 3.25), k)
    np.testing.assert_array_equal(got["topk_ids"], np.tile(np.arange(k), (5, 1)))


def test_tie_kat_lower_index_k1(cuda):
    # test_topk.py:230-246 pattern: equal maxima, the lower index wins
    got = _run(cuda, np.array([[4.0, 7.0, 1.0, 7.0], [9.0, 1.0, 9.0, 8.0]]), 1)
    np.testing.assert_array_equal(got["topk_ids"][:, 0], [1, 0])


def test_adjacent_floats_are_not_ties(cuda):
    nxt = np.nextafter(np.float32(10.0), np.float32(np.inf))
    got = _run(cuda, np.array([[10.0, nxt, 9.0]], dtype=np.float32), 1)
    np.testing.assert_array_equal(got["topk_ids"], [[1]])


def test_k_equals_e_is_full_order(cuda):
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((20, 8)).astype(np.float32)
    got = _run(cuda, logits, 8, normalize=True)
    np.testing.assert_array_equal(got["topk_ids"], np.argsort(-logits, axis=1, kind="stable"))
    np.testing.assert_allclose(got["topk_w"].sum(axis=1), 1.0, rtol=1e-6)


def test_normalize_k1_gives_unit_weight(cuda):
    rng = np.random.default_rng(4)
    got = _run(cuda, rng.standard_normal((33, 8)), 1, normalize=True)
    np.testing.assert_array_equal(got["topk_w"], np.ones((33, 1), np.float32))


def test_zipf_skewed_routing(cuda):
    """Skewed load (a few hot experts hold most rows) at the Qwen3 shape."""
    from onnxruntime_musa_amd.workloads import CONFIGS, make_problem
    p = make_problem(CONFIGS["c5_moe_f16_qwen3"], 8192, seed=1, device=cuda, hidden=64, inter=64)
    logits = p.inputs["router_probs"].float().cpu().numpy()
    got = _run(cuda, logits, 8, "f16", normalize=True)
    counts = np.diff(got["offsets"])
    assert counts.max() > 4 * counts.mean()
