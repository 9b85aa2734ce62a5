"""Shared helpers for the parity tests.

compare_outputs() follows the reference's run_and_compare semantics
(test/ops/op_test_utils.py:274-308): same shape, then same dtype, then
assert_allclose(actual, expected, rtol, atol).  Tolerances come from the
build target: fp32 max-abs 1e-4; fp16/bf16 rtol = atol = 2e-2.
"""
from __future__ import annotations

import numpy as np
import torch

from onnxruntime_musa_amd.workloads import Problem, to_host
from oracle import oracle

TOL = {"f32": (0.0, 1e-4), "f16": (2e-2, 2e-2), "bf16": (2e-2, 2e-2)}


def compare_outputs(got: np.ndarray, exp: np.ndarray, dtype: str, what: str, rows=None):
    assert got.shape == exp.shape, f"{what}: shape {got.shape} vs {exp.shape}"
    assert got.dtype == exp.dtype, f"{what}: dtype {got.dtype} vs {exp.dtype}"
    g = oracle.to_f32(got, dtype)
    e = oracle.to_f32(exp, dtype)
    if rows is not None:
        g, e = g[rows], e[rows]
    rtol, atol = TOL[dtype]
    assert np.all(np.isfinite(g)), f"{what}: non-finite output"
    np.testing.assert_allclose(g, e, rtol=rtol, atol=atol, err_msg=what)
    return float(np.max(np.abs(g - e))) if g.size else 0.0


def tolerance_margin(got: np.ndarray, exp: np.ndarray, dtype: str) -> float:
    """max over elements of |got - exp| / (atol + rtol |exp|): the share of
    the tolerance the worst element uses (the test fails above 1)."""
    g = oracle.to_f32(got, dtype).astype(np.float64)
    e = oracle.to_f32(exp, dtype).astype(np.float64)
    rtol, atol = TOL[dtype]
    return float(np.max(np.abs(g - e) / (atol + rtol * np.abs(e)))) if g.size else 0.0


def run_op(problem: Problem, path: str = "auto", with_workspace: bool = False, prepack: bool = False):
    op = problem.make_op(expert_path=path)
    inputs = problem.schema_inputs()
    if prepack:
        assert op.prepack_all(*inputs), "no expert weight was pre-packed"
    ws = None
    layout = None
    if with_workspace:
        nbytes = op.workspace_size(*inputs)
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=inputs[0].device)
        layout = op.workspace_layout(*inputs)
    y = op(*inputs, workspace=ws)
    torch.cuda.synchronize()
    routing = None
    if with_workspace:
        T, k, E = problem.tokens, problem.cfg.k, problem.cfg.experts

        def view(off, n, dt):
            return ws[off:off + n * 4].view(dt)[:n].cpu().numpy()

        routing = dict(topk_ids=view(layout["topk_ids"], T * k, torch.int32).reshape(T, k),
                       topk_w=view(layout["topk_w"], T * k, torch.float32).reshape(T, k),
                       offsets=view(layout["offsets"], E + 1, torch.int32),
                       perm=view(layout["perm"], T * k, torch.int32),
                       inv_perm=view(layout["inv_perm"], T * k, torch.int32))
    return y, routing


def check_problem(problem: Problem, path: str = "auto", sample_tokens=None, seed=0, threads=0, prepack=False,
                  report=False):
    """Runs the HIP op and the oracle on the same inputs and compares.
    sample_tokens: compute the oracle's expert FFN for this many sampled tokens
    only (routing is still checked for every token).  report: print the
    largest error and the share of the tolerance it uses."""
    y, routing = run_op(problem, path, with_workspace=True, prepack=prepack)
    host = {n: to_host(t) for n, t in problem.inputs.items()}
    T = problem.tokens
    mask, rows = None, None
    if sample_tokens is not None and sample_tokens < T:
        rng = np.random.default_rng(seed)
        rows = np.sort(rng.choice(T, size=sample_tokens, replace=False))
        mask = np.zeros(T, np.uint8)
        mask[rows] = 1
    ref = oracle.forward_problem(problem.cfg, host, token_mask=mask, threads=threads)
    # routing: bit-exact ids, offsets and permutation; weights to fp32 rounding
    np.testing.assert_array_equal(routing["topk_ids"], ref["topk_ids"], err_msg="topk ids")
    np.testing.assert_array_equal(routing["offsets"], ref["offsets"], err_msg="expert offsets")
    np.testing.assert_array_equal(routing["perm"], ref["perm"], err_msg="dispatch permutation")
    if T:
        np.testing.assert_array_equal(routing["inv_perm"][routing["perm"]], np.arange(T * problem.cfg.k),
                                      err_msg="inverse permutation")
    np.testing.assert_allclose(routing["topk_w"], ref["topk_w"], rtol=2e-6, atol=1e-7, err_msg="routing weights")
    what = f"{problem.cfg.name} T={T} path={path}"
    got = to_host(y)
    if report:
        g, e = (got, ref["out"]) if rows is None else (got[rows], ref["out"][rows])
        err = float(np.max(np.abs(oracle.to_f32(g, problem.cfg.dtype) - oracle.to_f32(e, problem.cfg.dtype))))
        print(f"[parity] {what}: max|err| {err:.3e}, worst element at "
              f"{tolerance_margin(g, e, problem.cfg.dtype):.3f} of the tolerance "
              f"({'all' if rows is None else len(rows)} tokens compared)", flush=True)
    return compare_outputs(got, ref["out"], problem.cfg.dtype, what, rows=rows)
