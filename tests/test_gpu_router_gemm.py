"""Router-GEMM fusion (moe_kernel_compute_fused_router) against the oracle.

The routing kernels compute logits = x W_gate^T (+ b) with fp32
accumulation, round them once to the activation type and route them in the
same launch.  Checks, per expert path and router kernel (single workgroup,
multi-workgroup):
  * exactly representable inputs (small dyadic x, W, b: every partial sum is
    exact in fp32, so any summation order gives the same value): logits equal
    the oracle's float64 matmul rounded once, bit for bit, and routing ids,
    offsets and permutation equal the oracle's bit for bit;
  * random inputs: logits within one unit in the last place of the oracle's
    (the kernel's fp32 summation order is not the float64 one), then the
    oracle routes the kernel's own logits: ids and permutation exact, output
    within the fp32 / fp16 / bf16 tolerance.
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

from moe_testutil import compare_outputs
from onnxruntime_musa_amd import MoeError
from onnxruntime_musa_amd.workloads import CONFIGS, make_problem, to_host
from oracle import oracle

pytestmark = pytest.mark.gpu

_TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
C1, C3, C4, C5 = (CONFIGS[n] for n in ("c1_moe_f32", "c3_qmoe_int4_mixtral", "c4_qmoe_int4_gptoss",
                                       "c5_moe_f16_qwen3"))


def _gate_inputs(cfg, T, seed, exact, bias):
    rng = np.random.default_rng(seed)
    H, E = cfg.hidden, cfg.experts
    if exact:
        x = rng.integers(-2, 3, size=(T, H)) * 0.25
        w = rng.integers(-3, 4, size=(E, H)) * 0.0625
        b = rng.integers(-8, 9, size=E) * 0.125
    else:
        x = rng.standard_normal((T, H))
        w = rng.standard_normal((E, H)) / np.sqrt(H)
        b = rng.standard_normal(E) * 0.5
    return x, w, (b if bias else None)


def _dev(a, dt, cuda):
    return None if a is None else torch.from_numpy(np.asarray(a, np.float32)).to(_TD[dt]).to(cuda).contiguous()


def _ulp(v: np.ndarray, dt: str) -> np.ndarray:
    if dt == "f32":
        return np.spacing(np.abs(v).astype(np.float32)).astype(np.float64)
    mant = 10 if dt == "f16" else 7
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -14)))
    return 2.0 ** (e - mant)


def run_case(cuda, cfg, T, path, exact, bias, seed=3):
    p = make_problem(cfg, T, seed=seed, device=cuda, gen="numpy")
    dt = cfg.dtype
    x, w, b = _gate_inputs(cfg, T, seed + 1, exact, bias)
    p.inputs["input"] = _dev(x, dt, cuda)
    wg, bg = _dev(w, dt, cuda), _dev(b, dt, cuda)
    op = p.make_op(expert_path=path)
    full = p.schema_inputs()  # router_probs of shape [T, E] for the workspace query
    ws = torch.empty((op.workspace_size(*full),), dtype=torch.uint8, device=cuda)
    lay = op.workspace_layout(*full)
    ins = list(full)
    ins[1] = None
    y = op.fused_router(*ins, router_weight=wg, router_bias=bg, workspace=ws)
    torch.cuda.synchronize()
    E, k = cfg.experts, cfg.k
    esz = 4 if dt == "f32" else 2
    raw = ws[lay["logits"]:lay["logits"] + T * E * esz].cpu()
    if dt == "f32":
        got_lg = raw.view(torch.float32).numpy().reshape(T, E)
    elif dt == "f16":
        got_lg = raw.view(torch.float16).numpy().reshape(T, E)
    else:
        got_lg = raw.view(torch.int16).numpy().view(np.uint16).reshape(T, E)
    host = {n: to_host(t) for n, t in p.inputs.items()}
    exp_lg = oracle.gate_logits(host["input"], to_host(wg), None if bg is None else to_host(bg), dt)
    g64, e64 = oracle.to_f32(got_lg, dt).astype(np.float64), oracle.to_f32(exp_lg, dt).astype(np.float64)
    if exact:
        np.testing.assert_array_equal(g64, e64, err_msg="fused router logits")
    else:
        # fp32 summation of H + 1 terms in another order than the float64 one:
        # the textbook forward error bound (H + 1) u sum |x w| (+ |b|), u =
        # 2^-24, then one rounding to the activation type (one unit in the
        # last place); near-zero logits of large cancelling terms are bound
        # by the first term, the others by the second
        xf = oracle.to_f32(host["input"], dt).astype(np.float64)
        wf = oracle.to_f32(to_host(wg), dt).astype(np.float64)
        bound = (cfg.hidden + 1) * 2.0 ** -24 * (np.abs(xf) @ np.abs(wf).T + (0 if b is None else np.abs(b)))
        r = np.abs(g64 - e64) / (bound + _ulp(e64, dt))
        i = np.unravel_index(np.argmax(r), r.shape)
        assert r[i] <= 1.0, f"fused router logit {i}: {g64[i]!r} vs {e64[i]!r}, beyond fp32 bound + one ulp"
    # the oracle routes the kernel's logits (equal to its own in the exact case)
    host["router_probs"] = got_lg
    ref = oracle.forward_problem(p.cfg, host, threads=8)

    def view(off, n, dtp):
        return ws[off:off + n * 4].view(dtp)[:n].cpu().numpy()
    np.testing.assert_array_equal(view(lay["topk_ids"], T * k, torch.int32).reshape(T, k), ref["topk_ids"])
    np.testing.assert_array_equal(view(lay["offsets"], E + 1, torch.int32), ref["offsets"])
    np.testing.assert_array_equal(view(lay["perm"], T * k, torch.int32), ref["perm"])
    compare_outputs(to_host(y), ref["out"], dt, f"fused router {cfg.name} T={T} path={path}")


SMALL3 = dict(hidden=512, inter=512)


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("cfg,over,T,path", [
    (C3, SMALL3, 16, "decode"),                               # one workgroup routes, decode experts
    (C3, SMALL3, 1, "decode"),
    (C3, SMALL3, 300, "prefill"),                             # multi-workgroup router
    (C3, dict(hidden=4096, inter=256, experts=16), 100, "auto"),  # T E H above the one-workgroup limit
    (C5, dict(hidden=256, inter=128, experts=128), 64, "auto"),   # 128 experts: 16 expert chunks per token
    (C1, {}, 64, "simt"),                                     # fp32
])
def test_fused_router(cuda, cfg, over, T, path, exact):
    run_case(cuda, replace(cfg, **over), T, path, exact, bias=False)


@pytest.mark.parametrize("T", [16, 300])
def test_fused_router_with_bias_bf16(cuda, T):
    # gpt-oss-shaped router (bias on), bf16, interleaved SwiGLU experts
    run_case(cuda, replace(C4, hidden=256, inter=256, experts=32), T, "auto", exact=True, bias=True)
    run_case(cuda, replace(C4, hidden=256, inter=256, experts=32), T, "auto", exact=False, bias=True, seed=9)


def test_fused_router_hidden_not_a_multiple_of_8(cuda):
    run_case(cuda, replace(C1, hidden=100), 20, "simt", exact=False, bias=True)


def test_fused_router_errors(cuda):
    p = make_problem(replace(C3, **SMALL3), 8, seed=1, device=cuda, gen="numpy")
    op = p.make_op()
    ins = p.schema_inputs()
    ins[1] = None
    x = p.inputs["input"]
    for bad in (torch.zeros((8, 511), dtype=x.dtype, device=cuda),      # hidden mismatch
                torch.zeros((8, 512), dtype=torch.float32, device=cuda)):  # type mismatch
        with pytest.raises(MoeError) as ei:
            op.fused_router(*ins, router_weight=bad)
        assert ei.value.code == 2
    with pytest.raises(MoeError) as ei:
        op.fused_router(*ins, router_weight=torch.zeros((8, 512), dtype=x.dtype, device=cuda),
                        router_bias=torch.zeros((7,), dtype=x.dtype, device=cuda))
    assert ei.value.code == 2
