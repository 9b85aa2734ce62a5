#!/usr/bin/env python3
"""MoE / QMoE layer benchmark on one MI355X.

A step is one QMoE layer invocation (router + dispatch + fc1/fc3 + activation
+ fc2 + finalize) over one batch of synthetic tokens whose inputs and weights
are already resident in HBM.  The headline workload is the configuration the
decode target is quoted on: QMoE int4 block-128 (fp16 scales), Mixtral shape
(H=4096, I=14336, E=8, top-2, SwiGLU fc1/fc3 unfused), fp16 activations, at
16 tokens (decode).  The other configurations are reported under "extra".

Decode workloads whose routed weights are smaller than twice the 256 MB
Infinity Cache (e.g. 2 Mixtral int4 experts at T=1) rotate through enough
copies of the expert weights (at least 4, together at least 1 GiB) that no
step can find the previous step's weights in a cache: every step reads its
weights from HBM.

Roofline: the dominant kernel's algorithmic bytes (decode) or FLOPs (prefill)
per launch divided by its mean duration, timed with HIP events recorded by the
library on the stream the kernels run on (moe_kernel_stage_times).

cpu_baseline: the oracle (C restatement, OpenMP) on the same inputs on the
host cores this process may use (its affinity mask, or OMP_NUM_THREADS where
that is smaller: the CPU share a GPU box allots).  It is a reported
baseline, not the target.  A second line times the prefill layer (C3 T=4096)
on a sample of its tokens.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extra] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "onnxruntime-musa_amd" / "python"))
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0   # MI355X HBM3E
PEAK_MFMA_TFLOPS = 2500.0  # MI355X dense fp16/bf16

METRIC = "QMoE layer tokens/s; HBM GB/s at decode, MFMA TFLOP/s at prefill, % roofline"
HEADLINE = ("c3_qmoe_int4_mixtral", 16)
CPU_PREFILL = ("c3_qmoe_int4_mixtral", 4096, 512)  # workload, tokens, tokens sampled on the CPU
MALL_BYTES = 256 << 20  # MI355X Infinity Cache
EXTRA = [("c2_qmoe_int8_mixtral", 1), ("c2_qmoe_int8_mixtral", 16), ("c2_qmoe_int8_mixtral", 4096),
         ("c3_qmoe_int4_mixtral", 1), ("c3_qmoe_int4_mixtral", 4096),
         ("c4_qmoe_int4_gptoss", 1), ("c4_qmoe_int4_gptoss", 16), ("c4_qmoe_int4_gptoss", 64),
         ("c4_qmoe_int4_gptoss", 8192), ("c5_moe_f16_qwen3", 8192), ("c1_moe_f32", 64),
         # extension: gpt-oss shape with MXFP4 experts (not a BASELINE config)
         ("x1_mxfp4_gptoss", 16), ("x1_mxfp4_gptoss", 8192)]


def esz(dt: str) -> int:
    return {"f32": 4, "e8m0": 1}.get(dt, 2)


def expert_bytes(cfg, part: str) -> int:
    """HBM bytes of one expert's weights + scales + biases for fc1 (incl. fc3) or fc2."""
    H, I = cfg.hidden, cfg.inter
    mats = [(cfg.n1, H)] + ([(I, H)] if cfg.use_fc3 else []) if part == "fc1" else [(H, I)]
    total = 0
    for n, k in mats:
        if cfg.bits:
            total += n * k * cfg.bits // 8
            total += n * (k // cfg.block_size if cfg.block_size else 1) * esz(cfg.scale_dtype)
        else:
            total += n * k * esz(cfg.dtype)
        if cfg.bias:
            total += n * esz(cfg.dtype)
    return total


def kernel_cost(cfg, T: int, hit: int):
    """Algorithmic bytes and FLOPs per launch of the fc1 and fc2 kernels."""
    rows = T * cfg.k
    a = esz(cfg.dtype)
    fc1_bytes = hit * expert_bytes(cfg, "fc1") + T * cfg.hidden * a + rows * cfg.inter * a
    fc2_bytes = hit * expert_bytes(cfg, "fc2") + rows * cfg.inter * a + rows * cfg.hidden * 4
    n1_total = cfg.n1 + (cfg.inter if cfg.use_fc3 else 0)
    fc1_flops = rows * 2 * n1_total * cfg.hidden
    fc2_flops = rows * 2 * cfg.hidden * cfg.inter
    layer_bytes = (hit * (expert_bytes(cfg, "fc1") + expert_bytes(cfg, "fc2")) + T * cfg.hidden * a * 2
                   + T * cfg.experts * a)
    return dict(fc1_bytes=fc1_bytes, fc2_bytes=fc2_bytes, fc1_flops=fc1_flops, fc2_flops=fc2_flops,
                layer_bytes=layer_bytes, layer_flops=fc1_flops + fc2_flops)


def measured_traffic(key: str):
    """HBM bytes per fc1 launch measured by two rocprofv3 PMC runs (FETCH_SIZE,
    WRITE_SIZE), each scaled by what the counter reads for a plain copy of
    known size; stored in profiles/traffic.json.  None when not measured."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    ent = json.loads(f.read_text()).get("workloads", {}).get(key)
    return ent["bytes"] if ent else None


WEIGHT_NAMES = ("fc1_experts_weights", "fc1_scales", "fc1_experts_bias", "fc2_experts_weights", "fc2_scales",
                "fc2_experts_bias", "fc3_experts_weights", "fc3_scales", "fc3_experts_bias")


def weight_copies(routed_bytes: int) -> int:
    """Copies of the expert weights a decode step rotates through: 1 when the
    routed weights are at least twice the Infinity Cache, else enough copies
    (at least 4, together at least 1 GiB) that a step never finds its weights
    still cached from an earlier step."""
    if routed_bytes >= 2 * MALL_BYTES:
        return 1
    return max(4, -(-(4 * MALL_BYTES) // max(routed_bytes, 1)))


def run_workload(name: str, T: int, steps: int, warmup: int, dev, keep_problem=False, prepack=True):
    import torch

    from onnxruntime_musa_amd.workloads import CONFIGS, make_problem

    cfg = CONFIGS[name]
    prob = make_problem(cfg, T, seed=1234, device=dev)
    inputs = prob.schema_inputs()
    names = prob.input_names[:len(inputs)]
    ws = out = None

    def build(ins):
        """One op over `ins`; session set-up: QMoE expert weights pre-packed
        once (not timed), as a plugin EP's PrePack does for constant
        initializers.  Returns (op, its call, packed input indices)."""
        nonlocal ws, out
        op = prob.make_op()
        packed = op.prepack_all(*ins) if prepack else []
        ins = [None if i in packed else t for i, t in enumerate(ins)]
        if ws is None:
            ws = torch.empty((op.workspace_size(*ins),), dtype=torch.uint8, device=dev)
            out = torch.empty_like(inputs[0])
        return op, op.bind(*ins, out=out, workspace=ws), packed

    op, call, packed = build(inputs)
    call()
    torch.cuda.synchronize()
    # routing of this workload: experts actually hit
    lay = op.workspace_layout(*[None if i in packed else t for i, t in enumerate(inputs)])
    offs = ws[lay["offsets"]:lay["offsets"] + 4 * (cfg.experts + 1)].view(torch.int32).cpu()
    hit = int((offs[1:] - offs[:-1] > 0).sum())
    cost = kernel_cost(cfg, T, hit)
    decode_sized = T <= 64
    ncopy = weight_copies(hit * (expert_bytes(cfg, "fc1") + expert_bytes(cfg, "fc2"))) if decode_sized else 1
    ops, calls = [op], [call]
    for _ in range(ncopy - 1):
        # the same weights at other addresses (the row-major copy is dropped
        # once packed)
        ins = [t.clone() if (t is not None and n in WEIGHT_NAMES) else t for n, t in zip(names, inputs)]
        o, c, _ = build(ins)
        ops.append(o)
        calls.append(c)
        del ins
    torch.cuda.synchronize()
    for i in range(warmup):
        calls[i % ncopy]()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        calls[i % ncopy]()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = max(start.elapsed_time(stop), wall * 1e3) / steps
    # per-stage timing pass (events recorded by the library on the kernels' stream)
    for o in ops:
        o.set_profiling(True)
    stages = []
    for i in range(steps):
        calls[i % ncopy]()
        stages.append(ops[i % ncopy].stage_times())
    for o in ops:
        o.set_profiling(False)
    path = stages[-1]["path"]
    st = {k: statistics.mean(s[k] for s in stages) for k in ("route_dispatch", "fc1", "fc2", "finalize")}
    decode = path != "prefill"
    traffic = measured_traffic(f"{name}:{T}")
    if decode:
        fc1_ach = cost["fc1_bytes"] / (st["fc1"] * 1e-3) / 1e9
        roof = dict(bound="hbm", achieved=round(fc1_ach, 1), peak=PEAK_HBM_GBS, unit="GB/s",
                    frac=round(fc1_ach / PEAK_HBM_GBS, 4), traffic=traffic)
    else:
        fc1_ach = cost["fc1_flops"] / (st["fc1"] * 1e-3) / 1e12
        roof = dict(bound="mfma", achieved=round(fc1_ach, 1), peak=PEAK_MFMA_TFLOPS, unit="TFLOP/s",
                    frac=round(fc1_ach / PEAK_MFMA_TFLOPS, 4), traffic=traffic)
    layer_s = ms_per_step * 1e-3
    res = dict(workload=name, tokens=T, path=path, prepacked=packed, ms_per_step=round(ms_per_step, 4),
               tokens_per_s=round(T / layer_s, 1), experts_hit=hit, weight_copies=ncopy,
               layer_hbm_gbs=round(cost["layer_bytes"] / layer_s / 1e9, 1),
               layer_tflops=round(cost["layer_flops"] / layer_s / 1e12, 2),
               stages_ms={k: round(v, 4) for k, v in st.items()},
               fc2=dict(achieved_gbs=round(cost["fc2_bytes"] / (st["fc2"] * 1e-3) / 1e9, 1),
                        achieved_tflops=round(cost["fc2_flops"] / (st["fc2"] * 1e-3) / 1e12, 2)),
               roofline=roof, algorithmic=dict(fc1_bytes=cost["fc1_bytes"], fc1_flops=cost["fc1_flops"]))
    del ops, calls, op, call, ws, out
    if keep_problem:
        torch.cuda.empty_cache()
        return res, prob
    del prob, inputs
    torch.cuda.empty_cache()
    return res, None


def run_op(spec: str, steps: int, warmup: int, dev) -> dict:
    """Times the stand-alone TopK or Softmax op on an fp32 [rows, dim] input
    along the last axis.  Algorithmic bytes: the input read once plus the
    outputs written once (TopK: k values and k int64 indices per row)."""
    import ctypes

    import torch

    from onnxruntime_musa_amd import _capi as C

    parts = spec.split(":")
    op = parts[0]
    rows, dim = (int(v) for v in parts[1].split("x"))
    k = int(parts[2]) if len(parts) > 2 else 8
    x = torch.randn((rows, dim), device=dev)
    lib = C.load_library()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    # buffers and parameters built once, so that the loop times the kernels
    # and not the Python wrapper's allocations
    if op == "topk":
        vals = torch.empty((rows, k), device=dev)
        idx = torch.empty((rows, k), dtype=torch.int64, device=dev)
        prm = C.MoeTopKParams(input=x.data_ptr(), elem_type=C.ELEM_FLOAT, largest=1, sorted=1, rows=rows, dim=dim,
                              inner=1, k=k, values=vals.data_ptr(), indices=idx.data_ptr())
        fn = lib.moe_topk_launch
        nbytes = rows * dim * 4 + rows * k * (4 + 8)
    elif op == "softmax":
        y = torch.empty_like(x)
        prm = C.MoeSoftmaxParams(input=x.data_ptr(), output=y.data_ptr(), elem_type=C.ELEM_FLOAT, outer=rows,
                                 dim=dim, inner=1)
        fn = lib.moe_softmax_launch
        nbytes = rows * dim * 4 * 2
    else:
        raise SystemExit(f"unknown op {op}")
    ref = ctypes.byref(prm)

    def call():
        C.check(fn(ref, stream))
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        call()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(op=op, rows=rows, dim=dim, k=k if op == "topk" else None, dtype="f32", ms_per_call=round(ms, 4),
                roofline=dict(bound="hbm", achieved=round(gbs, 1), peak=PEAK_HBM_GBS, unit="GB/s",
                              frac=round(gbs / PEAK_HBM_GBS, 4)))


ROUTER_FUSION = [("c3_qmoe_int4_mixtral", 16), ("c3_qmoe_int4_mixtral", 4096), ("c4_qmoe_int4_gptoss", 16)]


def run_router_fusion(name: str, T: int, steps: int, warmup: int, dev) -> dict:
    """The router GEMM fused into the op (moe_kernel_compute_fused_router)
    against the unfused pair it replaces: the graph's gate MatMul (torch's,
    hipBLASLt) writing the logits, then the op reading them.  Random
    [E, H] gate weights of the activation type."""
    import torch

    from onnxruntime_musa_amd.workloads import CONFIGS, make_problem

    cfg = CONFIGS[name]
    prob = make_problem(cfg, T, seed=1234, device=dev)
    x = prob.inputs["input"]
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    wg = (torch.randn((cfg.experts, cfg.hidden), generator=g, device=dev) / cfg.hidden ** 0.5).to(x.dtype)
    wt = wg.t().contiguous()  # the MatMul's [H, E] operand
    op = prob.make_op()
    ins = prob.schema_inputs()
    packed = op.prepack_all(*ins)
    ins = [None if i in packed else t for i, t in enumerate(ins)]
    ws = torch.empty((op.workspace_size(*ins),), dtype=torch.uint8, device=dev)
    out = torch.empty_like(x)
    logits = torch.empty_like(prob.inputs["router_probs"])
    ins_u = list(ins)
    ins_u[1] = logits
    call_u = op.bind(*ins_u, out=out, workspace=ws)
    ins_f = list(ins)
    ins_f[1] = None
    call_f = op.bind_fused_router(*ins_f, router_weight=wg, out=out, workspace=ws)

    def unfused():
        torch.matmul(x, wt, out=logits)
        call_u()

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / steps

    tu, tf = timed(unfused), timed(call_f)
    res = dict(workload=name, tokens=T, unfused_ms=round(tu, 4), fused_ms=round(tf, 4),
               saved_us=round((tu - tf) * 1e3, 1))
    del op, ws, out, prob, ins, ins_u, ins_f, call_u, call_f
    torch.cuda.empty_cache()
    return res


def cpu_model() -> str:
    """The host CPU's model name (lscpu's "Model name", from /proc/cpuinfo)."""
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(prob, budget_s: float = 12.0, sample_tokens=None):
    """Times the oracle on a workload on this host's cores: every core of
    the affinity mask, or OMP_NUM_THREADS where that is smaller (the CPU
    share a GPU box allots).  sample_tokens: compute the expert FFN for that
    many seeded token samples only (routing for every token); tokens/s is
    then sample_tokens / time."""
    import numpy as np

    from onnxruntime_musa_amd.workloads import to_host
    from oracle import oracle

    affinity = len(os.sched_getaffinity(0))
    cores = min(affinity, int(os.environ.get("OMP_NUM_THREADS") or affinity))
    host = {n: to_host(t) for n, t in prob.inputs.items()}
    T = prob.tokens
    mask, counted = None, T
    if sample_tokens is not None and sample_tokens < T:
        rows = np.random.default_rng(0).choice(T, size=sample_tokens, replace=False)
        mask = np.zeros(T, np.uint8)
        mask[rows] = 1
        counted = sample_tokens
    oracle.forward_problem(prob.cfg, host, token_mask=mask, threads=cores)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 and (not times or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        oracle.forward_problem(prob.cfg, host, token_mask=mask, threads=cores)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    what = f"{T} tokens" if mask is None else f"{counted} of {T} tokens (seeded sample; routing for all)"
    return dict(value=round(counted / med, 2), unit="tokens/s", cores=cores, kind="port",
                sample=f"{prob.cfg.name} layer, {what}, {len(times)} timed runs (median {med * 1e3:.1f} ms), "
                       f"OpenMP fp32 restatement on {cores} threads of {affinity} in the affinity mask, "
                       f"{cpu_model()}")


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--workload", default=None, help="name:tokens to run instead of the headline")
    ap.add_argument("--no-prepack", action="store_true", help="keep the expert weights in the op's row-major layout")
    ap.add_argument("--op", default=None, metavar="OP:ROWSxDIM[:K]",
                    help="time the stand-alone topk or softmax op on a [rows, dim] fp32 input instead "
                         "(e.g. topk:8192x128:8, softmax:8192x4096)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the MoE layer runs on a single MI355X; multi-GPU sharding is design-only).", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.copy_probe:
        n = args.copy_probe << 20
        src = torch.ones((n,), dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "copies": args.steps}), flush=True)
        return
    if args.op:
        print(json.dumps(run_op(args.op, args.steps, args.warmup, dev)), flush=True)
        return
    name, T = HEADLINE
    if args.workload:
        name, t = args.workload.split(":")
        T = int(t)
    head, prob = run_workload(name, T, args.steps, args.warmup, dev, keep_problem=True,
                              prepack=not args.no_prepack)
    print(f"[bench] {name} T={T}: {head['tokens_per_s']} tok/s, {head['ms_per_step']} ms, "
          f"fc1 {head['roofline']['achieved']} {head['roofline']['unit']}", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(prob)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)
    del prob
    torch.cuda.empty_cache()
    extra = []
    cpu_prefill = None
    if not args.no_extra and not args.workload:
        for wname, wT in EXTRA:
            keep = not args.no_cpu and (wname, wT) == CPU_PREFILL[:2]
            r, wprob = run_workload(wname, wT, max(10, args.steps // 2), max(3, args.warmup // 2), dev,
                                    keep_problem=keep, prepack=not args.no_prepack)
            if wprob is not None:
                cpu_prefill = cpu_baseline(wprob, sample_tokens=CPU_PREFILL[2])
                cpu_prefill["gpu_tokens_per_s"] = r["tokens_per_s"]
                print(f"[bench] cpu baseline (prefill): {cpu_prefill}", file=sys.stderr, flush=True)
                del wprob
                torch.cuda.empty_cache()
            extra.append(r)
            print(f"[bench] {wname} T={wT}: {r['tokens_per_s']} tok/s, {r['ms_per_step']} ms, path={r['path']}, "
                  f"fc1 {r['roofline']['achieved']} {r['roofline']['unit']} ({r['roofline']['frac']:.1%})",
                  file=sys.stderr, flush=True)
    fusion = []
    if not args.no_extra and not args.workload:
        for wname, wT in ROUTER_FUSION:
            r = run_router_fusion(wname, wT, max(10, args.steps // 2), max(3, args.warmup // 2), dev)
            fusion.append(r)
            print(f"[bench] router GEMM fusion {wname} T={wT}: unfused {r['unfused_ms']} ms, fused {r['fused_ms']} ms",
                  file=sys.stderr, flush=True)
    from onnxruntime_musa_amd.workloads import CONFIGS
    cfg = CONFIGS[name]
    line = {
        "metric": METRIC,
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype,
        "data": "synthetic",
        "config": {"workload": name, "tokens": T, "hidden": cfg.hidden, "inter": cfg.inter,
                   "experts": cfg.experts, "k": cfg.k,
                   "weights": (f"int{cfg.bits} " + (f"block {cfg.block_size}" if cfg.block_size else "per-channel")
                               + f", {cfg.scale_dtype} scales") if cfg.bits else cfg.dtype,
                   "path": head["path"], "experts_hit": head["experts_hit"],
                   "weight_copies": head["weight_copies"],
                   "prepacked_inputs": head["prepacked"]},
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "cpu_baseline_prefill": cpu_prefill,
        "stages_ms": head["stages_ms"],
        "layer_hbm_gbs": head["layer_hbm_gbs"],
        "extra": extra,
        "router_gemm_fusion": fusion,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
