"""Writes the golden fixtures of tests/golden/ with the oracle.

Inputs are not stored: each fixture records the config, shape overrides and
seed from which onnxruntime_musa_amd.workloads.make_problem(gen="numpy")
regenerates them (numpy PCG64 streams), plus the first input values as a
drift check, and the expected routing and fp32 output.

    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT / "onnxruntime-musa_amd" / "python"), str(ROOT)]

from onnxruntime_musa_amd.workloads import CONFIGS, make_problem, to_host  # noqa: E402
from oracle import oracle  # noqa: E402

HERE = Path(__file__).resolve().parent


def write(path, name, T, seed, **over):
    p = make_problem(CONFIGS[name], T, seed=seed, device="cpu", gen="numpy", **over)
    h = {n: to_host(t) for n, t in p.inputs.items()}
    r = oracle.forward_problem(p.cfg, h, threads=1)
    np.savez_compressed(path, config=np.array(name), tokens=T, seed=seed,
                        hidden=p.cfg.hidden, inter=p.cfg.inter, experts=p.cfg.experts,
                        input_head=h["input"].reshape(-1)[:16], topk_ids=r["topk_ids"], perm=r["perm"],
                        out=r["out_f32"])
    print("wrote", path)


if __name__ == "__main__":
    write(HERE / "c1_moe_f32_seed0.npz", "c1_moe_f32", 64, 0)
    write(HERE / "qmoe_int4_b128_small.npz", "c3_qmoe_int4_mixtral", 16, 11, hidden=128, inter=256, experts=4)
    write(HERE / "qmoe_int8_chan_small.npz", "c2_qmoe_int8_mixtral", 16, 12, hidden=128, inter=256, experts=4)
