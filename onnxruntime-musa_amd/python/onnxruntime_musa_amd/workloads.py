"""Synthetic MoE / QMoE workloads: the five benchmark configurations, seeded
input generation and symmetric weight quantisation.

Draw order per problem: x -> router logits -> W1 -> b1 -> W3 -> b3 -> W2 -> b2.
x ~ N(0,1); logits ~ N(0,1) (or Zipf-skewed, below); weights ~ N(0, 1/fan_in)
(std 1/sqrt(fan_in), fan_in = H for fc1/fc3 and I for fc2); biases likewise.
Small problems draw with numpy's PCG64 (`gen="numpy"`), large ones with a
seeded torch generator on the GPU (`gen="torch"`), so that full Mixtral-size
weights are generated in HBM in seconds.

Quantisation (symmetric, the QMoE encoding): int8 per output channel
s = max|w_row| / 127, q = clamp(round(w / s), -128, 127) + 128; int4 per block
of `block_size` along K, s = max|w_block| / 7, q = clamp(round(w / s), -8, 7) + 8,
two values per byte with the even-k value in the low nibble.

MXFP4 (OCP Microscaling Formats v1.0; the library extension for gpt-oss
style experts): per block of 32 along K a shared E8M0 exponent
e = floor(log2 max|w|) - 2 (uint8 scale byte e + 127), elements w / 2^e
rounded to the nearest FP4 E2M1 value (ties to the even code, saturating at
+-6), two per byte with the even-k element in the low nibble.

Zipf routing (the Qwen3-MoE-shaped config): p_e ~ r_e^-s with r a seeded
permutation of 1..E, logits = log p_e + Gumbel(0, 1); by the Gumbel-top-k trick
each token's top-k is a draw without replacement proportional to p.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, replace
from typing import Dict, List, Optional

import numpy as np
import torch

from .ops import MOE_INPUTS, QMOE_INPUTS, MoE, QMoE

_TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


@dataclass(frozen=True)
class MoEConfig:
    name: str
    hidden: int
    inter: int
    experts: int
    k: int
    dtype: str = "f16"           # activation / bias type T
    bits: int = 0                # 0 = MoE (float weights); 4 / 8 = QMoE
    block_size: int = 0          # 0 = per output channel
    scale_dtype: str = "f16"     # T2 ("e8m0": uint8 MXFP4 scales)
    weight_format: str = "int"   # "int" (QMoE zero-point integers) | "mxfp4" (bits 4, block 32, e8m0)
    activation: str = "swiglu"
    swiglu_fusion: int = 0       # 0 with use_fc3, 1 interleaved, 2 chunked
    use_fc3: bool = True
    swiglu_limit: Optional[float] = None
    alpha: float = 1.0
    beta: float = 0.0
    normalize: int = 1
    router_sigmoid: int = 0      # library extension: sigmoid routing instead of softmax
    bias: bool = False
    router: str = "normal"       # "normal" | "zipf"
    zipf_s: float = 1.2
    tokens: tuple = (16,)

    @property
    def op_type(self) -> str:
        return "QMoE" if self.bits else "MoE"

    @property
    def fused(self) -> bool:
        return self.activation == "swiglu" and not self.use_fc3

    @property
    def n1(self) -> int:
        return 2 * self.inter if self.fused else self.inter

    def weight_bytes_per_expert(self) -> int:
        """HBM bytes of one expert's weights, scales and biases."""
        H, I, n1 = self.hidden, self.inter, self.n1
        rows_k = [(n1, H), (H, I)] + ([(I, H)] if self.use_fc3 else [])
        esz = {"f32": 4, "f16": 2, "bf16": 2, "e8m0": 1}
        total = 0
        for n, kk in rows_k:
            if self.bits == 0:
                total += n * kk * esz[self.dtype]
            else:
                total += n * kk * self.bits // 8
                nblk = kk // self.block_size if self.block_size else 1
                total += n * nblk * esz[self.scale_dtype]
        if self.bias:
            total += (n1 + H + (I if self.use_fc3 else 0)) * esz[self.dtype]
        return total

    def flops_per_row(self) -> int:
        """Multiply-add FLOPs of one (token, expert) pair: 2 * (N1*H + H*I) (+ fc3)."""
        n1 = self.n1 + (self.inter if self.use_fc3 else 0)
        return 2 * (n1 * self.hidden + self.hidden * self.inter)

    def op_kwargs(self) -> dict:
        kw = dict(k=self.k, activation_type=self.activation, normalize_routing_weights=self.normalize,
                  swiglu_fusion=self.swiglu_fusion, swiglu_limit=self.swiglu_limit,
                  activation_alpha=self.alpha, activation_beta=self.beta, router_sigmoid=self.router_sigmoid)
        if self.bits:
            kw.update(expert_weight_bits=self.bits, block_size=self.block_size)
        return kw


CONFIGS: Dict[str, MoEConfig] = {
    # the CPU-runnable fp32 MoE
    "c1_moe_f32": MoEConfig("c1_moe_f32", hidden=128, inter=256, experts=8, k=2, dtype="f32",
                            activation="silu", use_fc3=False, normalize=1, bias=True, tokens=(64,)),
    # QMoE int8 per-channel, Mixtral shape
    "c2_qmoe_int8_mixtral": MoEConfig("c2_qmoe_int8_mixtral", hidden=4096, inter=14336, experts=8, k=2,
                                      dtype="f16", bits=8, block_size=0, scale_dtype="f16",
                                      tokens=(1, 16, 4096)),
    # QMoE int4 block 128, Mixtral shape
    "c3_qmoe_int4_mixtral": MoEConfig("c3_qmoe_int4_mixtral", hidden=4096, inter=14336, experts=8, k=2,
                                      dtype="f16", bits=4, block_size=128, scale_dtype="f16",
                                      tokens=(1, 16, 4096)),
    # QMoE int4 block 32, gpt-oss shape, interleaved SwiGLU with clamp, bias, bf16
    "c4_qmoe_int4_gptoss": MoEConfig("c4_qmoe_int4_gptoss", hidden=2880, inter=2880, experts=32, k=4,
                                     dtype="bf16", bits=4, block_size=32, scale_dtype="bf16",
                                     swiglu_fusion=1, use_fc3=False, swiglu_limit=7.0, alpha=1.702, beta=1.0,
                                     bias=True, tokens=tuple(2 ** i for i in range(14))),
    # MoE fp16, Qwen3-MoE shape, Zipf-skewed routing
    "c5_moe_f16_qwen3": MoEConfig("c5_moe_f16_qwen3", hidden=2048, inter=768, experts=128, k=8, dtype="f16",
                                  router="zipf", tokens=(8192,)),
    # extension (not a BASELINE config): configs[3]'s gpt-oss shape with MXFP4
    # experts (E2M1 elements, E8M0 block-32 scales), the format gpt-oss ships
    "x1_mxfp4_gptoss": MoEConfig("x1_mxfp4_gptoss", hidden=2880, inter=2880, experts=32, k=4,
                                 dtype="bf16", bits=4, block_size=32, scale_dtype="e8m0", weight_format="mxfp4",
                                 swiglu_fusion=1, use_fc3=False, swiglu_limit=7.0, alpha=1.702, beta=1.0,
                                 bias=True, tokens=(1, 16, 64, 8192)),
}


def quantize_int8_per_channel(w: torch.Tensor, scale_dtype: torch.dtype):
    """w [..., N, K] float -> (q uint8 [..., N, K], s [..., N])."""
    amax = w.abs().amax(dim=-1)
    s = amax / 127.0
    safe = torch.where(s > 0, s, torch.ones_like(s))
    q = torch.clamp(torch.round(w / safe.unsqueeze(-1)), -128, 127) + 128
    return q.to(torch.uint8), s.to(scale_dtype)


def quantize_int4_block(w: torch.Tensor, block: int, scale_dtype: torch.dtype):
    """w [..., N, K] float -> (packed uint8 [..., N, K/2], s [..., N, K/block])."""
    *lead, N, K = w.shape
    wb = w.reshape(*lead, N, K // block, block)
    s = wb.abs().amax(dim=-1) / 7.0
    safe = torch.where(s > 0, s, torch.ones_like(s))
    q = (torch.clamp(torch.round(wb / safe.unsqueeze(-1)), -8, 7) + 8).to(torch.uint8).reshape(*lead, N, K)
    packed = q[..., 0::2] | (q[..., 1::2] << 4)
    return packed.contiguous(), s.to(scale_dtype)


def quantize_int4_per_channel(w: torch.Tensor, scale_dtype: torch.dtype):
    s = w.abs().amax(dim=-1) / 7.0
    safe = torch.where(s > 0, s, torch.ones_like(s))
    q = (torch.clamp(torch.round(w / safe.unsqueeze(-1)), -8, 7) + 8).to(torch.uint8)
    return (q[..., 0::2] | (q[..., 1::2] << 4)).contiguous(), s.to(scale_dtype)


def quantize_int8_block(w: torch.Tensor, block: int, scale_dtype: torch.dtype):
    *lead, N, K = w.shape
    wb = w.reshape(*lead, N, K // block, block)
    s = wb.abs().amax(dim=-1) / 127.0
    safe = torch.where(s > 0, s, torch.ones_like(s))
    q = (torch.clamp(torch.round(wb / safe.unsqueeze(-1)), -128, 127) + 128).to(torch.uint8).reshape(*lead, N, K)
    return q.contiguous(), s.to(scale_dtype)


_E2M1_GRID = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def quantize_mxfp4(w: torch.Tensor):
    """w [..., N, K] float -> (packed uint8 [..., N, K/2] E2M1 nibbles,
    uint8 [..., N, K/32] E8M0 scales), the MX v1.0 quantizer."""
    *lead, N, K = w.shape
    wb = w.reshape(*lead, N, K // 32, 32).to(torch.float64)
    amax = wb.abs().amax(dim=-1)
    e = torch.where(amax > 0, torch.floor(torch.log2(amax.clamp_min(2.0 ** -200))) - 2,
                    torch.full_like(amax, -127.0)).clamp(-127, 127)
    a = (wb.abs() / torch.exp2(e).unsqueeze(-1)).clamp(max=6.0)
    grid = torch.tensor(_E2M1_GRID, dtype=torch.float64, device=w.device)
    # nearest grid value; a tie goes to the even code (odd codes lose by 1e-9)
    odd = (torch.arange(8, device=w.device) % 2).to(torch.float64) * 1e-9
    code = ((a.unsqueeze(-1) - grid).abs() + odd).argmin(dim=-1)
    nib = (code | ((wb < 0).to(torch.int64) << 3)).to(torch.uint8).reshape(*lead, N, K)
    packed = nib[..., 0::2] | (nib[..., 1::2] << 4)
    return packed.contiguous(), (e + 127).to(torch.uint8).contiguous()


def quantize(w: torch.Tensor, bits: int, block: int, scale_dtype: torch.dtype):
    if bits == 8:
        return quantize_int8_block(w, block, scale_dtype) if block else quantize_int8_per_channel(w, scale_dtype)
    return quantize_int4_block(w, block, scale_dtype) if block else quantize_int4_per_channel(w, scale_dtype)


class _Draw:
    """Seeded normal draws, numpy (host) or torch (device)."""

    def __init__(self, gen: str, seed: int, device):
        self.gen, self.device = gen, device
        if gen == "numpy":
            self.rng = np.random.default_rng(seed)
        else:
            self.g = torch.Generator(device=device)
            self.g.manual_seed(seed)

    def normal(self, shape, std=1.0) -> torch.Tensor:
        if self.gen == "numpy":
            a = self.rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std)
            return torch.from_numpy(a).to(self.device)
        return torch.randn(shape, generator=self.g, device=self.device, dtype=torch.float32) * std

    def uniform(self, shape) -> torch.Tensor:
        if self.gen == "numpy":
            return torch.from_numpy(self.rng.random(size=shape, dtype=np.float32)).to(self.device)
        return torch.rand(shape, generator=self.g, device=self.device, dtype=torch.float32)

    def permutation(self, n) -> torch.Tensor:
        if self.gen == "numpy":
            return torch.from_numpy(self.rng.permutation(n)).to(self.device)
        return torch.randperm(n, generator=self.g, device=self.device)


@dataclass
class Problem:
    """One seeded MoE/QMoE invocation, inputs resident on `device`."""
    cfg: MoEConfig
    tokens: int
    seed: int
    inputs: Dict[str, Optional[torch.Tensor]] = field(default_factory=dict)

    @property
    def input_names(self) -> List[str]:
        return list(QMOE_INPUTS if self.cfg.bits else MOE_INPUTS)

    def schema_inputs(self) -> List[Optional[torch.Tensor]]:
        """Inputs in op-schema order, trailing absent optionals dropped."""
        vals = [self.inputs.get(n) for n in self.input_names]
        while vals and vals[-1] is None:
            vals.pop()
        return vals

    def make_op(self, **overrides):
        kw = self.cfg.op_kwargs()
        kw.update(overrides)
        return (QMoE if self.cfg.bits else MoE)(**kw)


def make_problem(cfg: MoEConfig, tokens: int, seed: int = 0, device="cuda", gen: Optional[str] = None,
                 **cfg_overrides) -> Problem:
    if cfg_overrides:
        cfg = replace(cfg, **cfg_overrides)
    if gen is None:
        gen = "numpy" if cfg.experts * cfg.hidden * cfg.inter <= (1 << 24) else "torch"
    d = _Draw(gen, seed, device)
    T, H, I, E, n1 = tokens, cfg.hidden, cfg.inter, cfg.experts, cfg.n1
    dt = _TORCH_DT[cfg.dtype]
    mx = cfg.weight_format == "mxfp4"
    if mx and (cfg.bits != 4 or cfg.block_size != 32):
        raise ValueError("MXFP4 experts need bits 4 and block_size 32")
    sdt = None if mx else _TORCH_DT[cfg.scale_dtype]
    p = Problem(cfg, tokens, seed)
    p.inputs["input"] = d.normal((T, H)).to(dt).contiguous()
    if cfg.router == "zipf":
        ranks = d.permutation(E).to(torch.float32) + 1.0
        logp = -cfg.zipf_s * torch.log(ranks)
        logp = logp - torch.logsumexp(logp, 0)
        u = d.uniform((T, E)).clamp_(1e-20, 1.0 - 1e-7)
        gumbel = -torch.log(-torch.log(u))
        p.inputs["router_probs"] = (logp.unsqueeze(0) + gumbel).to(dt).contiguous()
    else:
        p.inputs["router_probs"] = d.normal((T, E)).to(dt).contiguous()

    def weight(n, kk):
        # one expert at a time keeps the fp32 staging small for Mixtral-size weights
        mats = [d.normal((n, kk), 1.0 / math.sqrt(kk)) for _ in range(E)]
        if cfg.bits == 0:
            return torch.stack([m.to(dt) for m in mats]).contiguous(), None
        qs = [quantize_mxfp4(m) if mx else quantize(m, cfg.bits, cfg.block_size, sdt) for m in mats]
        return torch.stack([q for q, _ in qs]).contiguous(), torch.stack([s for _, s in qs]).contiguous()

    def bias(n, fan_in):
        return d.normal((E, n), 1.0 / math.sqrt(fan_in)).to(dt).contiguous() if cfg.bias else None

    w1, s1 = weight(n1, H)
    b1 = bias(n1, H)
    w3 = s3 = b3 = None
    if cfg.use_fc3:
        w3, s3 = weight(I, H)
        b3 = bias(I, H)
    w2, s2 = weight(H, I)
    b2 = bias(H, I)
    p.inputs.update({"fc1_experts_weights": w1, "fc1_experts_bias": b1, "fc2_experts_weights": w2,
                     "fc2_experts_bias": b2, "fc3_experts_weights": w3, "fc3_experts_bias": b3})
    if cfg.bits:
        p.inputs.update({"fc1_scales": s1, "fc2_scales": s2, "fc3_scales": s3})
    return p


def to_host(t: Optional[torch.Tensor]) -> Optional[np.ndarray]:
    """Device tensor -> numpy; bf16 becomes its raw uint16 payload."""
    if t is None:
        return None
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


__all__ = ["MoEConfig", "CONFIGS", "Problem", "make_problem", "quantize", "quantize_mxfp4", "to_host"]
