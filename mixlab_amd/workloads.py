"""Synthetic inputs for the benchmark configurations of the MoE layer.

The configurations are the five of the benchmark plan (moe_tiny-scale fp32,
near-uniform bf16, Zipf-skewed bf16, fine-grained d=2048/64e/top-8 bf16, and
the int8-weight decode shape).  Inputs are seeded: x ~ N(0, 1), router and
expert weights ~ N(0, 0.02) (mixlab's `weight_init: "normal"`); bf16
configurations round the fp32 draws to bf16 (nearest-even).

The Zipf configuration realises its skew inside the op's semantics, since
mixlab's router has no bias (docs/config-reference.md:477): the last feature
of x is a constant c = 1 and router_w[D-1, e] = b_e, with b_e calibrated on
the seed so that top-k loads follow p_e ~ (e+1)^-1.2.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .moe import MOE_ACT_SILU, MOE_EXPERT_SWIGLU


@dataclass
class MoEConfig:
    name: str
    B: int
    T: int
    D: int
    E: int
    K: int
    F: int
    dtype: str  # "fp32" | "bf16"
    expert_type: int = MOE_EXPERT_SWIGLU
    activation: int = MOE_ACT_SILU
    leaky_slope: float = 0.0
    seed: int = 0
    zipf_s: float = 0.0  # > 0: calibrate router skew to Zipf(s)
    int8_weights: bool = False
    note: str = ""

    @property
    def N(self) -> int:
        return self.B * self.T

    @property
    def wpe(self) -> int:
        return 2 if self.expert_type == 2 else 3

    @property
    def int_params(self) -> list:
        return [self.B, self.T, self.D, self.E, self.K, self.expert_type, self.F, self.activation]

    def flops(self) -> dict:
        """Algorithmic FLOPs (top-k experts only), as arch/moe.go:215-236 counts them."""
        n, d, e, k, f = self.N, self.D, self.E, self.K, self.F
        up = k * (4 if self.wpe == 3 else 2) * n * d * f
        down = k * 2 * n * f * d
        return dict(router=2 * n * d * e, up=up, down=down, experts=up + down)


CONFIGS = {
    "C1": MoEConfig("C1", 8, 128, 128, 4, 2, 512, "fp32", seed=0,
                    note="moe_tiny-scale fp32, d=128, 4 experts top-2, F=512, 1024 tokens"),
    "C2": MoEConfig("C2", 16, 1024, 512, 8, 2, 2048, "bf16", seed=2,
                    note="bf16 d=512, 8 experts top-2, F=2048, 16384 tokens"),
    "C3": MoEConfig("C3", 32, 2048, 1024, 16, 2, 4096, "bf16", seed=3, zipf_s=1.2,
                    note="bf16 d=1024, 16 experts top-2 Zipf(1.2) load, F=4096, 65536 tokens"),
    "C4": MoEConfig("C4", 32, 2048, 2048, 64, 8, 1024, "bf16", seed=4,
                    note="bf16 d=2048, 64 experts top-8, F=1024 gated, 65536 tokens"),
    "C5": MoEConfig("C5", 1, 64, 2048, 64, 8, 1408, "bf16", seed=5, int8_weights=True,
                    note="decode: 64 tokens, d=2048, 64 experts top-8, F=1408, int8 weights"),
}


def round_bf16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    r = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def bf16_bits(a: np.ndarray) -> np.ndarray:
    return (round_bf16(a).view(np.uint32) >> 16).astype(np.uint16)


def quantize_int8(w: np.ndarray):
    """Symmetric per-output-channel int8 of a [in, out] matrix:
    s_j = max_k |w[k, j]| / 127, q = clamp(round(w / s), -127, 127)."""
    amax = np.abs(w).max(axis=0)
    s = np.where(amax > 0, amax / 127.0, 1.0).astype(np.float32)
    q = np.clip(np.rint(w / s), -127, 127).astype(np.int8)
    return q, s


@dataclass
class Workload:
    cfg: MoEConfig
    x: np.ndarray            # [N, D] fp32 values (bf16-representable for bf16 configs)
    router_w: np.ndarray     # [D, E]
    experts: list            # per expert [w_gate, w_up, w_down] (fp32 values)
    q8: list = field(default_factory=list)  # per expert [(q, s), ...] for int8 configs
    zipf_bias: np.ndarray = None

    def x_bits(self) -> np.ndarray:
        return bf16_bits(self.x)


def _zipf_bias(rng, x, wr, cfg: MoEConfig, iters: int = 40) -> np.ndarray:
    """Per-expert logit bias so that top-k loads follow p_e ~ (e+1)^-s."""
    E, K = cfg.E, cfg.K
    target = (np.arange(1, E + 1, dtype=np.float64)) ** (-cfg.zipf_s)
    target = target / target.sum()
    sample = x[: min(len(x), 16384)].astype(np.float64)
    base = sample[:, :-1] @ wr[:-1].astype(np.float64)
    b = np.log(target) - np.log(target).mean()
    for _ in range(iters):
        bb = round_bf16(b.astype(np.float32)).astype(np.float64) if cfg.dtype == "bf16" else b
        logits = base + bb[None, :]
        top = np.argpartition(-logits, K - 1, axis=1)[:, :K]
        load = np.bincount(top.ravel(), minlength=E) / top.size
        b = b + 0.8 * (np.log(target) - np.log(np.maximum(load, 1e-6)))
        b -= b.mean()
    return b.astype(np.float32)


def make_workload(cfg: MoEConfig, n_tokens: int = None) -> Workload:
    rng = np.random.default_rng(cfg.seed)
    N = cfg.N if n_tokens is None else n_tokens
    D, E, F = cfg.D, cfg.E, cfg.F
    x = rng.standard_normal((N, D), dtype=np.float32)
    wr = (rng.standard_normal((D, E), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    experts = []
    for _ in range(E):
        mats = []
        for j in range(cfg.wpe):
            shape = (F, D) if j == cfg.wpe - 1 else (D, F)
            mats.append((rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)))
        experts.append(mats)
    bias = None
    if cfg.zipf_s > 0:
        x[:, D - 1] = 1.0
        bias = _zipf_bias(rng, x, wr, cfg)
        wr[D - 1, :] = bias
    q8 = []
    if cfg.int8_weights:
        deq = []
        for mats in experts:
            qs = [quantize_int8(w) for w in mats]
            q8.append(qs)
            deq.append([q.astype(np.float32) * s[None, :] for q, s in qs])
        experts = deq
    if cfg.dtype == "bf16":
        x = round_bf16(x)
        wr = round_bf16(wr)
        experts = [[round_bf16(w) for w in mats] for mats in experts]
    return Workload(cfg, x, wr, experts, q8, bias)
