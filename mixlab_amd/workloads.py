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

import os
from concurrent.futures import ThreadPoolExecutor
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
    # not a benchmark-plan configuration: C4 at the reference's default expert
    # width ffnDim(2048, 2.67) = 5468 (arch/weight_shapes.go:11,56-65), which
    # the MFMA kernels run at 5504 with zero weights in the padding
    "C4F": MoEConfig("C4F", 32, 2048, 2048, 64, 8, 5468, "bf16", seed=6,
                     note="bf16 d=2048, 64 experts top-8, F=5468 (default mlp_mult 2.67) "
                          "gated, 65536 tokens"),
}


def round_bf16(a: np.ndarray) -> np.ndarray:
    """Round finite fp32 values to the nearest bf16 (ties to even), as fp32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    r = (u >> 16) & np.uint32(1)
    r += u
    r += np.uint32(0x7FFF)
    r &= np.uint32(0xFFFF0000)
    return r.view(np.float32)


def bf16_bits(a: np.ndarray) -> np.ndarray:
    return (round_bf16(a).view(np.uint32) >> 16).astype(np.uint16)


def from_bits(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b).astype(np.uint32) << 16).view(np.float32)


def quantize_int8(w: np.ndarray):
    """Symmetric per-output-channel int8 of a [in, out] matrix:
    s_j = max_k |w[k, j]| / 127, q = clamp(round(w / s), -127, 127)."""
    amax = np.abs(w).max(axis=0)
    s = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(w / s), -127, 127).astype(np.int8)
    return q, s


@dataclass
class Workload:
    """Seeded inputs of one configuration.  Expert matrices are stored once:
    as bf16 bit patterns (bf16 configs) or fp32 (fp32 configs), shaped
    [E, wpe, rows*cols] in the x.W layout of arch/moe.go:126-142."""

    cfg: MoEConfig
    x: np.ndarray                   # [N, D] fp32 values (bf16-representable for bf16)
    router_w: np.ndarray            # [D, E]
    store: np.ndarray               # [E, wpe, D*F] uint16 bits or fp32
    q8: list = field(default_factory=list)  # per expert [(q [in,out] int8, s [out] fp32), ...]
    zipf_bias: np.ndarray = None

    def shape(self, j: int) -> tuple:
        D, F = self.cfg.D, self.cfg.F
        return (F, D) if j == self.cfg.wpe - 1 else (D, F)

    def matrix(self, e: int, j: int) -> np.ndarray:
        """Expert e's j-th matrix as fp32 values."""
        m = self.store[e, j]
        if m.dtype == np.uint16:
            m = from_bits(m)
        return m.reshape(self.shape(j))

    def matrix_upload(self, e: int, j: int) -> np.ndarray:
        """Expert e's j-th matrix in the form uploaded to the device."""
        return self.store[e, j].reshape(self.shape(j))

    @property
    def experts(self) -> list:
        return [[self.matrix(e, j) for j in range(self.cfg.wpe)] for e in range(self.cfg.E)]

    def packed_f32(self) -> np.ndarray:
        """All expert matrices as one flat fp32 array (the oracle's packing)."""
        return from_bits(self.store).ravel() if self.store.dtype == np.uint16 else self.store.ravel()

    def x_upload(self) -> np.ndarray:
        return bf16_bits(self.x) if self.cfg.dtype == "bf16" else self.x

    def router_upload(self) -> np.ndarray:
        return bf16_bits(self.router_w) if self.cfg.dtype == "bf16" else self.router_w


def _zipf_bias(x, wr, cfg: MoEConfig, iters: int = 200) -> np.ndarray:
    """Per-expert logit bias so that top-k loads follow p_e ~ (e+1)^-s
    (damped multiplicative fitting of the realised loads on a token sample)."""
    E, K = cfg.E, cfg.K
    target = (np.arange(1, E + 1, dtype=np.float64)) ** (-cfg.zipf_s)
    target = target / target.sum()
    sample = x[: min(len(x), 16384)].astype(np.float64)
    base = sample[:, :-1] @ wr[:-1].astype(np.float64)
    b = np.zeros(E)
    for _ in range(iters):
        bb = round_bf16(b.astype(np.float32)).astype(np.float64) if cfg.dtype == "bf16" else b
        logits = base + bb[None, :]
        top = np.argpartition(-logits, K - 1, axis=1)[:, :K]
        load = np.bincount(top.ravel(), minlength=E) / top.size
        step = np.clip(np.log(target) - np.log(np.maximum(load, 0.5 / top.size)), -0.5, 0.5)
        b = b + 0.5 * step
        b -= b.mean()
    return b.astype(np.float32)


_X_CHUNK = 4096


def make_workload(cfg: MoEConfig, n_tokens: int = None, threads: int = None) -> Workload:
    """Seeded inputs; independent child streams per expert and per 4096-row
    block of x (numpy SeedSequence.spawn), generated on a thread pool."""
    N = cfg.N if n_tokens is None else n_tokens
    D, E, F, wpe = cfg.D, cfg.E, cfg.F, cfg.wpe
    root = np.random.SeedSequence(cfg.seed)
    s_x, s_r, s_e = root.spawn(3)
    x_seeds = s_x.spawn((N + _X_CHUNK - 1) // _X_CHUNK)
    e_seeds = s_e.spawn(E)
    threads = threads or min(16, os.cpu_count() or 1)
    bf16 = cfg.dtype == "bf16"

    x = np.empty((N, D), np.float32)

    def gen_x(i):
        r0, r1 = i * _X_CHUNK, min(N, (i + 1) * _X_CHUNK)
        np.random.default_rng(x_seeds[i]).standard_normal(out=x[r0:r1], dtype=np.float32)

    wr = np.random.default_rng(s_r).standard_normal((D, E), dtype=np.float32) * np.float32(0.02)
    store = np.empty((E, wpe, D * F), np.uint16 if bf16 else np.float32)
    q8 = [None] * E

    def gen_e(e):
        rng = np.random.default_rng(e_seeds[e])
        buf = np.empty(D * F, np.float32)
        qs = []
        for j in range(wpe):
            rng.standard_normal(out=buf, dtype=np.float32)
            buf *= np.float32(0.02)
            w = buf
            if cfg.int8_weights:
                q, s = quantize_int8(buf.reshape((F, D) if j == wpe - 1 else (D, F)))
                qs.append((q, s))
                w = (q.astype(np.float32) * s[None, :]).ravel()
            store[e, j] = bf16_bits(w) if bf16 else w
        if cfg.int8_weights:
            q8[e] = qs

    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(gen_x, range(len(x_seeds))))
        list(ex.map(gen_e, range(E)))
    bias = None
    if cfg.zipf_s > 0:
        x[:, D - 1] = 1.0
        bias = _zipf_bias(x, wr, cfg)
        wr[D - 1, :] = bias
    if bf16:
        x = round_bf16(x)
        wr = round_bf16(wr)
    return Workload(cfg, x, wr, store, q8 if cfg.int8_weights else [], bias)
