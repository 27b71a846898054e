"""Dense fp32 restatement of moe_feed_forward (gpu/ir.cpp:1073-1164) on
numpy/OpenBLAS -- the CPU baseline timed beside the GPU.

TEST INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and the tests).

Like the reference, it runs every expert FFN on every row and masks with the
per-row gate (gpu/ir.cpp:1118-1148), so it executes E/K times the algorithmic
expert FLOPs; matrix products are BLAS sgemm, the way MLX on Linux links
OpenBLAS (gpu/mlx_linux.go:11).  Its results are checked against the C
restatement (oracle/moe_oracle.c) in tests/test_oracle.py.
"""
from __future__ import annotations

import numpy as np


def _act(v: np.ndarray, activation: int, slope: float) -> np.ndarray:
    if activation == 0:
        return v / (np.float32(1) + np.exp(-v))
    if activation == 1:
        return np.float32(0.5) * v * (np.float32(1) + np.tanh(np.float32(0.7978845608) * (v + np.float32(0.044715) * v * v)))
    if activation == 2:
        return np.maximum(v, np.float32(0))
    y = np.where(v > 0, v, v * np.float32(slope))
    return y * y


def dense_forward(x, router_w, expert_matrix, E: int, K: int, expert_type: int = 0,
                  activation: int = 0, slope: float = 0.0):
    """x [n, D] fp32, router_w [D, E] fp32, expert_matrix(e, j) -> fp32 matrix.
    Returns (delta [n, D], aux, entropy)."""
    x = np.asarray(x, np.float32)
    n = x.shape[0]
    logits = x @ router_w
    m = logits.max(axis=1, keepdims=True)
    ex = np.exp(logits - m)
    probs = ex / ex.sum(axis=1, keepdims=True)
    top = np.argsort(-probs, axis=1, kind="stable")[:, :K]
    top_p = np.take_along_axis(probs, top, axis=1)
    top_norm = top_p / np.maximum(top_p.sum(axis=1, keepdims=True), np.float32(1e-12))
    out = np.zeros_like(x)
    aux = np.float32(0)
    for e in range(E):
        sel = top == e
        gate = np.where(sel, top_norm, np.float32(0)).sum(axis=1, keepdims=True)
        if expert_type == 2:
            h = _act(x @ expert_matrix(e, 0), activation, slope)
            y = h @ expert_matrix(e, 1)
        else:
            g = x @ expert_matrix(e, 0)
            a = np.float32(1) / (np.float32(1) + np.exp(-g)) if expert_type == 0 else _act(g, 1, 0.0)
            y = (a * (x @ expert_matrix(e, 1))) @ expert_matrix(e, 2)
        out += y * gate
        aux += probs[:, e].mean() * (sel.sum(axis=1) / np.float32(K)).mean()
    aux *= np.float32(E)
    ent = -np.mean(np.sum(probs * np.log(np.maximum(probs, np.float32(1e-12))), axis=1))
    return out, float(aux), float(ent)
