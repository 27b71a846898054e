"""Float64 restatement of op 74's backward (TEST INFRASTRUCTURE ONLY: the
checker of mxm_moe_backward; only tests/ import it).

The forward is gpu/ir.cpp:1106-1162 with the top-k indices held fixed (they
carry no gradient); the backward is what autodiff through those operations
gives (the reference exercises it in gpu/moe_feed_forward_test.go:84-151).
``forward64`` and ``backward64`` share no code with the GPU path; the
backward is pinned by central finite differences of ``forward64`` in
tests/test_backward.py.
"""
from __future__ import annotations

import numpy as np

EPS = 1e-12
GELU_C, GELU_K = 0.7978845608, 0.044715


def _sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


def _gelu(v):
    t = np.tanh(GELU_C * (v + GELU_K * v ** 3))
    d = 0.5 * (1.0 + t) + 0.5 * v * (1.0 - t * t) * GELU_C * (1.0 + 3.0 * GELU_K * v * v)
    return 0.5 * v * (1.0 + t), d


def _act(u, act, slope):
    """mlp activation (gpu/ir.cpp:1053-1071) and its derivative."""
    if act == 0:
        s = _sigmoid(u)
        return u * s, s * (1.0 + u * (1.0 - s))
    if act == 1:
        return _gelu(u)
    if act == 2:
        return np.maximum(u, 0.0), (u > 0).astype(np.float64)
    y = np.where(u > 0, u, u * slope)
    return y * y, 2.0 * y * np.where(u > 0, 1.0, slope)


def forward64(x, wr, experts, top_idx, etype=0, act=0, slope=0.0):
    """delta, aux, entropy and the intermediates, in float64, for fixed top_idx."""
    x = np.asarray(x, np.float64)
    wr = np.asarray(wr, np.float64)
    N, D = x.shape
    E = wr.shape[1]
    K = top_idx.shape[1]
    logits = x @ wr
    z = logits - logits.max(axis=1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=1, keepdims=True)
    tp = np.take_along_axis(p, top_idx, axis=1)
    S = tp.sum(axis=1, keepdims=True)
    gates = tp / np.maximum(S, EPS)
    delta = np.zeros((N, D))
    slots = []
    for n in range(N):
        for k in range(K):
            e = int(top_idx[n, k])
            ws = [np.asarray(w, np.float64) for w in experts[e]]
            if etype == 2:
                u = x[n] @ ws[0]
                h, dact = _act(u, act, slope)
                g = None
                y = h @ ws[1]
            else:
                g = x[n] @ ws[0]
                u = x[n] @ ws[1]
                a, dact = (_sigmoid(g), None) if etype == 0 else _gelu(g)
                h = a * u
                y = h @ ws[2]
            delta[n] += gates[n, k] * y
            slots.append((n, k, e, g, u, h, y))
    counts = np.bincount(top_idx.ravel(), minlength=E)
    aux = E * np.sum(p.mean(axis=0) * counts / (K * N))
    ent = -np.mean(np.sum(p * np.log(np.maximum(p, EPS)), axis=1))
    return dict(delta=delta, aux=float(aux), entropy=float(ent), p=p, tp=tp, S=S, gates=gates,
                counts=counts, slots=slots)


def backward64(x, wr, experts, top_idx, d_delta, d_aux=0.0, d_ent=0.0, etype=0, act=0,
               slope=0.0):
    """(dx, d_router_w, d_experts) of L = <d_delta, delta> + d_aux*aux + d_ent*entropy."""
    x = np.asarray(x, np.float64)
    wr = np.asarray(wr, np.float64)
    dD = np.asarray(d_delta, np.float64)
    f = forward64(x, wr, experts, top_idx, etype, act, slope)
    N, D = x.shape
    E = wr.shape[1]
    K = top_idx.shape[1]
    p, tp, S = f["p"], f["tp"], f["S"]
    dx = np.zeros_like(x)
    dexp = [[np.zeros(np.shape(w)) for w in ws] for ws in experts]
    dgates = np.zeros((N, K))
    for (n, k, e, g, u, h, y) in f["slots"]:
        ws = [np.asarray(w, np.float64) for w in experts[e]]
        dgates[n, k] = dD[n] @ y
        dy = f["gates"][n, k] * dD[n]
        wd = ws[-1]
        dh = wd @ dy
        dexp[e][-1] += np.outer(h, dy)
        if etype == 2:
            _, dact = _act(u, act, slope)
            du = dh * dact
            dexp[e][0] += np.outer(x[n], du)
            dx[n] += ws[0] @ du
        else:
            if etype == 0:
                a = _sigmoid(g)
                da = a * (1.0 - a)
            else:
                a, da = _gelu(g)
            dg = dh * u * da
            du = dh * a
            dexp[e][0] += np.outer(x[n], dg)
            dexp[e][1] += np.outer(x[n], du)
            dx[n] += ws[0] @ dg + ws[1] @ du
    Sc = np.maximum(S, EPS)
    T = np.sum(dgates * tp, axis=1, keepdims=True)
    dtp = dgates / Sc - np.where(S > EPS, T / (Sc * Sc), 0.0)
    dp = np.zeros((N, E))
    np.add.at(dp, (np.repeat(np.arange(N), K), top_idx.ravel()), dtp.ravel())
    dp += d_aux * E * f["counts"][None, :] / (K * N) / N
    dp -= d_ent / N * (np.log(np.maximum(p, EPS)) + (p > EPS))
    dlogits = p * (dp - np.sum(p * dp, axis=1, keepdims=True))
    dwr = x.T @ dlogits
    dx += dlogits @ wr.T
    return dx, dwr, dexp
