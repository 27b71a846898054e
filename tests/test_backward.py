"""The float64 backward restatement (oracle/backward.py) against central
finite differences of its forward, with the routing held fixed (CPU)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle.backward import backward64, forward64


def _problem(seed, N, D, E, F, etype):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((N, D))
    wr = rng.standard_normal((D, E)) * 0.5
    shapes = [(D, F), (F, D)] if etype == 2 else [(D, F), (D, F), (F, D)]
    experts = [[rng.standard_normal(s) * 0.4 for s in shapes] for _ in range(E)]
    dD = rng.standard_normal((N, D))
    return x, wr, experts, dD


def _loss(x, wr, experts, top_idx, dD, d_aux, d_ent, etype, act, slope):
    f = forward64(x, wr, experts, top_idx, etype, act, slope)
    return float(np.sum(dD * f["delta"]) + d_aux * f["aux"] + d_ent * f["entropy"])


@pytest.mark.parametrize("etype,act,slope", [(0, 0, 0.0), (1, 1, 0.0), (2, 0, 0.0), (2, 1, 0.0),
                                             (2, 3, 0.3)])
def test_backward_matches_finite_differences(etype, act, slope):
    N, D, E, K, F = 5, 4, 4, 2, 3
    x, wr, experts, dD = _problem(40 + etype + act, N, D, E, F, etype)
    fwd = oracle.moe_forward(x.astype(np.float32), wr.astype(np.float32),
                             [[w.astype(np.float32) for w in ws] for ws in experts], top_k=K,
                             expert_type=etype, activation=act, leaky_slope=slope)
    top_idx = fwd["top_idx"].astype(np.int64)
    d_aux, d_ent = 0.7, -0.4
    dx, dwr, dexp = backward64(x, wr, experts, top_idx, dD, d_aux, d_ent, etype, act, slope)
    h = 1e-6

    def fd(arr, idx, setter):
        old = arr[idx]
        arr[idx] = old + h
        lp = setter()
        arr[idx] = old - h
        lm = setter()
        arr[idx] = old
        return (lp - lm) / (2 * h)

    L = lambda: _loss(x, wr, experts, top_idx, dD, d_aux, d_ent, etype, act, slope)  # noqa: E731
    rng = np.random.default_rng(1)
    for _ in range(12):
        i = tuple(rng.integers(0, s) for s in x.shape)
        assert abs(fd(x, i, L) - dx[i]) <= 1e-6 * (1 + abs(dx[i]))
        j = tuple(rng.integers(0, s) for s in wr.shape)
        assert abs(fd(wr, j, L) - dwr[j]) <= 1e-6 * (1 + abs(dwr[j]))
        e = int(rng.integers(0, E))
        m = int(rng.integers(0, len(experts[e])))
        w = experts[e][m]
        q = tuple(rng.integers(0, s) for s in w.shape)
        assert abs(fd(w, q, L) - dexp[e][m][q]) <= 1e-6 * (1 + abs(dexp[e][m][q]))


def test_unrouted_experts_get_no_gradient():
    x, wr, experts, dD = _problem(50, 6, 4, 5, 3, 0)
    top_idx = np.array([[0, 1]] * 6)
    _, _, dexp = backward64(x, wr, experts, top_idx, dD)
    for e in (2, 3, 4):
        assert all(not np.any(g) for g in dexp[e])
    assert any(np.any(g) for g in dexp[0])


def test_router_gradient_nonzero_and_finite():
    """gpu/moe_feed_forward_test.go:84-151 asks for finite gradients and a
    non-zero router gradient with top_k = 1."""
    x, wr, experts, dD = _problem(51, 3, 3, 2, 4, 0)
    fwd = oracle.moe_forward(x.astype(np.float32), wr.astype(np.float32),
                             [[w.astype(np.float32) for w in ws] for ws in experts], top_k=1)
    dx, dwr, dexp = backward64(x, wr, experts, fwd["top_idx"].astype(np.int64), dD, 0.01)
    assert np.all(np.isfinite(dx)) and np.all(np.isfinite(dwr))
    assert np.max(np.abs(dwr)) > 0
