"""Pins of the CPU restatement in oracle/ (the checker of libmixmoe).

The restatement is trusted only as far as these checks reach:
  * the reference's known-answer procedure (gpu/moe_feed_forward_test.go:14-82,
    L_inf <= 2e-5) and its extensions, against float64 fixtures written by
    tests/golden/gen_golden.py, an independent numpy restatement;
  * planted mistakes (swapped operands, permuted experts, a wrong expert kind
    or slope) that these fixtures must reject;
  * closed forms and invariants: K = E (dense softmax mixture), K = 1 (argmax,
    gate 1), E = K = 1 (the plain sigmoid-GLU FFN), ties to the lower expert,
    dense == sparse bit for bit, permutation and count invariants;
  * the exp used by the routing (within 2 ulp of the correctly rounded value
    on a dense sweep) and bf16 rounding (ties to even, against brute force).
No GPU is used here.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

import oracle
from oracle.dense_blas import dense_forward

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import gen_golden  # noqa: E402  (the fixture generator doubles as a float64 reference)

CASES = json.loads((GOLDEN / "moe_known_answer.json").read_text())["cases"]


def _case_arrays(c):
    x = np.asarray(c["x"], np.float32)
    wr = np.asarray(c["router_w"], np.float32)
    experts = [[np.asarray(w, np.float32) for w in ws] for ws in c["experts"]]
    return x, wr, experts


def _run(c, experts=None, etype=None, slope=None, K=None, wr=None):
    x, wr0, ex0 = _case_arrays(c)
    B, T, D, E, K0, et0, F, act = c["int_params"]
    return oracle.moe_forward(x, wr0 if wr is None else wr, ex0 if experts is None else experts,
                              top_k=K0 if K is None else K,
                              expert_type=et0 if etype is None else etype, activation=act,
                              leaky_slope=c["float_params"][0] if slope is None else slope)


def _delta_ok(got, want) -> bool:
    """The reference's bar (L_inf <= 2e-5) and, since several fixtures have
    deltas near 1e-4, a relative bar of 2e-5 of the largest magnitude."""
    want = np.asarray(want)
    err = float(np.max(np.abs(got - want)))
    return err <= 2e-5 and err <= 2e-5 * float(np.max(np.abs(want))) + 1e-9


def test_fixture_inputs_follow_patterned_floats():
    c = CASES[0]
    x, wr, experts = _case_arrays(c)
    np.testing.assert_array_equal(x.ravel(), gen_golden.patterned_floats(12, 0.17))
    np.testing.assert_array_equal(wr.ravel(), gen_golden.patterned_floats(9, 0.23))
    np.testing.assert_array_equal(experts[2][1].ravel(), gen_golden.patterned_floats(12, 0.17))
    assert c["int_params"] == [1, 4, 3, 3, 1, 0, 4, 0]


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_matches_golden(case):
    got = _run(case)
    want = case["want"]
    np.testing.assert_array_equal(got["top_idx"], np.asarray(want["top_idx"]))
    np.testing.assert_array_equal(got["counts"], np.asarray(want["counts"]))
    np.testing.assert_allclose(got["gates"], np.asarray(want["gates"]), rtol=2e-6, atol=1e-7)
    assert _delta_ok(got["delta"], want["delta"]), np.max(np.abs(got["delta"] - want["delta"]))
    assert abs(got["aux"] - want["aux"]) <= 2e-5
    assert abs(got["entropy"] - want["entropy"]) <= 2e-5


def _case(name):
    return next(c for c in CASES if c["name"] == name)


@pytest.mark.parametrize("mistake", ["swap_gate_up", "permute_experts", "reverse_router_columns",
                                     "geglu_as_swiglu", "wrong_leaky_slope", "top_k_minus_one",
                                     "transpose_down"])
def test_golden_rejects_planted_mistakes(mistake):
    """Each plausible slip, planted in the oracle's inputs, fails the fixture check."""
    if mistake == "swap_gate_up":
        c = _case("known_answer_swiglu_k2")
        _, _, ex = _case_arrays(c)
        got = _run(c, experts=[[u, g, d] for g, u, d in ex])
    elif mistake == "permute_experts":
        c = _case("wide_swiglu_k3")
        _, _, ex = _case_arrays(c)
        got = _run(c, experts=ex[1:] + ex[:1])
    elif mistake == "reverse_router_columns":
        c = _case("known_answer_swiglu_k2")
        _, wr, _ = _case_arrays(c)
        got = _run(c, wr=np.ascontiguousarray(wr[:, ::-1]))
    elif mistake == "geglu_as_swiglu":
        c = _case("large_geglu_k2")
        got = _run(c, etype=0)
    elif mistake == "wrong_leaky_slope":
        c = _case("large_mlp_leaky_relu_sq_k2")
        got = _run(c, slope=0.5)
    elif mistake == "top_k_minus_one":
        c = _case("known_answer_swiglu_k2")
        got = _run(c, K=1)
    else:  # a square down projection read transposed
        c = _case("large_swiglu_k2")
        _, _, ex = _case_arrays(c)
        got = _run(c, experts=[[g, u, np.ascontiguousarray(d.T)] for g, u, d in ex])
    want = c["want"]
    same_routing = (got["top_idx"].shape == np.asarray(want["top_idx"]).shape
                    and np.array_equal(got["top_idx"], np.asarray(want["top_idx"])))
    assert not (same_routing and _delta_ok(got["delta"], want["delta"])
                and abs(got["aux"] - want["aux"]) <= 2e-5)


def _rand_problem(rng, N, D, E, F, etype=0, wscale=0.1):
    x = rng.standard_normal((N, D), dtype=np.float32)
    wr = (rng.standard_normal((D, E), dtype=np.float32) * np.float32(0.3)).astype(np.float32)
    shapes = [(D, F), (D, F), (F, D)] if etype != 2 else [(D, F), (F, D)]
    experts = [[(rng.standard_normal(s, dtype=np.float32) * np.float32(wscale)) for s in shapes]
               for _ in range(E)]
    return x, wr, experts


def _ffn64(x, ws, etype=0, act=0, slope=0.0):
    x = x.astype(np.float64)
    ws = [w.astype(np.float64) for w in ws]
    if etype in (0, 1):
        g, u = x @ ws[0], x @ ws[1]
        h = (gen_golden.sigmoid(g) if etype == 0 else gen_golden.gelu_tanh(g)) * u
        return h @ ws[2]
    return gen_golden.activation(x @ ws[0], act, slope) @ ws[1]


def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def test_k_equals_e_is_dense_softmax_mixture():
    rng = np.random.default_rng(1)
    x, wr, ex = _rand_problem(rng, 40, 24, 5, 16)
    got = oracle.moe_forward(x, wr, ex, top_k=5)
    lg = x.astype(np.float64) @ wr.astype(np.float64)
    p = np.exp(lg - lg.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    want = sum(p[:, e:e + 1] * _ffn64(x, ex[e]) for e in range(5))
    assert _rel(got["delta"], want) <= 1e-5
    np.testing.assert_allclose(got["gates"].sum(1), 1.0, rtol=1e-6)
    assert abs(got["aux"] - 1.0) <= 1e-6  # every expert selected by every token


def test_k1_is_argmax_with_unit_gate():
    rng = np.random.default_rng(2)
    x, wr, ex = _rand_problem(rng, 64, 16, 6, 8)
    got = oracle.moe_forward(x, wr, ex, top_k=1)
    np.testing.assert_array_equal(got["gates"], 1.0)
    np.testing.assert_array_equal(got["top_idx"][:, 0], np.argmax(got["probs"], axis=1))
    want = np.stack([_ffn64(x[n:n + 1], ex[got["top_idx"][n, 0]])[0] for n in range(64)])
    assert _rel(got["delta"], want) <= 1e-5


@pytest.mark.parametrize("etype,act,slope", [(0, 0, 0.0), (1, 1, 0.0), (2, 0, 0.0), (2, 1, 0.0),
                                             (2, 2, 0.0), (2, 3, 0.4)])
def test_single_expert_is_plain_ffn(etype, act, slope):
    """E = K = 1: the plain expert FFN (for swiglu, the `swiglu` block of
    arch/blocks.go:656-680), gate 1, aux 1, entropy 0."""
    rng = np.random.default_rng(3)
    x, wr, ex = _rand_problem(rng, 32, 16, 1, 24, etype=etype, wscale=0.4)
    got = oracle.moe_forward(x, wr, ex, top_k=1, expert_type=etype, activation=act,
                             leaky_slope=slope)
    assert _rel(got["delta"], _ffn64(x, ex[0], etype, act, slope)) <= 1e-5
    assert got["aux"] == 1.0 and got["entropy"] == 0.0
    np.testing.assert_array_equal(got["top_idx"], 0)


def test_ties_go_to_lower_expert():
    rng = np.random.default_rng(4)
    x, wr, ex = _rand_problem(rng, 48, 8, 6, 8)
    wr[:, 4] = wr[:, 1]
    wr[:, 5] = wr[:, 1]
    got = oracle.moe_forward(x, wr, ex, top_k=3)
    for n in range(48):
        row = list(got["top_idx"][n])
        for a, b in ((1, 4), (4, 5), (1, 5)):
            if a in row and b in row:
                assert row.index(a) < row.index(b)
        if 4 in row:
            assert 1 in row
        if 5 in row:
            assert 4 in row


@pytest.mark.parametrize("bf16", [False, True])
def test_dense_equals_sparse_bitwise(bf16):
    rng = np.random.default_rng(5)
    x, wr, ex = _rand_problem(rng, 50, 32, 6, 24)
    a = oracle.moe_forward(x, wr, ex, top_k=2, bf16=bf16)
    b = oracle.moe_forward(x, wr, ex, top_k=2, bf16=bf16, dense=True)
    np.testing.assert_array_equal(a["delta"].view(np.uint32), b["delta"].view(np.uint32))
    assert a["aux"] == b["aux"] and a["entropy"] == b["entropy"]


def test_dispatch_invariants():
    rng = np.random.default_rng(6)
    N, E, K = 300, 7, 3
    x, wr, ex = _rand_problem(rng, N, 16, E, 8)
    got = oracle.moe_forward(x, wr, ex, top_k=K, want_delta=False)
    counts, offsets, perm, top = got["counts"], got["offsets"], got["perm"], got["top_idx"]
    assert counts.sum() == N * K
    np.testing.assert_array_equal(counts, np.bincount(top.ravel(), minlength=E))
    np.testing.assert_array_equal(offsets, np.concatenate([[0], np.cumsum(counts)]))
    assert all(len(set(r)) == K for r in top.tolist())  # distinct experts per token
    for e in range(E):
        seg = perm[offsets[e]:offsets[e + 1]]
        assert np.all(np.diff(seg) > 0)  # ascending token within the expert
        np.testing.assert_array_equal(np.sort(seg), np.nonzero((top == e).any(1))[0])
    np.testing.assert_allclose(got["gates"].sum(1), 1.0, rtol=2e-6)


def test_bf16_flow_tracks_float64():
    rng = np.random.default_rng(7)
    x, wr, ex = _rand_problem(rng, 64, 64, 8, 64)
    got = oracle.moe_forward(x, wr, ex, top_k=2, bf16=True)
    xr, wrr = oracle.round_bf16(x), oracle.round_bf16(wr)
    exr = [[oracle.round_bf16(w) for w in ws] for ws in ex]
    want = np.zeros((64, 64))
    for n in range(64):
        for k in range(2):
            e = got["top_idx"][n, k]
            want[n] += got["gates"][n, k] * _ffn64(xr[n:n + 1], exr[e])[0]
    assert _rel(got["delta"], want) <= 2e-2
    del wrr


def test_exp_within_two_ulp():
    """exp as used by softmax, sigmoid and tanh: within 2 ulp of the correctly
    rounded value on [-86.5, 88]; below -86.5 (results near the bottom of the
    normal range) it returns +0, the routing's flush-to-zero contract."""
    xs = np.linspace(-86.5, 88.0, 400_001, dtype=np.float32)
    xs = np.concatenate([xs, np.float32(-np.arange(0, 2000, dtype=np.float32) * 2.0 ** -20),
                         np.float32(np.arange(0, 2000, dtype=np.float32) * 2.0 ** -20)])
    got = oracle.exp(xs).astype(np.float64)
    ref = np.exp(xs.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert float(np.max(np.abs(got - ref) / ulp)) <= 2.0
    assert oracle.exp(np.zeros(1, np.float32))[0] == 1.0
    np.testing.assert_array_equal(oracle.exp(np.array([-86.6, -100.0, -np.inf], np.float32)), 0.0)
    assert np.isinf(oracle.exp(np.array([89.0], np.float32))[0])


def test_round_bf16_ties_to_even_and_brute_force():
    one = np.float32(1.0)
    cases = {1.0 + 2.0 ** -8: 1.0, 1.0 + 3 * 2.0 ** -8: 1.0 + 2.0 ** -6,
             -(1.0 + 2.0 ** -8): -1.0, 1.0 + 2.0 ** -8 + 2.0 ** -20: 1.0 + 2.0 ** -7}
    for v, w in cases.items():
        assert oracle.round_bf16(np.array([v], np.float32))[0] == np.float32(w)
    assert np.isnan(oracle.round_bf16(np.array([np.nan], np.float32))[0])
    assert np.isinf(oracle.round_bf16(np.array([np.finfo(np.float32).max], np.float32))[0])
    rng = np.random.default_rng(8)
    bits = rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f) & (np.abs(f) < np.float32(3e38))]
    got = oracle.round_bf16(f)
    lo = (f.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32).astype(np.float64)
    hi_bits = (f.view(np.uint32) & np.uint32(0xFFFF0000)) + np.uint32(0x10000)
    hi = hi_bits.view(np.float32).astype(np.float64)
    fd = f.astype(np.float64)
    dlo, dhi = np.abs(fd - lo), np.abs(hi - fd)
    lo_even = ((f.view(np.uint32) >> 16) & 1) == 0
    want = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi, np.where(lo_even, lo, hi)))
    np.testing.assert_array_equal(got.astype(np.float64), want)
    # the C and numpy roundings agree bit for bit
    c = np.empty_like(f)
    oracle._load().oracle_round_bf16_array(oracle._p(f), oracle._p(c), f.size)
    np.testing.assert_array_equal(c.view(np.uint32), got.view(np.uint32))
    del one


def test_dense_blas_baseline_matches_oracle():
    rng = np.random.default_rng(9)
    x, wr, ex = _rand_problem(rng, 96, 32, 6, 48)
    want = oracle.moe_forward(x, wr, ex, top_k=2)
    delta, aux, ent = dense_forward(x, wr, lambda e, j: ex[e][j], 6, 2, 0, 0, 0.0)
    assert _rel(delta, want["delta"].astype(np.float64)) <= 1e-5
    assert abs(aux - want["aux"]) <= 1e-5 and abs(ent - want["entropy"]) <= 1e-5


# ---- block level: RMSNorm (gpu/ir.cpp:4949-4960) and the residual block ----

def _rms64(x, scale, eps):
    x64 = x.astype(np.float64)
    return x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + eps) * scale.astype(np.float64)


@pytest.mark.parametrize("D", [3, 64, 300, 2048])
def test_rmsnorm_matches_float64(D):
    rng = np.random.default_rng(10 + D)
    x = rng.standard_normal((17, D), dtype=np.float32) * np.float32(3.0)
    scale = (np.float32(1.0) + rng.standard_normal(D, dtype=np.float32) * np.float32(0.1))
    got = oracle.rmsnorm(x, scale, 1e-5)
    want = _rms64(x, scale, 1e-5)
    assert float(np.max(np.abs(got - want) / (np.abs(want) + 1e-30))) <= 2e-6
    # dropping eps, or averaging over D-1, is visible at this tolerance
    xs = x * np.float32(1e-3)
    got_small = oracle.rmsnorm(xs, scale, 1e-5)
    assert float(np.max(np.abs(got_small - _rms64(xs, scale, 0.0)))) > 1e-3
    if D > 3:
        alt = xs.astype(np.float64) / np.sqrt((xs.astype(np.float64) ** 2).sum(1, keepdims=True)
                                              / (D - 1) + 1e-5) * scale
        assert float(np.max(np.abs(got_small - alt) / np.abs(alt))) > 1e-4


def test_rmsnorm_invariances():
    """Power-of-two scalings are exact through every step, so they commute
    with the norm bit for bit (eps = 0 so it does not break the scaling)."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((9, 513), dtype=np.float32)
    scale = rng.standard_normal(513, dtype=np.float32)
    a = oracle.rmsnorm(x, scale, 0.0)
    np.testing.assert_array_equal(oracle.rmsnorm(x * np.float32(8.0), scale, 0.0), a)
    np.testing.assert_array_equal(oracle.rmsnorm(x, scale * np.float32(0.25), 0.0),
                                  a * np.float32(0.25))
    # a constant row normalises to sign * scale / sqrt(1 + eps / c^2)
    c = np.full((1, 256), 3.0, np.float32)
    np.testing.assert_allclose(oracle.rmsnorm(c, np.ones(256, np.float32), 0.0), 1.0, rtol=1e-7)
    # bf16 output is the rounding of the fp32 output
    np.testing.assert_array_equal(oracle.rmsnorm(x, scale, 1e-5, out_bf16=True),
                                  oracle.round_bf16(oracle.rmsnorm(x, scale, 1e-5)))


@pytest.mark.parametrize("with_scale", [False, True])
def test_block_forward_composition(with_scale):
    """arch/moe.go:152-213: x + moe_scale * MoE(RMSNorm(x)), aux scaled by
    the load-balance weight; against float64 evaluation of each step."""
    rng = np.random.default_rng(12)
    x, wr, ex = _rand_problem(rng, 48, 32, 6, 24)
    ns = (np.float32(1.0) + rng.standard_normal(32, dtype=np.float32) * np.float32(0.1))
    ms = rng.standard_normal(32, dtype=np.float32) if with_scale else None
    got = oracle.block_forward(x, ns, wr, ex, top_k=2, moe_scale=ms, aux_weight=0.05)
    xn64 = _rms64(x, ns, 1e-5)
    np.testing.assert_allclose(got["xn"], xn64, rtol=2e-6, atol=1e-7)
    want = np.zeros((48, 32))
    for n in range(48):
        for k in range(2):
            e = got["top_idx"][n, k]
            want[n] += got["gates"][n, k] * _ffn64(xn64[n:n + 1], ex[e])[0]
    if with_scale:
        want = want * ms
    assert _rel(got["x_out"] - x, want) <= 2e-5
    assert abs(got["aux"] - 0.05 * got["aux_raw"]) <= 1e-8
