"""Pins of the oracle's bf16 dtype flow.

The reference runs op 74 under compute_dtype "bf16" with every weight cast to
bf16 (gpu/ir_trainer.cpp:1395-1412), so MLX's promotion rules fix where the
values are rounded (gpu/ir.cpp:1106-1162): logits = x.Wr and probs =
softmax(logits) are bf16; argsort ranks the bf16 probabilities; the top-p sum
is bf16 and the renorm fp32 (the 1e-12 floor is an fp32 array); the per-expert
mean probability of aux is bf16; entropy is fp32 over the bf16 probabilities
(the fp32 floor promotes); the expert projections are bf16 matmuls; swiglu's
sigmoid and product, mlp-silu and relu stay bf16, while gelu (its float
scalars) and leaky_relu_sq (its fp32 slope array) promote to fp32, and y is
bf16 exactly when the hidden is.

Each pin below recomputes one of those steps independently -- numpy lexsort,
float64 softmax and sums, float64 activations rounded at the flow's rounding
points -- from the values the restatement returns, and each is shown to
reject a planted slip (a build of oracle/moe_oracle.c with one ORACLE_PLANT_*
macro defined): a rounding dropped or a decision taken on unrounded values.
Where an independent float64 value lies within the fp32 evaluation error of a
bf16 rounding boundary, the two roundings may legitimately differ; such
elements are held to one bf16 ulp plus that error bound, and every other
element must match bit for bit.  No GPU is used here.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle

PLANTS = ["LOGITS_FP32", "PROBS_FP32", "TOPK_FP32", "TOPSUM_FP32", "AUX_MEAN_FP32",
          "ENTROPY_FP32", "PROJ_FP32", "SWIGLU_SIG", "SWIGLU_PROD", "GEGLU_SQ", "SILU_SIG",
          "GELU_SQ", "Y_FP32", "Y_BF16"]
# (expert type, activation, slope) of the six expert kinds (arch/moe.go:53-80)
KINDS = [(0, 0, 0.0), (1, 1, 0.0), (2, 0, 0.0), (2, 1, 0.0), (2, 2, 0.0), (2, 3, 0.4)]
KIND_IDS = ["swiglu", "geglu", "mlp_silu", "mlp_gelu", "mlp_relu", "mlp_leaky_relu_sq"]
GELU_A = float(np.float32(0.044715))
GELU_C = float(np.float32(0.7978845608))


@pytest.fixture(scope="module")
def planted(tmp_path_factory):
    d = tmp_path_factory.mktemp("oracle_plants")
    with ThreadPoolExecutor(max_workers=8) as ex:
        paths = list(ex.map(lambda p: oracle.build_planted(p, d), PLANTS))
    return dict(zip(PLANTS, paths))


# ---- bf16 helpers (float64 in, exact) ----

def rb(v) -> np.ndarray:
    """Nearest bf16 (ties to even) of float64 values, via their float32."""
    return oracle.round_bf16(np.asarray(v, np.float64).astype(np.float32)).astype(np.float64)


def is_bf16(a) -> bool:
    a = np.asarray(a, np.float32)
    return bool(np.all((a.view(np.uint32) & np.uint32(0xFFFF)) == 0))


def bf16_ulp(v) -> np.ndarray:
    """Spacing of bf16 values at |v| (8 significant bits)."""
    v = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(v, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def near_bf16_boundary(v, tol) -> np.ndarray:
    """True where float64 v is within tol of a bf16 rounding midpoint."""
    v = np.asarray(v, np.float64)
    f = v.astype(np.float32)
    lo = (f.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32).astype(np.float64)
    hi = ((f.view(np.uint32) & np.uint32(0xFFFF0000)) + np.uint32(0x10000)).view(
        np.float32).astype(np.float64)
    mid = 0.5 * (lo + hi)
    return np.abs(v - mid) <= tol


def match_rounding(got, exact64, tol) -> bool:
    """got == rb(exact64) except within tol (the fp32 evaluation's error
    bound) of a midpoint, where got may be the rounding of any value within
    tol of exact64: one bf16 ulp plus tol."""
    got = np.asarray(got, np.float64)
    tol = np.broadcast_to(np.asarray(tol, np.float64), np.shape(exact64))
    want = rb(exact64)
    near = near_bf16_boundary(exact64, tol)
    if not np.array_equal(got[~near], want[~near]):
        return False
    return bool(np.all(np.abs(got[near] - exact64[near])
                       <= bf16_ulp(exact64[near]) + tol[near]))


# ---- routing pins (gpu/ir.cpp:1106-1111, 1150-1162) ----

def routing_problem(seed, N=512, D=64, E=16, wscale=0.002, dup=True):
    """Near-uniform routing: small router weights put the probabilities close
    to 1/E, where bf16 holds few distinct values, so ties are common; two
    duplicated router columns add exact ties."""
    rng = np.random.default_rng(seed)
    x = oracle.round_bf16(rng.standard_normal((N, D), dtype=np.float32))
    wr = rng.standard_normal((D, E), dtype=np.float32) * np.float32(wscale)
    if dup:
        wr[:, E - 1] = wr[:, 1]
        wr[:, E - 2] = wr[:, 3]
    return x, oracle.round_bf16(wr)


def pin_logits(x, wr, res) -> bool:
    lg = res["logits"]
    if not is_bf16(lg):
        return False
    x64, w64 = x.astype(np.float64), wr.astype(np.float64)
    dot = x64 @ w64
    bound = 2.0 ** -22 * (np.abs(x64) @ np.abs(w64)) + 1e-30  # fp32 accumulation error
    return match_rounding(lg, dot, bound)


def pin_probs(res) -> bool:
    p = res["probs"]
    if not is_bf16(p):
        return False
    lg = res["logits"].astype(np.float64)
    ex = np.exp(lg - lg.max(1, keepdims=True))
    sm = ex / ex.sum(1, keepdims=True)
    return match_rounding(p, sm, 1e-5 * sm)


def pin_topk(res, K) -> bool:
    p = res["probs"]
    E = p.shape[1]
    for n in range(p.shape[0]):
        order = np.lexsort((np.arange(E), -p[n].astype(np.float64)))  # p desc, then e asc
        if not np.array_equal(order[:K], res["top_idx"][n]):
            return False
    return True


def pin_gates(res) -> bool:
    ti, p = res["top_idx"], res["probs"]
    ps = np.take_along_axis(p, ti, axis=1)
    s = ps.astype(np.float64).sum(axis=1)  # exact: a few bf16 values
    den = np.maximum(rb(s), 1e-12).astype(np.float32)
    want = ps.astype(np.float32) / den[:, None]  # fp32 division, correctly rounded
    return np.array_equal(res["gates"], want)


def pin_aux(res, K) -> bool:
    p, ti = res["probs"].astype(np.float64), res["top_idx"]
    N, E = p.shape
    pm = rb(p.mean(axis=0))  # MLX: mean of a bf16 column is bf16
    cnt = np.bincount(ti.ravel(), minlength=E).astype(np.float64)
    aux = E * np.sum(pm * cnt / K / N)
    return abs(res["aux"] - aux) <= 2e-6 * abs(aux) + 1e-9


def pin_entropy(res) -> bool:
    p = res["probs"].astype(np.float64)
    ent = -np.mean(np.sum(p * np.log(np.maximum(p, 1e-12)), axis=1))
    return abs(res["entropy"] - ent) <= 2e-6 * abs(ent) + 1e-9


ROUTING_CASES = [(11, 512, 64, 16, 4, 0.002), (12, 256, 96, 64, 8, 0.001),
                 (13, 300, 32, 8, 2, 0.05), (14, 1024, 128, 64, 8, 0.02)]


def _route(case, lib=None):
    seed, N, D, E, K, ws = case
    x, wr = routing_problem(seed, N, D, E, ws)
    experts = np.zeros(E * 3 * D * 8, np.float32)  # F = 8; the FFN plays no part here
    res = oracle.moe_forward(x, wr, experts, top_k=K, bf16=True, prerounded=True,
                             want_delta=False, lib=lib)
    return x, wr, K, res


@pytest.mark.parametrize("case", ROUTING_CASES, ids=lambda c: f"N{c[1]}_D{c[2]}_E{c[3]}_K{c[4]}")
def test_bf16_routing_pins(case):
    x, wr, K, res = _route(case)
    assert pin_logits(x, wr, res)
    assert pin_probs(res)
    assert pin_topk(res, K)
    assert pin_gates(res)
    assert pin_aux(res, K)
    assert pin_entropy(res)


def test_routing_inputs_have_bf16_ties():
    """The pins are only as sharp as the inputs: at least a quarter of the
    rows must have a bf16 tie across their top-K boundary (the planted
    fp32-ranked top-k shows that ranking inside such ties changes picks)."""
    x, wr, K, res = _route(ROUTING_CASES[0])
    p = res["probs"]
    ties = 0
    for n in range(p.shape[0]):
        srt = np.sort(p[n])[::-1]
        ties += int(srt[K - 1] == srt[K])
    assert ties >= p.shape[0] // 4


ROUTING_PLANTS = {
    "LOGITS_FP32": lambda x, wr, K, r: pin_logits(x, wr, r),
    "PROBS_FP32": lambda x, wr, K, r: pin_probs(r),
    "TOPK_FP32": lambda x, wr, K, r: pin_topk(r, K),
    "TOPSUM_FP32": lambda x, wr, K, r: pin_gates(r),
    "AUX_MEAN_FP32": lambda x, wr, K, r: pin_aux(r, K),
    "ENTROPY_FP32": lambda x, wr, K, r: pin_entropy(r),
}


@pytest.mark.parametrize("plant", list(ROUTING_PLANTS))
def test_routing_pins_reject_planted_mistakes(planted, plant):
    x, wr, K, res = _route(ROUTING_CASES[0], lib=planted[plant])
    assert not ROUTING_PLANTS[plant](x, wr, K, res)


# ---- hidden activations (gpu/ir.cpp:1053-1071, 1130-1145) ----

def sigmoid64(v):
    return 1.0 / (1.0 + np.exp(-v))


def gelu64(v, sq):
    return 0.5 * v * (1.0 + np.tanh(GELU_C * (v + GELU_A * v * sq)))


def hidden_inputs(seed, n=200_000):
    rng = np.random.default_rng(seed)
    g = oracle.round_bf16(rng.standard_normal(n, dtype=np.float32) * np.float32(2.5))
    u = oracle.round_bf16(rng.standard_normal(n, dtype=np.float32) * np.float32(2.5))
    g[:4] = [0.0, -0.0, 8.0, -8.0]
    u[:4] = [1.0, -1.0, 0.0, 3.0]
    return g, u


def pin_hidden(kind, g, u, h) -> bool:
    """h from the restatement against an independent float64 evaluation of
    the kind's bf16 flow."""
    et, act, slope = kind
    g64, u64, h64 = g.astype(np.float64), u.astype(np.float64), h.astype(np.float64)

    def bf16_glu(a, b):  # rbf(rbf(sigmoid(a)) * b): swiglu and mlp-silu
        s = sigmoid64(a)
        near = near_bf16_boundary(s, 4e-7 * s)  # fp32 exp + division error
        want = rb(rb(s) * b)
        ok = np.array_equal(h64[~near], want[~near])
        return ok and bool(np.all(np.abs(h64[near] - s[near] * b[near])
                                  <= 2 * bf16_ulp(s[near] * b[near]) + 1e-30))

    def fp32_gelu(v, mul):
        want = gelu64(v, rb(v * v)) * mul
        scale = np.abs(0.5 * v * mul) * 2.0 + 1e-30
        return bool(np.all(np.abs(h64 - want) <= 1e-6 * scale))

    if et == 0:
        return is_bf16(h) and bf16_glu(g64, u64)
    if et == 1:
        return fp32_gelu(g64, u64)
    if act == 0:
        return is_bf16(h) and bf16_glu(u64, u64)
    if act == 1:
        return fp32_gelu(u64, 1.0)
    if act == 2:
        return np.array_equal(h64, np.maximum(u64, 0.0))
    y = np.where(u > 0, u, (u * np.float32(slope)).astype(np.float32)).astype(np.float32)
    return np.array_equal(h, (y * y).astype(np.float32))


@pytest.mark.parametrize("kind", KINDS, ids=KIND_IDS)
def test_hidden_bf16_pins(kind):
    g, u = hidden_inputs(21)
    h = oracle.hidden(True, *kind, g, u)
    assert pin_hidden(kind, g, u, h)


HIDDEN_PLANTS = {"SWIGLU_SIG": KINDS[0], "SWIGLU_PROD": KINDS[0], "GEGLU_SQ": KINDS[1],
                 "SILU_SIG": KINDS[2], "GELU_SQ": KINDS[3]}


@pytest.mark.parametrize("plant", list(HIDDEN_PLANTS))
def test_hidden_pins_reject_planted_mistakes(planted, plant):
    kind = HIDDEN_PLANTS[plant]
    g, u = hidden_inputs(21)
    h = oracle.hidden(True, *kind, g, u, lib=planted[plant])
    assert not pin_hidden(kind, g, u, h)


# ---- the expert FFN and combine of the bf16 flow (gpu/ir.cpp:1118-1148) ----

def hidden_is_bf16(et, act):
    return et == 0 or (et == 2 and act in (0, 2))


def ffn_bf16_flow64(xr, ws, kind):
    """Expert FFN of one row block in float64, rounded at the bf16 flow's
    rounding points: projections, the kind's activation steps, and y when
    the hidden is bf16."""
    et, act, slope = kind
    ws = [w.astype(np.float64) for w in ws]
    x64 = xr.astype(np.float64)
    if et in (0, 1):
        g, u = rb(x64 @ ws[0]), rb(x64 @ ws[1])
        h = rb(rb(sigmoid64(g)) * u) if et == 0 else gelu64(g, rb(g * g)) * u
    else:
        u = rb(x64 @ ws[0])
        if act == 0:
            h = rb(u * rb(sigmoid64(u)))
        elif act == 1:
            h = gelu64(u, rb(u * u))
        elif act == 2:
            h = np.maximum(u, 0.0)
        else:
            y = np.where(u > 0, u, u * np.float32(slope))
            h = y * y
    y = h @ ws[-1]
    return rb(y) if hidden_is_bf16(et, act) else y


def ffn_plain64(xr, ws, kind):
    """The same FFN in float64 with no rounding at all."""
    et, act, slope = kind
    ws = [w.astype(np.float64) for w in ws]
    x64 = xr.astype(np.float64)
    if et in (0, 1):
        g, u = x64 @ ws[0], x64 @ ws[1]
        h = (sigmoid64(g) if et == 0 else gelu64(g, g * g)) * u
    else:
        u = x64 @ ws[0]
        h = {0: lambda: u * sigmoid64(u), 1: lambda: gelu64(u, u * u),
             2: lambda: np.maximum(u, 0.0)}.get(act, lambda: np.where(u > 0, u, u * slope) ** 2)()
    return h @ ws[-1]


def ffn_problem(seed, kind, N=96, D=64, E=6, F=64):
    rng = np.random.default_rng(seed)
    x = oracle.round_bf16(rng.standard_normal((N, D), dtype=np.float32))
    wr = oracle.round_bf16(rng.standard_normal((D, E), dtype=np.float32) * np.float32(0.3))
    shapes = [(D, F), (D, F), (F, D)] if kind[0] != 2 else [(D, F), (F, D)]
    experts = [[oracle.round_bf16(rng.standard_normal(s, dtype=np.float32) * np.float32(0.15))
                for s in shapes] for _ in range(E)]
    return x, wr, experts


def delta_from(res, x, experts, kind, ffn):
    N, D = x.shape
    want = np.zeros((N, D))
    for n in range(N):
        for k in range(res["top_idx"].shape[1]):
            e = res["top_idx"][n, k]
            want[n] += np.float64(res["gates"][n, k]) * ffn(x[n:n + 1], experts[e], kind)[0]
    return want


def rel_l2(a, b) -> float:
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


# Measured on these inputs: the restatement sits within 6e-6 of the float64
# flow with the same roundings; each dropped or added rounding in FFN_PLANTS
# moves it by 1.6e-3 or more.  (A dropped rounding of geglu's square moves the
# delta by only 2e-5; the hidden-activation pin rejects it.)
TIGHT = 1e-4


def _ffn_run(kind, lib=None):
    x, wr, ex = ffn_problem(31, kind)
    res = oracle.moe_forward(x, wr, ex, top_k=2, expert_type=kind[0], activation=kind[1],
                             leaky_slope=kind[2], bf16=True, prerounded=True, lib=lib)
    return x, ex, res


@pytest.mark.parametrize("kind", KINDS, ids=KIND_IDS)
def test_bf16_flow_delta_pins(kind):
    x, ex, res = _ffn_run(kind)
    # the flow's roundings, restated in float64
    assert rel_l2(res["delta"], delta_from(res, x, ex, kind, ffn_bf16_flow64)) <= TIGHT
    # and the float64 band of the unrounded FFN (the bf16 bar)
    assert rel_l2(res["delta"], delta_from(res, x, ex, kind, ffn_plain64)) <= 2e-2


FFN_PLANTS = {"PROJ_FP32": KINDS[0], "SWIGLU_PROD": KINDS[0], "Y_FP32": KINDS[0],
              "Y_BF16": KINDS[1], "SILU_SIG": KINDS[2]}


@pytest.mark.parametrize("plant", list(FFN_PLANTS))
def test_bf16_flow_delta_pins_reject_planted_mistakes(planted, plant):
    kind = FFN_PLANTS[plant]
    x, ex, res = _ffn_run(kind, lib=planted[plant])
    assert rel_l2(res["delta"], delta_from(res, x, ex, kind, ffn_bf16_flow64)) > TIGHT
