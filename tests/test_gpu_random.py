"""A seeded sweep of op shapes through every flow, against the restatement.

The other GPU tests pin chosen edges (tile multiples, router limits, padded
widths, decode sizes).  This sweep draws its shapes at random -- tokens,
model and expert widths off every tile, expert counts and top-k, all six
expert kinds, fp32 / bf16 / int8 weights -- so that the interactions of the
executor's choices (MFMA or SIMT family and tile, padding, router path,
decode flow) meet shapes nobody chose.  Bars, per flow:
* routing (top-k indices, gates, counts, offsets, permutation) bit-exact;
* fp32, and bf16 on the SIMT kernels: delta bit-exact (the exact-order
  kernels follow the restatement's summation order);
* bf16 on the MFMA kernels: delta within 1e-3 relative L2 (accumulation
  order only);
* int8: delta within 1e-3 of the restatement fed the exact products q * s;
* aux and entropy within 1e-5 (fp32) or 1e-2 / 1e-4 (bf16 flows).
The cases are fixed by the seed; each prints its shape before it runs.
"""
import numpy as np
import pytest

import oracle
from mixlab_amd import _lib
from mixlab_amd.workloads import bf16_bits, quantize_int8, round_bf16
from tests.moe_testutil import assert_routing_equal, random_case, rel_l2, run_gpu, run_oracle, same_bits

pytestmark = pytest.mark.gpu

KINDS = [(0, 0), (1, 1), (2, 0), (2, 1), (2, 2), (2, 3)]  # (expert type, activation)


def _cases(n=36, seed=2026, max_e=80, max_k=8):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        flow = ("fp32", "bf16", "int8")[len(cases) % 3]
        etype, act = KINDS[int(rng.integers(len(KINDS)))]
        E = int(rng.integers(1, max_e + 1))
        K = int(rng.integers(1, min(E, max_k) + 1))
        N = int(rng.integers(1, 4001))
        D = int(rng.integers(16, 1100))
        F = int(rng.integers(16, 1500))
        wpe = 2 if etype == 2 else 3
        if N * K * D * F * wpe > 4e9:  # keeps each restatement run to about a second
            continue
        slope = float(np.round(rng.uniform(0.1, 0.5), 3)) if act == 3 else 0.0
        cases.append((flow, N, D, E, K, F, etype, act, slope, int(rng.integers(1 << 30))))
    return cases


# the common regime, then wide routers: up to 256 experts (several expert
# groups per lane) and top-k past one combine chunk of 8 slots
CASES = _cases() + _cases(n=12, seed=2029, max_e=256, max_k=24)


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-N{c[1]}-D{c[2]}-E{c[3]}-K{c[4]}-F{c[5]}-k{c[6]}{c[7]}"
                                             for c in CASES])
def test_random_shapes(gpu_lib, case):
    from mixlab_amd.op import MoEFeedForward

    flow, N, D, E, K, F, etype, act, slope, seed = case
    print(f"case {case}", flush=True)
    x, wr, experts = random_case(seed, N, D, E, F, expert_type=etype)
    if flow == "fp32":
        delta, aux, ent, routing, info = run_gpu(x, wr, experts, B=1, T=N, K=K, expert_type=etype,
                                                 activation=act, slope=slope)
        want = run_oracle(x, wr, experts, K=K, expert_type=etype, activation=act, slope=slope)
        assert_routing_equal(routing, want)
        assert same_bits(delta, want["delta"])
        assert abs(aux - want["aux"]) <= 1e-5 * abs(want["aux"]) + 1e-7
        assert abs(ent - want["entropy"]) <= 1e-5 * abs(want["entropy"]) + 1e-7
        return
    x, wr = round_bf16(x), round_bf16(wr)
    if flow == "bf16":
        experts = [[round_bf16(m) for m in ws] for ws in experts]
        delta, aux, ent, routing, info = run_gpu(x, wr, experts, B=1, T=N, K=K, expert_type=etype,
                                                 activation=act, slope=slope, bf16=True)
        want = run_oracle(x, wr, experts, K=K, expert_type=etype, activation=act, slope=slope,
                          bf16=True)
        assert_routing_equal(routing, want)
        if info["mfma"]:
            err = rel_l2(delta, want["delta"])
            print(f"  mfma (widths {info['ffn_kernel']} / {info['d_kernel']}): rel L2 {err:.2e}")
            assert err <= 1e-3
        else:
            assert same_bits(delta, want["delta"])
    else:
        wpe = 2 if etype == 2 else 3
        q8 = [[quantize_int8(m) for m in ws] for ws in experts]
        with MoEFeedForward([1, N, D, E, K, etype, F, act], [slope], compute_dtype="bf16",
                            flags=_lib.MXM_FLAG_INT8_WEIGHTS) as op:
            op.set_input(1, bf16_bits(wr))
            for e in range(E):
                for j in range(wpe):
                    op.set_input_q8(2 + e * wpe + j, *q8[e][j])
            delta, aux, ent = op.forward_host(bf16_bits(x))
            routing = op.routing()
            info = op.info()
        exact = [[(q.astype(np.float32) * s[None, :]).astype(np.float32) for q, s in ws]
                 for ws in q8]
        want = oracle.moe_forward(x, wr, exact, top_k=K, expert_type=etype, activation=act,
                                  leaky_slope=slope, bf16=True, prerounded=True)
        assert_routing_equal(routing, want)
        err = rel_l2(delta, want["delta"])
        print(f"  int8 (route flow {info['route_flow']}): rel L2 {err:.2e}")
        assert err <= 1e-3
    assert abs(aux - want["aux"]) <= 1e-2 * abs(want["aux"]) + 1e-6
    assert abs(ent - want["entropy"]) <= 1e-4 * abs(want["entropy"]) + 1e-6


def _bw_cases(n=16, seed=2027):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        flow = ("fp32", "bf16")[len(cases) % 2]
        etype, act = KINDS[int(rng.integers(len(KINDS)))]
        E = int(rng.integers(1, 41))
        K = int(rng.integers(1, min(E, 8) + 1))
        N = int(rng.integers(1, 1500))
        D = int(rng.integers(16, 700))
        F = int(rng.integers(16, 900))
        wpe = 2 if etype == 2 else 3
        if N * K * D * F * wpe > 1.5e9:  # the float64 restatement's products stay small
            continue
        slope = float(np.round(rng.uniform(0.1, 0.5), 3)) if act == 3 else 0.0
        cases.append((flow, N, D, E, K, F, etype, act, slope, int(rng.integers(1 << 30))))
    return cases


BW_CASES = _bw_cases()


@pytest.mark.parametrize("case", BW_CASES,
                         ids=[f"{c[0]}-N{c[1]}-D{c[2]}-E{c[3]}-K{c[4]}-F{c[5]}-k{c[6]}{c[7]}"
                              for c in BW_CASES])
def test_random_shapes_backward(gpu_lib, case):
    """mxm_moe_backward at random shapes (fp32, and bf16 on whichever kernels
    the executor picks) against the float64 restatement (oracle/backward.py,
    pinned by finite differences), routing held at the forward's: dx, d
    router_w and every expert matrix within 1e-4 relative L2 (fp32) or 2e-2
    (the bf16 flow's roundings)."""
    from mixlab_amd.op import MoEFeedForward
    from oracle.backward import backward64

    flow, N, D, E, K, F, etype, act, slope, seed = case
    print(f"case {case}", flush=True)
    bf16 = flow == "bf16"
    x, wr, experts = random_case(seed, N, D, E, F, expert_type=etype, wscale=0.1)
    if bf16:
        x, wr = round_bf16(x), round_bf16(wr)
        experts = [[round_bf16(m) for m in ws] for ws in experts]
    dD = np.random.default_rng(seed + 1).standard_normal((N, D), dtype=np.float32)
    up = bf16_bits if bf16 else (lambda a: a)
    with MoEFeedForward([1, N, D, E, K, etype, F, act], [slope],
                        compute_dtype="bf16" if bf16 else "fp32") as op:
        op.set_weights(up(wr), [[up(m) for m in ws] for ws in experts])
        dx, dwr, dexp = op.backward_host(x, dD, d_aux=0.3, d_entropy=-0.2)
        routing = op.routing()
        info = op.info()
    want = run_oracle(x, wr, experts, K=K, expert_type=etype, activation=act, slope=slope,
                      bf16=bf16)
    assert_routing_equal(routing, want)
    rdx, rdwr, rdexp = backward64(x, wr, experts, want["top_idx"].astype(np.int64), dD, 0.3, -0.2,
                                  etype, act, slope)
    tol = 2e-2 if bf16 else 1e-4
    errs = [rel_l2(dx, rdx), rel_l2(dwr, rdwr)]
    for m in range(len(experts[0])):
        got = np.concatenate([dexp[e][m].ravel() for e in range(E)])
        ref = np.concatenate([np.asarray(rdexp[e][m], np.float64).ravel() for e in range(E)])
        errs.append(rel_l2(got, ref) if np.any(ref) else float(np.any(got)))
    print(f"  {'mfma' if info['mfma'] else 'simt'}: rel L2 dx {errs[0]:.2e} dwr {errs[1]:.2e} "
          f"experts {max(errs[2:]):.2e}")
    assert max(errs) <= tol, errs


def _block_cases(n=12, seed=2028):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        flow = ("fp32", "bf16", "int8")[len(cases) % 3]
        etype, act = KINDS[int(rng.integers(len(KINDS)))]
        E = int(rng.integers(1, 65))
        K = int(rng.integers(1, min(E, 8) + 1))
        N = int(rng.integers(1, 3000))
        D = int(rng.integers(16, 1100))
        F = int(rng.integers(16, 1500))
        wpe = 2 if etype == 2 else 3
        if N * K * D * F * wpe > 4e9:
            continue
        slope = float(np.round(rng.uniform(0.1, 0.5), 3)) if act == 3 else 0.0
        with_scale = bool(rng.integers(2))
        cases.append((flow, N, D, E, K, F, etype, act, slope, with_scale, int(rng.integers(1 << 30))))
    return cases


BLOCK_CASES = _block_cases()


@pytest.mark.parametrize("case", BLOCK_CASES,
                         ids=[f"{c[0]}-N{c[1]}-D{c[2]}-E{c[3]}-K{c[4]}-F{c[5]}-k{c[6]}{c[7]}"
                              f"{'-scale' if c[9] else ''}" for c in BLOCK_CASES])
def test_random_blocks(gpu_lib, case):
    """The fused block (RMSNorm, op 74, moe_scale, residual, aux weight) at
    random shapes against the restatement: routing bit-exact (so the norm is
    too); x_out bit-exact in fp32 (SIMT experts), the block's delta within
    2e-2 (bf16) or 1e-3 (int8, against the exact products q * s)."""
    from mixlab_amd.op import MoEFeedForward

    flow, N, D, E, K, F, etype, act, slope, with_scale, seed = case
    print(f"case {case}", flush=True)
    rng = np.random.default_rng(seed)
    x, wr, experts = random_case(seed, N, D, E, F, expert_type=etype)
    x = x * np.float32(2.5)
    ns = np.float32(1.0) + rng.standard_normal(D, dtype=np.float32) * np.float32(0.2)
    ms = rng.standard_normal(D, dtype=np.float32) if with_scale else None
    wpe = 2 if etype == 2 else 3
    bf16 = flow != "fp32"
    if bf16:
        x, wr, ns = round_bf16(x), round_bf16(wr), round_bf16(ns)
        ms = None if ms is None else round_bf16(ms)
    conv = bf16_bits if bf16 else (lambda a: np.ascontiguousarray(a, np.float32))
    flags = _lib.MXM_FLAG_INT8_WEIGHTS if flow == "int8" else 0
    with MoEFeedForward([1, N, D, E, K, etype, F, act], [slope],
                        compute_dtype="bf16" if bf16 else "fp32", flags=flags) as op:
        op.set_input(1, conv(wr))
        if flow == "int8":
            q8 = [[quantize_int8(m) for m in ws] for ws in experts]
            for e in range(E):
                for j in range(wpe):
                    op.set_input_q8(2 + e * wpe + j, *q8[e][j])
            feed = [[(q.astype(np.float32) * s[None, :]).astype(np.float32) for q, s in ws]
                    for ws in q8]
        else:
            if bf16:
                experts = [[round_bf16(m) for m in ws] for ws in experts]
            for e in range(E):
                for j in range(wpe):
                    op.set_input(2 + e * wpe + j, conv(experts[e][j]))
            feed = experts
        out, aux, ent = op.block_forward_host(conv(x), conv(ns), None if ms is None else conv(ms),
                                              eps=1e-5, aux_weight=0.03)
        routing = op.routing()
    want = oracle.block_forward(x, ns, wr, feed, top_k=K, expert_type=etype, activation=act,
                                leaky_slope=slope, moe_scale=ms, eps=1e-5, aux_weight=0.03,
                                bf16=bf16, prerounded=flow == "int8")
    assert_routing_equal(routing, want)
    if flow == "fp32":
        assert same_bits(out, want["x_out"])
    else:
        err = rel_l2(out - x, want["x_out"] - x)
        print(f"  {flow}: block delta rel L2 {err:.2e}")
        assert err <= (1e-3 if flow == "int8" else 2e-2)
    assert abs(aux - want["aux"]) <= (1e-5 if flow == "fp32" else 1e-2) * abs(want["aux"]) + 1e-7
    assert abs(ent - want["entropy"]) <= 1e-3 * abs(want["entropy"]) + 1e-7
