"""Expert and model widths that are not multiples of the kernels' tiles.

The reference's default expert width is ffnDim = round(D * 2.67)
(arch/weight_shapes.go:11,56-65): 1,367 / 2,734 / 5,468 at D = 512 / 1,024 /
2,048, none a multiple of 64.  The library pads such widths with zero
weights (zero gate / up columns and W_down rows: the hidden of a zero
projection is 0 for every expert kind, so y is unchanged; zero W_down
columns for a padded model width), so these ops run on the MFMA and int8
kernels instead of the SIMT ones.  Each case is held to the same bars as the
tile-aligned ones: routing bit-exact against the restatement, the delta
within 1e-3 of it (sampled rows at the widest shapes, where the scalar
restatement takes seconds per row group) and, on every row, within 1e-3 of
the exact-order SIMT kernels run on the same op shape.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from mixlab_amd import _lib, moe
from mixlab_amd.workloads import bf16_bits, quantize_int8, round_bf16
from tests.moe_testutil import assert_routing_equal, random_case, rel_l2, run_gpu, run_oracle

BF16_TOL = 2e-2
MFMA_TIGHT = 1e-3


def _ffn(D, mult=2.67):
    return moe.ffn_dim(D, mult)


def _round_up(v, m):
    return (v + m - 1) // m * m


def _case(seed, N, D, E, F, etype=0):
    x, wr, experts = random_case(seed, N, D, E, F, expert_type=etype)
    return round_bf16(x), round_bf16(wr), [[round_bf16(m) for m in ws] for ws in experts]


def _check(N, D, E, K, F, etype=0, act=0, slope=0.0, sample=None, seed=5):
    x, wr, experts = _case(seed, N, D, E, F, etype)
    print(f"N {N} D {D} E {E} K {K} F {F} kind {etype}/{act}", flush=True)
    delta, aux, ent, routing, info = run_gpu(x, wr, experts, B=1, T=N, K=K, expert_type=etype,
                                             activation=act, slope=slope, bf16=True)
    assert info["mfma"], info
    assert info["ffn_kernel"] == _round_up(F, 128)
    assert info["d_kernel"] == _round_up(D, 128) and info["d_reduce"] == _round_up(D, 64)
    rows = None
    if sample:
        rows = np.sort(np.random.default_rng(seed).choice(N, size=sample, replace=False))
        rows = rows.astype(np.int32)
    want = run_oracle(x, wr, experts, K=K, expert_type=etype, activation=act, slope=slope,
                      bf16=True, rows=rows)
    assert_routing_equal(routing, want)
    sel = rows if rows is not None else slice(None)
    err = rel_l2(delta[sel], want["delta"][sel])
    assert abs(aux - want["aux"]) <= 1e-2 * abs(want["aux"])
    # every row against the exact-order SIMT kernels (unpadded) on the same op
    sdelta, _, _, srouting, sinfo = run_gpu(x, wr, experts, B=1, T=N, K=K, expert_type=etype,
                                            activation=act, slope=slope, bf16=True,
                                            flags=_lib.MXM_FLAG_FORCE_SIMT)
    assert not sinfo["mfma"]
    assert_routing_equal(srouting, want)
    err_all = rel_l2(delta, sdelta)
    print(f"  delta rel L2 {err:.2e} vs the restatement, {err_all:.2e} vs SIMT on all rows")
    assert err <= MFMA_TIGHT and err_all <= MFMA_TIGHT
    return delta


@pytest.mark.gpu
@pytest.mark.parametrize("D", [512, 1024, 2048])
def test_default_expert_width_on_mfma(gpu_lib, D):
    """D in {512, 1024, 2048} with the default mlp_mult 2.67: F = 1367 / 2734 /
    5468 run on the MFMA kernels at F rounded up to 128."""
    F = _ffn(D)
    assert F == {512: 1367, 1024: 2734, 2048: 5468}[D]
    _check(N=1024, D=D, E=8, K=2, F=F, sample=None if D == 512 else 16)


KINDS = [(0, 0, 0.0), (1, 1, 0.0), (2, 0, 0.0), (2, 1, 0.0), (2, 2, 0.0), (2, 3, 0.3)]


@pytest.mark.gpu
@pytest.mark.parametrize("etype,act,slope", KINDS)
def test_padded_width_every_kind(gpu_lib, etype, act, slope):
    """Every expert kind at a padded width, including those whose hidden is
    fp32 in the bf16 flow (two bf16 planes of Fk columns each)."""
    _check(N=512, D=256, E=6, K=2, F=333, etype=etype, act=act, slope=slope)


@pytest.mark.gpu
@pytest.mark.parametrize("D,F", [(320, 640), (544, 1452), (160, 427), (192, 513)])
def test_padded_model_width(gpu_lib, D, F):
    """Model widths that are not multiples of 128: the down projection runs
    at D rounded up to 128 (zero W_down columns, y read D of Dk columns), and
    where D is not a multiple of 64 either (544, 160) the up projection reads
    a zero-padded copy of x's rows.  544 is one of the reference's example
    widths (examples/*.json model_dim)."""
    _check(N=700, D=D, E=8, K=2, F=F)


@pytest.mark.gpu
@pytest.mark.parametrize("shape,etype,act", [((1, 600, 512, 8, 1367, 2), 0, 0),
                                             ((1, 600, 256, 6, 333, 2), 1, 1),
                                             ((1, 600, 256, 6, 333, 2), 2, 0),
                                             ((1, 500, 320, 8, 640, 2), 0, 0)])
def test_backward_padded_widths(gpu_lib, shape, etype, act):
    """The bf16 backward at padded widths.  A padded expert width keeps the
    MFMA backward (the padded units' gradients are zero and not stored, so
    d_experts keeps the op's [D][F] layout); a padded model width takes the
    fp32 backward kernels on the bf16 flow's values.  Against the SIMT
    backward on the same op (which shares nothing but the routing) and the
    float64 restatement."""
    from mixlab_amd.op import MoEFeedForward
    from oracle.backward import backward64

    B, T, D, E, F, K = shape
    N = B * T
    x, wr, experts = random_case(120 + etype, N, D, E, F, expert_type=etype, wscale=0.1)
    x, wr = round_bf16(x), round_bf16(wr)
    experts = [[round_bf16(w) for w in ws] for ws in experts]
    dD = np.random.default_rng(121).standard_normal((N, D), dtype=np.float32)

    def run(flags):
        with MoEFeedForward([B, T, D, E, K, etype, F, act], [0.0], compute_dtype="bf16",
                            flags=flags) as op:
            op.set_weights(bf16_bits(wr), [[bf16_bits(w) for w in ws] for ws in experts])
            out = op.backward_host(x, dD, d_aux=0.3, d_entropy=-0.2)
            return out, op.routing(), op.info()

    (dx, dwr, dexp), routing, info = run(0)
    assert info["mfma"] and info["ffn_kernel"] == _round_up(F, 128)
    (sdx, sdwr, sdexp), srouting, sinfo = run(_lib.MXM_FLAG_FORCE_SIMT)
    assert not sinfo["mfma"]
    want = run_oracle(x, wr, experts, K=K, expert_type=etype, bf16=True)
    assert_routing_equal(routing, want)
    assert_routing_equal(srouting, want)
    rdx, rdwr, rdexp = backward64(x, wr, experts, want["top_idx"].astype(np.int64), dD, 0.3, -0.2,
                                  etype, act, 0.0)
    assert rel_l2(dx, rdx) <= BF16_TOL and rel_l2(dwr, rdwr) <= BF16_TOL
    assert rel_l2(dx, sdx) <= 1e-2
    for m in range(len(experts[0])):
        assert dexp[0][m].shape == experts[0][m].shape
        got = np.concatenate([dexp[e][m].ravel() for e in range(E)])
        ref = np.concatenate([np.asarray(rdexp[e][m], np.float64).ravel() for e in range(E)])
        sim = np.concatenate([sdexp[e][m].ravel() for e in range(E)])
        print(f"  matrix {m}: rel L2 {rel_l2(got, ref):.2e} vs float64, "
              f"{rel_l2(got, sim):.2e} vs SIMT")
        assert rel_l2(got, ref) <= BF16_TOL and rel_l2(got, sim) <= 1e-2, m


def _int8_check(N, D, E, K, F, etype=0, act=0, seed=140):
    from mixlab_amd.op import MoEFeedForward

    rng = np.random.default_rng(seed)
    wpe = 2 if etype == 2 else 3
    x = round_bf16(rng.standard_normal((N, D), dtype=np.float32))
    wr = round_bf16(rng.standard_normal((D, E), dtype=np.float32) * np.float32(0.08))
    q8 = [[quantize_int8(rng.standard_normal(((F, D) if j == wpe - 1 else (D, F)),
                                             dtype=np.float32) * np.float32(0.02))
           for j in range(wpe)] for _ in range(E)]
    print(f"int8 N {N} D {D} E {E} K {K} F {F}", flush=True)
    with MoEFeedForward([1, N, D, E, K, etype, F, act], [0.0], compute_dtype="bf16",
                        flags=_lib.MXM_FLAG_INT8_WEIGHTS) as op:
        op.set_input(1, bf16_bits(wr))
        for e in range(E):
            for j in range(wpe):
                op.set_input_q8(2 + e * wpe + j, *q8[e][j])
        info = op.info()
        assert info["int8"] and info["ffn_kernel"] == _round_up(F, 64)
        delta, aux, ent = op.forward_host(bf16_bits(x))
        routing = op.routing()
    exact = [[(q.astype(np.float32) * s[None, :]).astype(np.float32) for q, s in ws] for ws in q8]
    rows = None if D * F <= 2048 * 1024 else np.arange(0, N, N // 16, dtype=np.int32)
    want = oracle.moe_forward(x, wr, exact, top_k=K, expert_type=etype, activation=act,
                              bf16=True, prerounded=True, rows=rows)
    assert_routing_equal(routing, want)
    sel = rows if rows is not None else slice(None)
    err = rel_l2(delta[sel], want["delta"][sel])
    print(f"  int8 delta rel L2 {err:.2e} vs the restatement fed q * s")
    assert err <= MFMA_TIGHT


@pytest.mark.gpu
@pytest.mark.parametrize("D,F,etype", [(2048, 5468, 0), (1024, 2734, 1), (544, 1452, 2),
                                       (2048, 2880, 0)])
def test_int8_wide_and_unaligned(gpu_lib, D, F, etype):
    """int8 experts past the old 2048 / multiple-of-64 limits: default widths
    (F = round(2.67 D)), a reduction longer than one LDS chunk of staged rows
    (the down projection over 5504 or 2880 k), and a model width that is not a
    multiple of 64 (544: x's rows padded to 576)."""
    _int8_check(N=64, D=D, E=8, K=2, F=F, etype=etype)
