"""CPU restatement of mixlab's MoE feed-forward op (IR op 74).

TEST INFRASTRUCTURE ONLY: the checker for libmixmoe.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this package;
the product path (mixlab_amd) never does.

``moe_forward`` wraps oracle/moe_oracle.c (a plain-C restatement of
gpu/ir.cpp:1073-1164, built by oracle/Makefile).  ``dense_blas`` in
oracle/dense_blas.py restates the same dense algorithm with numpy/BLAS in
fp32 and serves as the timed CPU baseline.

Parity pins (see tests/test_oracle.py):
  * the reference's known-answer procedure gpu/moe_feed_forward_test.go:14-82
    (patternedFloats inputs, K in {1, 2}, L_inf <= 2e-5) against float64
    fixtures in tests/golden/;
  * the float64 export oracle train/export_hf_ffn_oracle_test.go:9-108
    (geglu and mlp leaky_relu_sq cases) against the same fixtures;
  * closed forms: K = E (dense softmax mixture), K = 1 (argmax, gate 1),
    E = K = 1 (plain sigmoid-GLU FFN), tie order of a stable argsort;
  * exp within 2 ulp of the correctly rounded value on a dense sweep;
  * dense (every expert on every row) == sparse bit for bit;
  * the bf16 dtype flow step by step (tests/test_oracle_bf16.py): bf16 logits
    and probabilities against float64 dot products and softmax, top-k against
    a lexsort of the bf16 probabilities, gates against the bf16 top-p sum,
    aux against the bf16 per-expert means, entropy over the bf16
    probabilities, each expert kind's activation against float64 rounded at
    the flow's rounding points, and the delta against a float64 restatement
    of the flow -- each shown to reject a planted slip (build_planted).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libmoe_oracle.so"

_libs: dict = {}


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def build_planted(plant: str, outdir) -> Path:
    """Compile a copy of the restatement with one planted mistake
    (ORACLE_PLANT_<plant>, see the list at the top of moe_oracle.c) into
    outdir; the tests use it to show that a pin rejects that mistake."""
    out = Path(outdir) / f"libmoe_oracle_plant_{plant.lower()}.so"
    cmd = ["gcc", "-O2", "-mfma", "-mavx2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
           "-fPIC", "-std=c11", "-shared", f"-DORACLE_PLANT_{plant.upper()}",
           "-o", str(out), str(HERE / "moe_oracle.c"), "-lm"]
    subprocess.run(cmd, check=True)
    return out


def _load(path=None):
    path = str(LIB_PATH if path is None else path)
    if path not in _libs:
        if path == str(LIB_PATH) and not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(path)
        f32p = ctypes.POINTER(ctypes.c_float)
        i32p = ctypes.POINTER(ctypes.c_int32)
        lib.oracle_moe_forward.restype = ctypes.c_int
        lib.oracle_moe_forward.argtypes = [
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int,
            f32p, f32p, f32p, i32p, ctypes.c_int, f32p, f32p, f32p, i32p, f32p, f32p, f32p,
            i32p, i32p, i32p,
        ]
        lib.oracle_exp.restype = ctypes.c_float
        lib.oracle_exp.argtypes = [ctypes.c_float]
        lib.oracle_round_bf16.restype = ctypes.c_float
        lib.oracle_round_bf16.argtypes = [ctypes.c_float]
        lib.oracle_exp_array.argtypes = [f32p, f32p, ctypes.c_int64]
        lib.oracle_round_bf16_array.argtypes = [f32p, f32p, ctypes.c_int64]
        lib.oracle_rmsnorm.argtypes = [ctypes.c_int, ctypes.c_int, f32p, f32p, ctypes.c_float,
                                       ctypes.c_int, f32p]
        lib.oracle_hidden_array.argtypes = [
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, f32p, f32p, f32p,
            ctypes.c_int64,
        ]
        _libs[path] = lib
    return _libs[path]


def _p(a, ctype=ctypes.c_float):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def round_bf16(a: np.ndarray) -> np.ndarray:
    """Round fp32 values to the nearest bf16 (ties to even), returned as fp32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    r = (u >> 16) & np.uint32(1)
    r += u
    r += np.uint32(0x7FFF)
    r &= np.uint32(0xFFFF0000)
    nan = np.isnan(a)
    if nan.any():
        r[nan] = (u[nan] | np.uint32(0x00400000)) & np.uint32(0xFFFF0000)
    return r.view(np.float32)


def to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) of fp32 values after round_bf16."""
    return (round_bf16(a).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def exp(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    _load().oracle_exp_array(_p(x), _p(y), x.size)
    return y


def hidden(bf16: bool, expert_type: int, activation: int, slope: float, g, u,
           lib=None) -> np.ndarray:
    """Hidden unit act(g, u) of gpu/ir.cpp:1130-1145 elementwise; g and u are
    the projections (bf16 values in the bf16 flow).  lib: a planted build."""
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    h = np.empty_like(u)
    _load(lib).oracle_hidden_array(int(bf16), expert_type, activation, slope, _p(g), _p(u), _p(h), u.size)
    return h


def pack_experts(expert_weights) -> np.ndarray:
    """Concatenate per-expert matrices [[w_gate, w_up, w_down] or [w_up, w_down], ...]."""
    return np.ascontiguousarray(
        np.concatenate([np.ascontiguousarray(w, dtype=np.float32).ravel()
                        for ws in expert_weights for w in ws]), dtype=np.float32)


def moe_forward(x, router_w, expert_weights, *, top_k: int, expert_type: int = 0,
                activation: int = 0, leaky_slope: float = 0.0, bf16: bool = False,
                dense: bool = False, rows=None, want_delta: bool = True,
                prerounded: bool = False, lib=None) -> dict:
    """Run the restatement.  x [N, D]; router_w [D, E]; expert_weights as in
    pack_experts (or already packed).  In the bf16 flow inputs are rounded to
    bf16 here.  Returns delta, aux, entropy, top_idx, gates, probs, logits,
    counts, offsets, perm (numpy arrays).  lib: a planted build (tests)."""
    lib = _load(lib)
    x = np.ascontiguousarray(x, dtype=np.float32)
    router_w = np.ascontiguousarray(router_w, dtype=np.float32)
    N, D = x.shape
    E = router_w.shape[1]
    if isinstance(expert_weights, np.ndarray) and expert_weights.ndim == 1:
        packed = np.ascontiguousarray(expert_weights, dtype=np.float32)
    else:
        packed = pack_experts(expert_weights)
    wpe = 2 if expert_type == 2 else 3
    F = packed.size // (E * wpe * D)
    if F * E * wpe * D != packed.size:
        raise ValueError("expert weight sizes do not match D, E and the expert type")
    if bf16 and not prerounded:
        x, router_w, packed = round_bf16(x), round_bf16(router_w), round_bf16(packed)
    K = top_k
    delta = np.zeros((N, D), np.float32) if want_delta else None
    aux = np.zeros(1, np.float32)
    ent = np.zeros(1, np.float32)
    top_idx = np.zeros((N, K), np.int32)
    gates = np.zeros((N, K), np.float32)
    probs = np.zeros((N, E), np.float32)
    logits = np.zeros((N, E), np.float32)
    counts = np.zeros(E, np.int32)
    offsets = np.zeros(E + 1, np.int32)
    perm = np.zeros(N * K, np.int32)
    rows_arr = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    rc = lib.oracle_moe_forward(
        N, D, E, K, expert_type, F, activation, leaky_slope, int(bf16), int(dense),
        _p(x), _p(router_w), _p(packed), _p(rows_arr, ctypes.c_int32),
        0 if rows_arr is None else rows_arr.size, _p(delta), _p(aux), _p(ent),
        _p(top_idx, ctypes.c_int32), _p(gates), _p(probs), _p(logits),
        _p(counts, ctypes.c_int32), _p(offsets, ctypes.c_int32), _p(perm, ctypes.c_int32))
    if rc != 0:
        raise ValueError("oracle_moe_forward: invalid arguments")
    return dict(delta=delta, aux=float(aux[0]), entropy=float(ent[0]), top_idx=top_idx,
                gates=gates, probs=probs, logits=logits, counts=counts, offsets=offsets,
                perm=perm)


def rmsnorm(x, scale, eps: float = 1e-5, out_bf16: bool = False) -> np.ndarray:
    """RMSNorm of gpu/ir.cpp:4949-4960 in the fixed summation order of
    oracle_rmsnorm.  x [N, D] and scale [D] hold the input values (bf16
    inputs as their exact fp32 values); the result is fp32, rounded to bf16
    values when out_bf16."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    N, D = x.shape
    out = np.empty_like(x)
    _load().oracle_rmsnorm(N, D, _p(x), _p(scale), eps, int(out_bf16), _p(out))
    return out


def block_forward(x, norm_scale, router_w, expert_weights, *, top_k: int,
                  moe_scale=None, eps: float = 1e-5, aux_weight: float = 0.01,
                  bf16: bool = False, **kw) -> dict:
    """The MoE block of arch/moe.go:152-213: xn = RMSNorm(x), op 74 on xn
    (moe_forward), delta *= moe_scale, x_out = x + delta (fp32), aux scaled by
    aux_weight.  x, norm_scale and moe_scale hold the input values (round
    them to bf16 first for the bf16 flow)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    xn = rmsnorm(x, norm_scale, eps, out_bf16=bf16)
    res = moe_forward(xn, router_w, expert_weights, top_k=top_k, bf16=bf16, **kw)
    delta = res["delta"]
    if moe_scale is not None:
        delta = delta * np.asarray(moe_scale, dtype=np.float32)[None, :]
    res["xn"] = xn
    res["aux_raw"] = res["aux"]
    res["aux"] = float(np.float32(res["aux"]) * np.float32(aux_weight))
    res["x_out"] = (x + delta).astype(np.float32)
    return res


def num_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
