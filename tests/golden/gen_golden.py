"""Write tests/golden/moe_known_answer.json: float64 expected outputs of op 74.

The reference keeps no stored vectors for this path; its known-answer
procedure is gpu/moe_feed_forward_test.go:14-82: patternedFloats inputs
(gpu/hgrn2_mlstm_scan_test.go:288-294), B=1, T=4, D=3, E=3, FFN=4, top_k in
{1, 2}, sigmoid-GLU experts, compared with a CPU oracle
(cpuMoESwiGLU, gpu/moe_feed_forward_test.go:188-240) at L_inf <= 2e-5.  This
script restates that procedure in float64 with numpy, independently of the
C restatement in oracle/, and extends it to the other expert types of
gpu/ir.cpp:1053-1148 (geglu with the tanh gelu, mlp with silu / gelu / relu /
leaky_relu_sq) and to a tie case and a wider case.  The top-k order is a
stable sort on descending probability (ties to the lower expert), as
sort.SliceStable in train/export_hf_ffn_oracle_test.go:40-42.

    python tests/golden/gen_golden.py        # rewrites the JSON fixture
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "moe_known_answer.json"


def patterned_floats(n: int, scale: float) -> np.ndarray:
    """gpu/hgrn2_mlstm_scan_test.go:288-294, rounded to float32 like the Go code."""
    return np.array([np.float32(scale * (math.sin(i + 1) * 0.7 + math.cos((i + 3) % 11) * 0.3))
                     for i in range(n)], dtype=np.float32)


def sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


def gelu_tanh(v):
    # gpu/ir.cpp:1054-1056
    return 0.5 * v * (1.0 + np.tanh(0.7978845608 * (v + 0.044715 * v * v * v)))


def activation(v, act: int, slope: float):
    # gpu/ir.cpp:1053-1071
    if act == 0:
        return v * sigmoid(v)
    if act == 1:
        return gelu_tanh(v)
    if act == 2:
        return np.maximum(v, 0.0)
    y = np.where(v > 0, v, v * slope)
    return y * y


def forward64(x, wr, experts, K: int, etype: int, act: int, slope: float) -> dict:
    """Op 74 in float64 (gpu/ir.cpp:1106-1162), sparse over the top-k experts."""
    x = x.astype(np.float64)
    wr = wr.astype(np.float64)
    N, D = x.shape
    E = wr.shape[1]
    logits = x @ wr
    m = logits.max(axis=1, keepdims=True)
    ex = np.exp(logits - m)
    probs = ex / ex.sum(axis=1, keepdims=True)
    top_idx = np.zeros((N, K), np.int64)
    gates = np.zeros((N, K))
    delta = np.zeros((N, D))
    for n in range(N):
        order = sorted(range(E), key=lambda e: -probs[n, e])  # stable: ties keep e order
        sel = order[:K]
        den = max(sum(probs[n, e] for e in sel), 1e-12)
        for k, e in enumerate(sel):
            top_idx[n, k] = e
            gates[n, k] = probs[n, e] / den
            ws = [w.astype(np.float64) for w in experts[e]]
            if etype in (0, 1):
                g = x[n] @ ws[0]
                u = x[n] @ ws[1]
                h = (sigmoid(g) if etype == 0 else gelu_tanh(g)) * u
                y = h @ ws[2]
            else:
                y = activation(x[n] @ ws[0], act, slope) @ ws[1]
            delta[n] += gates[n, k] * y
    counts = np.bincount(top_idx.ravel(), minlength=E)
    aux = E * sum(probs[:, e].mean() * (counts[e] / K) / N for e in range(E))
    ent = -np.mean(np.sum(probs * np.log(np.maximum(probs, 1e-12)), axis=1))
    return dict(delta=delta, aux=float(aux), entropy=float(ent), top_idx=top_idx, gates=gates,
                counts=counts, probs=probs)


def make_case(name, B, T, D, E, K, F, etype=0, act=0, slope=0.0, tie_cols=None, gain=1.0):
    """patternedFloats inputs in the layout of gpu/moe_feed_forward_test.go:29-38
    (gain > 1 scales x so the projections reach the activations' curved and
    negative ranges)."""
    x = patterned_floats(B * T * D, 0.17 * gain).reshape(B * T, D)
    wr = patterned_floats(D * E, 0.23).reshape(D, E)
    if tie_cols is not None:
        a, b = tie_cols
        wr[:, b] = wr[:, a]
    experts = []
    for e in range(E):
        gate = patterned_floats(D * F, 0.09 + e * 0.03).reshape(D, F)
        up = patterned_floats(D * F, 0.11 + e * 0.03).reshape(D, F)
        down = patterned_floats(F * D, 0.13 + e * 0.03).reshape(F, D)
        experts.append([gate, up, down] if etype in (0, 1) else [up, down])
    want = forward64(x, wr, experts, K, etype, act, slope)
    return {
        "name": name,
        "int_params": [B, T, D, E, K, etype, F, act],
        "float_params": [slope],
        "x": x.tolist(),
        "router_w": wr.tolist(),
        "experts": [[w.tolist() for w in ws] for ws in experts],
        "want": {
            "delta": want["delta"].tolist(),
            "aux": want["aux"],
            "entropy": want["entropy"],
            "top_idx": want["top_idx"].tolist(),
            "gates": want["gates"].tolist(),
            "counts": want["counts"].tolist(),
        },
    }


def main() -> None:
    cases = [
        # the reference's own known-answer case (gpu/moe_feed_forward_test.go:19-27)
        make_case("known_answer_swiglu_k1", 1, 4, 3, 3, 1, 4),
        make_case("known_answer_swiglu_k2", 1, 4, 3, 3, 2, 4),
        # the same procedure over the other expert kinds of gpu/ir.cpp:1126-1145
        make_case("known_answer_geglu_k2", 1, 4, 3, 3, 2, 4, etype=1, act=1),
        make_case("known_answer_mlp_silu_k2", 1, 4, 3, 3, 2, 4, etype=2, act=0),
        make_case("known_answer_mlp_gelu_k2", 1, 4, 3, 3, 2, 4, etype=2, act=1),
        make_case("known_answer_mlp_relu_k2", 1, 4, 3, 3, 2, 4, etype=2, act=2),
        make_case("known_answer_mlp_leaky_relu_sq_k2", 1, 4, 3, 3, 2, 4, etype=2, act=3, slope=0.5),
        # two experts with identical router columns: ties go to the lower index
        make_case("tie_columns_k2", 1, 6, 5, 4, 2, 6, tie_cols=(1, 3)),
        # wider: several row blocks, K=3 of E=8
        make_case("wide_swiglu_k3", 2, 8, 16, 8, 3, 24),
        # larger activations (|projection| up to a few units)
        make_case("large_swiglu_k2", 1, 8, 8, 4, 2, 8, gain=12.0),
        make_case("large_geglu_k2", 1, 8, 8, 4, 2, 8, etype=1, act=1, gain=12.0),
        make_case("large_mlp_gelu_k2", 1, 8, 8, 4, 2, 8, etype=2, act=1, gain=12.0),
        make_case("large_mlp_relu_k2", 1, 8, 8, 4, 2, 8, etype=2, act=2, gain=12.0),
        make_case("large_mlp_leaky_relu_sq_k2", 1, 8, 8, 4, 2, 8, etype=2, act=3, slope=0.3,
                  gain=12.0),
    ]
    OUT.write_text(json.dumps({
        "source": "tests/golden/gen_golden.py (float64 restatement of the "
                  "gpu/moe_feed_forward_test.go:14-82 procedure)",
        "cases": cases,
    }, separators=(",", ":")))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(cases)} cases)")


if __name__ == "__main__":
    main()
