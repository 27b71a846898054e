"""Helpers shared by the parity tests: run one op on the GPU through the C ABI
and compare with the CPU restatement in oracle/."""
from __future__ import annotations

import numpy as np

import oracle
from mixlab_amd import _lib
from mixlab_amd.workloads import bf16_bits


# examples/moe_tiny.json of the reference (two MoE blocks: D 64, mlp_mult 2.0,
# 4 experts, top-2; 1024 tokens per step), with one JSONC comment added
MOE_TINY = """{
  "name": "moe-tiny",
  "model_dim": 64,
  "vocab_size": 1024,
  "seq_len": 128,
  "mlp_mult": 2.0,
  // a JSONC comment, as stripJSONComments allows
  "blocks": [
    {"type": "plain", "heads": 4},
    {"type": "moe", "num_experts": 4, "top_k": 2, "expert_block": {"type": "swiglu"},
     "router": "linear", "load_balance_loss_weight": 0.01},
    {"type": "plain", "heads": 4},
    {"type": "moe", "num_experts": 4, "top_k": 2, "expert_block": {"type": "swiglu"}}
  ],
  "training": {"steps": 200, "lr": 0.0003, "batch_tokens": 1024, "grad_clip": 1.0,
               "weight_decay": 0.01}
}"""


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def run_gpu(x, router_w, experts, *, B, T, K, expert_type=0, activation=0, slope=0.0,
            bf16=False, flags=0, want_probs=False):
    """One op-74 forward through libmixmoe.  Inputs are fp32 arrays (values
    already bf16-representable in the bf16 flow); bf16 runs upload bit
    patterns.  Returns (delta, aux, entropy, routing dict, info dict)."""
    from mixlab_amd.op import MoEFeedForward

    N, D = x.shape
    E = router_w.shape[1]
    F = experts[0][0].shape[1]
    ip = [B, T, D, E, K, expert_type, F, activation]
    if want_probs:
        flags |= _lib.MXM_FLAG_DEBUG_PROBS
    conv = bf16_bits if bf16 else (lambda a: np.ascontiguousarray(a, np.float32))
    with MoEFeedForward(ip, [slope], compute_dtype="bf16" if bf16 else "fp32", flags=flags) as op:
        op.set_weights(conv(router_w), [[conv(w) for w in ws] for ws in experts])
        delta, aux, ent = op.forward_host(conv(x))
        routing = op.routing()
        if want_probs:
            routing["probs"] = op.probs()
        info = op.info()
    return delta, aux, ent, routing, info


def run_oracle(x, router_w, experts, *, K, expert_type=0, activation=0, slope=0.0, bf16=False,
               rows=None):
    return oracle.moe_forward(x, router_w, experts, top_k=K, expert_type=expert_type,
                              activation=activation, leaky_slope=slope, bf16=bf16, rows=rows)


def assert_routing_equal(got: dict, want: dict) -> None:
    np.testing.assert_array_equal(got["top_idx"], want["top_idx"])
    assert same_bits(got["gates"], want["gates"]), "gates differ bitwise"
    np.testing.assert_array_equal(got["counts"], want["counts"])
    np.testing.assert_array_equal(got["offsets"], want["offsets"])
    np.testing.assert_array_equal(got["perm"], want["perm"])


def random_case(seed, N, D, E, F, expert_type=0, wscale=0.02):
    rng = np.random.default_rng(seed)
    wpe = 2 if expert_type == 2 else 3
    x = rng.standard_normal((N, D), dtype=np.float32)
    wr = rng.standard_normal((D, E), dtype=np.float32) * np.float32(wscale * 4)
    experts = []
    for _ in range(E):
        experts.append([rng.standard_normal(((F, D) if j == wpe - 1 else (D, F)), dtype=np.float32)
                        * np.float32(wscale) for j in range(wpe)])
    return x, wr, experts


def run_gpu_workload(w, flags=0):
    """Forward of a generated Workload, uploading its stored bits directly
    (int8 configurations upload q and the per-output-channel scales)."""
    from mixlab_amd.op import MoEFeedForward

    cfg = w.cfg
    if cfg.int8_weights:
        flags |= _lib.MXM_FLAG_INT8_WEIGHTS
    with MoEFeedForward(cfg.int_params, [cfg.leaky_slope], compute_dtype=cfg.dtype,
                        flags=flags) as op:
        op.set_input(1, w.router_upload())
        idx = 2
        for e in range(cfg.E):
            for j in range(cfg.wpe):
                if cfg.int8_weights:
                    q, sc = w.q8[e][j]
                    op.set_input_q8(idx, q, sc)
                else:
                    op.set_input(idx, w.matrix_upload(e, j))
                idx += 1
        delta, aux, ent = op.forward_host(w.x_upload())
        routing = op.routing()
        info = op.info()
    return delta, aux, ent, routing, info


def run_oracle_workload(w, rows=None):
    cfg = w.cfg
    return oracle.moe_forward(w.x, w.router_w, w.packed_f32(), top_k=cfg.K,
                              expert_type=cfg.expert_type, activation=cfg.activation,
                              leaky_slope=cfg.leaky_slope, bf16=cfg.dtype == "bf16", rows=rows,
                              prerounded=True)
