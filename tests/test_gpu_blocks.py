"""GPU runs of whole MoE blocks as configs and checkpoints describe them:
the reference's examples/moe_tiny.json, and an int8 block read from the
reference's quantized checkpoint format (train/export.go:203-352).  Checked
against the CPU restatement (oracle/) on the same weights."""
import numpy as np
import pytest

import oracle
from mixlab_amd import _lib, moe
from mixlab_amd.workloads import bf16_bits, round_bf16
from tests.moe_testutil import MOE_TINY, assert_routing_equal, rel_l2, same_bits

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


def _normal_weights(rng, metas):
    """weight_init "normal": N(0, 0.02) matrices, norm and residual scales 1."""
    ws = []
    for m in metas:
        if m.name in ("moe_norm_scale", "moe_scale"):
            ws.append(np.ones(m.shape, np.float32))
        else:
            ws.append(rng.standard_normal(m.shape, dtype=np.float32) * np.float32(0.02))
    return ws


@pytest.mark.parametrize("flow", ["fp32", "bf16"])
def test_moe_tiny_blocks(gpu_lib, flow):
    """Both MoE blocks of examples/moe_tiny.json (D 64, F = ffnDim(64, 2.0) =
    128, 4 experts, top-2, 1024 tokens = batch_tokens / seq_len rows of
    seq_len) through the fused block.  D = 64 is below the MFMA tiles' 128
    columns, so both flows run the exact-order SIMT kernels and match the
    restatement bit for bit."""
    from mixlab_amd.op import MoEBlock

    cfg = moe.parse_model_config(MOE_TINY, "moe_tiny.json")
    B, T, D = cfg.batch_tokens // cfg.seq_len, cfg.seq_len, cfg.model_dim
    bf16 = flow == "bf16"
    r = round_bf16 if bf16 else (lambda a: a)
    rng = np.random.default_rng(64)
    x = rng.standard_normal((B * T, D), dtype=np.float32)
    for idx, spec in enumerate(cfg.blocks):
        if moe.block_type_key(spec) != "moe":
            continue
        print(f"moe_tiny block {idx} {flow}", flush=True)
        with MoEBlock(spec, B, T, D, mlp_mult=cfg.mlp_mult, block_scales=cfg.block_scales,
                      compute_dtype=flow) as blk:
            assert not blk.op.info()["mfma"]
            ws = _normal_weights(rng, blk.metas)
            blk.set_weights(ws)
            xin = r(x)
            out, aux, ent = blk.forward_host(bf16_bits(xin) if bf16 else xin)
            routing = blk.op.routing()
        K = moe.effective_moe_top_k(spec)
        F = moe.ffn_dim(D, cfg.mlp_mult)
        assert F == 128 and K == 2
        experts = [[r(w) for w in ws[2 + 3 * e:5 + 3 * e]] for e in range(spec.num_experts)]
        want = oracle.block_forward(xin, r(ws[0]), r(ws[1]), experts, top_k=K, eps=blk.eps,
                                    aux_weight=blk.aux_weight, bf16=bf16)
        assert_routing_equal(routing, want)
        assert same_bits(out, want["x_out"])
        assert abs(aux - want["aux"]) <= 1e-6 * abs(want["aux"])
        assert abs(ent - want["entropy"]) <= 1e-5 * abs(want["entropy"])
        x = out  # the next block's input, as the stream carries it


@pytest.mark.parametrize("mode,D,mult", [("int8", 256, 2.0), ("int6", 256, 2.0),
                                         ("int8", 512, 2.67)])
def test_int8_block_from_quantized_checkpoint(gpu_lib, tmp_path, mode, D, mult):
    """An MoE block written by the reference's quantized export (per-row
    int8 / int6 matrices, F32 norm and moe_scale), read back and run on the
    int8 expert kernels.  Routing is bit-exact against the restatement fed
    the router as the file dequantises it; the delta is checked against the
    restatement fed the executor's per-channel weights and against the one
    fed the file's own per-row dequantised weights (what the reference would
    compute from this file), both within the bf16 bar.  The third case is a
    block at the reference's default expert width (mlp_mult 2.67: F =
    ffnDim(512, 2.67) = 1367, which the int8 kernels run at 1408)."""
    from mixlab_amd.op import MoEBlock
    from mixlab_amd.weights import (QuantizedWeight, export_safetensors_quantized,
                                    load_quantized_weights)

    spec = moe.BlockSpec.from_json('{"type":"moe","num_experts":6,"top_k":2,'
                                   '"residual_scale_init":0.5}')
    B, T = 1, 64
    rng = np.random.default_rng(77)
    with MoEBlock(spec, B, T, D, mlp_mult=mult, block_scales=True, compute_dtype="bf16",
                  flags=_lib.MXM_FLAG_INT8_WEIGHTS) as blk:
        ws = _normal_weights(rng, blk.metas)
        ws[1] = ws[1] * np.float32(4.0)  # a router with some spread
        ws[-1] = np.full(D, 0.5, np.float32)
        path = str(tmp_path / "q.safetensors")
        export_safetensors_quantized(path, blk.metas, ws, mode, first_index=3)
        blk.load_quantized(path, first_index=3)
        info = blk.op.info()
        assert info["int8"] and info["ffn_kernel"] == (moe.ffn_dim(D, mult) + 63) // 64 * 64
        x = round_bf16(rng.standard_normal((B * T, D), dtype=np.float32))
        out, aux, ent = blk.forward_host(bf16_bits(x))
        routing = blk.op.routing()
    got = load_quantized_weights(path, blk.metas, first_index=3)
    assert isinstance(got[1], QuantizedWeight) and isinstance(got[2], QuantizedWeight)
    router = round_bf16(got[1].dequantize())
    ns, ms = round_bf16(got[0]), round_bf16(got[-1])
    n_exp = spec.num_experts
    per_channel = []
    per_row = []
    for e in range(n_exp):
        mats = got[2 + 3 * e:5 + 3 * e]
        per_channel.append([round_bf16(q.astype(np.float32) * s[None, :])
                            for q, s in (m.per_channel() for m in mats)])
        per_row.append([round_bf16(m.dequantize()) for m in mats])
    want = oracle.block_forward(x, ns, router, per_channel, top_k=2, moe_scale=ms, eps=blk.eps,
                                aux_weight=blk.aux_weight, bf16=True)
    assert_routing_equal(routing, want)
    err_exec = rel_l2(out - x, want["x_out"] - x)
    want_rows = oracle.block_forward(x, ns, router, per_row, top_k=2, moe_scale=ms, eps=blk.eps,
                                     aux_weight=blk.aux_weight, bf16=True)
    err_file = rel_l2(out - x, want_rows["x_out"] - x)
    print(f"{mode}: delta rel L2 {err_exec:.3e} vs executor weights, {err_file:.3e} vs file")
    assert err_exec <= BF16_TOL and err_file <= BF16_TOL
    assert abs(aux - want["aux"]) <= 1e-2 * abs(want["aux"])
