"""Weight I/O on either side of op 74 (no GPU): the native checkpoint format
of train/export.go:20-80 / train/import.go:20-146, the int8 conversions, and
the aux / entropy aggregation of arch/loss_emit.go:244-303."""
from __future__ import annotations

import numpy as np
import pytest

from mixlab_amd import moe
from mixlab_amd.weights import (CheckpointError, checkpoint_name, dequantize_per_row,
                                export_safetensors, load_safetensors, load_weights,
                                per_row_to_per_channel, quantize_per_channel)


def _metas(block_scales=True):
    spec = moe.BlockSpec.from_json('{"type":"moe","num_experts":3,"top_k":2}')
    return moe.moe_weight_shapes(spec, 16, 2.0, block_scales)


def _weights(metas, seed=0):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal(m.shape, dtype=np.float32) for m in metas]


def test_checkpoint_round_trip(tmp_path):
    metas = _metas()
    w = _weights(metas)
    path = str(tmp_path / "block.safetensors")
    export_safetensors(path, metas, w, {"name": "t"}, first_index=5)
    got = load_weights(path, metas, first_index=5)
    for a, b in zip(got, w):
        np.testing.assert_array_equal(a, b)
    names = set(load_safetensors(path))
    assert checkpoint_name(5, "moe_norm_scale") == "w5_moe_norm_scale"
    assert names == {f"w{5 + i}_{m.name}" for i, m in enumerate(metas)}


def test_checkpoint_is_standard_safetensors(tmp_path):
    """A file the safetensors library reads back with the same names,
    values and metadata."""
    from safetensors import safe_open

    metas = _metas(False)
    w = _weights(metas, 1)
    path = str(tmp_path / "b.safetensors")
    export_safetensors(path, metas, w)
    with safe_open(path, framework="numpy") as f:
        assert f.metadata()["format"] == "mixlab_v1"
        for i, m in enumerate(metas):
            np.testing.assert_array_equal(f.get_tensor(f"w{i}_{m.name}"), w[i])


def test_checkpoint_errors(tmp_path):
    """train/import_test.go:76-175 cases and the checks of decode."""
    with pytest.raises(CheckpointError):
        load_safetensors(str(tmp_path / "nonexistent.safetensors"))
    for name, data in (("empty", b""), ("small", bytes([1, 2, 3]))):
        p = tmp_path / f"{name}.safetensors"
        p.write_bytes(data)
        with pytest.raises(CheckpointError, match="too small"):
            load_safetensors(str(p))
    p = tmp_path / "long.safetensors"
    p.write_bytes((1000).to_bytes(8, "little") + b"{}")
    with pytest.raises(CheckpointError, match="exceeds file size"):
        load_safetensors(str(p))
    metas = _metas(False)
    path = str(tmp_path / "w.safetensors")
    export_safetensors(path, metas, _weights(metas))
    extra = list(metas) + [moe.WeightMeta("extra", [16])]
    with pytest.raises(CheckpointError, match='missing tensor "w11_extra"'):
        load_weights(path, extra)
    bad = list(metas)
    bad[1] = moe.WeightMeta("router_w", [16, 4])
    with pytest.raises(CheckpointError, match="shape mismatch"):
        load_weights(path, bad)
    from safetensors.numpy import save_file
    p16 = str(tmp_path / "f16.safetensors")
    save_file({"w0_moe_norm_scale": np.ones(16, np.float16)}, p16)
    with pytest.raises(CheckpointError, match="only F32"):
        load_weights(p16, metas[:1])


def test_quantize_per_channel():
    rng = np.random.default_rng(2)
    w = rng.standard_normal((64, 48), dtype=np.float32)
    w[:, 7] = 0.0
    q, s = quantize_per_channel(w)
    assert q.dtype == np.int8 and s.shape == (48,)
    assert q.min() >= -127 and q.max() <= 127
    assert s[7] == 1.0 and not q[:, 7].any()
    assert np.all(np.abs(q.astype(np.float32) * s - w) <= s / 2 + 1e-7)
    np.testing.assert_array_equal(np.abs(q).max(axis=0)[np.arange(48) != 7], 127)


def test_per_row_to_per_channel():
    """The reference exports per input row (train/quantize.go:99-118); the
    conversion dequantises (DequantizePerRow) and requantises per column."""
    rng = np.random.default_rng(3)
    q_rows = rng.integers(-127, 128, size=(32, 24), dtype=np.int64).astype(np.int8)
    row_s = rng.uniform(0.01, 0.05, 32).astype(np.float32)
    w = dequantize_per_row(q_rows, row_s)
    assert w[3, 5] == np.float32(q_rows[3, 5]) * row_s[3]
    q, s = per_row_to_per_channel(q_rows, row_s)
    assert np.all(np.abs(q.astype(np.float32) * s - w) <= s / 2 + 1e-7)


def test_aux_entropy_aggregation():
    """arch/loss_emit.go:244-303 over a program with two MoE blocks."""
    spec = moe.BlockSpec.from_json('{"type":"moe","num_experts":4,"top_k":2}')
    prog = moe.Program()
    wi = moe.emit_moe_ir(prog, spec, "x", 0, 16, 4, 1, 0, mlp_mult=2.0)
    moe.emit_moe_ir(prog, spec, "x", wi, 16, 4, 1, 1, mlp_mult=2.0)
    aux, ent = moe.collect_moe_auxiliary_outputs(prog)
    assert aux == ["x_moe_0_moe_aux_loss", "x_moe_1_moe_aux_loss"]
    assert ent == ["x_moe_0_moe_router_entropy", "x_moe_1_moe_router_entropy"]
    start = len(prog.ops)
    assert moe.emit_moe_auxiliary_aggregates_ir(prog, task_loss_has_eval_loss=False)
    outs = [op.outputs[0] for op in prog.ops[start:]]
    assert outs == ["eval_loss", "task_loss", "moe_aux_accum_1", "moe_aux_loss",
                    "moe_entropy_accum_1", "moe_router_entropy", "loss"]
    vals = {"loss": 2.5, aux[0]: 0.011, aux[1]: 0.013, ent[0]: 1.2, ent[1]: 1.3}
    moe.evaluate_scalar_ops(prog, vals, start)
    f = np.float32
    assert vals["moe_aux_loss"] == float(f(0.011) + f(0.013))
    assert vals["moe_router_entropy"] == float((f(1.2) + f(1.3)) * f(0.5))
    assert vals["loss"] == float(f(2.5) + f(vals["moe_aux_loss"]))
    # no MoE block: nothing emitted
    assert not moe.emit_moe_auxiliary_aggregates_ir(moe.Program(), False)


# ---- HF export names (train/export_hf.go:544-604) ----

def _moe_metas(expert_type="swiglu", E=2, D=8):
    from mixlab_amd.weights import moe_block_metas
    spec = moe.BlockSpec(type="moe", num_experts=E, top_k=min(2, E),
                         expert_block=moe.BlockSpec(type=expert_type))
    return spec, moe_block_metas(spec, D, 4.0)


@pytest.mark.parametrize("expert_type,kinds", [("swiglu", ("gate", "up", "down")),
                                               ("geglu", ("gate", "up", "down")),
                                               ("mlp", ("up", "down"))])
def test_hf_moe_names(expert_type, kinds):
    from mixlab_amd.weights import hf_moe_weight_map
    spec, metas = _moe_metas(expert_type)
    got = hf_moe_weight_map(4, spec, metas, first_index=10)
    want_hf = ["blocks.4.norm.weight", "blocks.4.router_w"] + [
        f"blocks.4.experts.{e}.w_{k}.weight" for e in range(2) for k in kinds]
    assert [g[1] for g in got] == want_hf
    assert [g[0] for g in got] == [f"w{10 + i}_{m.name}" for i, m in enumerate(metas)]
    assert [g[2] for g in got] == [list(m.shape) for m in metas]


def test_hf_moe_default_expert_is_swiglu():
    from mixlab_amd.weights import hf_moe_weight_map, moe_block_metas
    spec = moe.BlockSpec(type="moe", num_experts=1, top_k=1)
    got = hf_moe_weight_map(0, spec, moe_block_metas(spec, 8, 4.0))
    assert got[2][1] == "blocks.0.experts.0.w_gate.weight"


def test_hf_moe_errors():
    from mixlab_amd.weights import hf_moe_weight_map
    spec, metas = _moe_metas("swiglu")
    with pytest.raises(CheckpointError, match="weight map exhausted while mapping moe block 1 expert 1"):
        hf_moe_weight_map(1, spec, metas[:-1])
    with pytest.raises(CheckpointError, match="weight map exhausted while mapping moe block 1$"):
        hf_moe_weight_map(1, spec, metas[:1])
    swapped = [metas[1], metas[0]] + list(metas[2:])
    with pytest.raises(CheckpointError, match="expected Mixlab weight 'moe_norm_scale' at index 3, got 'router_w'"):
        hf_moe_weight_map(1, spec, swapped, first_index=3)
    bad = moe.BlockSpec(type="moe", num_experts=1, top_k=1, expert_block=moe.BlockSpec(type="conv"))
    with pytest.raises(CheckpointError, match="unsupported HF export moe expert type 'conv'"):
        hf_moe_weight_map(0, bad, metas)
    # block scales: moe_scale has no HF name, so the map stops short of the
    # block's metas and the export fails (train/export_hf.go:733-735)
    scaled = moe.moe_weight_shapes(spec, 8, 4.0, block_scales=True)
    assert scaled[-1].name == "moe_scale"
    with pytest.raises(CheckpointError, match="did not consume all weights: next_unmapped=10 "
                                              "total=11"):
        hf_moe_weight_map(0, spec, scaled, first_index=2)


def test_hf_export_round_trip(tmp_path):
    from mixlab_amd.weights import export_hf_safetensors, hf_moe_weight_map, load_safetensors
    spec, metas = _moe_metas("mlp", E=3)
    rng = np.random.default_rng(3)
    ws = [rng.standard_normal(m.shape).astype(np.float32) for m in metas]
    mapping = hf_moe_weight_map(2, spec, metas)
    path = str(tmp_path / "hf.safetensors")
    export_hf_safetensors(path, mapping, ws, {"name": "t", "model_dim": "8"})
    tensors = load_safetensors(path)
    for (_, hf, shape), w in zip(mapping, ws):
        assert tensors[hf].dtype == "F32" and tensors[hf].shape == shape
        np.testing.assert_array_equal(np.frombuffer(tensors[hf].data, "<f4").reshape(shape), w)
    with open(path, "rb") as f:
        import json, struct
        n = struct.unpack("<Q", f.read(8))[0]
        meta = json.loads(f.read(n))["__metadata__"]
    assert meta == {"format": "pt", "name": "t", "model_dim": "8"}


def test_training_step_outputs_and_component_losses():
    """gpu/ir_trainer.cpp:1540-1585: the loss first, then the captured scalars
    the program writes; the telemetry's component_losses carries
    moe_aux_loss only when the graph has it."""
    spec = moe.BlockSpec.from_json('{"type":"moe","num_experts":4,"top_k":2}')
    prog = moe.Program()
    assert moe.training_step_output_names(prog) == ["loss"]
    wi = moe.emit_moe_ir(prog, spec, "x", 0, 16, 4, 1, 0, mlp_mult=2.0)
    moe.emit_moe_ir(prog, spec, "x", wi, 16, 4, 1, 1, mlp_mult=2.0)
    assert moe.training_step_output_names(prog) == ["loss"]  # per-block names only so far
    assert moe.emit_moe_auxiliary_aggregates_ir(prog, task_loss_has_eval_loss=False)
    assert moe.training_step_output_names(prog) == ["loss", "moe_aux_loss", "moe_router_entropy"]
    assert moe.training_step_output_names(prog, "total") == ["total", "moe_aux_loss",
                                                             "moe_router_entropy"]
    assert moe.moe_component_losses({"loss": 1.0}) == {}
    assert moe.moe_component_losses({"moe_aux_loss": np.float32(0.25)}) == {"moe_aux_loss": 0.25}
