"""The reference's MoE config and op-encoding surface, restated in
mixlab_amd.moe (no device).  Mirrors arch/moe_test.go:8-198 and the
validation branch arch/config_validate.go:519-556."""
from __future__ import annotations

import json

import pytest

from mixlab_amd import moe
from mixlab_amd.moe import BlockSpec, ConfigError
from tests.moe_testutil import MOE_TINY


def _block(body: str) -> BlockSpec:
    return BlockSpec.from_json(body)


def test_defaults():
    """arch/moe_test.go:8-32: top_k 2, aux weight 0.01, swiglu experts."""
    spec = _block('{"type":"moe","num_experts":4}')
    moe.validate_moe_block(spec)
    assert moe.effective_moe_top_k(spec) == 2
    assert moe.effective_moe_load_balance_loss_weight(spec) == 0.01
    assert moe.effective_moe_expert_block(spec).type == "swiglu"
    assert moe.moe_router(spec) == "linear"
    # a single expert defaults to top-1 (arch/moe.go:28-36)
    assert moe.effective_moe_top_k(_block('{"type":"moe","num_experts":1}')) == 1


def test_explicit_zero_aux_weight_disables_aux():
    """arch/config.go:229-249 presence flag: an explicit 0 stays 0."""
    spec = _block('{"type":"moe","num_experts":3,"load_balance_loss_weight":0}')
    assert spec.load_balance_loss_weight_set
    assert moe.effective_moe_load_balance_loss_weight(spec) == 0.0


@pytest.mark.parametrize("body,want", [
    ('{"type":"moe","num_experts":0}', "num_experts > 0"),
    ('{"type":"moe","num_experts":2,"top_k":3}', "invalid top_k"),
    ('{"type":"moe","num_experts":2,"router":"hash"}', "invalid router"),
    ('{"type":"moe","num_experts":2,"load_balance_loss_weight":-0.1}', "load_balance_loss_weight"),
    ('{"type":"moe","num_experts":2,"expert_block":{"type":"plain","heads":2}}', "expert_block.type"),
    ('{"type":"moe","num_experts":2,"expert_block":{"type":"mlp","activation":"bogus"}}',
     "invalid activation"),
    ('{"type":"moe","num_experts":2,"expert_block":{"type":"mlp","leaky_slope":-1}}',
     "invalid leaky_slope"),
    ('{"type":"moe","num_experts":2,"expert_block":{"type":"swiglu","weight_group":"g"}}',
     "cannot set weight_group"),
    ('{"type":"moe","num_experts":2,"expert_block":{"type":"swiglu","parallel_residual":true}}',
     "cannot set parallel_residual"),
])
def test_validation_error_substrings(body, want):
    """arch/moe_test.go:34-60 (substrings) and arch/config_validate.go:519-556."""
    with pytest.raises(ConfigError) as ei:
        moe.validate_moe_block(_block(body))
    assert want in str(ei.value)


@pytest.mark.parametrize("expert,want", [
    ('{"type":"swiglu"}', (0, 0, 0.0)),
    ('{"type":"geglu","activation":"relu"}', (1, 1, 0.0)),  # GLU kinds ignore activation
    ('{"type":"mlp"}', (2, 0, 0.0)),
    ('{"type":"mlp","activation":"gelu"}', (2, 1, 0.0)),
    ('{"type":"mlp","activation":"ReLU "}', (2, 2, 0.0)),
    ('{"type":"mlp","activation":"leaky_relu_sq"}', (2, 3, 0.5)),  # default slope
    ('{"type":"mlp","activation":"leaky_relu_sq","leaky_slope":0.25}', (2, 3, 0.25)),
])
def test_expert_type_and_activation(expert, want):
    """arch/moe.go:53-80."""
    spec = _block('{"type":"moe","num_experts":2,"expert_block":%s}' % expert)
    assert moe.moe_expert_type_and_activation(spec) == want


def test_weight_shapes_and_order():
    """arch/moe_test.go:62-84 (geglu, 4 experts, D=32, mlp_mult 2, block scales)."""
    spec = _block('{"type":"moe","num_experts":4,"top_k":2,"expert_block":{"type":"geglu"}}')
    metas = moe.moe_weight_shapes(spec, 32, 2.0, block_scales=True)
    assert len(metas) == 2 + 4 * 3 + 1
    assert metas[0].name == "moe_norm_scale" and metas[0].is_norm_scale and metas[0].init_one
    assert metas[1].name == "router_w" and metas[1].shape == [32, 4]
    assert [m.name for m in metas[2:5]] == ["expert_0_w_gate", "expert_0_w_up", "expert_0_w_down"]
    assert metas[2].shape == [32, 64] and metas[4].shape == [64, 32]
    assert metas[-1].name == "moe_scale" and metas[-1].init_one
    mlp = _block('{"type":"moe","num_experts":3,"expert_block":{"type":"mlp"}}')
    names = [m.name for m in moe.moe_weight_shapes(mlp, 16, 4.0)]
    assert names == ["moe_norm_scale", "router_w", "expert_0_w_up", "expert_0_w_down",
                     "expert_1_w_up", "expert_1_w_down", "expert_2_w_up", "expert_2_w_down"]
    assert moe.moe_weight_count(mlp) == 2 + 3 * 2


@pytest.mark.parametrize("D,mult,want", [(128, 4.0, 512), (64, 2.67, 171), (512, 4.0, 2048),
                                         (32, 0.5, 32), (10, 1.25, 13), (8, 0.0, 21)])
def test_ffn_dim(D, mult, want):
    """arch/weight_shapes.go:56-65: round half away from zero, at least D,
    non-positive multipliers use the default 2.67."""
    assert moe.ffn_dim(D, mult) == want


def test_op_encoding_and_block_emission():
    """arch/moe.go:152-213, arch/ir.go:692-698: RMSNorm, op 74, aux scaling,
    optional moe_scale, residual add."""
    spec = _block('{"type":"moe","num_experts":3,"top_k":1,"load_balance_loss_weight":0.05,'
                  '"expert_block":{"type":"mlp","activation":"leaky_relu_sq"}}')
    prog = moe.Program()
    next_wi = moe.emit_moe_ir(prog, spec, "x", 7, 16, 4, 2, 0, mlp_mult=2.0, block_scales=True)
    codes = [op.code for op in prog.ops]
    assert codes == [moe.OP_RMSNORM, moe.OP_MOE_FEED_FORWARD, moe.OP_SCALAR_MUL, moe.OP_MUL,
                     moe.OP_ADD]
    norm, ff, scal, mul, add = prog.ops
    assert norm.inputs == ["x", "w7"] and norm.float_params == [1e-5]
    assert ff.inputs == ["x_moe_0_x_norm"] + [f"w{i}" for i in range(8, 8 + 1 + 3 * 2)]
    assert ff.outputs == ["x_moe_0_delta", "x_moe_0_moe_aux_loss_raw", "x_moe_0_moe_router_entropy"]
    assert ff.int_params == [2, 4, 16, 3, 1, 2, 32, 3]  # B,T,D,E,topK,expertType,ffn,activation
    assert ff.float_params == [0.5]
    assert scal.inputs == ["x_moe_0_moe_aux_loss_raw"] and scal.float_params == [0.05]
    assert scal.outputs == ["x_moe_0_moe_aux_loss"]
    assert mul.inputs == ["x_moe_0_delta", "w15"]
    assert add.inputs == ["x", "x_moe_0_scaled"] and add.outputs == ["x"]
    assert next_wi == 16


def test_parallel_residual_member_emission():
    """arch/moe.go:168-171 (arch/parallel_residual.go:461-462): no norm and no
    residual add of its own; op 74 on the pair's normalised rows, the aux
    scaling, optional moe_scale, the delta returned under the
    `<x_norm>_parallel_moe_<idx>` prefix."""
    spec = _block('{"type":"moe","num_experts":2,"top_k":2}')
    prog = moe.Program()
    delta, next_wi = moe.emit_moe_parallel_delta_ir(prog, spec, "h_norm", 3, 16, 4, 1, 5,
                                                    mlp_mult=2.0, block_scales=True)
    codes = [op.code for op in prog.ops]
    assert codes == [moe.OP_MOE_FEED_FORWARD, moe.OP_SCALAR_MUL, moe.OP_MUL]
    ff, scal, mul = prog.ops
    assert ff.inputs == ["h_norm"] + [f"w{i}" for i in range(3, 3 + 1 + 2 * 3)]
    assert ff.outputs == ["h_norm_parallel_moe_5_delta", "h_norm_parallel_moe_5_moe_aux_loss_raw",
                          "h_norm_parallel_moe_5_moe_router_entropy"]
    assert scal.outputs == ["h_norm_parallel_moe_5_moe_aux_loss"]
    assert mul.inputs == ["h_norm_parallel_moe_5_delta", "w10"]
    assert delta == "h_norm_parallel_moe_5_scaled" and next_wi == 11
    prog2 = moe.Program()
    delta2, wi2 = moe.emit_moe_parallel_delta_ir(prog2, spec, "h_norm", 0, 16, 4, 1, 0,
                                                 mlp_mult=2.0)
    assert delta2 == "h_norm_parallel_moe_0_delta" and wi2 == 7


def test_flop_estimates():
    """arch/moe.go:215-236 counts the router and top_k active experts."""
    spec = _block('{"type":"moe","num_experts":64,"top_k":8}')
    B, T, D = 32, 2048, 2048
    F = moe.ffn_dim(D, 0.5)
    got = moe.estimate_moe_block_flops(spec, B, T, D, 0.5)
    N = B * T
    assert got == 2 * N * D * 64 + 8 * 6 * N * D * F
    assert moe.op_flops([B, T, D, 64, 8, 0, F, 0]) == got


def test_parse_round_trip():
    raw = {"type": "moe", "num_experts": 8, "top_k": 2, "expert_block": {"type": "swiglu"}}
    spec = moe.parse_moe_block(json.dumps(raw))
    assert spec.num_experts == 8 and spec.expert_block.type == "swiglu"


# ---- parallel-residual follower, residual scale init, config loading ----

def test_parallel_residual_follower_omits_norm_scale():
    """arch/moe_test.go:160-198 and arch/weight_shapes.go:498-551: the second
    block of a parallel-residual pair drops moe_norm_scale; the first keeps
    it, and the counts follow (arch/parallel_residual.go:242-264)."""
    spec = _block('{"type":"moe","num_experts":2,"top_k":1}')
    lead = moe.moe_parallel_weight_shapes(spec, False, 32)
    follow = moe.moe_parallel_weight_shapes(spec, True, 32)
    assert lead[0].name == "moe_norm_scale"
    assert "moe_norm_scale" not in [m.name for m in follow]
    assert [m.name for m in follow] == [m.name for m in lead[1:]]
    for scales in (False, True):
        assert moe.moe_parallel_weight_count(spec, True, scales) == len(
            moe.moe_parallel_weight_shapes(spec, True, 32, block_scales=scales))
        assert moe.moe_parallel_weight_count(spec, False, scales) == len(
            moe.moe_parallel_weight_shapes(spec, False, 32, block_scales=scales))
    # the follower's metas still end with moe_scale under block scales
    assert moe.moe_parallel_weight_shapes(spec, True, 32, block_scales=True)[-1].name == "moe_scale"


@pytest.mark.parametrize("body,one,zero,value", [
    ('{"type":"moe","num_experts":2}', True, False, 0.0),
    ('{"type":"moe","num_experts":2,"residual_scale_init":0}', False, True, 0.0),
    ('{"type":"moe","num_experts":2,"residual_scale_init":0.1}', False, False,
     float(__import__("numpy").float32(0.1))),
])
def test_moe_scale_follows_residual_scale_init(body, one, zero, value):
    """arch/weight_shapes.go:75-87: moe_scale inits to 1, to zero for an
    explicit 0, else to the given value as fp32."""
    meta = moe.moe_weight_shapes(_block(body), 16, block_scales=True)[-1]
    assert meta.name == "moe_scale" and meta.shape == [16]
    assert (meta.init_one, meta.init_zero, meta.init_value) == (one, zero, value)





def test_parse_model_config_moe_tiny():
    """examples/moe_tiny.json: two MoE blocks of D 64, F = ffnDim(64, 2.0) =
    128, 4 experts, top-2; 1024 tokens per step."""
    cfg = moe.parse_model_config(MOE_TINY, "moe_tiny.json")
    assert (cfg.model_dim, cfg.seq_len, cfg.batch_tokens, cfg.mlp_mult) == (64, 128, 1024, 2.0)
    blocks = [b for b in cfg.blocks if moe.block_type_key(b) == "moe"]
    assert len(blocks) == 2
    assert moe.ffn_dim(cfg.model_dim, cfg.mlp_mult) == 128
    assert [moe.effective_moe_load_balance_loss_weight(b) for b in blocks] == [0.01, 0.01]


def test_parse_model_config_rejects_unknown_top_level_field():
    """arch/config_test.go:934-943 (TestUnknownFieldRejected)."""
    bad = MOE_TINY.replace('"seq_len": 128,', '"seq_len": 128, "bogus_field": true,')
    with pytest.raises(ConfigError, match='parse config "t": json: unknown field "bogus_field"'):
        moe.parse_model_config(bad, "t")


def test_unknown_block_keys_are_ignored_like_the_reference():
    """Inside a block the reference does not reject unknown keys: BlockSpec's
    own UnmarshalJSON (arch/config.go:229-249) re-decodes with a plain
    json.Unmarshal, which the outer DisallowUnknownFields does not reach.  A
    misspelled MoE key therefore falls back to its default, as there."""
    cfg = moe.parse_model_config(MOE_TINY.replace('"top_k": 2, "expert_block": {"type": "swiglu"}}',
                                                  '"topk": 3, "expert_block": {"type": "swiglu"}}'))
    spec = cfg.blocks[3]
    assert spec.extra == {"topk": 3}
    assert moe.effective_moe_top_k(spec) == 2


def test_parse_model_config_validates_moe_blocks():
    bad = MOE_TINY.replace('"num_experts": 4, "top_k": 2, "expert_block": {"type": "swiglu"},\n'
                           '     "router": "linear"',
                           '"num_experts": 4, "top_k": 2, "expert_block": {"type": "swiglu"},\n'
                           '     "router": "hash"')
    with pytest.raises(ConfigError, match=r'blocks\[1\] type=moe has invalid router="hash"'):
        moe.parse_model_config(bad, "t")
