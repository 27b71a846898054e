"""mixlab's MoE block surface: config fields, defaults, validation, weight
shapes, op-74 encoding and FLOP estimate.

The reference implements this in Go (arch/moe.go, arch/config.go,
arch/config_validate.go, arch/weight_shapes.go, arch/ir.go); Go is not part
of this build's toolchain, so the same surface is restated here with the same
names, defaults, parameter order and error substrings, and it drives the
op-74 executor in mixlab_amd.op.  Nothing here touches a device.
"""
from __future__ import annotations

import json
import math
from dataclasses import dataclass, field
from typing import Any, Optional

import numpy as np

# arch/ir.go:10-67 (op codes are a stable ABI shared with gpu/ir.h)
OP_ADD = 3
OP_MUL = 4
OP_SCALAR_MUL = 5
OP_DROPOUT = 15
OP_RMSNORM = 33
OP_MOE_FEED_FORWARD = 74
DROPOUT_KEYS_INPUT = "dropout_keys"  # arch/ir.go:97

# arch/moe.go:8-19
MOE_EXPERT_SWIGLU, MOE_EXPERT_GEGLU, MOE_EXPERT_MLP = 0, 1, 2
MOE_ACT_SILU, MOE_ACT_GELU, MOE_ACT_RELU, MOE_ACT_LEAKY_RELU_SQ = 0, 1, 2, 3

DEFAULT_FFN_MULTIPLIER = 2.67  # arch/weight_shapes.go:11


class ConfigError(ValueError):
    pass


@dataclass
class BlockSpec:
    """The MoE-relevant fields of arch.BlockSpec (arch/config.go:150-161)."""

    type: str = ""
    num_experts: int = 0
    top_k: int = 0
    expert_block: Optional["BlockSpec"] = None
    router: str = ""
    load_balance_loss_weight: float = 0.0
    activation: str = ""
    leaky_slope: float = 0.0
    weight_group: str = ""
    parallel_residual: Optional[bool] = None
    heads: int = 0
    residual_scale_init: Optional[float] = None
    # keys outside the fields above.  arch.BlockSpec has its own UnmarshalJSON
    # (arch/config.go:229-249), which re-decodes the block with a plain
    # json.Unmarshal: the outer decoder's DisallowUnknownFields
    # (arch/config_load.go:115) does not reach into a block, so unknown keys
    # inside a block are ignored by the reference, not rejected.
    extra: dict = field(default_factory=dict)
    # presence flag recorded by BlockSpec.UnmarshalJSON (arch/config.go:229-249)
    load_balance_loss_weight_set: bool = False

    @classmethod
    def from_dict(cls, raw: dict) -> "BlockSpec":
        known = {"type", "num_experts", "top_k", "expert_block", "router",
                 "load_balance_loss_weight", "activation", "leaky_slope", "weight_group",
                 "parallel_residual", "heads", "residual_scale_init"}
        rsi = raw.get("residual_scale_init")
        spec = cls(
            type=str(raw.get("type", "")),
            num_experts=int(raw.get("num_experts", 0)),
            top_k=int(raw.get("top_k", 0)),
            expert_block=cls.from_dict(raw["expert_block"]) if raw.get("expert_block") is not None else None,
            router=str(raw.get("router", "")),
            load_balance_loss_weight=float(raw.get("load_balance_loss_weight", 0.0)),
            activation=str(raw.get("activation", "")),
            leaky_slope=float(raw.get("leaky_slope", 0.0)),
            weight_group=str(raw.get("weight_group", "")),
            parallel_residual=raw.get("parallel_residual"),
            heads=int(raw.get("heads", 0)),
            residual_scale_init=None if rsi is None else float(rsi),
            extra={k: v for k, v in raw.items() if k not in known},
        )
        spec.load_balance_loss_weight_set = "load_balance_loss_weight" in raw
        return spec

    @classmethod
    def from_json(cls, text: str) -> "BlockSpec":
        return cls.from_dict(json.loads(text))


def block_type_key(spec: BlockSpec) -> str:
    """arch/registry.go:64-70 (blockTypeName)."""
    key = spec.type.strip().lower()
    return "gated_linear_ssm" if key == "mamba3" else key


def effective_moe_expert_block(spec: BlockSpec) -> BlockSpec:
    """arch/moe.go:21-26."""
    return spec.expert_block if spec.expert_block is not None else BlockSpec(type="swiglu")


def effective_moe_top_k(spec: BlockSpec) -> int:
    """arch/moe.go:28-36."""
    if spec.top_k > 0:
        return spec.top_k
    return 1 if spec.num_experts <= 1 else 2


def effective_moe_load_balance_loss_weight(spec: BlockSpec) -> float:
    """arch/moe.go:38-43: an explicit 0 disables the aux loss, omitted gives 0.01."""
    if not spec.load_balance_loss_weight_set and spec.load_balance_loss_weight == 0:
        return 0.01
    return spec.load_balance_loss_weight


def moe_router(spec: BlockSpec) -> str:
    """arch/moe.go:45-51."""
    r = spec.router.strip().lower()
    return r or "linear"


def moe_expert_type_and_activation(spec: BlockSpec) -> tuple[int, int, float]:
    """arch/moe.go:53-80 -> (expertType, activation, leakySlope)."""
    expert = effective_moe_expert_block(spec)
    key = block_type_key(expert)
    if key == "swiglu":
        return MOE_EXPERT_SWIGLU, MOE_ACT_SILU, 0.0
    if key == "geglu":
        return MOE_EXPERT_GEGLU, MOE_ACT_GELU, 0.0
    if key == "mlp":
        act = expert.activation.strip().lower()
        if act in ("", "silu"):
            return MOE_EXPERT_MLP, MOE_ACT_SILU, 0.0
        if act == "gelu":
            return MOE_EXPERT_MLP, MOE_ACT_GELU, 0.0
        if act == "relu":
            return MOE_EXPERT_MLP, MOE_ACT_RELU, 0.0
        if act == "leaky_relu_sq":
            slope = expert.leaky_slope if expert.leaky_slope != 0 else 0.5
            return MOE_EXPERT_MLP, MOE_ACT_LEAKY_RELU_SQ, float(slope)
        raise ConfigError(f'unsupported moe mlp activation "{expert.activation}"')
    raise ConfigError(f'unsupported moe expert block type "{expert.type}"')


def moe_expert_weight_count(spec: BlockSpec) -> int:
    """arch/moe.go:82-95."""
    etype, _, _ = moe_expert_type_and_activation(spec)
    return 2 if etype == MOE_EXPERT_MLP else 3


def moe_weight_count(spec: BlockSpec, block_scales: bool = False) -> int:
    """arch/moe.go:97-110: norm + router + expert weights (+ moe_scale)."""
    if spec.num_experts <= 0:
        raise ConfigError("moe requires num_experts > 0")
    return 2 + spec.num_experts * moe_expert_weight_count(spec) + (1 if block_scales else 0)


def ffn_dim(D: int, multiplier: float) -> int:
    """arch/weight_shapes.go:56-65: round(D*mult) (half away from zero), at least D."""
    if multiplier <= 0:
        multiplier = DEFAULT_FFN_MULTIPLIER
    v = D * multiplier
    f = int(math.floor(v + 0.5)) if v >= 0 else -int(math.floor(-v + 0.5))
    return D if f < D else f


@dataclass
class WeightMeta:
    """The fields of arch.WeightMeta this block sets (arch/weight_shapes.go)."""

    name: str
    shape: list
    is_norm_scale: bool = False
    init_one: bool = False
    init_zero: bool = False
    init_value: float = 0.0


def residual_scale_weight_meta(spec: BlockSpec, name: str, dim: int) -> WeightMeta:
    """arch/weight_shapes.go:75-87: init 1 unless residual_scale_init is set;
    an explicit 0 inits to zero, any other value inits to that value (fp32)."""
    meta = WeightMeta(name, [dim], init_one=True)
    if spec.residual_scale_init is None:
        return meta
    meta.init_one = False
    if spec.residual_scale_init == 0:
        meta.init_zero = True
        return meta
    meta.init_value = float(np.float32(spec.residual_scale_init))
    return meta


def moe_weight_shapes(spec: BlockSpec, D: int, mlp_mult: float = DEFAULT_FFN_MULTIPLIER,
                      block_scales: bool = False) -> list[WeightMeta]:
    """arch/moe.go:116-150 (names, shapes and order; x.W layout [in, out])."""
    if spec.num_experts <= 0:
        raise ConfigError("moe requires num_experts > 0")
    etype, _, _ = moe_expert_type_and_activation(spec)
    F = ffn_dim(D, mlp_mult)
    metas = [WeightMeta("moe_norm_scale", [D], is_norm_scale=True, init_one=True),
             WeightMeta("router_w", [D, spec.num_experts])]
    for i in range(spec.num_experts):
        if etype in (MOE_EXPERT_SWIGLU, MOE_EXPERT_GEGLU):
            metas += [WeightMeta(f"expert_{i}_w_gate", [D, F]),
                      WeightMeta(f"expert_{i}_w_up", [D, F]),
                      WeightMeta(f"expert_{i}_w_down", [F, D])]
        else:
            metas += [WeightMeta(f"expert_{i}_w_up", [D, F]),
                      WeightMeta(f"expert_{i}_w_down", [F, D])]
    if block_scales:
        metas.append(residual_scale_weight_meta(spec, "moe_scale", D))
    return metas


def moe_parallel_weight_shapes(spec: BlockSpec, paired_second: bool, D: int,
                               mlp_mult: float = DEFAULT_FFN_MULTIPLIER,
                               block_scales: bool = False) -> list[WeightMeta]:
    """arch/weight_shapes.go:498-551 for an MoE block: the second block of a
    parallel-residual pair runs on the pair's shared normalised rows, so its
    own moe_norm_scale is stripped (pinned by arch/moe_test.go:160-198)."""
    metas = moe_weight_shapes(spec, D, mlp_mult, block_scales)
    if paired_second:
        if not metas or metas[0].name != "moe_norm_scale":
            raise ConfigError("parallel_residual FFN block has unexpected weight layout")
        metas = metas[1:]
    return metas


def moe_parallel_weight_count(spec: BlockSpec, paired_second: bool,
                              block_scales: bool = False) -> int:
    """arch/parallel_residual.go:242-264: a paired MoE follower omits one
    weight (its norm scale)."""
    n = moe_weight_count(spec, block_scales)
    return n - 1 if paired_second else n


def validate_moe_block(b: BlockSpec, source: str = "config", group: str = "blocks",
                       idx: int = 0) -> None:
    """The MoE branch of validateBlockSpec, arch/config_validate.go:519-556."""
    if block_type_key(b) != "moe":
        return
    where = f'config "{source}" {group}[{idx}] type=moe'
    if b.num_experts <= 0:
        raise ConfigError(f"{where} requires num_experts > 0")
    top_k = effective_moe_top_k(b)
    if top_k < 1 or top_k > b.num_experts:
        raise ConfigError(f"{where} has invalid top_k={top_k} (must be in [1,num_experts={b.num_experts}])")
    if moe_router(b) != "linear":
        raise ConfigError(f'{where} has invalid router="{b.router}" (v1 supports "linear")')
    lbw = effective_moe_load_balance_loss_weight(b)
    if lbw < 0:
        raise ConfigError(f"{where} has invalid load_balance_loss_weight={lbw:g} (must be >= 0)")
    expert = effective_moe_expert_block(b)
    if expert.weight_group:
        raise ConfigError(f"{where} expert_block cannot set weight_group")
    if expert.parallel_residual is not None:
        raise ConfigError(f"{where} expert_block cannot set parallel_residual")
    key = block_type_key(expert)
    if key in ("swiglu", "geglu"):
        return
    if key == "mlp":
        act = expert.activation.strip().lower()
        if act not in ("", "silu", "gelu", "relu", "leaky_relu_sq"):
            raise ConfigError(f'{where} expert_block has invalid activation "{expert.activation}"')
        if expert.leaky_slope < 0:
            raise ConfigError(f"{where} expert_block has invalid leaky_slope={expert.leaky_slope:g} (must be >= 0)")
        return
    raise ConfigError(f'{where} expert_block.type must be swiglu, geglu, or mlp (got "{expert.type}")')


def parse_moe_block(text: str, source: str = "config", idx: int = 0) -> BlockSpec:
    spec = BlockSpec.from_json(text)
    validate_moe_block(spec, source=source, idx=idx)
    return spec


# JSON names of arch.ArchConfig's fields (arch/config.go:18-87): the
# top-level keys ParseArchConfig accepts; any other top-level key is an error
# (DisallowUnknownFields, arch/config_load.go:115).
ARCH_CONFIG_FIELDS = frozenset((
    "name", "model_dim", "vocab_size", "seq_len", "mlp_mult", "tie_embeddings", "block_scales",
    "resid_mix", "parallel_residual", "unet", "rc_equivariant", "smear_embeddings",
    "smear_embeddings_gate_shape", "char_vocab_size", "char_dim", "char_max_per_token",
    "positional_embedding", "max_positions", "embedding_dropout", "input_adapter",
    "hf_export_format", "bigram_vocab_size", "bigram_dim", "trigram_vocab_size", "trigram_dim",
    "logit_softcap", "dropout", "attn_dropout", "hidden_dropout", "tie_dropout", "mlm_head",
    "norm_type", "norm_eps", "norm_affine", "batchnorm_momentum", "norm_placement", "final_norm",
    "ffn_internal_norm", "layer_aggregation", "mtp", "backout", "data", "blocks", "recurrence",
    "recurrence_phases", "execution_order", "recurrence_phase_activations", "training", "eval"))


@dataclass
class ModelConfig:
    """The top-level fields of arch.ArchConfig that size and place MoE blocks."""

    name: str
    model_dim: int
    seq_len: int
    mlp_mult: float
    block_scales: bool
    parallel_residual: bool
    batch_tokens: int
    blocks: list


def _strip_json_comments(text: str) -> str:
    """arch/config_load.go stripJSONComments: drop // line comments outside
    strings (JSONC)."""
    out, in_str, esc, i = [], False, False, 0
    while i < len(text):
        c = text[i]
        if in_str:
            out.append(c)
            if esc:
                esc = False
            elif c == "\\":
                esc = True
            elif c == '"':
                in_str = False
        elif c == '"':
            in_str = True
            out.append(c)
        elif c == "/" and text[i + 1:i + 2] == "/":
            while i < len(text) and text[i] != "\n":
                i += 1
            continue
        else:
            out.append(c)
        i += 1
    return "".join(out)


def parse_model_config(text: str, source: str = "config") -> ModelConfig:
    """The part of ParseArchConfig (arch/config_load.go:98-136, comments per
    stripJSONComments at :49-92) this path
    needs: JSONC comments stripped, unknown top-level keys rejected with the
    reference's wording, then each MoE block validated
    (arch/config_validate.go:519-556).  Other block kinds are returned
    unvalidated; the nested objects (training, data, ...) are not checked."""
    try:
        raw = json.loads(_strip_json_comments(text))
    except json.JSONDecodeError as err:
        raise ConfigError(f'parse config "{source}": {err}') from None
    if not isinstance(raw, dict):
        raise ConfigError(f'parse config "{source}": top level is not an object')
    for key in raw:
        if key not in ARCH_CONFIG_FIELDS:
            raise ConfigError(f'parse config "{source}": json: unknown field "{key}" '
                              "(check field names against docs/config-reference.md)")
    blocks = [BlockSpec.from_dict(b) for b in raw.get("blocks", [])]
    for i, b in enumerate(blocks):
        validate_moe_block(b, source=source, idx=i)
    training = raw.get("training") or {}
    return ModelConfig(name=str(raw.get("name", "")), model_dim=int(raw.get("model_dim", 0)),
                       seq_len=int(raw.get("seq_len", 0)),
                       mlp_mult=float(raw.get("mlp_mult", 0.0)),
                       block_scales=bool(raw.get("block_scales", False)),
                       parallel_residual=bool(raw.get("parallel_residual", False)),
                       batch_tokens=int(training.get("batch_tokens", 0)), blocks=blocks)


@dataclass
class Op:
    """arch/ir.go:126-133."""

    code: int
    inputs: list
    outputs: list
    float_params: list
    int_params: list


@dataclass
class Program:
    """The slice of arch.Program the MoE emitter uses (arch/ir.go:166-174)."""

    ops: list = field(default_factory=list)

    def add_op(self, code, inputs, outputs, float_params=None, int_params=None):
        self.ops.append(Op(code, list(inputs), list(outputs), list(float_params or []),
                           list(int_params or [])))

    def moe_feed_forward(self, inputs, delta, aux_loss, entropy, B, T, D, experts, top_k,
                         expert_type, ffn, activation, leaky_slope):
        """arch/ir.go:692-698."""
        self.add_op(OP_MOE_FEED_FORWARD, inputs, [delta, aux_loss, entropy], [leaky_slope],
                    [B, T, D, experts, top_k, expert_type, ffn, activation])

    def rms_norm(self, x, scale, output, eps):
        self.add_op(OP_RMSNORM, [x, scale], [output], [eps])  # arch/ir.go:437-439

    def scalar_mul(self, a, s, output):
        self.add_op(OP_SCALAR_MUL, [a], [output], [s])  # arch/ir.go:230-232

    def add(self, a, b, output):
        self.add_op(OP_ADD, [a, b], [output])  # arch/ir.go:200-202

    def mul(self, a, b, output):
        self.add_op(OP_MUL, [a, b], [output])  # arch/ir.go:225-227

    def dropout(self, a, rate, output):
        ordinal = sum(1 for op in self.ops if op.code == OP_DROPOUT)
        self.add_op(OP_DROPOUT, [a, DROPOUT_KEYS_INPUT], [output], [rate], [ordinal])


def weight_name(i: int) -> str:
    return f"w{i}"  # arch/ir.go:901-903


def tmp_name(base: str, idx: int) -> str:
    return f"{base}_{idx}"  # arch/ir.go:906-908


def emit_moe_delta_ir(prog: Program, spec: BlockSpec, x_norm: str, wi: int, D: int, T: int, B: int,
                      idx: int, mlp_mult: float, block_scales: bool, dropout: float,
                      prefix: str) -> tuple[str, int]:
    """arch/moe.go:173-213."""
    experts = spec.num_experts
    top_k = effective_moe_top_k(spec)
    etype, act, slope = moe_expert_type_and_activation(spec)
    ffn = ffn_dim(D, mlp_mult)
    inputs = [x_norm, weight_name(wi)]
    wi += 1
    per = moe_expert_weight_count(spec)
    for _ in range(experts * per):
        inputs.append(weight_name(wi))
        wi += 1
    delta = prefix + "_delta"
    aux = prefix + "_moe_aux_loss_raw"
    ent = prefix + "_moe_router_entropy"
    prog.moe_feed_forward(inputs, delta, aux, ent, B, T, D, experts, top_k, etype, ffn, act, slope)
    prog.scalar_mul(aux, float(effective_moe_load_balance_loss_weight(spec)), prefix + "_moe_aux_loss")
    if block_scales:
        scaled = prefix + "_scaled"
        prog.mul(delta, weight_name(wi), scaled)
        wi += 1
        delta = scaled
    if dropout > 0:
        dropped = prefix + "_dropout"
        prog.dropout(delta, dropout, dropped)
        delta = dropped
    return delta, wi


def emit_moe_ir(prog: Program, spec: BlockSpec, x: str, wi: int, D: int, T: int, B: int, idx: int,
                mlp_mult: float = DEFAULT_FFN_MULTIPLIER, block_scales: bool = False,
                dropout: float = 0.0) -> int:
    """arch/moe.go:152-166 (adaLN and layer aggregation are no-ops when unset)."""
    prefix = tmp_name(x + "_moe", idx)
    x_norm = prefix + "_x_norm"
    prog.rms_norm(x, weight_name(wi), x_norm, 1e-5)
    wi += 1
    delta, next_wi = emit_moe_delta_ir(prog, spec, x_norm, wi, D, T, B, idx, mlp_mult,
                                       block_scales, dropout, prefix)
    prog.add(x, delta, x)
    return next_wi


def emit_moe_parallel_delta_ir(prog: Program, spec: BlockSpec, x_norm: str, wi: int, D: int, T: int,
                               B: int, idx: int, mlp_mult: float = DEFAULT_FFN_MULTIPLIER,
                               block_scales: bool = False, dropout: float = 0.0) -> tuple[str, int]:
    """arch/moe.go:168-171, the MoE member of a parallel-residual pair
    (arch/parallel_residual.go:461-462): the pair's shared normalised rows
    go straight into op 74 and the delta is returned for the pair to add."""
    prefix = tmp_name(x_norm + "_parallel_moe", idx)
    return emit_moe_delta_ir(prog, spec, x_norm, wi, D, T, B, idx, mlp_mult, block_scales,
                             dropout, prefix)


def estimate_moe_block_flops(block: BlockSpec, B: int, T: int, D: int, mlp_mult: float) -> int:
    """arch/moe.go:215-236: router + top_k active experts (the algorithmic count)."""
    if block.num_experts <= 0:
        return 0
    ffn = ffn_dim(D, mlp_mult)
    top_k = effective_moe_top_k(block)
    try:
        etype, _, _ = moe_expert_type_and_activation(block)
    except ConfigError:
        return 0
    total = 2 * B * T * D * block.num_experts
    if etype in (MOE_EXPERT_SWIGLU, MOE_EXPERT_GEGLU):
        per = 2 * 2 * B * T * D * ffn + 2 * B * T * ffn * D
    else:
        per = 2 * B * T * D * ffn + 2 * B * T * ffn * D
    return total + top_k * per


def op_flops(int_params) -> int:
    """Algorithmic FLOPs of one op-74 forward from its IntParams."""
    B, T, D, E, K, etype, F, _ = int_params[:8]
    N = B * T
    per = (6 if etype != MOE_EXPERT_MLP else 4) * N * D * F
    return 2 * N * D * E + K * per


# ---- aux / entropy aggregation into the loss (arch/loss_emit.go:244-303) ----

def collect_moe_auxiliary_outputs(prog: Program) -> tuple[list, list]:
    """arch/loss_emit.go:244-258: per-block outputs suffixed _moe_aux_loss /
    _moe_router_entropy, in program order."""
    aux, ent = [], []
    for op in prog.ops:
        for out in op.outputs:
            if out.endswith("_moe_aux_loss") and out != "moe_aux_loss":
                aux.append(out)
            elif out.endswith("_moe_router_entropy") and out != "moe_router_entropy":
                ent.append(out)
    return aux, ent


def emit_moe_auxiliary_aggregates_ir(prog: Program, task_loss_has_eval_loss: bool) -> bool:
    """arch/loss_emit.go:260-303: moe_aux_loss = sum of the blocks' aux
    losses (left to right), moe_router_entropy = their mean (sum times
    1/count), loss = task_loss + moe_aux_loss."""
    aux, ent = collect_moe_auxiliary_outputs(prog)
    if not aux:
        return False
    if not task_loss_has_eval_loss:
        prog.scalar_mul("loss", 1.0, "eval_loss")
    prog.scalar_mul("loss", 1.0, "task_loss")
    acc = aux[0]
    for i in range(1, len(aux)):
        nxt = f"moe_aux_accum_{i}"
        prog.add(acc, aux[i], nxt)
        acc = nxt
    prog.scalar_mul(acc, 1.0, "moe_aux_loss")
    if ent:
        acc = ent[0]
        for i in range(1, len(ent)):
            nxt = f"moe_entropy_accum_{i}"
            prog.add(acc, ent[i], nxt)
            acc = nxt
        prog.scalar_mul(acc, float(np.float32(1.0) / np.float32(len(ent))), "moe_router_entropy")
    prog.add("task_loss", "moe_aux_loss", "loss")
    return True


def training_step_output_names(prog: Program, loss_name: str = "loss") -> list:
    """gpu/ir_trainer.cpp:1540-1585: the outputs a training step reads back --
    the loss, then each of magnitudes, x_hidden, logits, qr, moe_aux_loss and
    moe_router_entropy that some op of the program writes, in that order."""
    written = {out for op in prog.ops for out in op.outputs}
    names = [loss_name]
    for name in ("magnitudes", "x_hidden", "logits", "qr", "moe_aux_loss", "moe_router_entropy"):
        if name in written:
            names.append(name)
    return names


def moe_component_losses(values: dict) -> dict:
    """The MoE entry of the telemetry's ``component_losses`` object
    (train/telemetry.go:48, docs/performance.md:158-163): ``moe_aux_loss``
    when the graph produced it; absent objectives add no key."""
    return {"moe_aux_loss": float(values["moe_aux_loss"])} if "moe_aux_loss" in values else {}


def evaluate_scalar_ops(prog: Program, values: dict, start: int = 0) -> dict:
    """Evaluate the scalar Add / ScalarMul ops of prog (from op index start)
    in fp32, as the interpreter does for [1]-shaped tensors; values maps
    names to floats and is extended in place."""
    for op in prog.ops[start:]:
        if op.code == OP_ADD:
            a, b = (np.float32(values[n]) for n in op.inputs)
            values[op.outputs[0]] = float(a + b)
        elif op.code == OP_SCALAR_MUL:
            values[op.outputs[0]] = float(np.float32(values[op.inputs[0]])
                                          * np.float32(op.float_params[0]))
    return values
