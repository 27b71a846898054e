"""Weight I/O on either side of op 74: mixlab's native checkpoint format and
the int8 expert format of this build.

Native checkpoints are safetensors files whose tensors are named
``w{index}_{name}`` after the model's weight metas (train/export.go:20-80
writes them, F32 little-endian, with ``__metadata__`` format "mixlab_v1";
train/import.go:20-146 reads them, F32 only).  An MoE block's weights are the
metas of arch/moe.go:112-150 at the block's offset: ``moe_norm_scale``,
``router_w``, ``expert_{e}_w_gate/up/down`` (mlp: up, down), then
``moe_scale`` with block scales.  The reader and writer here follow the same
layout and the same checks, with the reference's error messages.

HF export (train/export_hf.go): an MoE block's weights keep their shapes
and data and are renamed ``blocks.{b}.norm.weight``, ``blocks.{b}.router_w``
and ``blocks.{b}.experts.{e}.w_{gate,up,down}.weight`` (``hf_moe_weight_map``,
``export_hf_safetensors``).

int8: the reference quantises for export per input row with clipping
(train/quantize.go:99-118; ``DequantizePerRow`` :191-200 undoes it); the
int8 executor (``mxm_moe_set_input_q8``) takes symmetric per-output-channel
scales instead.  ``per_row_to_per_channel`` converts the former into the
latter through the dequantised fp32 weights.
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from .moe import BlockSpec, WeightMeta, effective_moe_expert_block, moe_weight_shapes


class CheckpointError(ValueError):
    pass


@dataclass
class SafeTensor:
    dtype: str
    shape: List[int]
    data: bytes


def load_safetensors(path: str) -> Dict[str, SafeTensor]:
    """Parse a safetensors file (train/import.go:20-67): 8-byte LE header
    length, JSON header, payload; offsets are checked against the payload."""
    try:
        with open(path, "rb") as f:
            blob = f.read()
    except OSError as e:
        raise CheckpointError(f'read safetensors "{path}": {e}') from e
    if len(blob) < 8:
        raise CheckpointError(f'invalid safetensors "{path}": too small ({len(blob)} bytes)')
    header_len = struct.unpack("<Q", blob[:8])[0]
    if header_len == 0:
        raise CheckpointError(f'invalid safetensors "{path}": empty header')
    if header_len > len(blob) - 8:
        raise CheckpointError(f'invalid safetensors "{path}": header length {header_len} '
                              f"exceeds file size {len(blob)}")
    try:
        raw = json.loads(blob[8:8 + header_len])
    except json.JSONDecodeError as e:
        raise CheckpointError(f'parse safetensors header "{path}": {e}') from e
    payload = blob[8 + header_len:]
    out = {}
    for name, ent in raw.items():
        if name == "__metadata__":
            continue
        offs = ent.get("data_offsets", [])
        if len(offs) != 2:
            raise CheckpointError(f'invalid offsets for "{name}" in "{path}": expected 2, '
                                  f"got {len(offs)}")
        start, end = int(offs[0]), int(offs[1])
        if end < start or end > len(payload):
            raise CheckpointError(f'invalid offsets for "{name}" in "{path}": start={start} '
                                  f"end={end} payload={len(payload)}")
        out[name] = SafeTensor(str(ent.get("dtype", "")), [int(v) for v in ent.get("shape", [])],
                               payload[start:end])
    return out


def decode_f32(name: str, want_shape: Sequence[int], tensors: Dict[str, SafeTensor]) -> np.ndarray:
    """train/import.go:119-146: F32 only, shape must match."""
    ent = tensors.get(name)
    if ent is None:
        raise CheckpointError(f'missing tensor "{name}" in safetensors file')
    if list(ent.shape) != list(want_shape):
        raise CheckpointError(f'shape mismatch for "{name}": file={ent.shape} '
                              f"expected={list(want_shape)}")
    n = int(np.prod(want_shape)) if len(want_shape) else 1
    if n <= 0:
        raise CheckpointError(f'invalid shape for "{name}": {list(want_shape)}')
    if ent.dtype != "F32":
        raise CheckpointError(f'unsupported dtype "{ent.dtype}" for "{name}" (only F32 '
                              "supported for weight loading)")
    if len(ent.data) != n * 4:
        raise CheckpointError(f'F32 payload size mismatch for "{name}": got={len(ent.data)} '
                              f"want={n * 4}")
    return np.frombuffer(ent.data, dtype="<f4").reshape(want_shape).astype(np.float32)


def checkpoint_name(index: int, meta_name: str) -> str:
    return f"w{index}_{meta_name}"  # train/export.go:36, train/import.go:79


def load_weights(path: str, metas: Sequence[WeightMeta], first_index: int = 0) -> List[np.ndarray]:
    """train/import.go:71-89 for a run of metas starting at global weight
    index first_index (a block's slice of the model's metas)."""
    tensors = load_safetensors(path)
    out = []
    for i, m in enumerate(metas):
        name = checkpoint_name(first_index + i, m.name)
        try:
            out.append(decode_f32(name, m.shape, tensors))
        except CheckpointError as e:
            raise CheckpointError(f"load weight {first_index + i} ({name}): {e}") from e
    return out


def export_safetensors(path: str, metas: Sequence[WeightMeta], weights: Sequence[np.ndarray],
                       metadata: Optional[Dict[str, str]] = None, first_index: int = 0) -> None:
    """train/export.go:20-80: F32 tensors named w{i}_{name}, header entries in
    weight order, ``__metadata__`` with format mixlab_v1; written atomically."""
    if len(metas) != len(weights):
        raise CheckpointError(f"shapes/weights count mismatch: {len(metas)} vs {len(weights)}")
    header = {}
    offset = 0
    arrays = []
    for i, (m, w) in enumerate(zip(metas, weights)):
        a = np.ascontiguousarray(w, dtype="<f4")
        if list(a.shape) != list(m.shape):
            raise CheckpointError(f"weight {i} ({m.name}) has shape {list(a.shape)}, "
                                  f"want {list(m.shape)}")
        header[checkpoint_name(first_index + i, m.name)] = {
            "dtype": "F32", "shape": list(m.shape), "data_offsets": [offset, offset + a.nbytes]}
        offset += a.nbytes
        arrays.append(a)
    meta = {"format": "mixlab_v1"}
    meta.update(metadata or {})
    header["__metadata__"] = meta
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    tmp = f"{path}.tmp{os.getpid()}"
    with open(tmp, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for a in arrays:
            f.write(a.tobytes())
    os.replace(tmp, path)


def hf_moe_weight_map(block_index: int, spec: BlockSpec, metas: Sequence[WeightMeta],
                      first_index: int = 0) -> List[Tuple[str, str, List[int]]]:
    """The HF export names of one MoE block (train/export_hf.go:544-604, with
    the positional checks of ``addExpected`` :247-255): walks the block's
    weight metas from global index ``first_index`` and returns
    (native checkpoint name, HF name, shape) per mapped weight.  The block's
    optional ``moe_scale`` is not mapped here, as in the reference's moe case."""
    mapping: List[Tuple[str, str, List[int]]] = []
    prefix = f"blocks.{block_index}"
    wi = 0

    def expect(want: str, hf: str, what: str) -> None:
        nonlocal wi
        if wi >= len(metas):
            raise CheckpointError(f"weight map exhausted while mapping {what}")
        got = metas[wi].name
        if got != want:
            raise CheckpointError(f"HF export weight map expected Mixlab weight {want!r} at index "
                                  f"{first_index + wi}, got {got!r}")
        mapping.append((checkpoint_name(first_index + wi, got), f"{prefix}.{hf}",
                        list(metas[wi].shape)))
        wi += 1

    for mix, hf in (("moe_norm_scale", "norm.weight"), ("router_w", "router_w")):
        expect(mix, hf, f"moe block {block_index}")
    expert_type = effective_moe_expert_block(spec).type.strip().lower() or "swiglu"
    if expert_type in ("swiglu", "geglu"):
        kinds = ("gate", "up", "down")
    elif expert_type == "mlp":
        kinds = ("up", "down")
    else:
        raise CheckpointError(f"unsupported HF export moe expert type "
                              f"{effective_moe_expert_block(spec).type!r}")
    for e in range(spec.num_experts):
        for k in kinds:
            expect(f"expert_{e}_w_{k}", f"experts.{e}.w_{k}.weight",
                   f"moe block {block_index} expert {e}")
    return mapping


def export_hf_safetensors(path: str, mapping: Sequence[Tuple[str, str, List[int]]],
                          weights: Sequence[np.ndarray],
                          metadata: Optional[Dict[str, str]] = None) -> None:
    """train/export_hf.go:772-800: F32 tensors under their HF names with the
    mapped shapes (no transposes), ``__metadata__`` format "pt" plus the
    model fields the caller passes (name, model_dim, vocab_size, seq_len)."""
    if len(mapping) != len(weights):
        raise CheckpointError(f"mapping/weights count mismatch: {len(mapping)} vs {len(weights)}")
    header = {}
    offset = 0
    arrays = []
    for (_, hf, shape), w in zip(mapping, weights):
        a = np.ascontiguousarray(w, dtype="<f4")
        if list(a.shape) != list(shape):
            raise CheckpointError(f"weight {hf} has shape {list(a.shape)}, want {list(shape)}")
        header[hf] = {"dtype": "F32", "shape": list(shape), "data_offsets": [offset, offset + a.nbytes]}
        offset += a.nbytes
        arrays.append(a)
    meta = {"format": "pt"}
    meta.update(metadata or {})
    header["__metadata__"] = meta
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    tmp = f"{path}.tmp{os.getpid()}"
    with open(tmp, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for a in arrays:
            f.write(a.tobytes())
    os.replace(tmp, path)


def moe_block_metas(spec: BlockSpec, D: int, mlp_mult: float, block_scales: bool = False):
    return moe_weight_shapes(spec, D, mlp_mult, block_scales)


def quantize_per_channel(w: np.ndarray):
    """Symmetric per-output-channel int8 of an x.W matrix [in, out]:
    s_j = max_k |w[k, j]| / 127 (1 for an all-zero column),
    q = clamp(rint(w / s), -127, 127).  Returns (q int8, s fp32)."""
    w = np.asarray(w, dtype=np.float32)
    amax = np.abs(w).max(axis=0)
    s = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(w / s), -127, 127).astype(np.int8)
    return q, s


def dequantize_per_row(q: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """train/quantize.go:191-200 (DequantizePerRow): w[r, c] = q[r, c] * s[r]."""
    return (np.asarray(q, np.int8).astype(np.float32) * np.asarray(scales, np.float32)[:, None])


def per_row_to_per_channel(q_rows: np.ndarray, row_scales: np.ndarray):
    """Convert the reference's per-row int8 export of an x.W matrix [in, out]
    (one scale per input row) into the executor's per-output-channel format."""
    return quantize_per_channel(dequantize_per_row(q_rows, row_scales))
