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
(train/quantize.go:99-118; ``DequantizePerRow`` :191-200 undoes it) and
writes ``w{i}_{name}`` as I8 plus ``w{i}_{name}.scale`` F32 per row
(``export_safetensors_quantized``, train/export.go:203-352); its own
importer reads F32 only.  ``load_quantized_weights`` reads such a file; the
int8 executor (``mxm_moe_set_input_q8``) takes symmetric per-output-channel
scales, and ``QuantizedWeight.per_channel`` / ``per_row_to_per_channel``
convert the former into the latter through the dequantised fp32 weights.
"""
from __future__ import annotations

import json
import math
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


def _align8(n: int) -> int:
    return (n + 7) // 8 * 8


def _write_safetensors(path: str, tensors: Sequence[Tuple[str, str, List[int], bytes]],
                       metadata: Dict[str, str]) -> None:
    """The layout of train/export.go:94-114,166-200: each tensor's data starts
    at an 8-byte aligned offset (zero padding after it), the JSON header (keys
    sorted, as Go marshals a map) is padded with spaces to a multiple of 8
    bytes; written to a temporary file and renamed into place."""
    header = {}
    offset = 0
    for name, dtype, shape, data in tensors:
        header[name] = {"dtype": dtype, "shape": list(shape),
                        "data_offsets": [offset, offset + len(data)]}
        offset = _align8(offset + len(data))
    header["__metadata__"] = dict(metadata)
    hb = json.dumps(header, separators=(",", ":"), sort_keys=True).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    tmp = f"{path}.tmp{os.getpid()}"
    with open(tmp, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for _, _, _, data in tensors:
            f.write(data)
            f.write(b"\0" * (_align8(len(data)) - len(data)))
    os.replace(tmp, path)


def export_safetensors(path: str, metas: Sequence[WeightMeta], weights: Sequence[np.ndarray],
                       metadata: Optional[Dict[str, str]] = None, first_index: int = 0) -> None:
    """train/export.go:20-80: F32 tensors named w{i}_{name} in weight order,
    ``__metadata__`` with format mixlab_v1; written atomically."""
    if len(metas) != len(weights):
        raise CheckpointError(f"shapes/weights count mismatch: {len(metas)} vs {len(weights)}")
    tensors = []
    for i, (m, w) in enumerate(zip(metas, weights)):
        a = np.ascontiguousarray(w, dtype="<f4")
        if list(a.shape) != list(m.shape):
            raise CheckpointError(f"weight {i} ({m.name}) has shape {list(a.shape)}, "
                                  f"want {list(m.shape)}")
        tensors.append((checkpoint_name(first_index + i, m.name), "F32", list(m.shape),
                        a.tobytes()))
    meta = {"format": "mixlab_v1"}
    meta.update(metadata or {})
    _write_safetensors(path, tensors, meta)


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
    if wi != len(metas):
        # train/export_hf.go:733-735: a weight the map leaves unmapped (an MoE
        # block's moe_scale has no HF name) fails the export
        raise CheckpointError(f"HF weight map did not consume all weights: "
                              f"next_unmapped={first_index + wi} total={first_index + len(metas)}")
    return mapping


def export_hf_safetensors(path: str, mapping: Sequence[Tuple[str, str, List[int]]],
                          weights: Sequence[np.ndarray],
                          metadata: Optional[Dict[str, str]] = None) -> None:
    """train/export_hf.go:772-800: F32 tensors under their HF names with the
    mapped shapes (no transposes), ``__metadata__`` format "pt" plus the
    model fields the caller passes (name, model_dim, vocab_size, seq_len)."""
    if len(mapping) != len(weights):
        raise CheckpointError(f"mapping/weights count mismatch: {len(mapping)} vs {len(weights)}")
    tensors = []
    for (_, hf, shape), w in zip(mapping, weights):
        a = np.ascontiguousarray(w, dtype="<f4")
        if list(a.shape) != list(shape):
            raise CheckpointError(f"weight {hf} has shape {list(a.shape)}, want {list(shape)}")
        tensors.append((hf, "F32", list(shape), a.tobytes()))
    meta = {"format": "pt"}
    meta.update(metadata or {})
    _write_safetensors(path, tensors, meta)


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


# ---- the reference's quantized export (train/export.go:203-352,
#      train/quantize.go) and a reader for it ----

QUANT_CLIP_Q = 0.9999             # train/quantize.go:10
QUANT_KEEP_FLOAT_1D_MAX = 256     # train/quantize.go:11
MIN_ROW_SCALE = np.float32(1.0 / 127.0)  # train/quantize.go:12


def _go_round(v: np.ndarray) -> np.ndarray:
    """Go's math.Round: half away from zero."""
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def should_quantize(shape: Sequence[int], total: int) -> bool:
    """train/quantize.go:175-183: tensors under 256 elements and 1-D tensors
    stay F32."""
    return total >= QUANT_KEEP_FLOAT_1D_MAX and len(shape) != 1


def clip_quant_abs(vals: np.ndarray, q: float = QUANT_CLIP_Q) -> np.float32:
    """train/quantize.go:21-39: the q-quantile of |v|, the element of rank
    ceil(q*n) - 1 (clamped to the array) in ascending order."""
    a = np.abs(np.asarray(vals, np.float32).ravel())
    if a.size == 0:
        return np.float32(0.0)
    idx = min(max(int(math.ceil(q * a.size)) - 1, 0), a.size - 1)
    return np.float32(np.partition(a, idx)[idx])


def quantize_clamp(q_raw: np.ndarray, mode: str) -> np.ndarray:
    """train/quantize.go:77-96: int8 clamps to [-127, 127]; int6 rounds to a
    multiple of 4 in [-128, 124]; the int8 conversion truncates."""
    q = np.asarray(q_raw, np.float32)
    if mode == "int6":
        q = (_go_round(q.astype(np.float64) / 4.0) * 4.0).astype(np.float32)
        q = np.clip(q, -128, 124)
    else:
        q = np.clip(q, -127, 127)
    return np.trunc(q).astype(np.int8)


def quantize_tensor_per_row(data: np.ndarray, mode: str = "int8"):
    """train/quantize.go:98-118: per row, scale = max(clip/127, 1/127) with
    clip the 0.9999 quantile of |row|; q = clamp(round(clip(v)/scale)).
    data [rows, cols] fp32 -> (q int8 [rows, cols], scales fp32 [rows])."""
    data = np.asarray(data, np.float32)
    rows = data.shape[0]
    q = np.empty(data.shape, np.int8)
    scales = np.empty(rows, np.float32)
    for r in range(rows):
        row = data[r]
        clip = clip_quant_abs(row)
        scale = np.float32(clip / np.float32(127.0))
        if scale < MIN_ROW_SCALE:
            scale = MIN_ROW_SCALE
        scales[r] = scale
        clipped = np.clip(row.astype(np.float64), -float(clip), float(clip)).astype(np.float32)
        q[r] = quantize_clamp(_go_round((clipped / scale).astype(np.float64)).astype(np.float32),
                              mode)
    return q, scales


def quantize_tensor_per_row_sdclip(data: np.ndarray, mode: str, k: float):
    """train/quantize.go:120-149: the clip is k standard deviations of the
    row (population std in float64), at least 1/127."""
    data = np.asarray(data, np.float32)
    rows, cols = data.shape
    q = np.empty(data.shape, np.int8)
    scales = np.empty(rows, np.float32)
    for r in range(rows):
        row = data[r]
        f = row.astype(np.float64)
        mean = f.sum() / cols
        std = math.sqrt((f * f).sum() / cols - mean * mean)
        clip = np.float32(float(np.float32(k)) * std)
        if clip < MIN_ROW_SCALE:
            clip = MIN_ROW_SCALE
        scale = np.float32(clip / np.float32(127.0))
        if scale < MIN_ROW_SCALE:
            scale = MIN_ROW_SCALE
        scales[r] = scale
        clipped = np.clip(f, -float(clip), float(clip)).astype(np.float32)
        q[r] = quantize_clamp(_go_round((clipped / scale).astype(np.float64)).astype(np.float32),
                              mode)
    return q, scales


def quantize_tensor_flat(data: np.ndarray, mode: str = "int8"):
    """train/quantize.go:151-171: one scale for the whole tensor (1 when the
    clip is 0)."""
    data = np.asarray(data, np.float32).ravel()
    if data.size == 0:
        return np.zeros(0, np.int8), np.float32(1.0)
    clip = clip_quant_abs(data)
    scale = np.float32(clip / np.float32(127.0)) if clip > 0 else np.float32(1.0)
    clipped = np.clip(data.astype(np.float64), -float(clip), float(clip)).astype(np.float32)
    return quantize_clamp(_go_round((clipped / scale).astype(np.float64)).astype(np.float32),
                          mode), scale


def export_safetensors_quantized(path: str, metas: Sequence[WeightMeta],
                                 weights: Sequence[np.ndarray], mode: str = "int8",
                                 quant_method: str = "quantile", k_matrix: float = 0.0,
                                 k_embed: float = 0.0,
                                 metadata: Optional[Dict[str, str]] = None,
                                 first_index: int = 0) -> None:
    """train/export.go:203-352 (exportSafetensorsQuantized): a 2-D tensor of
    256 or more elements becomes ``w{i}_{name}`` I8 [rows, cols] plus
    ``w{i}_{name}.scale`` F32 [rows]; other shapes of 256 or more elements
    (not 1-D) become I8 plus a scalar F32 scale; the rest stay F32.
    ``__metadata__`` adds quantize, quant_method (and quant_k, quant_k_embed
    for sdclip) to format mixlab_v1."""
    if mode not in ("int8", "int6"):
        raise CheckpointError(f'unsupported quantize mode "{mode}"')
    quant_method = quant_method or "quantile"
    if quant_method not in ("quantile", "sdclip"):
        raise CheckpointError(f'unsupported quantization method "{quant_method}"')
    if len(metas) != len(weights):
        raise CheckpointError(f"shapes/weights count mismatch: {len(metas)} vs {len(weights)}")
    tensors = []
    for i, (m, w) in enumerate(zip(metas, weights)):
        name = checkpoint_name(first_index + i, m.name)
        a = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
        if a.size != int(np.prod(m.shape)):
            raise CheckpointError(f"tensor {name} shape/data mismatch: shape={list(m.shape)} "
                                  f"data={a.size}")
        if not should_quantize(m.shape, a.size):
            tensors.append((name, "F32", list(m.shape), a.astype("<f4").tobytes()))
            continue
        if len(m.shape) == 2:
            mat = a.reshape(m.shape)
            if quant_method == "sdclip":
                k = k_embed if "embed" in m.name.lower() else k_matrix
                q, sc = quantize_tensor_per_row_sdclip(mat, mode, k)
            else:
                q, sc = quantize_tensor_per_row(mat, mode)
            tensors.append((name, "I8", list(m.shape), q.tobytes()))
            tensors.append((name + ".scale", "F32", [m.shape[0]], sc.astype("<f4").tobytes()))
        else:
            q, sc = quantize_tensor_flat(a, mode)
            tensors.append((name, "I8", list(m.shape), q.tobytes()))
            tensors.append((name + ".scale", "F32", [], np.float32(sc).astype("<f4").tobytes()))
    meta = {"format": "mixlab_v1", "quantize": mode, "quant_method": quant_method}
    if quant_method == "sdclip":
        meta["quant_k"] = f"{k_matrix:g}"
        meta["quant_k_embed"] = f"{k_embed:g}"
    meta.update(metadata or {})
    _write_safetensors(path, tensors, meta)


@dataclass
class QuantizedWeight:
    """One weight of a quantized checkpoint: int8 values and their scales as
    the file holds them (per input row for a matrix, one scalar otherwise)."""

    q: np.ndarray       # int8, the weight's shape
    scales: np.ndarray  # fp32 [rows] (2-D) or [] (flat)

    def dequantize(self) -> np.ndarray:
        """train/quantize.go:191-210 (DequantizePerRow / DequantizeFlat)."""
        if self.q.ndim == 2:
            return dequantize_per_row(self.q, self.scales)
        return (self.q.astype(np.float32) * np.float32(self.scales)).astype(np.float32)

    def per_channel(self):
        """(q, scales) in the int8 executor's per-output-channel format
        (mxm_moe_set_input_q8), through the dequantised values."""
        if self.q.ndim != 2:
            raise CheckpointError("per-output-channel int8 needs a matrix")
        return quantize_per_channel(self.dequantize())


def _read_metadata(path: str) -> Dict[str, str]:
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        raw = json.loads(f.read(n))
    return raw.get("__metadata__", {}) or {}


def load_quantized_weights(path: str, metas: Sequence[WeightMeta], first_index: int = 0):
    """Read a run of weights from a checkpoint written by
    exportSafetensorsQuantized (train/export.go:203-352; the reference's own
    importer, train/import.go:119-146, reads F32 only).  Each weight comes
    back as an fp32 array (tensors the export kept as F32) or a
    QuantizedWeight (I8 data plus its ``.scale`` tensor).  The file must
    declare ``quantize`` int8 or int6 in its metadata."""
    mode = _read_metadata(path).get("quantize", "")
    if mode not in ("int8", "int6"):
        raise CheckpointError(f'"{path}" is not a quantized mixlab checkpoint '
                              f'(metadata quantize="{mode}")')
    tensors = load_safetensors(path)
    out: List[object] = []
    for i, m in enumerate(metas):
        name = checkpoint_name(first_index + i, m.name)
        ent = tensors.get(name)
        if ent is None:
            raise CheckpointError(f'load weight {first_index + i} ({name}): missing tensor '
                                  f'"{name}" in safetensors file')
        if ent.dtype == "F32":
            out.append(decode_f32(name, m.shape, tensors))
            continue
        if ent.dtype != "I8":
            raise CheckpointError(f'unsupported dtype "{ent.dtype}" for "{name}" (F32 or I8 '
                                  "expected in a quantized checkpoint)")
        if list(ent.shape) != list(m.shape):
            raise CheckpointError(f'shape mismatch for "{name}": file={ent.shape} '
                                  f"expected={list(m.shape)}")
        n = int(np.prod(m.shape))
        if len(ent.data) != n:
            raise CheckpointError(f'I8 payload size mismatch for "{name}": got={len(ent.data)} '
                                  f"want={n}")
        q = np.frombuffer(ent.data, dtype=np.int8).reshape(m.shape).copy()
        scale_shape = [m.shape[0]] if len(m.shape) == 2 else []
        sent = tensors.get(name + ".scale")
        if sent is None:
            raise CheckpointError(f'missing tensor "{name}.scale" in safetensors file')
        if sent.dtype != "F32" or list(sent.shape) != scale_shape:
            raise CheckpointError(f'"{name}.scale" must be F32 {scale_shape}, file has '
                                  f"{sent.dtype} {sent.shape}")
        k = max(1, int(np.prod(scale_shape)) if scale_shape else 1)
        if len(sent.data) != 4 * k:
            raise CheckpointError(f'F32 payload size mismatch for "{name}.scale"')
        sc = np.frombuffer(sent.data, dtype="<f4").astype(np.float32)
        out.append(QuantizedWeight(q, sc.reshape(scale_shape) if scale_shape else sc[0]))
    return out
