"""The reference's quantized checkpoint format (train/export.go:203-352,
train/quantize.go) restated in mixlab_amd.weights, and the reader that feeds
it to the int8 expert executor.  Known answers are the reference's own test
tables (train/quantize_test.go, train/export_test.go:95-118); the quantizer is
further pinned by brute force on small rows.  No GPU."""
from __future__ import annotations

import json
import math
import struct

import numpy as np
import pytest

from mixlab_amd import weights as W
from mixlab_amd.moe import BlockSpec, WeightMeta, moe_weight_shapes


@pytest.mark.parametrize("raw,want", [(0, 0), (50, 50), (-50, -50), (127, 127), (-127, -127),
                                      (200, 127), (-200, -127), (50.6, 50)])
def test_quantize_clamp_int8(raw, want):
    """train/quantize_test.go:355-379."""
    assert int(W.quantize_clamp(np.float32(raw), "int8")) == want


@pytest.mark.parametrize("raw,want", [(0, 0), (4, 4), (-4, -4), (5, 4), (6, 8), (3, 4),
                                      (124, 124), (-128, -128), (200, 124), (-200, -128),
                                      (125, 124), (126, 124)])
def test_quantize_clamp_int6(raw, want):
    """train/quantize_test.go:381-409 (Go's Round: 1.5 -> 2)."""
    assert int(W.quantize_clamp(np.float32(raw), "int6")) == want


def test_quantize_clamp_int6_multiples_of_four():
    """train/quantize_test.go:411-419."""
    raw = np.arange(-200, 200.5, 0.5, dtype=np.float32)
    assert np.all(W.quantize_clamp(raw, "int6").astype(np.int32) % 4 == 0)


@pytest.mark.parametrize("vals,q,want", [([], 0.99, 0.0), ([-5.0], 0.9999, 5.0),
                                         ([0, 0, 0, 0], 0.9999, 0.0), ([3.0] * 4, 0.9999, 3.0),
                                         ([-1.0, -2.0, -3.0, -4.0], 0.9999, 4.0),
                                         ([10.0], 0.9, 10.0)])
def test_clip_quant_abs(vals, q, want):
    """train/quantize_test.go:421-478."""
    assert W.clip_quant_abs(np.asarray(vals, np.float32), q) == np.float32(want)


def test_clip_quant_abs_rank_brute_force():
    """The quantile is the element of rank ceil(q n) - 1 of the sorted |v|."""
    rng = np.random.default_rng(3)
    for n in (1, 7, 100, 10_001, 20_000):
        v = rng.standard_normal(n).astype(np.float32)
        idx = min(max(math.ceil(0.9999 * n) - 1, 0), n - 1)
        assert W.clip_quant_abs(v) == np.sort(np.abs(v))[idx]


def test_quantize_flat_zero_and_empty():
    """train/quantize_test.go:480-505."""
    q, s = W.quantize_tensor_flat(np.zeros(256, np.float32))
    assert s == 1.0 and not q.any()
    q, s = W.quantize_tensor_flat(np.zeros(0, np.float32))
    assert q.size == 0 and s == 1.0


@pytest.mark.parametrize("shape,want", [([64, 128], True), ([4, 4], False), ([256], False),
                                        ([32], False)])
def test_should_quantize(shape, want):
    """train/quantize_test.go:162-184."""
    assert W.should_quantize(shape, int(np.prod(shape))) == want


def _gauss(seed, shape, scale):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def _rel_rms(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return math.sqrt(((a - b) ** 2).sum() / (a ** 2).sum())


def test_per_row_round_trip_bounds():
    """train/quantize_test.go:15-85: int8 under 5 %, int6 under 15 % and
    worse than int8; flat int8 under 1 % (:135-160)."""
    data = _gauss(42, (256, 512), 0.1)
    q8, s8 = W.quantize_tensor_per_row(data, "int8")
    q6, s6 = W.quantize_tensor_per_row(data, "int6")
    e8 = _rel_rms(data, W.dequantize_per_row(q8, s8))
    e6 = _rel_rms(data, W.dequantize_per_row(q6, s6))
    assert e8 <= 0.05 and e6 <= 0.15 and e6 > e8
    flat = _gauss(99, 512, 0.05)
    qf, sf = W.quantize_tensor_flat(flat)
    assert _rel_rms(flat, qf.astype(np.float32) * sf) <= 0.01


def test_per_row_quantizer_brute_force():
    """Each row: scale = max(quantile/127, 1/127) in fp32; every value lands
    on the nearest multiple of the scale of its clipped value (ties away from
    zero), within [-127, 127]."""
    rng = np.random.default_rng(5)
    data = (rng.standard_normal((40, 300)) * rng.uniform(0.001, 3.0, (40, 1))).astype(np.float32)
    data[3] = 0.0
    q, s = W.quantize_tensor_per_row(data, "int8")
    for r in range(data.shape[0]):
        a = np.sort(np.abs(data[r]))
        clip = a[math.ceil(0.9999 * a.size) - 1]
        want_s = max(np.float32(clip / np.float32(127.0)), np.float32(1.0 / 127.0))
        assert s[r] == np.float32(want_s)
        for c in range(0, data.shape[1], 7):
            v = float(np.clip(data[r, c], -clip, clip))
            t = float(np.float32(np.float32(v) / s[r]))
            k = math.floor(abs(t) + 0.5) * (1 if t >= 0 else -1)
            assert int(q[r, c]) == max(-127, min(127, k))


def test_sdclip_known_answers():
    """train/quantize_test.go:87-133."""
    d = np.array([[-4, -2, 0, 2, 4], [-8, -4, 0, 4, 8]], np.float32)
    _, lo = W.quantize_tensor_per_row_sdclip(d, "int8", 1.5)
    _, hi = W.quantize_tensor_per_row_sdclip(d, "int8", 3.0)
    assert np.all(hi > lo)
    _, s = W.quantize_tensor_per_row_sdclip(np.array([[-3, -1, 1, 3]], np.float32), "int8", 2.0)
    assert abs(float(s[0]) - 2.0 * math.sqrt(5) / 127.0) <= 1e-6
    row = np.array([[-1, -0.5, 0, 0.5, 50]], np.float32)
    assert not np.array_equal(W.quantize_tensor_per_row(row, "int8")[0],
                              W.quantize_tensor_per_row_sdclip(row, "int8", 1.0)[0])


def _header(path):
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        return n, json.loads(f.read(n))


def test_export_header_dtypes_scales_and_alignment(tmp_path):
    """train/quantize_test.go:249-345 and train/export_test.go:95-118: a 2-D
    tensor becomes I8 with an F32 per-row .scale, a 1-D tensor stays F32 with
    no scale; header length and every data offset are 8-byte aligned."""
    metas = [WeightMeta("embed", [128, 32]), WeightMeta("norm", [32]), WeightMeta("wq", [32, 32]),
             WeightMeta("odd", [3, 5])]
    ws = [_gauss(7 + i, m.shape, 0.1) for i, m in enumerate(metas)]
    p = tmp_path / "q.safetensors"
    W.export_safetensors_quantized(str(p), metas, ws, "int8")
    n, hdr = _header(p)
    assert n % 8 == 0
    assert hdr["w0_embed"]["dtype"] == "I8" and hdr["w2_wq"]["dtype"] == "I8"
    assert hdr["w1_norm"]["dtype"] == "F32" and "w1_norm.scale" not in hdr
    assert hdr["w0_embed.scale"] == {**hdr["w0_embed.scale"], "dtype": "F32", "shape": [128]}
    assert hdr["w3_odd"]["dtype"] == "F32"  # 15 elements: below the 256 floor
    for name, ent in hdr.items():
        if name != "__metadata__":
            assert ent["data_offsets"][0] % 8 == 0
    assert hdr["__metadata__"]["quantize"] == "int8"
    assert hdr["__metadata__"]["quant_method"] == "quantile"
    assert hdr["__metadata__"]["format"] == "mixlab_v1"
    with pytest.raises(W.CheckpointError, match='unsupported quantize mode "int4"'):
        W.export_safetensors_quantized(str(p), metas, ws, "int4")
    # the plain F32 export keeps the same alignment
    W.export_safetensors(str(tmp_path / "f.safetensors"), metas, ws)
    n, hdr = _header(tmp_path / "f.safetensors")
    assert n % 8 == 0 and all(e["data_offsets"][0] % 8 == 0
                              for k, e in hdr.items() if k != "__metadata__")
    got = W.load_weights(str(tmp_path / "f.safetensors"), metas)
    for a, b in zip(got, ws):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("mode", ["int8", "int6"])
def test_moe_block_round_trip(tmp_path, mode):
    """An MoE block written by the quantized export and read back: the norm
    scale (1-D) and the router (64 x 3 = 192 elements, under the 256 floor)
    exactly as F32, every expert matrix as int8 + per-row scales equal to the
    quantizer's, and its per-output-channel form for the int8 executor."""
    spec = BlockSpec.from_json('{"type":"moe","num_experts":3}')
    D = 64
    metas = moe_weight_shapes(spec, D, 2.0)
    ws = [np.ones(D, np.float32)] + [_gauss(20 + i, m.shape, 0.02) for i, m in
                                      enumerate(metas[1:])]
    p = tmp_path / "moe.safetensors"
    W.export_safetensors_quantized(str(p), metas, ws, mode, first_index=5)
    got = W.load_quantized_weights(str(p), metas, first_index=5)
    np.testing.assert_array_equal(got[0], ws[0])
    np.testing.assert_array_equal(got[1], ws[1])
    for g, w, m in zip(got[2:], ws[2:], metas[2:]):
        assert isinstance(g, W.QuantizedWeight)
        q, s = W.quantize_tensor_per_row(w, mode)
        np.testing.assert_array_equal(g.q, q)
        np.testing.assert_array_equal(g.scales, s)
        np.testing.assert_array_equal(g.dequantize(), W.dequantize_per_row(q, s))
        qc, sc = g.per_channel()
        assert qc.shape == tuple(m.shape) and sc.shape == (m.shape[1],)
        # requantising per output channel keeps within half a channel step
        assert np.all(np.abs(qc.astype(np.float32) * sc - g.dequantize()) <= sc * 0.5 + 1e-7)


def test_reader_errors(tmp_path):
    metas = [WeightMeta("wq", [32, 32])]
    ws = [_gauss(1, [32, 32], 0.1)]
    plain = tmp_path / "plain.safetensors"
    W.export_safetensors(str(plain), metas, ws)
    with pytest.raises(W.CheckpointError, match="not a quantized mixlab checkpoint"):
        W.load_quantized_weights(str(plain), metas)
    p = tmp_path / "q.safetensors"
    W.export_safetensors_quantized(str(p), metas, ws)
    with pytest.raises(W.CheckpointError, match='shape mismatch for "w0_wq"'):
        W.load_quantized_weights(str(p), [WeightMeta("wq", [16, 64])])
    with pytest.raises(W.CheckpointError, match='missing tensor "w1_wq"'):
        W.load_quantized_weights(str(p), metas, first_index=1)
    # the F32 importer refuses I8, as train/import.go:119-146 does
    with pytest.raises(W.CheckpointError, match='unsupported dtype "I8"'):
        W.load_weights(str(p), metas)
    # a file whose scale tensor is missing
    n, hdr = _header(p)
    del hdr["w0_wq.scale"]
    blob = p.read_bytes()
    hb = json.dumps(hdr).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(struct.pack("<Q", len(hb)) + hb + blob[8 + n:])
    with pytest.raises(W.CheckpointError, match='missing tensor "w0_wq.scale"'):
        W.load_quantized_weights(str(bad), metas)
