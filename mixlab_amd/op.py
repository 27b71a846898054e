"""Host-side executor of op 74 on libmixmoe.

``MoEFeedForward`` plays the part of the reference's `case
OP_MOE_FEED_FORWARD` (gpu/ir.cpp:4816-4824): it is built from an op's
parameters (arch/ir.go:692-698), binds the weight inputs by their position in
Op.Inputs (gpu/ir.cpp:3730-3734 resolves them by name w<i>), and returns the
op's three outputs.  All compute runs in libmixmoe's HIP kernels.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import numpy as np

from . import _lib
from .moe import (DEFAULT_FFN_MULTIPLIER, MOE_EXPERT_MLP, OP_MOE_FEED_FORWARD, OP_RMSNORM, BlockSpec,
                  Op, Program, effective_moe_load_balance_loss_weight, emit_moe_ir,
                  moe_weight_shapes)

_DTYPES = {"fp32": _lib.MXM_DTYPE_F32, "float32": _lib.MXM_DTYPE_F32,
           "bf16": _lib.MXM_DTYPE_BF16, "bfloat16": _lib.MXM_DTYPE_BF16}


def _np_dtype_code(a: np.ndarray) -> int:
    if a.dtype == np.float32:
        return _lib.MXM_DTYPE_F32
    if a.dtype == np.uint16:  # bf16 bit patterns
        return _lib.MXM_DTYPE_BF16
    raise TypeError(f"unsupported array dtype {a.dtype} (fp32 or bf16 bits as uint16)")


class MoEFeedForward:
    def __init__(self, int_params: Sequence[int], float_params: Sequence[float] = (0.0,),
                 n_inputs: Optional[int] = None, compute_dtype: str = "fp32", flags: int = 0):
        self._lib = _lib.init()
        ip = [int(v) for v in int_params]
        if len(ip) >= 8:
            B, T, D, E, K, etype, F, act = ip[:8]
            wpe = 2 if etype == MOE_EXPERT_MLP else 3
            if n_inputs is None:
                n_inputs = 2 + E * wpe
            self.B, self.T, self.D, self.E, self.K, self.F = B, T, D, E, K, F
            self.expert_type, self.activation = etype, act
            self.N = B * T
        if n_inputs is None:
            n_inputs = 0
        self.compute_dtype = compute_dtype
        iarr = (ctypes.c_int32 * max(1, len(ip)))(*ip)
        fp = [float(v) for v in float_params]
        farr = (ctypes.c_float * max(1, len(fp)))(*fp)
        self.handle = self._lib.mxm_moe_create(farr, len(fp), iarr, len(ip), int(n_inputs),
                                               _DTYPES[compute_dtype], int(flags))
        if not self.handle:
            raise _lib.MixMoEError(_lib.last_error())
        self.n_inputs = n_inputs

    @classmethod
    def from_op(cls, op: Op, compute_dtype: str = "fp32", flags: int = 0) -> "MoEFeedForward":
        if op.code != OP_MOE_FEED_FORWARD:
            raise ValueError(f"op code {op.code} is not OP_MOE_FEED_FORWARD ({OP_MOE_FEED_FORWARD})")
        return cls(op.int_params, op.float_params, len(op.inputs), compute_dtype, flags)

    # -- weights ---------------------------------------------------------
    def set_input(self, input_index: int, w) -> None:
        """Bind Op.Inputs[input_index] (1 = router_w, then expert matrices).
        `w` is a numpy array (fp32, or uint16 bf16 bits) or a
        (DeviceBuffer, dtype_code, shape) triple for device-resident data."""
        if isinstance(w, tuple):
            buf, code, shape = w
            shp = (ctypes.c_int64 * len(shape))(*shape)
            rc = self._lib.mxm_moe_set_input(self.handle, input_index, code, shp, len(shape),
                                             ctypes.c_void_p(buf.value), 1)
        else:
            a = np.ascontiguousarray(w)
            shp = (ctypes.c_int64 * a.ndim)(*a.shape)
            rc = self._lib.mxm_moe_set_input(self.handle, input_index, _np_dtype_code(a), shp,
                                             a.ndim, ctypes.c_void_p(a.ctypes.data), 0)
        _lib.check(rc, f"mxm_moe_set_input({input_index})")

    def set_input_q8(self, input_index: int, q: np.ndarray, scales: np.ndarray) -> None:
        """Bind an expert matrix as int8 q [in, out] with fp32 per-output-channel
        scales [out] (W = q * scales); the op must use MXM_FLAG_INT8_WEIGHTS."""
        q = np.ascontiguousarray(q, dtype=np.int8)
        sc = np.ascontiguousarray(scales, dtype=np.float32)
        shp = (ctypes.c_int64 * 2)(*q.shape)
        rc = self._lib.mxm_moe_set_input_q8(self.handle, input_index, ctypes.c_void_p(q.ctypes.data),
                                            ctypes.c_void_p(sc.ctypes.data), shp, 2, 0)
        _lib.check(rc, f"mxm_moe_set_input_q8({input_index})")

    def set_weights(self, router_w, expert_weights) -> None:
        """router_w [D, E]; expert_weights: per expert (w_gate, w_up, w_down) or (w_up, w_down)."""
        self.set_input(1, router_w)
        i = 2
        for ws in expert_weights:
            for w in ws:
                self.set_input(i, w)
                i += 1

    # -- forward -----------------------------------------------------------
    def forward_host(self, x: np.ndarray):
        """x [B*T, D] (fp32 or bf16 bits) -> (delta [B*T, D] fp32, aux, entropy)."""
        x = np.ascontiguousarray(x)
        delta = np.empty((x.shape[0], self.D), np.float32)
        aux = np.zeros(1, np.float32)
        ent = np.zeros(1, np.float32)
        rc = self._lib.mxm_moe_forward_host(self.handle, ctypes.c_void_p(x.ctypes.data),
                                            _np_dtype_code(x), x.shape[0],
                                            ctypes.c_void_p(delta.ctypes.data),
                                            ctypes.c_void_p(aux.ctypes.data),
                                            ctypes.c_void_p(ent.ctypes.data))
        _lib.check(rc, "mxm_moe_forward_host")
        return delta, float(aux[0]), float(ent[0])

    def forward(self, x_ptr: int, x_dtype: int, rows: int, delta_ptr: int,
                aux_ptr: int = 0, ent_ptr: int = 0) -> None:
        """Asynchronous forward on device pointers (ints)."""
        rc = self._lib.mxm_moe_forward(self.handle, ctypes.c_void_p(x_ptr), x_dtype, rows,
                                       ctypes.c_void_p(delta_ptr),
                                       ctypes.c_void_p(aux_ptr) if aux_ptr else None,
                                       ctypes.c_void_p(ent_ptr) if ent_ptr else None)
        _lib.check(rc, "mxm_moe_forward")

    def block_forward_host(self, x: np.ndarray, norm_scale: np.ndarray,
                           moe_scale: Optional[np.ndarray] = None, eps: float = 1e-5,
                           aux_weight: float = 0.01):
        """The MoE block of arch/moe.go:152-213 on host arrays: RMSNorm, op 74,
        optional moe_scale, residual add.  x [B*T, D] fp32 or bf16 bits; the
        scales [D] fp32 or bf16 bits (both the same dtype).  Returns
        (x_out [B*T, D] fp32, aux = aux_weight * aux_raw, entropy)."""
        x = np.ascontiguousarray(x)
        ns = np.ascontiguousarray(norm_scale)
        ms = None if moe_scale is None else np.ascontiguousarray(moe_scale, dtype=ns.dtype)
        out = np.empty((x.shape[0], self.D), np.float32)
        aux = np.zeros(1, np.float32)
        ent = np.zeros(1, np.float32)
        vp = lambda a: None if a is None else ctypes.c_void_p(a.ctypes.data)  # noqa: E731
        rc = self._lib.mxm_moe_block_forward_host(
            self.handle, vp(x), _np_dtype_code(x), x.shape[0], vp(ns), vp(ms), _np_dtype_code(ns),
            float(eps), float(aux_weight), vp(out), vp(aux), vp(ent))
        _lib.check(rc, "mxm_moe_block_forward_host")
        return out, float(aux[0]), float(ent[0])

    def block_forward(self, x_ptr: int, x_dtype: int, rows: int, norm_scale_ptr: int,
                      moe_scale_ptr: int, scale_dtype: int, eps: float, aux_weight: float,
                      out_ptr: int, aux_ptr: int = 0, ent_ptr: int = 0) -> None:
        """Asynchronous block forward on device pointers (ints; moe_scale_ptr 0 = none)."""
        vp = lambda p: ctypes.c_void_p(p) if p else None  # noqa: E731
        rc = self._lib.mxm_moe_block_forward(self.handle, vp(x_ptr), x_dtype, rows,
                                             vp(norm_scale_ptr), vp(moe_scale_ptr), scale_dtype,
                                             float(eps), float(aux_weight), vp(out_ptr),
                                             vp(aux_ptr), vp(ent_ptr))
        _lib.check(rc, "mxm_moe_block_forward")

    def backward_host(self, x: np.ndarray, d_delta: np.ndarray, d_aux: float = 0.0,
                      d_entropy: float = 0.0):
        """Gradients of op 74: returns (dx [B*T, D], d_router_w [D, E],
        d_experts: per expert a list of the weight gradients in Op.Inputs
        order, x.W layout).  x is fp32 (rounded to bf16 by the library under
        bf16 compute); the gradients are computed in fp32."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        dd = np.ascontiguousarray(d_delta, dtype=np.float32)
        wpe = 2 if self.expert_type == MOE_EXPERT_MLP else 3
        dx = np.empty_like(x)
        dwr = np.empty((self.D, self.E), np.float32)
        dw = np.empty(self.E * wpe * self.D * self.F, np.float32)
        vp = lambda a: ctypes.c_void_p(a.ctypes.data)  # noqa: E731
        rc = self._lib.mxm_moe_backward_host(self.handle, vp(x), _lib.MXM_DTYPE_F32, x.shape[0],
                                             vp(dd), float(d_aux), float(d_entropy), vp(dx),
                                             vp(dwr), vp(dw))
        _lib.check(rc, "mxm_moe_backward_host")
        D, F = self.D, self.F
        shapes = [(D, F), (D, F), (F, D)] if wpe == 3 else [(D, F), (F, D)]
        experts, off = [], 0
        for _ in range(self.E):
            ws = []
            for shp in shapes:
                ws.append(dw[off:off + D * F].reshape(shp))
                off += D * F
            experts.append(ws)
        return dx, dwr, experts

    def synchronize(self) -> None:
        _lib.check(self._lib.mxm_moe_synchronize(self.handle), "mxm_moe_synchronize")

    # -- inspection ----------------------------------------------------------
    def routing(self) -> dict:
        N, K, E = self.N, self.K, self.E
        top_idx = np.empty((N, K), np.int32)
        gates = np.empty((N, K), np.float32)
        counts = np.empty(E, np.int32)
        offsets = np.empty(E + 1, np.int32)
        perm = np.empty(N * K, np.int32)
        vp = lambda a: ctypes.c_void_p(a.ctypes.data)  # noqa: E731
        rc = self._lib.mxm_moe_routing(self.handle, vp(top_idx), vp(gates), vp(counts),
                                       vp(offsets), vp(perm), 1)
        _lib.check(rc, "mxm_moe_routing")
        return dict(top_idx=top_idx, gates=gates, counts=counts, offsets=offsets, perm=perm)

    def probs(self) -> np.ndarray:
        p = np.empty((self.N, self.E), np.float32)
        _lib.check(self._lib.mxm_moe_probs(self.handle, ctypes.c_void_p(p.ctypes.data)),
                   "mxm_moe_probs")
        return p

    def set_profiling(self, enable: bool, repeats: int = 1) -> None:
        """Record per-stage events in later forwards; with repeats > 1 each
        stage is launched that many times between its events."""
        code = 0 if not enable else max(1, int(repeats))
        _lib.check(self._lib.mxm_moe_set_profiling(self.handle, code), "set_profiling")

    def stage_times(self) -> dict:
        """Mean per-stage milliseconds over the forwards since set_profiling(True)."""
        ms = (ctypes.c_float * _lib.MXM_NUM_STAGES)()
        count = self._lib.mxm_moe_stage_times(self.handle, ms, _lib.MXM_NUM_STAGES)
        if count <= 0:
            _lib.check(count if count < 0 else -1, "mxm_moe_stage_times")
        out = {name: float(ms[i]) for i, name in enumerate(_lib.STAGE_NAMES)}
        out["forwards"] = count
        return out

    def info(self) -> dict:
        """mfma: the op's bf16 expert weights are on the MFMA family (bf16_stream:
        at these decode sizes the forward streams them through the decode
        kernels instead of the tiles); int8: the op's expert weights are int8
        (int8_kernels: on the int8 kernels, else on the MFMA tiles with the
        integers as bf16); ffn_kernel, d_kernel and
        d_reduce: the expert width, the down projection's output width and
        the up projection's reduction length the kernels run at (the op's
        ffn and D, or those rounded up to the tiles with zero weights);
        route_flow: how the last forward routed (0 tiled router + scan +
        scatter, 1 the one-launch router, 2 the int8 decode flow, -1 before
        any forward)."""
        arr = (ctypes.c_int64 * 8)()
        self._lib.mxm_moe_info(self.handle, arr, 8)
        kind = int(arr[0])
        return dict(mfma=kind in (1, 3, 4), int8=kind in (2, 3), int8_kernels=kind == 2,
                    bf16_stream=kind == 4,
                    workspace_bytes=int(arr[1]),
                    gemm_bm=int(arr[2]), router_tiles=int(arr[3]), ffn_kernel=int(arr[4]),
                    d_kernel=int(arr[5]), d_reduce=int(arr[6]), route_flow=int(arr[7]))

    def close(self) -> None:
        if getattr(self, "handle", 0):
            self._lib.mxm_moe_destroy(self.handle)
            self.handle = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class MoEBlock:
    """One MoE block as the emitter builds it (arch/moe.go:152-213): RMSNorm,
    op 74, aux weight, optional moe_scale, residual add -- run as one fused
    call (mxm_moe_block_forward).  Weights follow the block's metas
    (arch/moe.go:112-150): moe_norm_scale, router_w, per-expert matrices,
    then moe_scale when block_scales is on."""

    def __init__(self, spec: BlockSpec, B: int, T: int, D: int,
                 mlp_mult: float = DEFAULT_FFN_MULTIPLIER, block_scales: bool = False,
                 compute_dtype: str = "fp32", flags: int = 0):
        prog = Program()
        emit_moe_ir(prog, spec, "x", 0, D, T, B, 0, mlp_mult, block_scales)
        norm = next(op for op in prog.ops if op.code == OP_RMSNORM)
        ff = next(op for op in prog.ops if op.code == OP_MOE_FEED_FORWARD)
        self.program = prog
        self.eps = float(norm.float_params[0])
        self.aux_weight = float(effective_moe_load_balance_loss_weight(spec))
        self.metas = moe_weight_shapes(spec, D, mlp_mult, block_scales)
        self.block_scales = block_scales
        self.bf16 = compute_dtype in ("bf16", "bfloat16")
        self._int8 = bool(flags & _lib.MXM_FLAG_INT8_WEIGHTS)
        self.op = MoEFeedForward.from_op(ff, compute_dtype=compute_dtype, flags=flags)
        self.norm_scale = None
        self.moe_scale = None

    def _conv(self, a):
        from .workloads import bf16_bits
        return bf16_bits(a) if self.bf16 else np.ascontiguousarray(a, dtype=np.float32)

    def set_weights(self, weights) -> None:
        """fp32 arrays in meta order (as the checkpoint holds them); under
        bf16 compute they are cast to bf16 (gpu/ir_trainer.cpp:1395-1412)."""
        if len(weights) != len(self.metas):
            raise ValueError(f"moe block takes {len(self.metas)} weights, got {len(weights)}")
        for m, w in zip(self.metas, weights):
            if list(np.shape(w)) != list(m.shape):
                raise ValueError(f"{m.name}: shape {list(np.shape(w))}, want {m.shape}")
        self.norm_scale = self._conv(weights[0])
        self.op.set_input(1, self._conv(weights[1]))
        n_exp = len(self.metas) - 2 - (1 if self.block_scales else 0)
        for i in range(n_exp):
            self.op.set_input(2 + i, self._conv(weights[2 + i]))
        self.moe_scale = self._conv(weights[-1]) if self.block_scales else None

    def load(self, path: str, first_index: int = 0) -> None:
        """Bind the block's weights from a native checkpoint (tensors
        w{first_index + i}_{meta name}, train/import.go:71-89)."""
        from .weights import load_weights
        self.set_weights(load_weights(path, self.metas, first_index))

    def load_quantized(self, path: str, first_index: int = 0) -> None:
        """Bind the block's weights from a checkpoint the reference's quantized
        export wrote (train/export.go:203-352: I8 matrices with per-row F32
        scales, small and 1-D tensors F32).  The block's op must use int8
        weights (MXM_FLAG_INT8_WEIGHTS): each expert matrix goes to the
        executor in its per-output-channel form (requantised from the
        dequantised values); the router, norm and moe_scale are bound as
        their dequantised values."""
        from .weights import QuantizedWeight, load_quantized_weights, quantize_per_channel
        if self.op.info()["mfma"] or not self._int8:
            raise ValueError("load_quantized needs a block created with int8 expert weights")
        got = load_quantized_weights(path, self.metas, first_index)
        dense = [g.dequantize() if isinstance(g, QuantizedWeight) else g for g in got]
        self.norm_scale = self._conv(dense[0])
        self.op.set_input(1, self._conv(dense[1]))
        n_exp = len(self.metas) - 2 - (1 if self.block_scales else 0)
        for i in range(n_exp):
            g = got[2 + i]
            q, sc = g.per_channel() if isinstance(g, QuantizedWeight) else quantize_per_channel(g)
            self.op.set_input_q8(2 + i, q, sc)
        self.moe_scale = self._conv(dense[-1]) if self.block_scales else None

    def forward_host(self, x: np.ndarray):
        """x [B*T, D] (fp32, or bf16 bits) -> (x + delta [B*T, D] fp32,
        aux = load-balance weight * aux_raw, router entropy)."""
        if self.norm_scale is None:
            raise ValueError("moe block weights are not set")
        return self.op.block_forward_host(x, self.norm_scale, self.moe_scale, self.eps,
                                          self.aux_weight)

    def close(self) -> None:
        self.op.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
