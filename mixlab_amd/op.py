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
from .moe import MOE_EXPERT_MLP, OP_MOE_FEED_FORWARD, Op

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

    def set_profiling(self, enable: bool) -> None:
        _lib.check(self._lib.mxm_moe_set_profiling(self.handle, int(enable)), "set_profiling")

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
        arr = (ctypes.c_int64 * 4)()
        self._lib.mxm_moe_info(self.handle, arr, 4)
        return dict(mfma=arr[0] == 1, int8=arr[0] == 2, workspace_bytes=int(arr[1]),
                    gemm_bm=int(arr[2]), router_tiles=int(arr[3]))

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
