"""ctypes binding of libmixmoe.so (include/mixmoe.h).

There is no CPU fallback: if the HIP library is missing or no GPU is present
the calls raise.  ``load()`` only needs the shared library (no device), so the
exported symbols can be checked on a machine without a GPU.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libmixmoe.so"

MXM_OK = 0
MXM_ERR = -1
MXM_ERR_ARGS = -10
MXM_ERR_INIT = -11
MXM_ERR_OP = -12
MXM_DTYPE_INT32 = 0
MXM_DTYPE_F32 = 1
MXM_DTYPE_BF16 = 2
MXM_DTYPE_I8 = 3
MXM_FLAG_FORCE_SIMT = 1
MXM_FLAG_DEBUG_PROBS = 2
MXM_FLAG_MFMA_TILE128 = 4
MXM_FLAG_MFMA_TILE256x128 = 8
MXM_FLAG_MFMA_TILE256x256 = 12
MXM_FLAG_INT8_WEIGHTS = 16
MXM_FLAG_KEEP_FOR_BACKWARD = 32
MXM_NUM_STAGES = 6
MXM_NOALLOC_MAX_BYTES = 64 << 20
STAGE_NAMES = ("router", "scan", "scatter", "gemm_up", "gemm_down", "combine")

# name -> (restype, argtypes); every function declared in include/mixmoe.h
_VP = ctypes.c_void_p
_I64P = ctypes.POINTER(ctypes.c_int64)
_I32P = ctypes.POINTER(ctypes.c_int32)
_F32P = ctypes.POINTER(ctypes.c_float)
SIGNATURES = {
    "mxm_init": (ctypes.c_int, []),
    "mxm_device_name": (ctypes.c_char_p, []),
    "mxm_last_error": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int]),
    "mxm_malloc": (ctypes.c_int, [ctypes.POINTER(_VP), ctypes.c_int64]),
    "mxm_free": (ctypes.c_int, [_VP]),
    "mxm_memcpy_h2d": (ctypes.c_int, [_VP, _VP, ctypes.c_int64]),
    "mxm_memcpy_d2h": (ctypes.c_int, [_VP, _VP, ctypes.c_int64]),
    "mxm_memcpy_d2d": (ctypes.c_int, [_VP, _VP, ctypes.c_int64]),
    "mxm_device_synchronize": (ctypes.c_int, []),
    "mxm_moe_create": (ctypes.c_int64, [_F32P, ctypes.c_int, _I32P, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int]),
    "mxm_moe_destroy": (ctypes.c_int, [ctypes.c_int64]),
    "mxm_moe_set_input": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int, ctypes.c_int, _I64P,
                                         ctypes.c_int, _VP, ctypes.c_int]),
    "mxm_moe_set_input_q8": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int, _VP, _VP, _I64P,
                                            ctypes.c_int, ctypes.c_int]),
    "mxm_moe_forward": (ctypes.c_int, [ctypes.c_int64, _VP, ctypes.c_int, ctypes.c_int64, _VP,
                                       _VP, _VP]),
    "mxm_moe_forward_host": (ctypes.c_int, [ctypes.c_int64, _VP, ctypes.c_int, ctypes.c_int64,
                                            _VP, _VP, _VP]),
    "mxm_moe_forward_noalloc": (ctypes.c_int, [ctypes.c_int64, _VP, ctypes.c_int,
                                               ctypes.c_int64, _VP, _VP, _VP]),
    "mxm_moe_block_forward": (ctypes.c_int, [ctypes.c_int64, _VP, ctypes.c_int, ctypes.c_int64,
                                             _VP, _VP, ctypes.c_int, ctypes.c_float,
                                             ctypes.c_float, _VP, _VP, _VP]),
    "mxm_moe_block_forward_host": (ctypes.c_int, [ctypes.c_int64, _VP, ctypes.c_int,
                                                  ctypes.c_int64, _VP, _VP, ctypes.c_int,
                                                  ctypes.c_float, ctypes.c_float, _VP, _VP, _VP]),
    "mxm_moe_backward": (ctypes.c_int, [ctypes.c_int64, _VP, ctypes.c_int, ctypes.c_int64, _VP,
                                        ctypes.c_float, ctypes.c_float, _VP, _VP, _VP]),
    "mxm_moe_backward_host": (ctypes.c_int, [ctypes.c_int64, _VP, ctypes.c_int, ctypes.c_int64,
                                             _VP, ctypes.c_float, ctypes.c_float, _VP, _VP, _VP]),
    "mxm_moe_backward_kept": (ctypes.c_int, [ctypes.c_int64, _VP, ctypes.c_float, ctypes.c_float,
                                             _VP, _VP, _VP]),
    "mxm_moe_synchronize": (ctypes.c_int, [ctypes.c_int64]),
    "mxm_moe_routing": (ctypes.c_int, [ctypes.c_int64, _VP, _VP, _VP, _VP, _VP, ctypes.c_int]),
    "mxm_moe_probs": (ctypes.c_int, [ctypes.c_int64, _VP]),
    "mxm_moe_set_profiling": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int]),
    "mxm_moe_stage_times": (ctypes.c_int, [ctypes.c_int64, _F32P, ctypes.c_int]),
    "mxm_moe_info": (ctypes.c_int, [ctypes.c_int64, _I64P, ctypes.c_int]),
}

_lib = None
_initialised = False


class MixMoEError(RuntimeError):
    pass


def load():
    """Load libmixmoe.so and bind every entry point (no device needed)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise MixMoEError(
                f"{LIB_PATH} is missing: build it with `python -m mixlab_amd.build` "
                "(hipcc, gfx950); there is no CPU fallback")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    lib = load()
    buf = ctypes.create_string_buffer(1024)
    lib.mxm_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != MXM_OK:
        raise MixMoEError(f"{what}: {last_error()} (rc={rc})")


def init() -> ctypes.CDLL:
    """Load the library and initialise the HIP device; raises without a GPU."""
    global _initialised
    lib = load()
    if not _initialised:
        check(lib.mxm_init(), "mxm_init")
        _initialised = True
    return lib


def device_name() -> str:
    return init().mxm_device_name().decode()


class DeviceBuffer:
    """Device memory from mxm_malloc, released on close()/garbage collection."""

    def __init__(self, nbytes: int):
        self._lib = init()
        self.ptr = ctypes.c_void_p()
        self.nbytes = int(nbytes)
        check(self._lib.mxm_malloc(ctypes.byref(self.ptr), self.nbytes), "mxm_malloc")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    @property
    def value(self) -> int:
        return self.ptr.value or 0

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("array larger than the device buffer")
        check(self._lib.mxm_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes), "mxm_memcpy_h2d")

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("requested more bytes than the device buffer holds")
        check(self._lib.mxm_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes), "mxm_memcpy_d2h")
        return out

    def close(self) -> None:
        if self.ptr.value:
            self._lib.mxm_free(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
