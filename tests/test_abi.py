"""libmixmoe's C ABI without a GPU: the library loads, exports every function
include/mixmoe.h declares with the binding's signatures, the header's
constants match the binding's, and op creation rejects bad parameters with
the reference's messages (gpu/ir.cpp:1076-1104) before touching a device.
Also: the product package never imports the CPU checker."""
from __future__ import annotations

import ast
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from mixlab_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = (ROOT / "include" / "mixmoe.h").read_text()


def _declared_functions() -> list[str]:
    body = re.sub(r"/\*.*?\*/", "", HEADER, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(mxm_[a-z_0-9]+)\s*\(", body, flags=re.M)


def _defines() -> dict:
    return {m.group(1): int(m.group(2))
            for m in re.finditer(r"^#define\s+(MXM_[A-Z0-9_a-z]+)\s+(-?\d+)", HEADER, flags=re.M)}


def test_header_declares_the_bound_functions():
    declared = _declared_functions()
    assert len(declared) == len(set(declared)) >= 20
    assert set(declared) == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT\s+(mxm_\w+)", out))
    assert set(_declared_functions()) <= exported


def test_header_constants_match_binding():
    d = _defines()
    for name in ("MXM_OK", "MXM_ERR", "MXM_ERR_ARGS", "MXM_ERR_INIT", "MXM_ERR_OP",
                 "MXM_DTYPE_INT32", "MXM_DTYPE_F32", "MXM_DTYPE_BF16", "MXM_DTYPE_I8",
                 "MXM_FLAG_FORCE_SIMT", "MXM_FLAG_DEBUG_PROBS", "MXM_FLAG_MFMA_TILE128",
                 "MXM_FLAG_MFMA_TILE256x128", "MXM_FLAG_MFMA_TILE256x256",
                 "MXM_FLAG_INT8_WEIGHTS", "MXM_FLAG_KEEP_FOR_BACKWARD", "MXM_NUM_STAGES"):
        assert d[name] == getattr(_lib, name), name
    assert d["MXM_OP_MOE_FEED_FORWARD"] == 74
    m = re.search(r"^#define\s+MXM_NOALLOC_MAX_BYTES\s+\((\d+)ll << (\d+)\)", HEADER, flags=re.M)
    assert m and int(m.group(1)) << int(m.group(2)) == _lib.MXM_NOALLOC_MAX_BYTES
    stage_defs = sorted((v, k) for k, v in d.items() if k.startswith("MXM_STAGE_"))
    assert [k[len("MXM_STAGE_"):].lower() for _, k in stage_defs] == list(_lib.STAGE_NAMES)


def _create(int_params, n_inputs, dtype=_lib.MXM_DTYPE_F32, flags=0, floats=(0.0,)):
    lib = _lib.load()
    ip = (ctypes.c_int32 * max(1, len(int_params)))(*int_params)
    fp = (ctypes.c_float * len(floats))(*floats)
    return lib.mxm_moe_create(fp, len(floats), ip, len(int_params), n_inputs, dtype, flags)


@pytest.mark.parametrize("int_params,n_inputs,dtype,flags,want", [
    ([1, 4, 3, 3, 2, 0, 4], 11, 1, 0, "requires B,T,D,E,topK,expertType,ffn,activation"),
    ([1, 4, 3, 3, 4, 0, 4, 0], 11, 1, 0, "invalid dimensions"),
    ([1, 4, 3, 3, 0, 0, 4, 0], 11, 1, 0, "invalid dimensions"),
    ([0, 4, 3, 3, 2, 0, 4, 0], 11, 1, 0, "invalid dimensions"),
    ([1, 4, 3, 3, 2, 0, 0, 0], 11, 1, 0, "invalid dimensions"),
    ([1, 4, 3, 3, 2, 5, 4, 0], 11, 1, 0, "unsupported expert type"),
    ([1, 4, 3, 3, 2, 2, 4, 9], 8, 1, 0, "unsupported activation"),
    ([1, 4, 3, 3, 2, 0, 4, 0], 10, 1, 0, "unexpected expert weight input count"),
    ([1, 4, 3, 3, 2, 2, 4, 0], 11, 1, 0, "unexpected expert weight input count"),
    ([1, 4, 3, 300, 2, 2, 4, 0], 602, 1, 0, "at most 256 experts"),
    ([1, 4, 64, 3, 2, 0, 64, 0], 11, 1, 16, "int8 weights need bf16 compute"),
    ([1, 4, 65536, 3, 2, 0, 65536, 0], 11, 2, 16, "fewer than 2^31 entries"),
    ([1, 4, 3, 3, 2, 0, 4, 0], 11, 7, 0, "compute dtype"),
    ([32768, 32768, 3, 3, 2, 0, 4, 0], 11, 1, 0, "routed slots exceeds 2147483647"),
])
def test_create_rejects_bad_parameters(int_params, n_inputs, dtype, flags, want):
    handle = _create(int_params, n_inputs, dtype, flags)
    assert handle == 0
    msg = _lib.last_error()
    assert msg.startswith("OP_MOE_FEED_FORWARD") and want in msg, msg


def test_status_code_classes():
    """gpu/mlx_bridge.cpp:814-823: -10 for an argument the call cannot take,
    -11 when the runtime cannot be initialised, -12 for a handle that is not
    live.  An argument error is reported before any device call."""
    lib = _lib.load()
    assert lib.mxm_malloc(None, 16) == _lib.MXM_ERR_ARGS
    assert "bad arguments" in _lib.last_error()
    assert lib.mxm_moe_backward_kept(987654321, None, 0.0, 0.0, None, None, None) == _lib.MXM_ERR_OP
    if not Path("/dev/kfd").exists():  # no GPU here: initialisation must fail as such
        assert lib.mxm_init() == _lib.MXM_ERR_INIT
        assert "device" in _lib.last_error()


def test_bad_handle_and_error_truncation():
    lib = _lib.load()
    assert lib.mxm_moe_synchronize(987654321) == -12
    assert "invalid handle" in _lib.last_error()
    full = lib.mxm_last_error(None, 0)
    buf = ctypes.create_string_buffer(8)
    assert lib.mxm_last_error(buf, 8) == full
    assert len(buf.value) == 7  # truncated and NUL terminated


def _oracle_imports(tree):
    for node in ast.walk(tree):
        if isinstance(node, ast.ImportFrom) and (node.module or "").split(".")[0] == "oracle":
            yield node
        elif isinstance(node, ast.Import) and any(a.name.split(".")[0] == "oracle"
                                                  for a in node.names):
            yield node


def test_product_never_imports_the_checker():
    for path in (ROOT / "mixlab_amd").rglob("*.py"):
        assert not list(_oracle_imports(ast.parse(path.read_text()))), path
    # bench.py loads the checker only inside its cpu_baseline leg
    tree = ast.parse((ROOT / "bench.py").read_text())
    inside = set()
    for fn in ast.walk(tree):
        if isinstance(fn, ast.FunctionDef) and fn.name == "cpu_baseline":
            inside = {id(n) for n in _oracle_imports(fn)}
    all_imports = list(_oracle_imports(tree))
    assert all_imports and all(id(n) in inside for n in all_imports)
