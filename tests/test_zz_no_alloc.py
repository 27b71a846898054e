"""mxm_moe_forward_noalloc (include/mixmoe.h) against mxm_moe_forward: the
same kernels on a per-GPU device scratch array instead of the op's own
workspace, so outputs and routing must match bit for bit.  Two calls in a
row share the scratch, the second with a smaller op; device memory must not
change across them; an op whose workspace exceeds the scratch is refused."""
import ctypes
import os

import numpy as np
import pytest

from mixlab_amd import _lib
from mixlab_amd.workloads import bf16_bits, quantize_int8, round_bf16

pytestmark = pytest.mark.gpu


def _hip_free_bytes() -> int:
    for name in ("/opt/rocm/lib/libamdhip64.so", "libamdhip64.so"):
        if name.startswith("/") and not os.path.exists(name):
            continue
        hip = ctypes.CDLL(name)
        free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
        assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
        return int(free.value)
    raise RuntimeError("HIP runtime library not found")


class Dev:
    """A device buffer from mxm_malloc."""

    def __init__(self, lib, nbytes):
        self.lib = lib
        self.p = ctypes.c_void_p()
        _lib.check(lib.mxm_malloc(ctypes.byref(self.p), max(int(nbytes), 4)), "mxm_malloc")
        self.nbytes = nbytes

    def put(self, a):
        a = np.ascontiguousarray(a)
        _lib.check(self.lib.mxm_memcpy_h2d(self.p, a.ctypes.data_as(ctypes.c_void_p), a.nbytes),
                   "h2d")

    def get(self, shape, dtype):
        out = np.empty(shape, dtype)
        _lib.check(self.lib.mxm_memcpy_d2h(out.ctypes.data_as(ctypes.c_void_p), self.p,
                                           out.nbytes), "d2h")
        return out

    def free(self):
        self.lib.mxm_free(self.p)


def _make_op(seed, B, T, D, E, K, F, etype=0, act=0, dtype="bf16", int8=False):
    from mixlab_amd.op import MoEFeedForward

    rng = np.random.default_rng(seed)
    wpe = 2 if etype == 2 else 3
    flags = _lib.MXM_FLAG_INT8_WEIGHTS if int8 else 0
    op = MoEFeedForward([B, T, D, E, K, etype, F, act], [0.3], compute_dtype=dtype, flags=flags)
    conv = bf16_bits if dtype == "bf16" else (lambda a: np.ascontiguousarray(a, np.float32))
    wr = round_bf16(rng.standard_normal((D, E), dtype=np.float32) * np.float32(0.1))
    op.set_input(1, conv(wr))
    for e in range(E):
        for j in range(wpe):
            shape = (F, D) if j == wpe - 1 else (D, F)
            w = rng.standard_normal(shape, dtype=np.float32) * np.float32(0.03)
            if int8:
                op.set_input_q8(2 + e * wpe + j, *quantize_int8(w))
            else:
                op.set_input(2 + e * wpe + j, conv(round_bf16(w) if dtype == "bf16" else w))
    x = rng.standard_normal((B * T, D), dtype=np.float32)
    xh = bf16_bits(round_bf16(x)) if dtype == "bf16" else x
    return op, xh


class IO:
    """Device input and output buffers of one op, allocated once."""

    def __init__(self, lib, op, xh):
        self.lib, self.op, self.xh = lib, op, xh
        self.x = Dev(lib, xh.nbytes)
        self.x.put(xh)
        self.delta = Dev(lib, op.N * op.D * 4)
        self.aux, self.ent = Dev(lib, 4), Dev(lib, 4)

    def forward(self, noalloc):
        code = _lib.MXM_DTYPE_BF16 if self.xh.dtype == np.uint16 else _lib.MXM_DTYPE_F32
        fn = self.lib.mxm_moe_forward_noalloc if noalloc else self.lib.mxm_moe_forward
        _lib.check(fn(self.op.handle, self.x.p, code, self.op.N, self.delta.p, self.aux.p,
                      self.ent.p), "forward")

    def results(self):
        """delta, aux, entropy and the routing of the op's last forward."""
        self.op.synchronize()
        return (self.delta.get((self.op.N, self.op.D), np.float32),
                float(self.aux.get(1, np.float32)[0]), float(self.ent.get(1, np.float32)[0]),
                self.op.routing())

    def free(self):
        for b in (self.x, self.delta, self.aux, self.ent):
            b.free()


# (name, big op, smaller op): each pair shares the device scratch, big first
FAMILIES = [
    ("bf16_mfma_tiled", dict(B=2, T=1100, D=512, E=8, K=2, F=1024),
     dict(B=1, T=1030, D=256, E=8, K=2, F=512)),
    ("bf16_mfma_decode", dict(B=1, T=700, D=512, E=16, K=4, F=512),
     dict(B=1, T=400, D=1024, E=8, K=2, F=256)),
    ("geglu_split", dict(B=1, T=1500, D=256, E=6, K=2, F=512, etype=1, act=1),
     dict(B=1, T=300, D=256, E=6, K=2, F=256, etype=1, act=1)),
    ("int8_decode", dict(B=1, T=512, D=1024, E=32, K=4, F=1024, int8=True),
     dict(B=1, T=64, D=512, E=8, K=2, F=512, int8=True)),
    # int8 weights at 96 or more rows per expert: the MFMA tiles, scaled
    ("int8_mfma", dict(B=1, T=1100, D=512, E=8, K=2, F=1024, int8=True),
     dict(B=1, T=700, D=256, E=4, K=2, F=512, int8=True)),
    ("fp32_simt", dict(B=1, T=2400, D=128, E=4, K=2, F=256, dtype="fp32"),
     dict(B=1, T=33, D=128, E=4, K=2, F=128, dtype="fp32")),
    # bf16 weights at decode sizes, streamed by the decode kernels (split
    # hidden: H in two planes, y fp32)
    ("bf16_stream", dict(B=1, T=600, D=512, E=64, K=2, F=1024, etype=1, act=1),
     dict(B=1, T=64, D=256, E=8, K=2, F=256)),
    # the tiled router's logits on the matrix cores (32 < E <= 64)
    ("bf16_router64", dict(B=1, T=1100, D=256, E=64, K=8, F=256),
     dict(B=1, T=1030, D=128, E=48, K=4, F=128)),
]


@pytest.mark.parametrize("name,big,small", FAMILIES, ids=[f[0] for f in FAMILIES])
def test_noalloc_matches_forward(gpu_lib, name, big, small):
    lib = _lib.init()
    print(f"no-alloc {name}", flush=True)
    ops = [_make_op(1, **big), _make_op(2, **small)]
    ios = [IO(lib, op, xh) for op, xh in ops]
    try:
        for op, _ in ops:
            assert op.info()["workspace_bytes"] <= _lib.MXM_NOALLOC_MAX_BYTES
        # the first op's workspace is well above the memory check's slack
        assert ops[0][0].info()["workspace_bytes"] > 6 << 20
        if big.get("int8"):  # the int8 kernels, or the MFMA tiles scaled
            for op, _ in ops:
                assert op.info()["int8_kernels"] == (name == "int8_decode")
        for op, _ in ops:
            assert op.info()["bf16_stream"] == (name == "bf16_stream")
        for io in ios:  # first launches: the runtime's own lazy setup
            io.forward(noalloc=True)
            io.results()
        free0 = _hip_free_bytes()
        got = []
        for io in ios:  # two calls in a row, the second op smaller
            io.forward(noalloc=True)
            got.append(io.results())
        free1 = _hip_free_bytes()
        want = []
        for io in ios:
            io.forward(noalloc=False)
            want.append(io.results())
        free2 = _hip_free_bytes()
        # no device memory taken by the no-alloc calls; the allocating
        # forwards take their ops' workspaces
        assert abs(free1 - free0) <= 2 << 20, (free0, free1)
        assert free1 - free2 >= ops[0][0].info()["workspace_bytes"] - (2 << 20), (free1, free2)
        for (d, a, e, r), (wd, wa, we, wr) in zip(got, want):
            assert np.array_equal(d.view(np.uint32), wd.view(np.uint32))
            assert a == wa and e == we
            for k in ("top_idx", "gates", "counts", "offsets", "perm"):
                assert np.array_equal(r[k], wr[k]), k
    finally:
        for io in ios:
            io.free()
        for op, _ in ops:
            op.close()


def _random_pairs(n=6, seed=2030):
    """Seeded pairs of op shapes over every flow, each workspace within the
    scratch array (the draw is repeated otherwise)."""
    rng = np.random.default_rng(seed)
    kinds = [(0, 0), (1, 1), (2, 0), (2, 1), (2, 2), (2, 3)]
    flows = [dict(dtype="fp32"), dict(dtype="bf16"), dict(dtype="bf16", int8=True)]

    def draw(flow):
        etype, act = kinds[int(rng.integers(len(kinds)))]
        E = int(rng.integers(1, 65))
        return dict(B=1, T=int(rng.integers(1, 3000)), D=int(rng.integers(16, 900)), E=E,
                    K=int(rng.integers(1, min(E, 8) + 1)), F=int(rng.integers(16, 1200)),
                    etype=etype, act=act, **flow)

    def fits(c):
        NK = c["T"] * c["K"]
        # a generous bound on the workspace (H and Y at 4 bytes per element
        # in padded widths, plus the routing tables)
        return NK * (2 * (c["F"] + 128) + (c["D"] + 128)) * 4 + (8 << 20) < (48 << 20)

    pairs = []
    while len(pairs) < n:
        flow = flows[len(pairs) % 3]
        first, second = draw(flow), draw(flow)
        if fits(first) and fits(second):
            pairs.append((first, second))
    return pairs


RANDOM_PAIRS = _random_pairs()


@pytest.mark.parametrize("first,second", RANDOM_PAIRS,
                         ids=[f"{b.get('dtype')}{'-int8' if b.get('int8') else ''}-T{b['T']}"
                              f"-D{b['D']}-E{b['E']}" for b, _ in RANDOM_PAIRS])
def test_noalloc_random_pairs(gpu_lib, first, second):
    """Random op shapes through the no-allocation forward, two ops in a row
    on the shared scratch: bit for bit the allocating forward's results."""
    lib = _lib.init()
    print(f"no-alloc random {first} then {second}", flush=True)
    ops = [_make_op(3, **first), _make_op(4, **second)]
    ios = [IO(lib, op, xh) for op, xh in ops]
    try:
        for op, _ in ops:
            assert op.info()["workspace_bytes"] <= _lib.MXM_NOALLOC_MAX_BYTES
        got = []
        for io in ios:
            io.forward(noalloc=True)
            got.append(io.results())
        want = []
        for io in ios:
            io.forward(noalloc=False)
            want.append(io.results())
        for (d, a, e, r), (wd, wa, we, wr) in zip(got, want):
            assert np.array_equal(d.view(np.uint32), wd.view(np.uint32))
            assert a == wa and e == we
            for k in ("top_idx", "gates", "counts", "offsets", "perm"):
                assert np.array_equal(r[k], wr[k]), k
    finally:
        for io in ios:
            io.free()
        for op, _ in ops:
            op.close()


def test_noalloc_refuses_oversized_workspace(gpu_lib):
    """2^17 tokens x top-2 x F 256 in bf16 needs 128 MiB for H alone."""
    from mixlab_amd.op import MoEFeedForward

    lib = _lib.init()
    N, D = 1 << 17, 256
    with MoEFeedForward([1, N, D, 2, 2, 0, 256, 0], [0.0], compute_dtype="bf16") as op:
        assert op.info()["workspace_bytes"] > _lib.MXM_NOALLOC_MAX_BYTES
        xd, dd = Dev(lib, N * D * 2), Dev(lib, N * D * 4)
        try:
            rc = lib.mxm_moe_forward_noalloc(op.handle, xd.p, _lib.MXM_DTYPE_BF16, N, dd.p, None,
                                             None)
        finally:
            xd.free()
            dd.free()
        assert rc != 0
        msg = _lib.last_error()
        assert "above the 67108864-byte device scratch" in msg, msg
