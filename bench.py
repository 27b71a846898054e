#!/usr/bin/env python3
"""MoE layer forward throughput on one MI355X (libmixmoe, op 74).

A step is one forward of the MoE feed-forward op (router, dispatch, grouped
expert FFN, combine) over the whole batch, with inputs and weights resident
in HBM.  The headline workload is C4: d_model 2048, 64 experts, top-8, gated
expert hidden 1024, 65,536 tokens, bf16; `roofline` is its grouped GEMM
(both launches) against the bf16 MFMA peak.  The same run also measures C2
and C3 (the near-uniform and the Zipf-ragged MFMA-bound configurations,
under "configs", with C2 also with int8 expert weights), C5, the decode
shape with int8 expert weights (64 tokens;
HBM-bound, under "decode_int8", with the same shape in bf16 under its
"bf16_weights"), the backward on the C2 shape (fp32 and
bf16), on the Zipf-ragged C3 shape and on the headline shape (bf16), and the
CPU baseline.  Prints one JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C4]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

METRIC = "MoE layer tokens/sec at d=2048,64e top-8; grouped-GEMM % MFMA peak"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA (AMD published)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E (AMD published)
PEAK_FP32_TFLOPS = 157.3    # MI355X fp32, matrix and vector (AMD published)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def stage_bytes(cfg) -> dict:
    """Algorithmic HBM bytes per launch of the memory-bound stages."""
    N, D, E, K = cfg.N, cfg.D, cfg.E, cfg.K
    xb = 2 if cfg.dtype == "bf16" else 4
    NK = N * K
    tiles = (N + 63) // 64
    return {
        # x read, router weights, top_idx + gates + ranks written, tile partials
        "router": N * D * xb + D * E * xb + NK * 12 + tiles * E * 8,
        # top_idx, ranks, tile bases read; perm, slot_pos written
        "scatter": NK * 4 * 2 + NK * 4 * 2,
        # K rows of y per token, gates + idx + pos, delta written fp32
        "combine": NK * D * (2 if cfg.dtype == "bf16" else 4) + NK * 12 + N * D * 4,
    }


def int8_weight_bytes(cfg, counts) -> dict:
    """Expert weight bytes the int8 kernels read: only experts with rows."""
    routed = int(np.count_nonzero(counts))
    D, F = cfg.D, cfg.F
    up = routed * ((2 if cfg.wpe == 3 else 1) * D * F + (2 if cfg.wpe == 3 else 1) * F * 4)
    down = routed * (F * D + D * 4)
    return {"routed_experts": routed, "gemm_up": up, "gemm_down": down}


def bf16_weight_bytes(cfg, counts) -> dict:
    """Expert weight bytes a bf16 decode forward streams: experts with rows."""
    routed = int(np.count_nonzero(counts))
    D, F = cfg.D, cfg.F
    up = routed * (2 if cfg.wpe == 3 else 1) * D * F * 2
    return {"routed_experts": routed, "gemm_up": up, "gemm_down": routed * F * D * 2}


def measured_traffic(workload: str, stage: str, flags: int):
    """HBM bytes per launch of a stage's kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (profiles/roofline_traffic.json); None
    when absent or when non-default flags select another kernel."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "roofline_traffic.json")
    if flags or not os.path.exists(path):
        return None
    with open(path) as f:
        entry = json.load(f).get(workload, {}).get(stage)
    return None if entry is None else int(entry["fetch_bytes"] + entry["write_bytes"])


CPU_RUNS = 5         # timed runs of the CPU baseline after one warm-up (median reported)
CPU_MIN_TOKENS = 4096  # smallest contiguous token slice timed


def gemm_traffic(workload: str, flags: int):
    """HBM bytes of the grouped GEMM of one forward (both launches)."""
    up, down = measured_traffic(workload, "gemm_up", flags), measured_traffic(workload,
                                                                               "gemm_down", flags)
    return None if up is None or down is None else up + down


def layer_traffic(workload: str, stages, flags: int):
    """HBM bytes of one whole forward: the sum over its launches."""
    parts = [measured_traffic(workload, s, flags) for s in stages]
    return None if any(p is None for p in parts) else sum(parts)


def cpu_baseline(w, cfg, target_s: float) -> dict:
    """Time the dense fp32 BLAS restatement of the reference algorithm
    (oracle/dense_blas.py: every expert on every token, gpu/ir.cpp:1118-1148)
    on the first n tokens of the same workload: n is at least 4,096 and
    grows until one run takes about target_s (the whole N if that fits); one
    warm-up, then the median of 5 runs, scaled to tokens/s (the dense cost is
    linear in n).  All host cores run the BLAS threads."""
    from threadpoolctl import threadpool_info

    from oracle.dense_blas import dense_forward

    blas_threads = max((p.get("num_threads", 1) for p in threadpool_info()
                        if p.get("user_api") == "blas"), default=1)
    mats = {}

    def mat(e, j):
        if (e, j) not in mats:
            mats[(e, j)] = np.ascontiguousarray(w.matrix(e, j), dtype=np.float32)
        return mats[(e, j)]

    def run(n):
        t0 = time.perf_counter()
        dense_forward(w.x[:n], w.router_w, mat, cfg.E, cfg.K, cfg.expert_type, cfg.activation,
                      cfg.leaky_slope)
        return time.perf_counter() - t0

    run(min(cfg.N, 64))  # converts the weights once
    n = min(cfg.N, 256)
    t = run(n)
    # the run time is linear in n: size the slice for target_s per run
    n = int(min(cfg.N, max(CPU_MIN_TOKENS, n * target_s / max(t, 1e-6))))
    n = min(cfg.N, max(CPU_MIN_TOKENS, n // 256 * 256))
    run(n)  # warm-up at the timed size
    times = [run(n) for _ in range(CPU_RUNS)]
    med = float(np.median(times))
    blas = next((f"{p.get('internal_api', 'blas')} {p.get('version', '')}".strip()
                 for p in threadpool_info() if p.get("user_api") == "blas"), "BLAS")
    nproc = os.cpu_count() or 1
    return {"value": n / med, "unit": "tokens/s", "cores": int(blas_threads), "kind": "port",
            "nproc": int(nproc), "blas_threads": int(blas_threads), "cpu_model": _cpu_model(),
            "blas": blas, "runs": CPU_RUNS, "run_s": [round(x, 3) for x in times],
            "sample": (f"first {n} of {cfg.N} tokens, dense fp32 (all {cfg.E} experts on every "
                       f"token, gpu/ir.cpp:1118-1148) with numpy sgemm ({blas}, "
                       f"{int(blas_threads)} threads; nproc {nproc}) on {_cpu_model()}; median "
                       f"of {CPU_RUNS} runs of {med:.2f} s after one warm-up")}


def _cpu_model() -> str:
    """The host CPU's model name (Linux /proc/cpuinfo), or 'unknown CPU'."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def grouped_gemm_summary(cfg, stages) -> dict:
    """The grouped GEMM of one forward (gate+up launch, then down launch):
    algorithmic FLOPs (6 K N D F for a GLU expert, 4 K N D F for an mlp
    expert; arch/moe.go:215-236) over the two launches' event times."""
    fl = cfg.flops()
    up = fl["up"] / (stages["gemm_up"] * 1e-3) / 1e12
    down = fl["down"] / (stages["gemm_down"] * 1e-3) / 1e12
    ms = stages["gemm_up"] + stages["gemm_down"]
    tf = fl["experts"] / (ms * 1e-3) / 1e12
    return {"ms": ms, "tflops": tf, "frac": tf / PEAK_BF16_TFLOPS, "up_tflops": up,
            "down_tflops": down, "up_frac": up / PEAK_BF16_TFLOPS,
            "down_frac": down / PEAK_BF16_TFLOPS, "flops": fl["experts"]}


def run_config(cfg, steps: int, warmup: int, flags: int = 0, stage_repeats: int = 1):
    """Upload a generated workload, run warm-up + timed forwards.  Returns
    (workload, result dict)."""
    from mixlab_amd import _lib
    from mixlab_amd.op import MoEFeedForward
    from mixlab_amd.workloads import make_workload

    t0 = time.time()
    w = make_workload(cfg)
    log(f"workload {cfg.name} generated in {time.time() - t0:.1f}s ({cfg.note})")
    if cfg.int8_weights:
        flags |= _lib.MXM_FLAG_INT8_WEIGHTS
    op = MoEFeedForward(cfg.int_params, [cfg.leaky_slope], compute_dtype=cfg.dtype, flags=flags)
    op.set_input(1, w.router_upload())
    idx = 2
    for e in range(cfg.E):
        for j in range(cfg.wpe):
            if cfg.int8_weights:
                op.set_input_q8(idx, *w.q8[e][j])
            else:
                op.set_input(idx, w.matrix_upload(e, j))
            idx += 1
    xdev = _lib.DeviceBuffer.from_array(w.x_upload())
    delta = _lib.DeviceBuffer(cfg.N * cfg.D * 4)
    aux = _lib.DeviceBuffer(4)
    ent = _lib.DeviceBuffer(4)
    xcode = _lib.MXM_DTYPE_BF16 if cfg.dtype == "bf16" else _lib.MXM_DTYPE_F32
    log(f"{cfg.name} weights uploaded; executor {op.info()}")

    def step():
        op.forward(xdev.value, xcode, cfg.N, delta.value, aux.value, ent.value)

    for _ in range(warmup):
        step()
    op.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    op.synchronize()
    elapsed = time.perf_counter() - t0
    # stage times from a second pass with HIP events between the stages (the
    # events add gaps between kernels, so they stay out of the timed pass);
    # short stages are launched `stage_repeats` times between their events
    op.set_profiling(True, stage_repeats)
    for _ in range(steps):
        step()
    op.synchronize()
    stages = op.stage_times()
    op.set_profiling(False)
    counts = op.routing()["counts"]
    info = op.info()
    op.close()
    ms = elapsed * 1e3 / steps
    log(f"{cfg.name}: {steps} steps, {ms:.4f} ms/step; stages {stages}")
    return w, {"ms_per_step": ms, "tokens_per_s": cfg.N / (ms * 1e-3), "stages": stages,
               "counts": counts, "info": info}


def vendor_gemm(cfg) -> dict:
    """The vendor library's dense bf16 GEMM (torch.matmul -> hipBLASLt) on the
    dense shapes of the grouped GEMM's two launches: [N*K, D] x [D, 2F] (gate
    and up together) and [N*K, F] x [F, D], every row one expert's, no gather.
    A reference point for the grouped kernel, not part of the op.  torch
    carries its own HIP runtime, so this runs in a child process that never
    loads libmixmoe (bench.py --vendor-gemm-only)."""
    import subprocess

    res = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor-gemm-only",
                          "--config", cfg.name], capture_output=True, text=True, timeout=600)
    sys.stderr.write(res.stderr)
    if res.returncode != 0:
        raise RuntimeError(f"vendor GEMM child exited with {res.returncode}")
    return json.loads(res.stdout.strip().splitlines()[-1])


def vendor_gemm_child(cfg, reps: int = 10) -> int:
    """--vendor-gemm-only: time torch.matmul on the two dense shapes and print
    one JSON line (this process loads torch and never libmixmoe)."""
    import torch

    out = {}
    M = cfg.N * cfg.K
    for name, (k, n) in {"gemm_up": (cfg.D, (2 if cfg.wpe == 3 else 1) * cfg.F),
                         "gemm_down": (cfg.F, cfg.D)}.items():
        a = torch.randn(M, k, device="cuda", dtype=torch.bfloat16)
        b = torch.randn(k, n, device="cuda", dtype=torch.bfloat16)
        for _ in range(3):
            c = a @ b
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            c = a @ b
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / reps
        tf = 2.0 * M * k * n / (ms * 1e-3) / 1e12
        out[name] = {"shape": [M, k, n], "ms": ms, "tflops": tf, "frac": tf / PEAK_BF16_TFLOPS}
        log(f"vendor dense GEMM {name} {M}x{k}x{n}: {ms:.3f} ms, {tf:.1f} TFLOP/s")
        del a, b, c
    print(json.dumps(out), flush=True)
    return 0


def copy_calibration(mib: int, reps: int = 5) -> int:
    """Copies of a known size: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on this
    run gives the counter-to-bytes factors used for roofline.traffic."""
    from mixlab_amd import _lib

    n = mib << 20
    src, dst = _lib.DeviceBuffer(n), _lib.DeviceBuffer(n)
    lib = _lib.init()
    for _ in range(reps):
        _lib.check(lib.mxm_memcpy_d2d(dst.ptr, src.ptr, n), "mxm_memcpy_d2d")
    _lib.check(lib.mxm_device_synchronize(), "sync")
    print(json.dumps({"copy_bytes": n, "reps": reps}), flush=True)
    return 0


def run_backward(cfg, steps: int, warmup: int, w=None, train: bool = False) -> dict:
    """Backward of op 74 (mxm_moe_backward: a forward with the routing kept,
    then the gradients of x, the router and every routed expert) on the
    configuration's compute dtype.  fp32: the routing of the forward, then
    every expert product as a ragged grouped bf16 MFMA product over the
    operands' hi / lo planes (three plane pairs per fp32 product); bf16 (MFMA
    weight family): every product on MFMA, the weight gradients on the
    ragged grouped weight-gradient kernel (fp32 out).
    train: a training step instead -- mxm_moe_forward on an op created with
    MXM_FLAG_KEEP_FOR_BACKWARD, then mxm_moe_backward_kept, which starts
    from the routing and projections that forward kept."""
    from mixlab_amd import _lib
    from mixlab_amd.op import MoEFeedForward
    from mixlab_amd.workloads import make_workload

    bf16 = cfg.dtype == "bf16"
    if w is None:
        w = make_workload(cfg)
    op = MoEFeedForward(cfg.int_params, [cfg.leaky_slope], compute_dtype=cfg.dtype,
                        flags=_lib.MXM_FLAG_KEEP_FOR_BACKWARD if train else 0)
    op.set_input(1, w.router_upload() if bf16 else np.ascontiguousarray(w.router_w, np.float32))
    idx = 2
    for e in range(cfg.E):
        for j in range(cfg.wpe):
            op.set_input(idx, w.matrix_upload(e, j) if bf16
                         else np.ascontiguousarray(w.matrix(e, j), np.float32))
            idx += 1
    rng = np.random.default_rng(7)
    xdev = _lib.DeviceBuffer.from_array(w.x_upload() if bf16
                                        else np.ascontiguousarray(w.x, np.float32))
    xcode = _lib.MXM_DTYPE_BF16 if bf16 else _lib.MXM_DTYPE_F32
    dd = _lib.DeviceBuffer.from_array(rng.standard_normal((cfg.N, cfg.D), dtype=np.float32))
    dx = _lib.DeviceBuffer(cfg.N * cfg.D * 4)
    dwr = _lib.DeviceBuffer(cfg.D * cfg.E * 4)
    dw = _lib.DeviceBuffer(cfg.E * cfg.wpe * cfg.D * cfg.F * 4)
    lib = _lib.init()
    mfma = op.info()["mfma"]

    delta = _lib.DeviceBuffer(cfg.N * cfg.D * 4) if train else None

    def step():
        if train:
            op.forward(xdev.value, xcode, cfg.N, delta.value)
            _lib.check(lib.mxm_moe_backward_kept(op.handle, dd.value, 0.01, 0.0, dx.value,
                                                 dwr.value, dw.value), "mxm_moe_backward_kept")
        else:
            _lib.check(lib.mxm_moe_backward(op.handle, xdev.value, xcode, cfg.N,
                                            dd.value, 0.01, 0.0, dx.value, dwr.value, dw.value),
                       "mxm_moe_backward")

    for _ in range(warmup):
        step()
    op.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    op.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    op.close()
    glu = cfg.expert_type != 2
    nkdf = cfg.N * cfg.K * cfg.D * cfg.F
    # The products the call runs, each 2*N*K*D*F FLOP (one D x F product over
    # all routed rows), plus the router's 2*N*D*E forward and 4*N*D*E
    # backward.  The backward call of the bf16 MFMA path runs its forward's
    # up projections (2 or 1) but not the down product (its gate gradients
    # come from dH' = dD W_down^T), then dH', dX (2 or 1) and the weight
    # gradients (3 or 2): 8 or 5.  A training step runs the whole forward (3
    # or 2) and that backward without the forward: 9 or 6.  The fp32 path's
    # backward call runs the whole forward before its backward: 9 or 6.
    fwd = 3 if glu else 2
    bwd = 1 + (2 if glu else 1) + (3 if glu else 2)
    units = fwd + bwd if (train or not (bf16 and mfma)) else fwd - 1 + bwd
    fl = 2 * nkdf * units + 6 * cfg.N * cfg.D * cfg.E
    tf = fl / (ms * 1e-3) / 1e12
    log(f"{'training step' if train else 'backward'} {cfg.name} {cfg.dtype}: {ms:.3f} ms/step, "
        f"{tf:.1f} TFLOP/s")
    if bf16 and mfma:
        roof = {"bound": "mfma", "kernel": ("forward + backward" if train else "whole backward")
                + " (MFMA grouped products and weight gradients)", "achieved": tf, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": tf / PEAK_BF16_TFLOPS, "traffic": None}
    else:
        # fp32 products as bf16 products over three plane pairs (hi.hi +
        # hi.lo + lo.hi): the MFMA executes three times the fp32 work
        roof = {"bound": "mfma",
                "kernel": "whole backward (each fp32 expert product as a bf16 MFMA grouped "
                          "product over three hi/lo plane pairs; router part on the VALU)",
                "achieved": 3 * tf, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": 3 * tf / PEAK_BF16_TFLOPS, "traffic": None,
                "fp32_equivalent_tflops": tf, "fp32_peak_tflops": PEAK_FP32_TFLOPS}
    return {"workload": f"{cfg.name} shape, {cfg.dtype} compute", "tokens": cfg.N,
            "ms_per_step": ms, "tokens_per_s": cfg.N / (ms * 1e-3),
            "expert_products_counted": units, "flop_per_step": fl, "roofline": roof}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C4", help="C1..C4 (C4 is the headline configuration)")
    ap.add_argument("--flags", type=int, default=0, help="mxm_moe_create flags (include/mixmoe.h)")
    ap.add_argument("--cpu-seconds", type=float, default=5.0,
                    help="target seconds per timed run of the CPU baseline (0 disables it)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the C1, C2fp32, C2, C2int8, C3 and C4F sections")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="also time hipBLASLt (torch.matmul) on the dense equivalents of the "
                         "grouped GEMM's two launches (in a child process)")
    ap.add_argument("--vendor-gemm-only", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--no-decode", action="store_true", help="skip the int8 decode (C5) section")
    ap.add_argument("--decode-steps", type=int, default=0, metavar="K",
                    help="timed (and stage-timed) C5 forwards; default max(steps, 200) with "
                         "max(warmup, 20) warm-up (counter collection runs want a few)")
    ap.add_argument("--no-backward", action="store_true", help="skip the backward section")
    ap.add_argument("--backward-only", nargs="?", const="C2", default=None, metavar="CONFIG",
                    help="only time the bf16 backward at the shape of CONFIG (default C2; 10 "
                         "steps after 3 warm-up, C3: 3 after 2) and print its JSON object (for "
                         "profiling)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run device-to-device copies of MIB MiB (the reference kernel "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if args.vendor_gemm_only:
        from mixlab_amd.workloads import CONFIGS
        return vendor_gemm_child(CONFIGS[args.config])
    if args.backward_only:
        from mixlab_amd.workloads import CONFIGS
        cfg = CONFIGS[args.backward_only]
        steps, warm = (10, 3) if cfg.N <= 16384 else (3, 2)
        print(json.dumps({"backward_bf16": run_backward(cfg, steps, warm)}), flush=True)
        return 0

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py runs on exactly one GPU: this build has no multi-GPU path "
              "(data parallelism over tokens would shard N with no collective; "
              "expert parallelism needs an all-to-all). Run with --gpus 1.", file=sys.stderr)
        return 2

    from mixlab_amd import _lib
    from mixlab_amd.workloads import CONFIGS

    cfg = CONFIGS[args.config]
    log(f"device: {_lib.device_name()}")
    # The decode layer is measured first, on a fresh allocator: after the
    # headline's multi-GB buffers are freed it measured 3-5 % slower (the
    # same kernels; 121 against 126-127 us per forward on one box)
    decode = None
    if not args.no_decode:
        c5 = CONFIGS["C5"]
        dsteps, dwarm = ((args.decode_steps, min(args.warmup, args.decode_steps))
                         if args.decode_steps else (max(args.steps, 200), max(args.warmup, 20)))
        _, d = run_config(c5, dsteps, dwarm, stage_repeats=10)
        ds = d["stages"]
        wb = int8_weight_bytes(c5, d["counts"])
        xb = c5.N * c5.D * 2
        total = wb["gemm_up"] + wb["gemm_down"] + sum(stage_bytes(c5).values()) + xb
        up_gbs = (wb["gemm_up"] + xb) / (ds["gemm_up"] * 1e-3) / 1e9
        layer_gbs = total / (d["ms_per_step"] * 1e-3) / 1e9
        decode = {
            "workload": "C5", "tokens": c5.N, "tokens_per_s": d["tokens_per_s"],
            "ms_per_step": d["ms_per_step"],
            "routed_experts": wb["routed_experts"],
            "hbm_gbs_forward": layer_gbs,
            # the decode layer as a whole: all launches of one forward
            "roofline": {"bound": "hbm", "kernel": "whole decode forward (all launches)",
                         "achieved": layer_gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": layer_gbs / PEAK_HBM_GBS,
                         "traffic": layer_traffic("C5", ("route_small", "gemm_up",
                                                         "gemm_down", "combine"), 0)},
            "up_roofline": {"bound": "hbm", "kernel": "gemm_up (int8 gate+up weight stream)",
                            "achieved": up_gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "frac": up_gbs / PEAK_HBM_GBS,
                            "traffic": measured_traffic("C5", "gemm_up", 0)},
            "gemm_down_gbs": (wb["gemm_down"]) / (ds["gemm_down"] * 1e-3) / 1e9,
            "stages_ms": {k: v for k, v in ds.items() if k != "forwards"},
        }
        # the same decode shape with bf16 expert weights (the reference's own
        # precision): the weights streamed through the decode kernels
        import dataclasses
        c5b = dataclasses.replace(c5, int8_weights=False, name="C5bf16")
        _, db = run_config(c5b, dsteps, dwarm, stage_repeats=10)
        dbs = db["stages"]
        wbb = bf16_weight_bytes(c5b, db["counts"])
        totb = wbb["gemm_up"] + wbb["gemm_down"] + sum(stage_bytes(c5b).values()) + xb
        decode["bf16_weights"] = {
            "tokens_per_s": db["tokens_per_s"], "ms_per_step": db["ms_per_step"],
            "hbm_gbs_forward": totb / (db["ms_per_step"] * 1e-3) / 1e9,
            "frac_hbm_forward": totb / (db["ms_per_step"] * 1e-3) / 1e9 / PEAK_HBM_GBS,
            "gemm_up_gbs": wbb["gemm_up"] / (dbs["gemm_up"] * 1e-3) / 1e9,
            "gemm_down_gbs": wbb["gemm_down"] / (dbs["gemm_down"] * 1e-3) / 1e9,
            "stages_ms": {k: v for k, v in dbs.items() if k != "forwards"},
            "executor": db["info"],
        }

    w, r = run_config(cfg, args.steps, args.warmup, args.flags)
    gg = grouped_gemm_summary(cfg, r["stages"])
    stages = r["stages"]
    sb = stage_bytes(cfg)
    hbm = {k: sb[k] / (stages[k] * 1e-3) / 1e9 for k in sb}

    cpu = None
    if args.cpu_seconds > 0:
        log("timing the CPU baseline")
        cpu = cpu_baseline(w, cfg, args.cpu_seconds)
        log(f"cpu baseline {cpu}")
    # the backward at the headline shape, on the same generated workload
    backward_bf16_main = train_bf16_main = None
    if not args.no_backward and cfg.dtype == "bf16" and not cfg.int8_weights:
        backward_bf16_main = run_backward(cfg, 3, 2, w=w)
        train_bf16_main = run_backward(cfg, 3, 2, w=w, train=True)
    del w

    # the other MFMA-bound configurations: near-uniform C2, Zipf-ragged C3 and
    # C4 at the reference's default expert width (F = 5468, padded to 5504
    # by the library; the figures count the op's own F)
    extra = {}
    if not args.no_configs:
        # C1, the reference's CPU-runnable moe_tiny-scale case: fp32 on the
        # exact-order SIMT kernels (no MFMA figure)
        c1 = CONFIGS["C1"]
        _, r1 = run_config(c1, max(args.steps, 100), max(args.warmup, 10))
        extra["C1"] = {"tokens": c1.N, "d_model": c1.D, "experts": c1.E, "top_k": c1.K,
                       "expert_hidden": c1.F, "dtype": c1.dtype,
                       "tokens_per_s": r1["tokens_per_s"], "ms_per_step": r1["ms_per_step"],
                       "stages_ms": {k: v for k, v in r1["stages"].items() if k != "forwards"},
                       "executor": r1["info"]}
        # the fp32 flow at C2's size: the exact-order kernels (fmaf chains in
        # ascending k, the 64 x 64 tile's on the fp32 matrix cores; bit-exact
        # against the oracle), against the fp32 dense peak
        import dataclasses
        c2f = dataclasses.replace(CONFIGS["C2"], dtype="fp32", name="C2fp32")
        _, rf = run_config(c2f, args.steps, args.warmup)
        flf = c2f.flops()
        gms = rf["stages"]["gemm_up"] + rf["stages"]["gemm_down"]
        extra["C2fp32"] = {"tokens": c2f.N, "d_model": c2f.D, "experts": c2f.E,
                           "top_k": c2f.K, "expert_hidden": c2f.F, "dtype": "fp32",
                           "tokens_per_s": rf["tokens_per_s"], "ms_per_step": rf["ms_per_step"],
                           "expert_gemm": {"ms": gms,
                                           "tflops": flf["experts"] / (gms * 1e-3) / 1e12,
                                           "frac_fp32_peak": flf["experts"] / (gms * 1e-3) / 1e12
                                           / PEAK_FP32_TFLOPS},
                           "stages_ms": {k: v for k, v in rf["stages"].items() if k != "forwards"},
                           "executor": rf["info"]}
        # C2int8: C2 with int8 expert weights, a prefill-sized int8 batch (256
        # routed rows per expert), which runs on the MFMA tiles with the
        # integers as bf16 and the scales in the epilogue
        c2q = dataclasses.replace(CONFIGS["C2"], int8_weights=True, name="C2int8")
        for name in ("C2", "C2int8", "C3", "C4F"):
            if name == cfg.name:
                continue
            c = c2q if name == "C2int8" else CONFIGS[name]
            _, rc = run_config(c, args.steps, args.warmup)
            counts = np.asarray(rc["counts"])
            extra[name] = {"tokens": c.N, "d_model": c.D, "experts": c.E, "top_k": c.K,
                           "expert_hidden": c.F,
                           "weights": "int8, fp32 per-output-channel scales"
                                      if c.int8_weights else c.dtype,
                           "tokens_per_s": rc["tokens_per_s"],
                           "ms_per_step": rc["ms_per_step"],
                           "grouped_gemm": grouped_gemm_summary(c, rc["stages"]),
                           "stages_ms": {k: v for k, v in rc["stages"].items() if k != "forwards"},
                           "expert_rows": {"max": int(counts.max()), "min": int(counts.min()),
                                           "mean": float(counts.mean())},
                           "executor": rc["info"]}

    vendor = vendor_gemm(cfg) if args.vendor_gemm else None

    backward = backward_bf16 = backward_bf16_c3 = None
    if not args.no_backward:
        import dataclasses
        backward = run_backward(dataclasses.replace(CONFIGS["C2"], dtype="fp32"), 5, 2)
        backward_bf16 = run_backward(CONFIGS["C2"], 10, 3)
        # skewed routing: one expert holds 37 % of the rows
        backward_bf16_c3 = run_backward(CONFIGS["C3"], 3, 2)

    line = {
        "metric": METRIC,
        "value": r["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype,
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02) weights)",
        "config": {"workload": cfg.name, "tokens": cfg.N, "d_model": cfg.D, "experts": cfg.E,
                   "top_k": cfg.K, "expert_hidden": cfg.F,
                   "expert": "sigmoid-GLU (swiglu)" if cfg.expert_type == 0 else str(cfg.expert_type),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma",
                     "kernel": "gemm_kernel, the grouped GEMM of one forward (gate+up launch "
                               "with GLU epilogue + down launch)",
                     "achieved": gg["tflops"], "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": gg["frac"], "traffic": gemm_traffic(cfg.name, args.flags)},
        "grouped_gemm": gg,
        "stages_ms": {k: v for k, v in stages.items() if k != "forwards"},
        "hbm_gbs": hbm,
        "configs": extra,
        "vendor_gemm": vendor,
        "decode_int8": decode,
        "backward_fp32": backward,
        "backward_bf16": backward_bf16,
        "backward_bf16_c3": backward_bf16_c3,
        f"backward_bf16_{cfg.name.lower()}": backward_bf16_main,
        f"train_step_bf16_{cfg.name.lower()}": train_bf16_main,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
