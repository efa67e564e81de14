#!/usr/bin/env python3
"""Benchmark of the fused attention hot path on one MI355X.

Metric: forward and forward+backward ms per call at b64 h6 s240 d64 fp32 through
the qkv path (the reference's headline, examples/compare.rs / bench/compare.py), plus the
achieved fraction of the fp32 matrix peak. A step is one forward + backward of the qkv op over
config 2's synthetic inputs (qkv [64, 240, 1152] ~ N(0, 1) and dout [64, 240, 384] ~ N(0, 1) drawn
by a CPU torch generator seeded 0, the reference's published inputs), resident in HBM before the
timed region. The op-level C ABI is called with preallocated outputs on torch's current stream.

Prints ONE JSON line. `--gpus N` with N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for p in (str(REPO), str(REPO / "candle-fused-attn_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "fwd & fwd+bwd ms at b64 h6 s240 d64 fp32; % of fp32 MFMA peak"
PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense fp32 matrix peak (public spec)
PEAK_HBM_GBS = 8000.0
B, H, S, D = 64, 6, 240, 64
SCALE = 0.125


def flops(b, h, s, d, causal):
    pairs = b * h * s * s if not causal else b * h * s * (s + 1) // 2
    return 4 * d * pairs, 10 * d * pairs


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # MI355X raises its clocks over the first ~20 ms of sustained work (a kernel trace shows the
    # forward going from 71 to 58 us per call over that time); 200 warm-up steps (~45 ms) put
    # the timed steps at the steady state a training loop runs at.
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--causal", action="store_true", help="config 3 instead of config 2")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-accuracy", action="store_true", help="skip the fp64 scoring")
    ap.add_argument("--cpu-threads", type=int, default=None)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one 256 MiB device-to-device copy (a kernel of known traffic, "
                         "to scale rocprofv3's FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one GPU "
              "(the op shards over (batch, head) with no communication; see DESIGN.md)",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import candle_fused_attn  # noqa: F401  (loads torch first, then libfattn)
    from candle_fused_attn import _lib

    if not torch.cuda.is_available():
        print("bench.py: no HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    L = _lib.lib()
    causal = bool(args.causal)

    # Inputs exactly as bench/compare.py:496-503 draws them.
    g = torch.Generator().manual_seed(0)
    qkv_cpu = torch.randn(B, S, 3 * H * D, generator=g)
    dout_cpu = torch.randn(B, S, H * D, generator=g)
    qkv = qkv_cpu.to(dev)
    dout = dout_cpu.to(dev)
    out = torch.empty(B, S, H * D, device=dev)
    lse = torch.empty(B, H, S, device=dev)
    dqkv = torch.empty_like(qkv)
    ws_bytes = int(L.fattn_bwd_workspace_bytes(B, H, S, D))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    shape, strides = _lib.arr(qkv.shape), _lib.arr(qkv.stride())
    gshape, gstrides = _lib.arr(dout.shape), _lib.arr(dout.stride())
    ci = int(causal)

    def fwd():
        _lib.check(L.fattn_qkv_forward(P(qkv), 0, shape, strides, H, SCALE, ci, P(out), P(lse),
                                       sp))

    def bwd():
        _lib.check(L.fattn_qkv_backward(P(qkv), 0, shape, strides, H, SCALE, ci, P(out), P(lse),
                                        P(dout), 0, gshape, gstrides, P(dqkv), P(ws), ws_bytes,
                                        sp))

    # Kernel-level views of the same operands, to time each kernel on its own.
    qst = _lib.arr([S * 3 * H * D, D, 3 * H * D])
    gst = _lib.arr([S * H * D, D, H * D])
    base = qkv.data_ptr()
    qp, kp, vp = (ctypes.c_void_p(base + i * H * D * 4) for i in range(3))

    def prep_k():
        _lib.check(L.fattn_bwd_prep_f32_d64(P(out), P(dout), gst, P(ws), ws_bytes, B, H, S, D,
                                            sp))

    def main_k():
        _lib.check(L.fattn_bwd_main_f32_d64(qp, kp, vp, P(out), P(dout), P(lse), P(dqkv), P(ws),
                                            ws_bytes, B, H, S, D, SCALE, ci, qst, qst, qst, gst,
                                            sp))

    def dq_k():
        _lib.check(L.fattn_bwd_dq_f32_d64(P(dqkv), P(ws), ws_bytes, B, H, S, D, SCALE, ci, sp))

    split = ws_bytes >= int(L.fattn_bwd_workspace_split_bytes(B, H, S, D))

    if args.calibrate_copy:
        src = torch.ones(64 * 1024 * 1024, device=dev)   # 256 MiB
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    log(f"bench: config {'3 (causal)' if causal else '2'} b{B} h{H} s{S} d{D}; "
        f"warmup {args.warmup}, steps {args.steps}")
    for _ in range(max(args.warmup, 1)):
        fwd()
        bwd()
    torch.cuda.synchronize()

    # roctx ranges name the timed windows (the reference brackets them with cuProfilerStart /
    # Stop for an nsys capture range, examples/compare.rs:261-277); `rocprofv3 --marker-trace`
    # records them. torch.cuda.nvtx is roctx on ROCm.
    def range_push(name):
        torch.cuda.nvtx.range_push(name)

    def range_pop():
        torch.cuda.nvtx.range_pop()

    def timed(fn, n, name):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        range_push(name)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / n
        range_pop()
        return e0.elapsed_time(e1) / n, wall

    K = max(args.steps, 1)
    step = lambda: (fwd(), bwd())  # noqa: E731
    fwd_bwd_ms, fwd_bwd_wall = timed(step, K, "fattn timed fwd+bwd")
    fwd_ms, _ = timed(fwd, K, "fattn timed fwd")
    log(f"bench: fwd+bwd {fwd_bwd_ms:.4f} ms (wall {fwd_bwd_wall:.4f}), fwd {fwd_ms:.4f} ms")

    # Per-kernel durations: K more steps, back to back as above, with the backward launched as
    # its kernel-level steps (the same kernels on the same arguments as fattn_qkv_backward) and a
    # HIP event on the launch stream between every two launches.
    # With a split workspace at d 64 step 1 launches nothing (step 2 computes D itself, and its
    # last workgroups sum dQ tiles); step 3 sums the tiles those left.
    kernels = [("fwd", fwd), ("bwd_prep", prep_k), ("bwd_main", main_k)]
    if split:
        kernels.append(("bwd_dq", dq_k))
    marks = []
    torch.cuda.synchronize()
    range_push("fattn kernel-level steps")
    for _ in range(K):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(kernels) + 1)]
        ev[0].record(stream)
        for i, (_, fn) in enumerate(kernels):
            fn()
            ev[i + 1].record(stream)
        marks.append(ev)
    torch.cuda.synchronize()
    range_pop()
    kus = {name: statistics.mean(ev[i].elapsed_time(ev[i + 1]) for ev in marks) * 1e3
           for i, (name, _) in enumerate(kernels)}
    steps_us = statistics.mean(ev[0].elapsed_time(ev[-1]) for ev in marks) * 1e3
    fwd_us, prep_us, main_us = kus["fwd"], kus.get("bwd_prep", 0.0), kus["bwd_main"]
    dq_us = kus.get("bwd_dq", 0.0)
    log(f"bench: kernels fwd {fwd_us:.1f} us, prep {prep_us:.1f} us, bwd main {main_us:.1f} us, "
        f"dq sum {dq_us:.1f} us ({'split' if split else 'turns'}); step {steps_us:.1f} us")

    f_fwd, f_bwd = flops(B, H, S, D, causal)
    fwd_tflops = f_fwd / (fwd_ms * 1e-3) / 1e12
    total_tflops = (f_fwd + f_bwd) / (fwd_bwd_ms * 1e-3) / 1e12
    main_tflops = f_bwd / (main_us * 1e-6) / 1e12
    bwd_steps_tflops = f_bwd / ((prep_us + main_us + dq_us) * 1e-6) / 1e12
    fwdk_tflops = f_fwd / (fwd_us * 1e-6) / 1e12

    traffic = None
    tfile = REPO / "profiles" / "traffic.json"
    if tfile.exists():
        try:
            traffic = json.loads(tfile.read_text()).get("bwd_main_bytes")
        except (OSError, ValueError):
            traffic = None

    result = {
        "metric": METRIC,
        "value": round(fwd_bwd_ms, 5),
        "unit": "ms",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(fwd_bwd_ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": ("qkv path forward+backward, qkv [64, 240, 1152] (h 6, d 64) and dout "
                         "[64, 240, 384] ~ N(0,1) seed 0, scale 1/8, "
                         + ("causal (config 3)" if causal else "non-causal (config 2)")),
            "b": B, "h": H, "s": S, "d": D, "causal": causal,
            "entry": "fattn_qkv_forward + fattn_qkv_backward",
        },
        "fwd_ms": round(fwd_ms, 5),
        "fwd_bwd_ms": round(fwd_bwd_ms, 5),
        "fwd_bwd_wall_ms": round(fwd_bwd_wall, 5),
        "fwd_tflops": round(fwd_tflops, 3),
        "fwd_bwd_tflops": round(total_tflops, 3),
        "frac_fp32_peak": round(total_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
        "kernels_us": {"fwd": round(fwd_us, 2), "bwd_prep": round(prep_us, 2),
                       "bwd_main": round(main_us, 2), "bwd_dq": round(dq_us, 2),
                       "step": round(steps_us, 2)},
        "dq_sum": "split" if split else "turns",
        "roofline": {
            "kernel": ("bwd_split_kernel<64> (fattn_bwd_main_f32_d64, split; its last "
                       "workgroups sum dQ tiles)" if split
                       else "bwd_kernel<false, 64> (fattn_bwd_main_f32_d64, turns)"),
            "bound": "mfma",
            "achieved": round(main_tflops, 3),
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(main_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": traffic,
            "flops_per_launch": f_bwd,
            "bwd_steps_1_3_achieved": round(bwd_steps_tflops, 3),
            "fwd_kernel_achieved": round(fwdk_tflops, 3),
            "fwd_kernel_frac": round(fwdk_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
        },
    }

    if not args.no_accuracy:
        from oracle import oracle as orc
        fwd()
        bwd()
        torch.cuda.synchronize()
        first = dqkv.clone()
        bwd()
        torch.cuda.synchronize()
        rerun_equal = bool(torch.equal(first.view(torch.int32), dqkv.view(torch.int32)))
        t0 = time.perf_counter()
        x, dd = qkv_cpu.numpy(), dout_cpu.numpy()
        ro, rl = orc.qkv_forward(x, H, SCALE, causal, dtype=np.float64)
        rg = orc.qkv_backward(x, H, SCALE, causal, ro, rl, dd, dtype=np.float64)
        go, gg = out.cpu().numpy(), dqkv.cpu().numpy()
        acc = {"o": orc.rel_fro(go, ro)}
        for name, a, r in zip(("dq", "dk", "dv"), np.split(gg, 3, axis=-1),
                              np.split(rg, 3, axis=-1)):
            acc[name] = orc.rel_fro(a, r)
        result["accuracy"] = {
            "normwise_vs_fp64": {k: float(f"{v:.3e}") for k, v in acc.items()},
            "tolerance": 2e-6,
            "within_tolerance": all(v <= 2e-6 for v in acc.values()),
            "bitwise_rerun": rerun_equal,
        }
        log(f"bench: accuracy {acc} (fp64 scoring {time.perf_counter() - t0:.1f} s), "
            f"bitwise rerun {rerun_equal}")

    if not args.no_cpu:
        from oracle import oracle as orc
        threads = args.cpu_threads or orc.default_threads()
        x, dd = qkv_cpu.numpy(), dout_cpu.numpy()

        def cpu_step(xx, gg, thr):
            o_, l_ = orc.qkv_forward(xx, H, SCALE, causal, dtype=np.float32, threads=thr)
            orc.qkv_backward(xx, H, SCALE, causal, o_, l_, gg, dtype=np.float32, threads=thr)

        cpu_step(x, dd, threads)
        ts = []
        t_start = time.perf_counter()
        while len(ts) < 5 and (time.perf_counter() - t_start < 20 or len(ts) < 1):
            t0 = time.perf_counter()
            cpu_step(x, dd, threads)
            ts.append((time.perf_counter() - t0) * 1e3)
        cpu_ms = statistics.median(ts)
        # One-thread figure on 4 of the 64 batches, scaled to the full call.
        t0 = time.perf_counter()
        cpu_step(x[:4], dd[:4], 1)
        one_ms = (time.perf_counter() - t0) * 1e3 * (B / 4)
        cpu_name = ""
        try:
            for line in Path("/proc/cpuinfo").read_text().splitlines():
                if line.startswith("model name"):
                    cpu_name = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
        result["cpu_baseline"] = {
            "value": round(cpu_ms, 2),
            "unit": "ms",
            "cores": threads,
            "kind": "port",
            "sample": (f"full config {'3' if causal else '2'} forward+backward, median of "
                       f"{len(ts)} after 1 warm-up, OpenMP over (b, h) on {threads} threads "
                       f"({cpu_name or 'unknown CPU'}, nproc {os.cpu_count()}); the C "
                       "restatement of the reference's composed CPU path (src/lib.rs:241-299)"),
            "one_thread_ms": round(one_ms, 1),
            "one_thread_sample": "batches 0-3 of 64, one thread, scaled x16",
            "gpu_speedup": round(cpu_ms / fwd_bwd_ms, 1),
        }
        log(f"bench: cpu baseline {cpu_ms:.1f} ms on {threads} threads; 1 thread {one_ms:.0f} ms")

    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
