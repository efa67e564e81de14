#!/usr/bin/env python3
"""Benchmark of the fused attention hot path on one MI355X.

Metric: forward and forward+backward ms per call at b64 h6 s240 d64 fp32 through
the qkv path (the reference's headline, examples/compare.rs / bench/compare.py), plus the
achieved fraction of the fp32 matrix peak. A step is one forward + backward of the qkv op over
config 2's synthetic inputs (qkv [64, 240, 1152] ~ N(0, 1) and dout [64, 240, 384] ~ N(0, 1) drawn
by a CPU torch generator seeded 0, the reference's published inputs), resident in HBM before the
timed region. The op-level C ABI is called with preallocated outputs on torch's current stream.

Configs 3-5 (causal, long causal, strided views) and config 2's shape at head_dim 32 and 128
are timed too, as extra keys of the same line (`configs`): op-level forward and
forward+backward, and each kernel on its own.

Order of the GPU work: W warm-up + K timed steps from an idle GPU (`fwd_bwd_from_idle_ms`),
configs 3-5, then W warm-up + K timed steps (`value`), K forwards (`fwd_ms`), K kernel-level
steps (`kernels_us`), K op-level backwards (`bwd_ms`), and last config 2 at head_dim 32 and 128.
`roofline` prices the op-level backward and forward windows: at config 2 each call is one launch
(step 2 alone, the forward kernel alone), so K calls back to back between two events give the
kernel's average launch duration plus the dispatch gap between launches; the kernel-level
steps, with an event between every two launches, add the gap between an event and the next
dispatch (about 3 us) to each kernel and are reported beside them. MI355X runs at
lower clocks for some tens of milliseconds after an idle second, so the headline steps come right
after sustained work, as in a training loop; the from-idle figure shows what a short run on an
idle GPU sees. The K timed steps run back to back with HIP events only before the first, after
the fifth, before the fifth-last and after the last (the means of the first and last 5 steps come
from those); an event between every two steps would add its own time to each (about 2 us).

Prints ONE JSON line. `--gpus N` with N > 1 exits: this build runs on one GPU.

`--traffic-from FETCH_CSV WRITE_CSV` does not touch a GPU: it turns two `rocprofv3 --pmc
FETCH_SIZE` / `--pmc WRITE_SIZE` counter files of a `--calibrate-copy` run into
profiles/traffic.json (HBM bytes per launch, scaled by the 256 MiB copy's counters, tagged with
the sha256 of the libfattn.so that was measured). `--trace-from KERNEL_TRACE_CSV` (no GPU either)
prints the per-kernel durations of the headline's timed and kernel-level steps from a
`rocprofv3 --kernel-trace` file of the same command.
"""
from __future__ import annotations

import argparse
import csv
import ctypes
import hashlib
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
SCALE = 0.125
TRAFFIC = REPO / "profiles" / "traffic.json"
LIB = REPO / "candle-fused-attn_amd" / "lib" / "libfattn.so"
COPY_KIB = 256 * 1024            # the --calibrate-copy kernel moves 256 MiB each way
KERNEL_NAMES = {"fwd": "fwd_kernel<64, 128, 32, 3, false>",
                "bwd_main": "bwd_split_kernel<64, 1, false>", "bwd_dq": "dq_kernel<64>"}
CAUSAL_FWD_NAME = "fwd_kernel<64, 64, 32, 3, true>"   # config 3's forward

# The BASELINE.json configurations this bench times: (name, kind, b, h, s, causal, seed, std).
CONFIGS = {
    2: ("config 2", "qkv", 64, 6, 240, False, 0, 1.0),
    3: ("config 3", "qkv", 64, 6, 240, True, 0, 1.0),
    4: ("config 4", "qkv", 8, 12, 2048, True, 2, 1.0),
    5: ("config 5", "strided", 16, 16, 1024, False, 3, 2.0),
}


def flops(b, h, s, d, causal):
    pairs = b * h * s * s if not causal else b * h * s * (s + 1) // 2
    return 4 * d * pairs, 10 * d * pairs


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def lib_sha256() -> str | None:
    try:
        return hashlib.sha256(LIB.read_bytes()).hexdigest()[:16]
    except OSError:
        return None


class Workload:
    """One configuration's operands, resident on the device, and closures over the C ABI: the
    op-level forward and backward (what a step runs) and the kernel-level launches of the same
    kernels on the same views (to time each kernel)."""

    def __init__(self, torch, L, _lib, dev, cfg: int, d: int = 64):
        import ctypes as C
        name, kind, b, h, s, causal, seed, std = CONFIGS[cfg]
        self.cfg, self.name, self.kind = cfg, name, kind
        self.b, self.h, self.s, self.d, self.causal = b, h, s, d, causal
        self.seed, self.std = seed, std
        P = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
        ci = int(causal)
        st = torch.cuda.current_stream(dev)
        sp = C.c_void_p(st.cuda_stream)
        self.stream = st
        hd = h * d
        if kind == "qkv":
            if cfg in (2, 3):
                # Exactly as bench/compare.py:496-503 draws them: qkv, then dout, on the CPU.
                g = torch.Generator().manual_seed(seed)
                self.qkv_cpu = torch.randn(b, s, 3 * hd, generator=g)
                self.dout_cpu = torch.randn(b, s, hd, generator=g)
                qkv, dout = self.qkv_cpu.to(dev), self.dout_cpu.to(dev)
            else:
                g = torch.Generator(device=dev).manual_seed(seed)
                qkv = torch.randn(b, s, 3 * hd, generator=g, device=dev)
                dout = torch.randn(b, s, hd, generator=g, device=dev)
            out = torch.empty(b, s, hd, device=dev)
            dqkv = torch.empty_like(qkv)
            shape, strides = _lib.arr(qkv.shape), _lib.arr(qkv.stride())
            gshape, gstrides = _lib.arr(dout.shape), _lib.arr(dout.stride())
            base = qkv.data_ptr()
            views = [C.c_void_p(base + i * hd * 4) for i in range(3)]
            vst = [_lib.arr([s * 3 * hd, d, 3 * hd])] * 3
            gst = _lib.arr([s * hd, d, hd])
            dout_p = P(dout)
        else:
            # q, k, v = transpose(1, 2) of [b, s, h, d] buffers ~ N(0, std^2), read in place
            # (strides [s h d, d, h d, 1]); dO [b, h, s, d] ~ N(0, 1).
            g = torch.Generator(device=dev).manual_seed(seed)
            bufs = [torch.randn(b, s, h, d, generator=g, device=dev) * std for _ in range(3)]
            do = torch.randn(b, h, s, d, generator=g, device=dev)
            qkv, dout = bufs, do
            out = torch.empty(b, s, h, d, device=dev)
            dqkv = torch.empty(b, s, 3, h, d, device=dev)
            bshape = _lib.arr([b, h, s, d])
            bstride = _lib.arr([s * h * d, d, h * d, 1])
            graw = do.transpose(1, 2)  # the gradient of the raw [b, s, h, d] output
            gshape, gstrides = _lib.arr(graw.shape), _lib.arr(graw.stride())
            views = [P(t) for t in bufs]
            vst = [_lib.arr([s * h * d, d, h * d])] * 3
            gst = _lib.arr([h * s * d, s * d, d])
            dout_p = P(do)
        lse = torch.empty(b, h, s, device=dev)
        ws_bytes = int(L.fattn_bwd_workspace_bytes(b, h, s, d))
        ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
        self.split = ws_bytes >= int(L.fattn_bwd_workspace_split_bytes(b, h, s, d))
        self.tensors = (qkv, dout, out, lse, dqkv, ws)  # kept alive
        self.out, self.lse, self.dqkv = out, lse, dqkv

        if kind == "qkv":
            def fwd():
                _lib.check(L.fattn_qkv_forward(P(qkv), 0, shape, strides, h, SCALE, ci, P(out),
                                               P(lse), sp))

            def bwd():
                _lib.check(L.fattn_qkv_backward(P(qkv), 0, shape, strides, h, SCALE, ci, P(out),
                                                P(lse), dout_p, 0, gshape, gstrides, P(dqkv),
                                                P(ws), ws_bytes, sp))
        else:
            args = []
            for t in bufs:
                args += [P(t), 0, bshape, bstride]

            def fwd():
                _lib.check(L.fattn_forward(*args, SCALE, ci, P(out), P(lse), sp))

            def bwd():
                _lib.check(L.fattn_backward(*args, SCALE, ci, P(out), P(lse), dout_p, 0, gshape,
                                            gstrides, P(dqkv), P(ws), ws_bytes, sp))

        # The kernel-level entries: the reference's names at d 64, the general ones elsewhere.
        kl = {n: getattr(L, f"fattn_{n}_f32_d64" if d == 64 else f"fattn_{n}_f32")
              for n in ("fwd", "bwd_prep", "bwd_main", "bwd_dq")}

        def fwd_k():
            _lib.check(kl["fwd"](*views, P(out), P(lse), b, h, s, d, SCALE, ci, *vst, sp))

        def prep_k():
            _lib.check(kl["bwd_prep"](P(out), dout_p, gst, P(ws), ws_bytes, b, h, s, d, sp))

        def main_k():
            _lib.check(kl["bwd_main"](*views, P(out), dout_p, P(lse), P(dqkv), P(ws), ws_bytes,
                                      b, h, s, d, SCALE, ci, *vst, gst, sp))

        def dq_k():
            _lib.check(kl["bwd_dq"](P(dqkv), P(ws), ws_bytes, b, h, s, d, SCALE, ci, sp))

        self.fwd, self.bwd = fwd, bwd
        # With a split workspace at d 64 step 1 launches nothing (step 2 computes D itself, and
        # its last workgroups sum dQ tiles); step 3 sums the tiles those left.
        self.kernels = [("fwd", fwd_k), ("bwd_prep", prep_k), ("bwd_main", main_k)]
        if self.split:
            self.kernels.append(("bwd_dq", dq_k))

    def step(self):
        self.fwd()
        self.bwd()

    def flops(self):
        return flops(self.b, self.h, self.s, self.d, self.causal)


def event_steps(torch, stream, fn, n, edge=5):
    """n calls of fn back to back, timed with HIP events on the launch stream: one before the first
    call, one after the last, one after the first `edge` calls and one before the last `edge`, and
    none between other calls (an event on the stream adds its own time to the call it follows:
    about 2 us per fwd+bwd step at config 2). Returns (mean ms per call over all n, (mean ms of the
    first `edge` calls, of the last `edge` calls), host wall ms per call)."""
    e = max(1, min(edge, n))
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    t0 = time.perf_counter()
    ev[0].record(stream)
    for i in range(n):
        if i == n - e:
            ev[2].record(stream)
        fn()
        if i == e - 1:
            ev[1].record(stream)
    ev[3].record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / n
    edges = (ev[0].elapsed_time(ev[1]) / e, ev[2].elapsed_time(ev[3]) / e)
    return ev[0].elapsed_time(ev[3]) / n, edges, wall


def kernel_steps(torch, stream, kernels, n):
    """n steps launched kernel by kernel, back to back, a HIP event between every two launches:
    mean us per kernel, and per step."""
    marks = []
    torch.cuda.synchronize()
    for _ in range(n):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(kernels) + 1)]
        ev[0].record(stream)
        for i, (_, fn) in enumerate(kernels):
            fn()
            ev[i + 1].record(stream)
        marks.append(ev)
    torch.cuda.synchronize()
    kus = {name: statistics.mean(ev[i].elapsed_time(ev[i + 1]) for ev in marks) * 1e3
           for i, (name, _) in enumerate(kernels)}
    kus["step"] = statistics.mean(ev[0].elapsed_time(ev[-1]) for ev in marks) * 1e3
    return kus


def traffic_entry():
    """roofline.traffic from profiles/traffic.json: the measured HBM bytes of step 2 when that file
    was measured on this very libfattn.so (same sha256), else null (stale; the old figure is kept
    under another key)."""
    sha = lib_sha256()
    try:
        t = json.loads(TRAFFIC.read_text())
    except (OSError, ValueError):
        return {"traffic": None, "lib_sha256": sha, "traffic_lib_sha256": None}
    tsha = t.get("lib_sha256")
    cur = tsha is not None and tsha == sha
    res = {"traffic": t.get("bwd_main_bytes") if cur else None, "lib_sha256": sha,
           "traffic_lib_sha256": tsha}
    if not cur:
        res["traffic_stale_bytes"] = t.get("bwd_main_bytes")
    return res


def traffic_path(cfg: int) -> Path:
    """Where the traffic summary of a config's run goes: profiles/traffic.json for config 2 (the
    headline's roofline.traffic), profiles/traffic_config<N>.json otherwise."""
    return TRAFFIC if cfg == 2 else TRAFFIC.with_name(f"traffic_config{cfg}.json")


# Kernel roles by name prefix (the traffic summary's keys).
KERNEL_ROLES = (("fwd", "fwd_kernel"), ("bwd_prep", "prep_kernel"),
                ("bwd_main", "bwd_split_kernel"), ("bwd_main", "bwd_kernel"),
                ("bwd_dq", "dq_kernel"))


def summarize_traffic(fetch_csv: str, write_csv: str, cfg: int = 2) -> int:
    """profiles/traffic.json (config 2) or profiles/traffic_config<N>.json from two counter runs
    of `bench.py --calibrate-copy --no-extra [--config N]` (one counter each): per kernel the mean
    FETCH_SIZE / WRITE_SIZE over its launches, in KiB, each scaled by what the same counter reads
    for the 256 MiB device copy (bytes it is known to move)."""
    def load(path, counter):
        vals: dict[str, list[float]] = {}
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                if r.get("Counter_Name") == counter:
                    vals.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return vals

    fetch, write = load(fetch_csv, "FETCH_SIZE"), load(write_csv, "WRITE_SIZE")
    copy = [k for k in fetch if "copyBuffer" in k]
    if not copy:
        print("bench.py: no copy kernel in the counter files (run with --calibrate-copy)",
              file=sys.stderr)
        return 1
    cf, cw = fetch[copy[0]][0], write[copy[0]][0]
    sf, sw = COPY_KIB / cf, COPY_KIB / cw
    name, kind, b, h, seq, causal, _, _ = CONFIGS[cfg]
    out = {"workload": f"{name}: {kind} b{b} h{h} s{seq} d64 "
                       + ("causal" if causal else "non-causal"),
           "lib_sha256": lib_sha256(), "copy_calibration_kib": COPY_KIB,
           "copy_fetch_kib": round(cf, 1), "copy_write_kib": round(cw, 1),
           "scale_fetch": round(sf, 5), "scale_write": round(sw, 5)}
    for key, prefix in KERNEL_ROLES:
        names = [n for n in fetch if _kernel_label(n).startswith(prefix) and n in write]
        if not names or key in out:
            continue
        fr, wr = statistics.mean(fetch[names[0]]), statistics.mean(write[names[0]])
        fb, wb = round(fr * 1024 * sf), round(wr * 1024 * sw)
        out[key] = {"kernel": _kernel_label(names[0]), "launches": len(fetch[names[0]]),
                    "fetch_kib_raw": round(fr, 2), "write_kib_raw": round(wr, 2),
                    "fetch_bytes": fb, "write_bytes": wb, "bytes": fb + wb}
    out["bwd_main_bytes"] = out.get("bwd_main", {}).get("bytes")
    out["fwd_bytes"] = out.get("fwd", {}).get("bytes")
    traffic_path(cfg).write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out, indent=1))
    return 0


def _kernel_label(raw: str) -> str:
    name = raw.split("fattn::(anonymous namespace)::", 1)[-1]
    return name.split("(", 1)[0].replace("void ", "")


def _headline_windows(rows: list, warmup: int, steps: int, cfg: int) -> dict | None:
    """The headline's windows from a time-ordered list of (start, kernel, workgroups, payload)
    dispatches of `bench.py --warmup W --steps K`: {"timed", "fwds", "kern", "bwds", "idle"}, each
    a list of steps, a step a list of (kernel, workgroups, payload); None if the run holds no such
    window. Configs 3-5 run the same kernel names, so the dispatches are split into steps (a step
    starts at a forward launch, or at a step-2 launch in a step that already holds one) and the
    main config's steps picked by the forward's name and grid; the headline's are the run of them
    after configs 3-5, its K forwards, K kernel-level steps and K backwards the steps after it."""
    b, h, s = CONFIGS[cfg][2], CONFIGS[cfg][3], CONFIGS[cfg][4]
    qb = 64 if CONFIGS[cfg][5] else 128
    main_fwd = (CAUSAL_FWD_NAME if CONFIGS[cfg][5] else KERNEL_NAMES["fwd"],
                ((s + qb - 1) // qb) * b * h)
    steps_seq: list[list] = []

    def step2(name):
        return name.startswith(("bwd_split_kernel", "bwd_kernel"))

    for _, name, wgs, payload in rows:
        if (name.startswith("fwd_kernel") or not steps_seq
                or (step2(name) and any(step2(n) for n, _, _ in steps_seq[-1]))):
            steps_seq.append([])
        steps_seq[-1].append((name, wgs, payload))
    is_main = [st[0][0] == main_fwd[0] and st[0][1] == main_fwd[1] for st in steps_seq]
    # Runs of consecutive main-config steps: the idle run opens the run (unless --no-extra, when
    # it is one run); the headline's is the first run after another config's steps that holds the
    # W warm-up, K timed, K forward and K kernel-level steps.
    runs, start = [], None
    for i, m in enumerate(is_main + [False]):
        if m and start is None:
            start = i
        elif not m and start is not None:
            runs.append((start, i))
            start = None
    need = warmup + 3 * steps
    if len(runs) == 1 and runs[0][0] == 0:
        first, idle = warmup + steps, steps_seq[warmup:warmup + steps]
    else:
        idle = (steps_seq[warmup:warmup + steps]
                if runs and runs[0][0] == 0 and runs[0][1] >= warmup + steps else [])
        later = [r for r in runs if r[0] > 0 and r[1] - r[0] >= need]
        first = later[0][0] if later else len(steps_seq)
    win = {
        "timed": steps_seq[first + warmup:first + warmup + steps],
        "fwds": steps_seq[first + warmup + steps:first + warmup + 2 * steps],
        "kern": steps_seq[first + warmup + 2 * steps:first + warmup + 3 * steps],
        "bwds": steps_seq[first + warmup + 3 * steps:first + warmup + 4 * steps],
        "idle": idle,
    }
    if len(win["timed"]) < steps or len(win["kern"]) < steps:
        return None
    if not (len(win["bwds"]) == steps and all(step2(st[0][0]) for st in win["bwds"])):
        win["bwds"] = []
    return win


def summarize_trace(trace_csv: str, warmup: int, steps: int, cfg: int = 2) -> int:
    """Per-kernel durations of the headline's GPU work, from a rocprofv3 --kernel-trace file of
    `bench.py --warmup W --steps K` (same W and K): the K timed forward+backward steps, the K
    op-level forwards and backwards (`fwd_ms`, `bwd_ms`, which price `roofline`), the K
    kernel-level steps (`kernels_us`), and the first K steps from idle (_headline_windows)."""
    rows = []
    with open(trace_csv, newline="") as f:
        for r in csv.DictReader(f):
            if "fattn::" not in r["Kernel_Name"]:
                continue
            wgs = int(r["Grid_Size_X"]) // max(int(r["Workgroup_Size_X"]), 1)
            rows.append((int(r["Start_Timestamp"]), _kernel_label(r["Kernel_Name"]), wgs,
                         (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    rows.sort()
    win = _headline_windows(rows, warmup, steps, cfg)
    if win is None:
        print(f"bench.py: the trace holds no run of {warmup + 3 * steps} config-{cfg} steps after "
              "the other configs", file=sys.stderr)
        return 1

    def table(title, seq):
        per: dict[str, list[float]] = {}
        for st in seq:
            for name, _, us in st:
                per.setdefault(name, []).append(us)
        total = sum(sum(v) for v in per.values())
        print(f"\n{title}\n")
        print("| kernel | calls | average (us) | median (us) | min (us) | max (us) | share |")
        print("|---|--:|--:|--:|--:|--:|--:|")
        for name, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
            print(f"| `{name}` | {len(v)} | {statistics.mean(v):.1f} | {statistics.median(v):.1f} "
                  f"| {min(v):.1f} | {max(v):.1f} | {100 * sum(v) / total:.1f} % |")

    table(f"The {steps} timed forward+backward steps (after {warmup} warm-up steps)", win["timed"])
    table(f"The {steps} op-level forwards (`fwd_ms`, `roofline.fwd_kernel_achieved`)", win["fwds"])
    if win["bwds"]:
        table(f"The {steps} op-level backwards (`bwd_ms`, `roofline.achieved`)", win["bwds"])
    table(f"The {steps} kernel-level steps (`kernels_us`)", win["kern"])
    if win["idle"]:
        table(f"The first {steps} steps from idle (after {warmup} warm-up steps; "
              "`fwd_bwd_from_idle_ms`)", win["idle"])
    return 0


# Counters per dispatch that the summary derives figures from (any subset may be present).
MFMA_CYCLES = 32            # v_mfma_f32_16x16x4_f32: 8 passes of 4 cycles on one SIMD
N_SIMDS, N_CUS, N_XCDS = 1024, 256, 8


def summarize_counters(csvs: list[str], warmup: int, steps: int, cfg: int = 2) -> int:
    """SQ / GRBM counters of the headline's K timed steps, per kernel, from the
    `counter_collection.csv` files of `rocprofv3 --pmc ... -- python3 bench.py --warmup W --steps K
    ...` runs (one file per counter pass; the same W, K and main config): each pass's dispatches
    are split into steps as _headline_windows does, the timed window's dispatches of each kernel
    averaged, and the passes merged. GRBM_GUI_ACTIVE comes summed over the 8 XCDs (per dispatch it
    reads 8 x the kernel's duration in GPU cycles), so the GPU-busy cycles of a dispatch are an
    eighth of it. Derived (where the counters are there): MFMA busy = SIMD cycles with the matrix
    core busy / (GPU-busy cycles x 1024 SIMDs); the MFMA instructions' own cycles (32 each)
    against that; waves per SIMD = 4 SQ_WAVE_CYCLES (quad-cycles) / (GPU-busy cycles x 1024
    SIMDs); non-MFMA VALU issue (4 cycles an instruction) as a share of SIMD cycles; per MFMA
    instruction: other VALU, SALU, LDS, transcendental instructions; executed MFMA GFLOP (512 FLOP
    per F32 MOPS unit); wave time waiting on a dependency (SQ_WAIT_ANY: memory, LDS, barrier),
    waiting to issue (SQ_WAIT_INST_ANY: its pipe busy with other waves) and issuing
    (SQ_ACTIVE_INST_ANY) as shares of the waves' cycles. Printed as a markdown table."""
    per: dict[str, dict[str, list[float]]] = {}
    calls: dict[str, int] = {}
    for path in csvs:
        disp: dict[int, dict] = {}
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                if "fattn::" not in r["Kernel_Name"]:
                    continue
                d = disp.setdefault(int(r["Dispatch_Id"]), {
                    "t": int(r["Start_Timestamp"]), "name": _kernel_label(r["Kernel_Name"]),
                    "wgs": int(r["Grid_Size"]) // max(int(r["Workgroup_Size"]), 1), "c": {}})
                d["c"][r["Counter_Name"]] = d["c"].get(r["Counter_Name"], 0.0) + float(
                    r["Counter_Value"])
        rows = sorted((d["t"], d["name"], d["wgs"], d["c"]) for d in disp.values())
        win = _headline_windows(rows, warmup, steps, cfg)
        if win is None:
            print(f"bench.py: {path} holds no run of {warmup + 3 * steps} config-{cfg} steps",
                  file=sys.stderr)
            return 1
        seen: dict[str, int] = {}
        for st in win["timed"]:
            for name, _, c in st:
                seen[name] = seen.get(name, 0) + 1
                slot = per.setdefault(name, {})
                for k, v in c.items():
                    slot.setdefault(k, []).append(v)
        for name, n in seen.items():
            calls[name] = max(calls.get(name, 0), n)
    mean = {n: {k: statistics.mean(v) for k, v in c.items()} for n, c in per.items()}

    def derived(c: dict) -> dict:
        out = {}
        gui = c.get("GRBM_GUI_ACTIVE", 0.0) / N_XCDS
        mfma = c.get("SQ_INSTS_MFMA")
        if gui and "SQ_VALU_MFMA_BUSY_CYCLES" in c:
            out["MFMA busy (% of SIMD cycles)"] = 100 * c["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui * N_SIMDS)
        if mfma and "SQ_VALU_MFMA_BUSY_CYCLES" in c:
            out["MFMA instruction cycles / MFMA busy cycles"] = (
                mfma * MFMA_CYCLES / c["SQ_VALU_MFMA_BUSY_CYCLES"])
        if gui and "SQ_WAVE_CYCLES" in c:
            out["waves per SIMD (average)"] = 4 * c["SQ_WAVE_CYCLES"] / (gui * N_SIMDS)
        if mfma and gui and "SQ_INSTS_VALU" in c:
            out["non-MFMA VALU issue (% of SIMD cycles)"] = (
                100 * 4 * (c["SQ_INSTS_VALU"] - mfma) / (gui * N_SIMDS))
        if mfma:
            if "SQ_INSTS_VALU" in c:
                out["other VALU per MFMA"] = (c["SQ_INSTS_VALU"] - mfma) / mfma
            for k, label in (("SQ_INSTS_SALU", "SALU per MFMA"), ("SQ_INSTS_LDS", "LDS per MFMA"),
                             ("SQ_INSTS_VALU_TRANS_F32", "transcendental per MFMA"),
                             ("SQ_INSTS_BRANCH", "branches per MFMA"),
                             ("SQ_INSTS_SMEM", "scalar loads per MFMA"),
                             ("SQ_INSTS_VMEM", "vector memory per MFMA")):
                if k in c:
                    out[label] = c[k] / mfma
        if "SQ_INSTS_VALU_MFMA_MOPS_F32" in c:
            out["MFMA GFLOP executed"] = c["SQ_INSTS_VALU_MFMA_MOPS_F32"] * 512 / 1e9
        if c.get("SQ_WAVE_CYCLES"):
            for k, label in (("SQ_WAIT_ANY", "wave cycles waiting (%)"),
                             ("SQ_WAIT_INST_ANY", "wave cycles waiting to issue (%)"),
                             ("SQ_ACTIVE_INST_ANY", "wave cycles issuing (%)")):
                if k in c:
                    out[label] = 100 * c[k] / c["SQ_WAVE_CYCLES"]
        if gui:
            out["GPU-busy cycles (GRBM_GUI_ACTIVE / 8)"] = gui
        return out

    names = sorted(mean, key=lambda n: -mean[n].get("GRBM_GUI_ACTIVE", 0.0))
    der = {n: derived(mean[n]) for n in names}
    print(f"\nThe {steps} timed steps after {warmup} warm-up steps (config {cfg}): mean per "
          f"dispatch over {len(csvs)} counter run(s)\n")
    print("| | " + " | ".join(f"`{n}`" for n in names) + " |")
    print("|---|" + "--:|" * len(names))
    print("| dispatches per run | " + " | ".join(str(calls[n]) for n in names) + " |")
    keys = []
    for n in names:
        keys += [k for k in der[n] if k not in keys]
    for k in keys:
        print(f"| {k} | " + " | ".join(f"{der[n][k]:.4g}" if k in der[n] else "" for n in names)
              + " |")
    raw = sorted({k for n in names for k in mean[n]})
    for k in raw:
        print(f"| {k} | " + " | ".join(f"{mean[n][k]:.6g}" if k in mean[n] else "" for n in names)
              + " |")
    return 0


def time_extra(torch, w: Workload, steps: int, warmup: int, warm_ms: float = 200.0) -> dict:
    """Op-level forward, backward and forward+backward ms, and each kernel's us, of one extra
    config, after at least `warmup` steps and at least `warm_ms` of back-to-back steps: the first
    calls on a new shape touch freshly allocated pages, and MI355X raises its clocks over some
    tens of milliseconds of sustained work (100 steps of config 3 are 14 ms, right after the
    headline's steps from idle)."""
    for _ in range(warmup):
        w.step()
    torch.cuda.synchronize()
    done, t0 = warmup, time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warm_ms:
        for _ in range(20):
            w.step()
        torch.cuda.synchronize()
        done += 20
    fb_ms, _, _ = event_steps(torch, w.stream, w.step, steps)
    f_ms, _, _ = event_steps(torch, w.stream, w.fwd, steps)
    kus = kernel_steps(torch, w.stream, w.kernels, steps)
    b_ms, _, _ = event_steps(torch, w.stream, w.bwd, steps)
    f_fwd, f_bwd = w.flops()
    bwd_us = kus.get("bwd_prep", 0.0) + kus["bwd_main"] + kus.get("bwd_dq", 0.0)
    return {
        "workload": f"{w.kind} b{w.b} h{w.h} s{w.s} d{w.d} "
                    + ("causal" if w.causal else "non-causal")
                    + (f", inputs ~N(0, {w.std ** 2:g})" if w.std != 1.0 else ""),
        "fwd_ms": round(f_ms, 5), "bwd_ms": round(b_ms, 5), "fwd_bwd_ms": round(fb_ms, 5),
        "fwd_bwd_tflops": round((f_fwd + f_bwd) / (fb_ms * 1e-3) / 1e12, 3),
        "fwd_frac": round(f_fwd / (f_ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
        "bwd_frac": round(f_bwd / (b_ms * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
        "kernels_us": {k: round(v, 2) for k, v in kus.items()},
        "bwd_main_frac": round(f_bwd / (kus["bwd_main"] * 1e-6) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
        "bwd_steps_frac": round(f_bwd / (bwd_us * 1e-6) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
        "fwd_kernel_frac": round(f_fwd / (kus["fwd"] * 1e-6) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
        "dq_sum": "split" if w.split else "turns",
        "steps": steps, "warmup": done,
    }


STEP_BENCH = REPO / "candle-fused-attn_amd" / "lib" / "cfa_step_bench"


def time_cxx_layer(b: int, h: int, s: int, d: int, causal: bool, warmup: int,
                   steps: int) -> dict | None:
    """Forward + backward steps through the C++ op layer (libcandle_fused_attn.so), timed by its
    own program in a child process (lib/cfa_step_bench: fused_attention_qkv and the node's bwd per
    step, outputs from the layer's memory pool, the node's kept workspace); None if it is not
    built or fails."""
    import subprocess
    if not STEP_BENCH.exists():
        log(f"bench: {STEP_BENCH} is not built: no C++ op layer step")
        return None
    cmd = [str(STEP_BENCH), str(b), str(h), str(s), str(d), str(int(causal)), str(warmup),
           str(steps)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    if res.returncode != 0:
        log(f"bench: C++ op layer step failed ({res.returncode}): {res.stderr.strip()[-400:]}")
        return None
    return json.loads(res.stdout.strip().splitlines()[-1])


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # MI355X raises its clocks over the first tens of milliseconds of sustained work (a kernel
    # trace shows the forward going from 71 to 58 us per call) and lowers them within a second of
    # idling. The line reports the first and last five timed steps, so a ramp shows.
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--causal", action="store_true", help="config 3 as the main workload")
    ap.add_argument("--config", type=int, choices=sorted(CONFIGS), default=None,
                    help="the main workload's config (default 2; --causal is config 3); the "
                         "driver's line is config 2's")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-accuracy", action="store_true", help="skip the fp64 scoring")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip timing configs 3-5 and config 2 at head_dim 32 / 128")
    ap.add_argument("--extra-steps", type=int, default=20)
    ap.add_argument("--cpu-threads", type=int, default=None)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one 256 MiB device-to-device copy (a kernel of known traffic, "
                         "to scale rocprofv3's FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write profiles/traffic.json from two counter files and exit (no GPU)")
    ap.add_argument("--counters-from", nargs="+", metavar="COUNTER_CSV",
                    help="no GPU: summarise rocprofv3 --pmc counter files of this command's "
                         "timed steps (same --warmup, --steps, --causal)")
    ap.add_argument("--trace-from", metavar="KERNEL_TRACE_CSV",
                    help="print per-kernel durations of the headline's steps from a rocprofv3 "
                         "kernel trace of this command with the same --warmup / --steps (and "
                         "--causal), and "
                         "exit (no GPU)")
    args = ap.parse_args()
    main_cfg = args.config or (3 if args.causal else 2)
    if args.traffic_from:
        return summarize_traffic(*args.traffic_from, cfg=main_cfg)
    if args.counters_from:
        return summarize_counters(args.counters_from, max(args.warmup, 1), max(args.steps, 1),
                                  main_cfg)
    if args.trace_from:
        return summarize_trace(args.trace_from, max(args.warmup, 1), max(args.steps, 1),
                               main_cfg)
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
    w = Workload(torch, L, _lib, dev, main_cfg)
    B, H, S, D, causal = w.b, w.h, w.s, w.d, w.causal

    if args.calibrate_copy:
        src = torch.ones(COPY_KIB * 256, device=dev)   # 256 MiB of f32
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    log(f"bench: config {main_cfg} b{B} h{H} s{S} d{D}; warmup {args.warmup}, "
        f"steps {args.steps}")
    K = max(args.steps, 1)
    n5 = min(5, K)

    # The same W + K steps from an idle GPU first ("cold"): MI355X lowers its clocks within a
    # second of idling and raises them again over some tens of milliseconds of sustained work, so
    # a short run started from idle measures the ramp. Then configs 3-5 are timed (about a second
    # of sustained work), and the headline's W warm-up and K timed steps follow them directly, at
    # the clocks a training loop runs at.
    for _ in range(max(args.warmup, 1)):
        w.step()
    torch.cuda.synchronize()
    cold_ms, cold_edges, _ = event_steps(torch, w.stream, w.step, K, n5)
    log(f"bench: from idle: fwd+bwd {cold_ms:.4f} ms (first {n5} steps {cold_edges[0]:.4f}, "
        f"last {n5} {cold_edges[1]:.4f})")

    extra = {}
    if not args.no_extra:
        for cfg in (2, 3, 4, 5):
            if cfg == main_cfg:
                continue
            xw = Workload(torch, L, _lib, dev, cfg)
            extra[f"config{cfg}"] = time_extra(torch, xw, max(args.extra_steps, 1), 100)
            log(f"bench: {CONFIGS[cfg][0]}: {json.dumps(extra[f'config{cfg}'])}")
            del xw
        torch.cuda.synchronize()

    for _ in range(max(args.warmup, 1)):
        w.step()
    torch.cuda.synchronize()

    # roctx ranges name the timed windows (the reference brackets them with cuProfilerStart /
    # Stop for an nsys capture range, examples/compare.rs:261-277); `rocprofv3 --marker-trace`
    # records them. torch.cuda.nvtx is roctx on ROCm.
    torch.cuda.nvtx.range_push("fattn timed fwd+bwd")
    fwd_bwd_ms, edges, fwd_bwd_wall = event_steps(torch, w.stream, w.step, K, n5)
    torch.cuda.nvtx.range_pop()
    torch.cuda.nvtx.range_push("fattn timed fwd")
    fwd_ms, _, _ = event_steps(torch, w.stream, w.fwd, K)
    torch.cuda.nvtx.range_pop()
    first5, last5 = edges
    log(f"bench: fwd+bwd {fwd_bwd_ms:.4f} ms (wall {fwd_bwd_wall:.4f}; first {n5} steps "
        f"{first5:.4f}, last {n5} {last5:.4f}), fwd {fwd_ms:.4f} ms")

    # Per-kernel durations: K more steps, back to back as above, with the backward launched as
    # its kernel-level steps (the same kernels on the same arguments as the op-level backward)
    # and a HIP event on the launch stream between every two launches.
    torch.cuda.nvtx.range_push("fattn kernel-level steps")
    kus = kernel_steps(torch, w.stream, w.kernels, K)
    torch.cuda.nvtx.range_pop()
    fwd_us, prep_us, main_us = kus["fwd"], kus.get("bwd_prep", 0.0), kus["bwd_main"]
    dq_us = kus.get("bwd_dq", 0.0)
    log(f"bench: kernels fwd {fwd_us:.1f} us, prep {prep_us:.1f} us, bwd main {main_us:.1f} us, "
        f"dq sum {dq_us:.1f} us ({'split' if w.split else 'turns'}); step {kus['step']:.1f} us")

    # The op-level backward alone, K calls back to back with events only at the window's ends.
    # With a split workspace at d <= 64 a call is one launch of step 2 (step 1 launches nothing,
    # and step 2 sums every dQ tile), so the window's mean is step 2's average launch duration
    # plus one dispatch gap; the forward window (`fwd_ms`) is the forward kernel's likewise.
    torch.cuda.nvtx.range_push("fattn timed bwd")
    bwd_ms, _, _ = event_steps(torch, w.stream, w.bwd, K)
    torch.cuda.nvtx.range_pop()
    one_launch = w.split and D <= 64
    log(f"bench: op-level bwd {bwd_ms:.4f} ms"
        + (" (one step-2 launch per call)" if one_launch else ""))

    if not args.no_extra:
        # The other head dims the kernels are built for, at the headline's shape: after the
        # headline (right before it, the heavier head_dim 128 work left the next 25 steps 4 %
        # slower in a kernel trace than the same kernels a few ms later).
        for d in (32, 128):
            xw = Workload(torch, L, _lib, dev, 2, d=d)
            extra[f"config2_d{d}"] = time_extra(torch, xw, max(args.extra_steps, 1), 100)
            log(f"bench: config 2 at d {d}: {json.dumps(extra[f'config2_d{d}'])}")
            del xw
        torch.cuda.synchronize()

    cxx = None
    if not args.no_extra:
        # The same step through the C++ op layer, in a child process once this one is idle: its
        # warm-up (at least 500 steps, about 0.1 s) brings the clocks back up after the child's
        # start-up.
        torch.cuda.synchronize()
        cxx = time_cxx_layer(B, H, S, D, causal, max(args.warmup, 500), K)
        if cxx:
            log(f"bench: C++ op layer step {cxx['fwd_bwd_ms']:.4f} ms "
                f"({cxx['fwd_bwd_ms'] / fwd_bwd_ms:.3f} x the C-ABI step)")

    f_fwd, f_bwd = w.flops()
    fwd_tflops = f_fwd / (fwd_ms * 1e-3) / 1e12
    total_tflops = (f_fwd + f_bwd) / (fwd_bwd_ms * 1e-3) / 1e12
    main_tflops = f_bwd / (main_us * 1e-6) / 1e12
    bwd_steps_tflops = f_bwd / ((prep_us + main_us + dq_us) * 1e-6) / 1e12
    fwdk_tflops = f_fwd / (fwd_us * 1e-6) / 1e12
    bwd_tflops = f_bwd / (bwd_ms * 1e-3) / 1e12
    # Step 2's rate: from the op-level backward window where a call is that one launch, else from
    # the kernel-level events around it.
    step2_tflops = bwd_tflops if one_launch else main_tflops
    traffic = traffic_entry()

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
            "workload": (f"qkv path forward+backward, qkv [{B}, {S}, {3 * H * D}] (h {H}, d {D}) "
                         f"and dout [{B}, {S}, {H * D}] ~ N(0,1) seed 0, scale 1/8, "
                         + ("causal (config 3)" if causal else "non-causal (config 2)")),
            "b": B, "h": H, "s": S, "d": D, "causal": causal,
            "entry": "fattn_qkv_forward + fattn_qkv_backward",
        },
        "fwd_ms": round(fwd_ms, 5),
        "bwd_ms": round(bwd_ms, 5),
        "fwd_bwd_ms": round(fwd_bwd_ms, 5),
        "fwd_bwd_wall_ms": round(fwd_bwd_wall, 5),
        "fwd_bwd_first5_ms": round(first5, 5),
        "fwd_bwd_last5_ms": round(last5, 5),
        "fwd_bwd_from_idle_ms": round(cold_ms, 5),
        "fwd_bwd_from_idle_first5_ms": round(cold_edges[0], 5),
        "fwd_bwd_from_idle_last5_ms": round(cold_edges[1], 5),
        "sequence": ("W warm-up + K timed steps from idle (fwd_bwd_from_idle_ms), "
                     + ("configs 3-5 timed (configs), " if extra else "")
                     + "W warm-up + K timed steps (value), K forwards, K kernel-level steps, "
                     + "K backwards"
                     + (", config 2 at d 32 / 128 timed (configs), the C++ op layer's step "
                        "(cxx_op_layer)" if extra else "")),
        "fwd_tflops": round(fwd_tflops, 3),
        "fwd_bwd_tflops": round(total_tflops, 3),
        "frac_fp32_peak": round(total_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
        "kernels_us": {"fwd": round(fwd_us, 2), "bwd_prep": round(prep_us, 2),
                       "bwd_main": round(main_us, 2), "bwd_dq": round(dq_us, 2),
                       "step": round(kus["step"], 2)},
        "dq_sum": "split" if w.split else "turns",
        "roofline": {
            "kernel": ("bwd_split_kernel<64, 1, false> (fattn_bwd_main_f32_d64, split; its last "
                       "workgroups sum dQ tiles)" if w.split
                       else "bwd_kernel<false, 64> (fattn_bwd_main_f32_d64, turns)"),
            "bound": "mfma",
            "achieved": round(step2_tflops, 3),
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(step2_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
            **traffic,
            "flops_per_launch": f_bwd,
            "achieved_from": (f"bwd_ms: {K} op-level backwards back to back, one step-2 launch "
                              "each, HIP events at the window's ends" if one_launch
                              else "kernels_us.bwd_main: kernel-level events"),
            "kernel_level_achieved": round(main_tflops, 3),
            "kernel_level_frac": round(main_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
            "bwd_steps_1_3_achieved": round(bwd_steps_tflops, 3),
            "fwd_kernel_achieved": round(fwd_tflops, 3),
            "fwd_kernel_frac": round(fwd_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
            "fwd_kernel_level_frac": round(fwdk_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
        },
    }

    if extra:
        result["configs"] = extra
    if cxx:
        result["cxx_op_layer"] = {
            "fwd_bwd_ms": round(cxx["fwd_bwd_ms"], 5),
            "vs_c_abi_step": round(cxx["fwd_bwd_ms"] / fwd_bwd_ms, 4),
            "steps": cxx["steps"], "warmup": cxx["warmup"],
            "how": ("candle_fused_attn::fused_attention_qkv + node->bwd per step "
                    "(libcandle_fused_attn.so; outputs from its memory pool, the node's kept "
                    "workspace), HIP events around K steps, in a child process "
                    "(lib/cfa_step_bench) after the C-ABI legs"),
        }

    if not args.no_accuracy:
        from oracle import oracle as orc
        w.step()
        torch.cuda.synchronize()
        first = w.dqkv.clone()
        w.bwd()
        torch.cuda.synchronize()
        rerun_equal = bool(torch.equal(first.view(torch.int32), w.dqkv.view(torch.int32)))
        t0 = time.perf_counter()
        x, dd = w.qkv_cpu.numpy(), w.dout_cpu.numpy()
        ro, rl = orc.qkv_forward(x, H, SCALE, causal, dtype=np.float64)
        rg = orc.qkv_backward(x, H, SCALE, causal, ro, rl, dd, dtype=np.float64)
        go, gg, gl = w.out.cpu().numpy(), w.dqkv.cpu().numpy(), w.lse.cpu().numpy()
        acc = {"o": orc.rel_fro(go, ro)}
        for name, a, r in zip(("dq", "dk", "dv"), np.split(gg, 3, axis=-1),
                              np.split(rg, 3, axis=-1)):
            acc[name] = orc.rel_fro(a, r)
        result["accuracy"] = {
            "normwise_vs_fp64": {k: float(f"{v:.3e}") for k, v in acc.items()},
            "lse_max_abs_vs_fp64": float(f"{orc.max_abs(gl, rl):.3e}"),
            "tolerance": 2e-6,
            "within_tolerance": all(v <= 2e-6 for v in acc.values()),
            "bitwise_rerun": rerun_equal,
        }
        log(f"bench: accuracy {acc}, L max-abs {orc.max_abs(gl, rl):.2e} "
            f"(fp64 scoring {time.perf_counter() - t0:.1f} s), bitwise rerun {rerun_equal}")

    if not args.no_cpu:
        from oracle import oracle as orc
        threads = args.cpu_threads or orc.default_threads()
        x, dd = w.qkv_cpu.numpy(), w.dout_cpu.numpy()

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
            "sample": (f"full config {main_cfg} forward+backward, median of "
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
