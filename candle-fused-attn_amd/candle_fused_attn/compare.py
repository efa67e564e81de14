"""Head-to-head of the fused attention with PyTorch-ROCm's own fp32 attentions on one MI355X.

This is the report the reference publishes for its CUDA build against PyTorch-CUDA
(bench/compare.py, bench/results/*-compare-v0.4.md): agreement with a float64 recompute, bit
equality of reruns, timing in alternated rounds with a decision rule, and per-call kernel time
from a profiler. Here every contender is Python on one device, so the design is in-process:

* Contenders. Each one maps the fused projection qkv [b, s, 3 h d] (a leaf tensor) to the merged
  output [b, s, h d], so head split and merge are part of every timed call:
    fattn.qkv        fused_attention_qkv (libfattn.so, hand-written gfx950 kernels)
    fattn.views      fused_attention on the q / k / v views of qkv, output merged back (the
                     views of one projection go to fused_attention_qkv's node)
    fattn.general    the same call with that routing switched off: fused_attention's own node,
                     whose three gradients autograd assembles into qkv's
    torch.eager      explicit softmax((q k^T) scale) v in torch ops (hipBLASLt matmuls)
    sdpa.math        scaled_dot_product_attention with the MATH backend forced
    sdpa.efficient   ... EFFICIENT_ATTENTION backend forced (AOTriton on ROCm)
    sdpa.flash       ... FLASH_ATTENTION backend forced (refuses fp32: recorded, not timed)
  The backward is out.backward(dout): the gradient arrives as given, with no loss head to time
  or subtract.
* Agreement. o, dq, dk, dv of every contender against float64 autograd of the same attention on
  the CPU (einsum formulation, independent of every contender): normwise relative error
  ||x - ref|| / ||ref|| and max-abs error; the floor row is the float64 result rounded to fp32.
  Reruns: a second forward + backward compared bit for bit.
* Timing. HIP events around `calls` back-to-back calls of one phase (`fwd` under no_grad, `step` =
  forward + backward) give one sample in ms per call. A round takes `reps` samples of every
  contender and phase in the order of one row of a cyclic Latin square over the contenders (row r
  for round r), so every contender runs in every position equally often; the round's value is the
  median of its samples.
* Decision rule (paired by round): A is faster than B on a phase when A's round value is below B's
  in every round; B faster when the reverse holds in every round; otherwise the pair is a tie at
  this number of rounds. The ratio reported is of the medians over rounds.
* Kernel time (--kernels): each contender and phase once more in a child process under
  `rocprofv3 --kernel-trace`; the dispatches of the last `--kernel-calls` calls (the first
  `--kernel-skip` of the fresh process run at ramping clocks and are dropped), summed per kernel
  and divided by the calls, give ms per call. A kernel whose launches are not a whole number per
  call is listed apart (allocator fills, one-off setup) and left out of the sum.

Run on one MI355X from the repository root:
    PYTHONPATH=candle-fused-attn_amd python3 -m candle_fused_attn.compare report --out DIR
Writes DIR/report.md and DIR/report.json.
"""
from __future__ import annotations

import argparse
import csv
import io
import json
import shutil
import statistics
import subprocess
import sys
import tempfile
import time
from dataclasses import dataclass
from pathlib import Path
from typing import Callable

PARTS = ("o", "dq", "dk", "dv")
PHASES = ("fwd", "step")
MINE = ("fattn.qkv", "fattn.views", "fattn.general")
SDPA_BACKENDS = {"sdpa.math": "MATH", "sdpa.efficient": "EFFICIENT_ATTENTION",
                 "sdpa.flash": "FLASH_ATTENTION"}


# --- statistics and the decision rule ---------------------------------------------------------

def latin_row(names, r: int) -> list:
    """Row `r` of the cyclic Latin square over `names`: the order of round r.

    >>> latin_row(["x", "y", "z", "w"], 2)
    ['z', 'w', 'x', 'y']
    >>> [latin_row("pq", r) for r in range(3)]
    [['p', 'q'], ['q', 'p'], ['p', 'q']]
    """
    names = list(names)
    k = r % len(names)
    return names[k:] + names[:k]


def round_value(samples: list[float]) -> float:
    """A round's value: the median of its samples.

    >>> round_value([5.0, 1.0, 3.0, 100.0])
    4.0
    """
    return statistics.median(samples)


def paired_rule(a: list[float], b: list[float]) -> int:
    """-1 if A's round value is below B's in every round (A faster), +1 if above in every round
    (B faster), 0 otherwise (a tie at this number of rounds). Rounds are paired by index.

    >>> paired_rule([0.20, 0.21, 0.19], [0.30, 0.22, 0.25])
    -1
    >>> paired_rule([0.40, 0.41], [0.30, 0.35])
    1
    >>> paired_rule([0.20, 0.26], [0.25, 0.22])
    0
    """
    if len(a) != len(b) or not a:
        raise ValueError("paired_rule: one value per round for both contenders")
    if all(x < y for x, y in zip(a, b)):
        return -1
    if all(x > y for x, y in zip(a, b)):
        return 1
    return 0


def head_to_head(name_a: str, a: list[float], name_b: str, b: list[float]) -> str:
    """The rule's outcome as a sentence, with the ratio of the medians over rounds.

    >>> head_to_head("fattn.qkv", [0.2, 0.21], "sdpa.math", [0.6, 0.63])
    'fattn.qkv ahead, 3.00x'
    >>> head_to_head("p", [0.9, 0.8], "q", [0.3, 0.35])
    'q ahead, 2.62x'
    >>> head_to_head("p", [0.2, 0.3], "q", [0.25, 0.26])
    'no separation in 2 rounds'
    """
    rule = paired_rule(a, b)
    ma, mb = statistics.median(a), statistics.median(b)
    if rule < 0:
        return f"{name_a} ahead, {mb / ma:.2f}x"
    if rule > 0:
        return f"{name_b} ahead, {ma / mb:.2f}x"
    return f"no separation in {len(a)} rounds"


def spread(xs: list[float]) -> str:
    """Median over rounds and its range, in ms.

    >>> spread([0.5, 0.25, 0.75])
    '0.5000 (0.2500..0.7500)'
    >>> spread([])
    'n/a'
    """
    if not xs:
        return "n/a"
    return f"{statistics.median(xs):.4f} ({min(xs):.4f}..{max(xs):.4f})"


# --- profiler output ----------------------------------------------------------------------------

def parse_kernel_trace(text: str, skip_calls: int, calls: int) -> list[tuple[str, int, float]]:
    """(kernel name, launches, total ns) over the last `calls` of `skip_calls + calls` calls, from
    rocprofv3's kernel_trace.csv (one row per dispatch). A kernel launched k times per call has
    k (skip_calls + calls) dispatches: its first k skip_calls (in time order) are dropped. A
    kernel whose count is not such a multiple is returned whole (then listed apart).

    >>> t = ('"Kernel_Name","Start_Timestamp","End_Timestamp"\\n'
    ...      '"a",0,50\\n"a",100,130\\n"a",200,220\\n"b",300,301\\n')
    >>> parse_kernel_trace(t, 1, 2)
    [('a', 2, 50.0), ('b', 1, 1.0)]
    """
    runs: dict[str, list[tuple[int, int]]] = {}
    for r in csv.DictReader(io.StringIO(text)):
        runs.setdefault(r["Kernel_Name"], []).append((int(r["Start_Timestamp"]),
                                                      int(r["End_Timestamp"])))
    rows = []
    for name, ds in runs.items():
        ds.sort()
        total = skip_calls + calls
        if len(ds) % total == 0:
            ds = ds[len(ds) // total * skip_calls:]
        rows.append((name, len(ds), float(sum(e - b for b, e in ds))))
    return rows


def kernel_time_per_call(rows: list[tuple[str, int, float]], calls: int) -> dict:
    """ms per call from kernels launched a multiple of `calls` times; the rest listed apart.

    >>> t = kernel_time_per_call([("a", 8, 1600.0), ("b", 4, 4000.0), ("z", 3, 90.0)], 4)
    >>> round(t["ms"], 6), t["other"], [(k["name"], k["per_call"]) for k in t["kernels"]]
    (0.0014, ['z'], [('b', 1), ('a', 2)])
    """
    kept, other, total = [], [], 0.0
    for name, n, ns in rows:
        if n and n % calls == 0:
            kept.append({"name": name, "per_call": n // calls, "us": ns / calls / 1e3})
            total += ns
        else:
            other.append(name)
    kept.sort(key=lambda k: -k["us"])
    return {"ms": total / calls / 1e6, "kernels": kept, "other": other}


def short_kernel(name: str) -> str:
    """A kernel's name without its return type, namespaces and argument list, for the report.

    >>> short_kernel("void fattn::(anonymous namespace)::fwd_kernel<64, 128>(FwdArgs)")
    'fwd_kernel<64, 128>'
    >>> short_kernel("__amd_rocclr_fillBufferAligned")
    '__amd_rocclr_fillBufferAligned'
    >>> short_kernel("void ew<4, at::native::Functor<float, float, float, Mul<float> > >(int)")
    'ew<4, at::native::Functor<float, float, fl...>'
    >>> short_kernel("Cijk_Ailk_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT240x256x16_MI16x16x1_SN_LDSB0")
    'Cijk_Ailk_Bljk_S_B_Bias_HA_S_SAV_UserArgs_MT240x256x16'
    """
    n = name.strip()
    if n.endswith(")"):  # drop the argument list: back to the '(' matching the last ')'
        depth = 0
        for i in range(len(n) - 1, -1, -1):
            depth += {")": 1, "(": -1}.get(n[i], 0)
            if depth == 0:
                n = n[:i]
                break
    depth, start = 0, 0
    for i, ch in enumerate(n):  # after the last ':' or ' ' outside <...> and (...)
        if ch in "<(":
            depth += 1
        elif ch in ">)":
            depth -= 1
        elif ch in ": " and depth == 0:
            start = i + 1
    n = n[start:]
    if n.startswith("Cijk_") and "_MT" in n:  # a Tensile GEMM: keep up to its macro tile
        head, _, tail = n.partition("_MT")
        return f"{head}_MT{tail.split('_')[0]}"
    return n if len(n) <= 48 else n[:42] + "...>"


# --- contenders ---------------------------------------------------------------------------------

@dataclass
class Contender:
    name: str
    forward: Callable  # qkv [b, s, 3 h d] -> out [b, s, h d]
    what: str


def make_contenders(heads: int, scale: float, causal: bool) -> list[Contender]:
    import torch
    import torch.nn.functional as F

    import candle_fused_attn as cfa

    def views(qkv):
        b, s, three_hd = qkv.shape
        d = three_hd // 3 // heads
        return qkv.view(b, s, 3, heads, d).permute(2, 0, 3, 1, 4).unbind(0)  # [b, h, s, d] each

    def merge(o):
        b, h, s, d = o.shape
        return o.transpose(1, 2).reshape(b, s, h * d)

    def fattn_views(qkv):
        q, k, v = views(qkv)
        return merge(cfa.fused_attention(q, k, v, scale, causal))

    def fattn_general(qkv):
        prev = cfa.ops.set_projection_route(False)
        try:
            return fattn_views(qkv)
        finally:
            cfa.ops.set_projection_route(prev)

    def eager(qkv):
        q, k, v = views(qkv)
        w = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
        if causal:
            s = q.shape[2]
            w = w.masked_fill(torch.ones(s, s, dtype=torch.bool, device=w.device).triu(1),
                              float("-inf"))
        return merge(torch.matmul(torch.softmax(w, dim=-1), v))

    def sdpa_with(backend_name):
        backend = getattr(torch.nn.attention.SDPBackend, backend_name)

        def run(qkv):
            q, k, v = views(qkv)
            with torch.nn.attention.sdpa_kernel([backend]):
                return merge(F.scaled_dot_product_attention(q, k, v, is_causal=causal,
                                                            scale=scale))
        return run

    out = [Contender("fattn.qkv", lambda x: cfa.fused_attention_qkv(x, heads, scale, causal),
                     "fused_attention_qkv (libfattn.so)"),
           Contender("fattn.views", fattn_views, "fused_attention on the q/k/v views"),
           Contender("fattn.general", fattn_general,
                     "fused_attention on the q/k/v views, its own node (no routing)"),
           Contender("torch.eager", eager, "softmax((q k^T) scale) v in torch ops")]
    for name, backend in SDPA_BACKENDS.items():
        out.append(Contender(name, sdpa_with(backend), f"scaled_dot_product_attention, {backend}"))
    return out


def reference64(qkv, dout, heads: int, scale: float, causal: bool) -> dict:
    """o, dq, dk, dv in float64 on the CPU (autograd of an einsum formulation)."""
    import torch
    x = qkv.detach().to("cpu", torch.float64).requires_grad_(True)
    b, s, three_hd = x.shape
    d = three_hd // 3 // heads
    q, k, v = x.view(b, s, 3, heads, d).unbind(2)                      # [b, s, h, d]
    logits = torch.einsum("bihc,bjhc->bhij", q, k) * scale
    if causal:
        logits = logits.masked_fill(torch.ones(s, s, dtype=torch.bool).triu(1), float("-inf"))
    o = torch.einsum("bhij,bjhc->bihc", torch.softmax(logits, dim=-1), v).reshape(b, s, heads * d)
    o.backward(dout.detach().to("cpu", torch.float64))
    dq, dk, dv = x.grad.view(b, s, 3, heads * d).unbind(2)
    return {"o": o.detach(), "dq": dq, "dk": dk, "dv": dv}


def agreement(got: dict, ref: dict) -> dict:
    """Per part: normwise relative error and max-abs error against `ref` (float64)."""
    res = {}
    for p in PARTS:
        r = ref[p]
        diff = got[p].to("cpu").double() - r
        den = float(r.norm())
        res[p] = {"rel": float(diff.norm()) / den if den else float(diff.norm()),
                  "max_abs": float(diff.abs().max()) if diff.numel() else 0.0}
    return res


def one_step(c: Contender, qkv, dout):
    """Forward + backward of a contender on a fresh leaf: (out, dq, dk, dv)."""
    x = qkv.detach().clone().requires_grad_(True)
    out = c.forward(x)
    out.backward(dout)
    hd = x.shape[-1] // 3
    return out.detach(), x.grad[..., :hd], x.grad[..., hd:2 * hd], x.grad[..., 2 * hd:]


# --- measurement --------------------------------------------------------------------------------

def phase_fn(torch, c: Contender, qkv, dout, phase: str):
    leaf = qkv.detach().clone().requires_grad_(phase == "step")

    def fwd():
        with torch.no_grad():
            c.forward(leaf)

    def step():
        leaf.grad = None
        c.forward(leaf).backward(dout)

    return fwd if phase == "fwd" else step


def event_block(torch, fn, calls: int) -> float:
    """ms per call over `calls` back-to-back calls, between two HIP events."""
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(calls):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / calls


def measure(torch, live: list[Contender], qkv, dout, rounds: int, reps: int, calls: int,
            warmup: int, log=print) -> dict:
    """{contender: {phase: [round values]}}, rounds ordered by the cyclic Latin square."""
    fns = {(c.name, p): phase_fn(torch, c, qkv, dout, p) for c in live for p in PHASES}
    for fn in fns.values():
        for _ in range(warmup):
            fn()
    torch.cuda.synchronize()
    by_name = {c.name: c for c in live}
    res = {c.name: {p: [] for p in PHASES} for c in live}
    for r in range(rounds):
        samples = {k: [] for k in fns}
        for _ in range(reps):
            for name in latin_row([c.name for c in live], r):
                for p in PHASES:
                    samples[(name, p)].append(event_block(torch, fns[(name, p)], calls))
        for (name, p), xs in samples.items():
            res[name][p].append(round_value(xs))
        log(f"compare: round {r + 1}/{rounds}: " + ", ".join(
            f"{n} {res[n]['step'][-1]:.4f}" for n in by_name))
    return res


def kernel_probe(args) -> None:
    """Child mode (run under rocprofv3): `calls` calls of one contender and phase, nothing else
    (the parent keeps the last ones: the first of a fresh process run at ramping clocks)."""
    import torch
    data = torch.load(args.inputs, weights_only=True)
    qkv, dout = data["qkv"].cuda(), data["dout"].cuda()
    c = {x.name: x for x in make_contenders(args.heads, args.scale, args.causal)}[args.contender]
    fn = phase_fn(torch, c, qkv, dout, args.phase)
    for _ in range(args.calls):
        fn()
    torch.cuda.synchronize()


def profile_kernels(args, name: str, phase: str, inputs: Path, work: Path) -> dict | None:
    rocprof = shutil.which("rocprofv3")
    if rocprof is None:
        return None
    tag = f"{name.replace('.', '_')}_{phase}"
    skip = args.kernel_skip
    cmd = [rocprof, "--kernel-trace", "--output-format", "csv", "-d", str(work / tag),
           "-o", "run", "--", sys.executable, "-m", "candle_fused_attn.compare", "probe",
           "--inputs", str(inputs), "--contender", name, "--phase", phase,
           "--calls", str(skip + args.kernel_calls), "--heads", str(args.heads),
           "--scale", str(args.scale)] + (["--causal"] if args.causal else [])
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    trace = sorted((work / tag).rglob("*kernel_trace.csv"))
    if not trace:
        return {"ms": None, "kernels": [], "other": [],
                "error": (res.stderr or res.stdout)[-400:]}
    rows = parse_kernel_trace(trace[0].read_text(), skip, args.kernel_calls)
    return kernel_time_per_call(rows, args.kernel_calls)


# --- the report ---------------------------------------------------------------------------------

def render(rep: dict) -> str:
    """The markdown report from the JSON result."""
    s = rep["setup"]
    lines = [f"# fused attention vs PyTorch-ROCm fp32 attention on {s['device']}", "",
             f"qkv [{s['b']}, {s['s']}, {3 * s['h'] * s['d']}] (h {s['h']}, d {s['d']}), "
             f"dout [{s['b']}, {s['s']}, {s['h'] * s['d']}], N(0, 1) from a CPU generator seeded "
             f"{s['seed']}, scale {s['scale']:g}, {'causal' if s['causal'] else 'non-causal'}. "
             f"{s['when']}; torch {s['torch']}, HIP {s['hip']}, fp32 matmul precision "
             f"{s['matmul_precision']}.", "",
             "## Contenders", "", "| name | what | status |", "|---|---|---|"]
    for name, st in rep["status"].items():
        lines.append(f"| {name} | {rep['what'][name]} | {st} |")
    live = [n for n, st in rep["status"].items() if st == "ran"]
    lines += ["", "## Agreement with float64 (normwise relative error / max-abs)", "",
              "| name | o | dq | dk | dv | rerun bit-equal |", "|---|--:|--:|--:|--:|:-:|"]
    for name in ["float64 rounded to fp32"] + live:
        e = rep["agreement"][name]
        cells = [f"{e[p]['rel']:.2e} / {e[p]['max_abs']:.1e}" for p in PARTS]
        eq = rep["rerun_equal"].get(name)
        lines.append(f"| {name} | " + " | ".join(cells) + f" | {'' if eq is None else ('yes' if eq else 'no')} |")
    t = rep["timing"]
    lines += ["", f"## Time per call, HIP events (ms; median over {t['rounds']} rounds, range)", "",
              f"Each round: {t['reps']} samples of {t['calls']} back-to-back calls per contender "
              f"and phase after {t['warmup']} warm-up calls, contenders ordered by one row of a "
              "cyclic Latin square; a round's value is its samples' median. `step` = forward + "
              "backward.", "", "| name | fwd | step |", "|---|--:|--:|"]
    for name in live:
        lines.append(f"| {name} | {spread(t['ms'][name]['fwd'])} | {spread(t['ms'][name]['step'])} |")
    lines += ["", "Head to head (A ahead when faster in every round):", "",
              "| A | B | fwd | step |", "|---|---|---|---|"]
    for a in MINE:
        for b in live:
            if b in MINE or a not in live:
                continue
            cells = [head_to_head(a, t["ms"][a][p], b, t["ms"][b][p]) for p in PHASES]
            lines.append(f"| {a} | {b} | " + " | ".join(cells) + " |")
    if rep.get("kernels"):
        lines += ["", f"## Kernel time per call, rocprofv3 (the last {rep['kernel_calls']} of "
                  f"{rep['kernel_skip'] + rep['kernel_calls']} calls per probe)",
                  "", "| name | phase | ms | kernels (launches per call, us per call) | not per call |",
                  "|---|---|--:|---|---|"]
        for key, k in rep["kernels"].items():
            name, phase = key.rsplit(":", 1)
            if k is None or k.get("ms") is None:
                lines.append(f"| {name} | {phase} | n/a | {(k or {}).get('error', 'no profiler')} | |")
                continue
            ks = "; ".join(f"{short_kernel(x['name'])} x{x['per_call']} {x['us']:.1f}"
                           for x in k["kernels"][:6])
            lines.append(f"| {name} | {phase} | {k['ms']:.4f} | {ks} | "
                         + ", ".join(short_kernel(o) for o in k["other"]) + " |")
    return "\n".join(lines) + "\n"


def report(args) -> int:
    import torch

    out = Path(args.out)
    out.mkdir(parents=True, exist_ok=True)
    torch.set_float32_matmul_precision("highest")
    dev = torch.device("cuda:0")
    b, h, s, d = args.batch, args.heads, args.seq, 64
    g = torch.Generator().manual_seed(args.seed)
    qkv_cpu = torch.randn(b, s, 3 * h * d, generator=g)
    dout_cpu = torch.randn(b, s, h * d, generator=g)
    qkv, dout = qkv_cpu.to(dev), dout_cpu.to(dev)
    log = lambda m: print(m, file=sys.stderr, flush=True)  # noqa: E731

    ref = reference64(qkv_cpu, dout_cpu, h, args.scale, args.causal)
    props = torch.cuda.get_device_properties(dev)
    device = f"{props.gcnArchName.split(':')[0]} ({props.multi_processor_count} CUs)"
    rep = {"setup": {"device": device, "b": b, "h": h, "s": s, "d": d,
                     "seed": args.seed, "scale": args.scale, "causal": args.causal,
                     "when": time.strftime("%Y-%m-%d %H:%M"), "torch": torch.__version__,
                     "hip": torch.version.hip,
                     "matmul_precision": torch.get_float32_matmul_precision()},
           "status": {}, "what": {}, "rerun_equal": {},
           "agreement": {"float64 rounded to fp32": agreement(
               {p: v.float() for p, v in ref.items()}, ref)}}
    contenders = make_contenders(h, args.scale, args.causal)
    live = []
    for c in contenders:
        rep["what"][c.name] = c.what
        try:
            first = one_step(c, qkv, dout)
            second = one_step(c, qkv, dout)
            torch.cuda.synchronize()
        except Exception as e:  # a backend that refuses these inputs is recorded, not timed
            rep["status"][c.name] = "refused: " + str(e).splitlines()[0][:160]
            torch.cuda.synchronize()
            continue
        rep["status"][c.name] = "ran"
        rep["agreement"][c.name] = agreement(dict(zip(PARTS, first)), ref)
        rep["rerun_equal"][c.name] = all(
            torch.equal(x.contiguous().view(torch.int32), y.contiguous().view(torch.int32))
            for x, y in zip(first, second))
        live.append(c)
        log(f"compare: {c.name}: " + " ".join(
            f"{p} {rep['agreement'][c.name][p]['rel']:.2e}" for p in PARTS))
    rep["timing"] = {"rounds": args.rounds, "reps": args.reps, "calls": args.calls,
                     "warmup": args.warmup,
                     "ms": measure(torch, live, qkv, dout, args.rounds, args.reps, args.calls,
                                   args.warmup, log)}
    if args.kernels:
        rep["kernel_calls"], rep["kernel_skip"] = args.kernel_calls, args.kernel_skip
        rep["kernels"] = {}
        with tempfile.TemporaryDirectory(dir=out) as tmp:
            work = Path(tmp)
            inputs = work / "inputs.pt"
            torch.save({"qkv": qkv_cpu, "dout": dout_cpu}, inputs)
            for c in live:
                for p in PHASES:
                    log(f"compare: rocprofv3 {c.name} {p}")
                    rep["kernels"][f"{c.name}:{p}"] = profile_kernels(args, c.name, p, inputs,
                                                                      work)
    (out / "report.json").write_text(json.dumps(rep, indent=1) + "\n")
    (out / "report.md").write_text(render(rep))
    log(f"compare: wrote {out / 'report.md'}")
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m candle_fused_attn.compare",
                                 description="fused attention vs PyTorch-ROCm fp32 attention")
    sub = ap.add_subparsers(dest="mode", required=True)
    r = sub.add_parser("report", help="measure every contender and write the report")
    r.add_argument("--out", required=True)
    r.add_argument("--batch", type=int, default=64)
    r.add_argument("--seq", type=int, default=240)
    r.add_argument("--seed", type=int, default=0)
    r.add_argument("--rounds", type=int, default=4)
    r.add_argument("--reps", type=int, default=5, help="samples per contender, phase and round")
    r.add_argument("--calls", type=int, default=20, help="back-to-back calls per sample")
    r.add_argument("--warmup", type=int, default=50)
    r.add_argument("--kernels", action="store_true", help="rocprofv3 kernel time per call")
    r.add_argument("--kernel-calls", type=int, default=100, help="calls kept per probe")
    # A fresh process's first ~100 calls run at ramping clocks: the probe's first calls are run
    # and dropped.
    r.add_argument("--kernel-skip", type=int, default=200, help="calls dropped per probe")
    p = sub.add_parser("probe", help="(child of --kernels) run one contender and phase")
    p.add_argument("--inputs", required=True)
    p.add_argument("--contender", required=True)
    p.add_argument("--phase", choices=PHASES, required=True)
    p.add_argument("--calls", type=int, default=20)
    for q in (r, p):
        q.add_argument("--heads", type=int, default=6)
        q.add_argument("--scale", type=float, default=0.125)
        q.add_argument("--causal", action="store_true")
    args = ap.parse_args(argv)
    if args.mode == "probe":
        kernel_probe(args)
        return 0
    return report(args)


if __name__ == "__main__":
    sys.exit(main())
