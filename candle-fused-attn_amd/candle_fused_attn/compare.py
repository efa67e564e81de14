"""The fused attention against PyTorch-ROCm's fp32 attentions on MI355X: accuracy and speed,
measured the same way for every candidate (the method of the reference's harness,
bench/compare.py:1-38, with rocprofv3 in place of nsys and every candidate in Python).

Every candidate computes the same unit of work: the fused projection qkv [b, s, 3 h 64] to the
merged output [b, s, h 64] (head split and merge included), and the backward from dout to dqkv
through the loss head sum(o * dout):
  fattn_qkv            fused_attention_qkv (libfattn.so)
  fattn_general        fused_attention on the q / k / v views of qkv, output merged back
  torch_composed       softmax((q scale) k^T) v written out in torch ops (bench/compare.py:278-289)
  torch_sdpa_math      scaled_dot_product_attention, MATH backend forced
  torch_sdpa_efficient scaled_dot_product_attention, EFFICIENT_ATTENTION backend forced
The FLASH backend is probed too; a backend that refuses these inputs is recorded with its reason
and left out of the timings.

Method (one child process per step; the parent never touches the GPU):
  1. inputs: qkv then dout ~ N(0, 1), fp32, drawn on the CPU by torch.Generator().manual_seed(seed)
     (bench/compare.py:496-503), saved once; every child reads them.
  2. accuracy: each candidate's o, dq, dk, dv against an fp64 recompute on the CPU (torch autograd
     of the composed math): max-abs and normwise relative error; the floor is the fp64 reference
     rounded to fp32. Determinism: a second forward + backward compared bit for bit.
  3. wall time: R rounds, the candidate order rotated each round; per candidate and phase, W warm-up
     calls, then S samples of N back-to-back calls between two device syncs (ms per call); phases
     fwd (no autograd), train (forward + head + backward), head (the head alone); net = train - head.
  4. decision rule: X is faster than Y on a phase iff X's worst round median is below Y's best
     round median (bench/compare.py:84-110); otherwise "not separated".
  5. kernel time (--kernels): one child per candidate and phase under
     `rocprofv3 --kernel-trace --stats`; per-call time = a kernel's total / its launches per call;
     kernels whose launch count is not a multiple of the calls are listed as irregular.

Run on one MI355X, from the repository root:
  PYTHONPATH=candle-fused-attn_amd python3 -m candle_fused_attn.compare run --out DIR [--kernels]
Writes DIR/report.md and DIR/report.json (the inputs and the candidates' outputs, about 100 MB
each at the default shape, go to DIR/data and are deleted at the end unless --keep-data).
"""
from __future__ import annotations

import argparse
import contextlib
import csv
import json
import os
import shutil
import statistics
import subprocess
import sys
import time
from pathlib import Path

HEAD_DIM = 64
OURS = ("fattn_qkv", "fattn_general")
TORCH = ("torch_composed", "torch_sdpa_math", "torch_sdpa_efficient")
PHASES = ("fwd", "train", "net")
PARTS = ("o", "dq", "dk", "dv")


# --- pure helpers ------------------------------------------------------------------------------

def summarize(xs: list[float]) -> dict[str, float]:
    """Median, quartiles (inclusive method), min and max.

    >>> summarize([3.0, 1.0, 2.0, 4.0])
    {'median': 2.5, 'q1': 1.75, 'q3': 3.25, 'min': 1.0, 'max': 4.0}
    >>> summarize([2.0])['q1']
    2.0
    """
    if len(xs) == 1:
        return {"median": xs[0], "q1": xs[0], "q3": xs[0], "min": xs[0], "max": xs[0]}
    q1, _, q3 = statistics.quantiles(xs, n=4, method="inclusive")
    return {"median": statistics.median(xs), "q1": q1, "q3": q3, "min": min(xs), "max": max(xs)}


def faster(xs: list[float], ys: list[float]) -> bool:
    """The decision rule: the worst of `xs` beats the best of `ys`.

    >>> faster([1.0, 1.2], [1.3, 1.5])
    True
    >>> faster([1.0, 1.4], [1.3, 1.5])
    False
    """
    return max(xs) < min(ys)


def verdict(name_x: str, xs: list[float], name_y: str, ys: list[float]) -> str:
    """The decision rule in words, with the ratio of medians.

    >>> verdict("a", [1.0], "b", [2.0])
    'a faster (x2.00)'
    >>> verdict("a", [2.0], "b", [1.0])
    'b faster (x2.00)'
    >>> verdict("a", [1.0, 2.0], "b", [1.5])
    'not separated'
    """
    mx, my = statistics.median(xs), statistics.median(ys)
    if faster(xs, ys):
        return f"{name_x} faster (x{my / mx:.2f})"
    if faster(ys, xs):
        return f"{name_y} faster (x{mx / my:.2f})"
    return "not separated"


def rotate(xs, k: int) -> list:
    """`xs` rotated left by `k` (round k's candidate order).

    >>> rotate(("a", "b", "c"), 1)
    ['b', 'c', 'a']
    >>> rotate(("a", "b"), 3)
    ['b', 'a']
    """
    return [xs[(i + k) % len(xs)] for i in range(len(xs))]


def fmt_range(xs: list[float]) -> str:
    """Median [min-max] in ms, or a dash.

    >>> fmt_range([0.25, 0.2, 0.3])
    '0.250 [0.200–0.300]'
    >>> fmt_range([])
    '—'
    """
    if not xs:
        return "—"
    return f"{statistics.median(xs):.3f} [{min(xs):.3f}–{max(xs):.3f}]"


def kernel_rows(stats_csv: str) -> list[tuple[str, int, int]]:
    """(name, total ns, launches) from rocprofv3's `*_kernel_stats.csv`.

    >>> kernel_rows('"Name","Calls","TotalDurationNs"\\n"k1",20,4000\\n"k2",3,60\\n')
    [('k1', 4000, 20), ('k2', 60, 3)]
    """
    rows = []
    for r in csv.DictReader(stats_csv.splitlines()):
        rows.append((r["Name"], int(float(r["TotalDurationNs"])), int(r["Calls"])))
    return rows


def per_call(rows: list[tuple[str, int, int]], calls: int) -> dict:
    """Kernel time per call: kernels launched a multiple of `calls` times count in the total (with
    their launches per call); the others are listed as irregular.

    >>> p = per_call([("k1", 4000, 20), ("k2", 60, 3)], 10)
    >>> p["ms"], p["irregular"], p["kernels"][0]["per_call"]
    (0.0004, ['k2'], 2.0)
    """
    regular, irregular, total = [], [], 0
    for name, ns, n in rows:
        if n % calls == 0:
            regular.append({"name": name, "per_call": n / calls, "us_per_call": ns / calls / 1e3})
            total += ns
        else:
            irregular.append(name)
    return {"ms": total / calls / 1e6, "kernels": regular, "irregular": irregular}


def short_name(kernel: str) -> str:
    """A kernel's name without its argument list and return type.

    >>> short_name("void fattn::(anonymous namespace)::bwd_kernel<true>(fattn::BwdArgs)")
    'fattn::(anonymous namespace)::bwd_kernel<true>'
    """
    name = kernel[5:] if kernel.startswith("void ") else kernel
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0 and not name[i:].startswith("(anonymous"):
            return name[:i]
    return name


# --- the candidates (child processes only) -----------------------------------------------------

def split_heads(qkv, heads: int):
    """q, k, v [b, h, s, d] as views of the [b, s, 3 h d] projection."""
    b, s, three_hd = qkv.shape
    hidden = three_hd // 3
    shape = (b, s, heads, hidden // heads)
    q, k, v = qkv.split(hidden, dim=-1)
    return tuple(t.view(shape).transpose(1, 2) for t in (q, k, v))


def composed(qkv, heads: int, scale: float, causal: bool):
    """softmax((q scale) k^T [+ causal mask]) v, merged back to [b, s, h d]; any float dtype."""
    import torch
    b, s, three_hd = qkv.shape
    q, k, v = split_heads(qkv, heads)
    scores = (q * scale) @ k.transpose(-2, -1)
    if causal:
        mask = torch.ones(s, s, dtype=torch.bool, device=qkv.device).triu(1)
        scores = scores.masked_fill(mask, float("-inf"))
    return (torch.softmax(scores, dim=-1) @ v).transpose(1, 2).reshape(b, s, three_hd // 3)


def sdpa(qkv, heads: int, scale: float, causal: bool):
    import torch
    b, s, three_hd = qkv.shape
    q, k, v = split_heads(qkv, heads)
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=scale)
    return o.transpose(1, 2).reshape(b, s, three_hd // 3)


def fattn_general(qkv, heads: int, scale: float, causal: bool):
    import candle_fused_attn as cfa
    b, s, three_hd = qkv.shape
    q, k, v = split_heads(qkv, heads)
    return cfa.fused_attention(q, k, v, scale, causal).transpose(1, 2).reshape(b, s, three_hd // 3)


def fattn_qkv(qkv, heads: int, scale: float, causal: bool):
    import candle_fused_attn as cfa
    return cfa.fused_attention_qkv(qkv, heads, scale, causal)


def backend_context(name: str):
    """The forced SDPA backend of candidate `name` (none for the others)."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    forced = {"torch_sdpa_math": SDPBackend.MATH,
              "torch_sdpa_efficient": SDPBackend.EFFICIENT_ATTENTION,
              "torch_sdpa_flash": SDPBackend.FLASH_ATTENTION}
    return sdpa_kernel([forced[name]]) if name in forced else contextlib.nullcontext()


ATTEND = {"fattn_qkv": fattn_qkv, "fattn_general": fattn_general, "torch_composed": composed,
          "torch_sdpa_math": sdpa, "torch_sdpa_efficient": sdpa, "torch_sdpa_flash": sdpa}


class Bench:
    """One candidate set on the saved inputs, in a child process."""

    def __init__(self, inputs: Path, heads: int, causal: bool) -> None:
        import torch
        from safetensors.torch import load_file
        t = load_file(str(inputs))
        self.qkv = t["qkv"].to("cuda").requires_grad_(True)
        self.dout = t["dout"].to("cuda")
        self.heads, self.causal = heads, causal
        self.scale = 1.0 / HEAD_DIM ** 0.5
        self.standin = torch.zeros_like(self.dout, requires_grad=True)

    def attend(self, name: str, qkv):
        return ATTEND[name](qkv, self.heads, self.scale, self.causal)

    def train(self, name: str):
        self.qkv.grad = None
        o = self.attend(name, self.qkv)
        (o * self.dout).sum().backward()
        return o, self.qkv.grad

    def call(self, name: str, phase: str) -> None:
        import torch
        if phase == "fwd":
            with torch.no_grad():
                self.attend(name, self.qkv)
        elif phase == "train":
            self.train(name)
        else:  # the head alone
            self.standin.grad = None
            (self.standin * self.dout).sum().backward()


def probe(bench: Bench, names) -> dict[str, str]:
    """Each candidate's forward + backward once: "ok", or the error that refused it."""
    import torch
    out = {}
    for name in names:
        try:
            with backend_context(name):
                bench.train(name)
            torch.cuda.synchronize()
            out[name] = "ok"
        except RuntimeError as e:
            out[name] = "refused: " + " ".join(str(e).split())[:300]
    return out


def side_accuracy(a) -> None:
    import torch
    from safetensors.torch import save_file
    torch.set_float32_matmul_precision("highest")
    bench = Bench(a.inputs, a.heads, a.causal)
    status = probe(bench, OURS + TORCH + ("torch_sdpa_flash",))
    rows = []
    for name in OURS + TORCH:
        if status[name] != "ok":
            continue
        with backend_context(name):
            o1, g1 = bench.train(name)
            o1, g1 = o1.detach().clone(), g1.clone()
            o2, g2 = bench.train(name)
        det = bool(torch.equal(o1, o2) and torch.equal(g1, g2))
        save_file({"o": o1.contiguous().cpu(), "dqkv": g1.contiguous().cpu()},
                  str(a.inputs.parent / f"{name}.safetensors"))
        rows.append({"name": name, "deterministic": det})
    env = {"torch": torch.__version__, "hip": torch.version.hip,
           "gpu": torch.cuda.get_device_name(0),
           "arch": getattr(torch.cuda.get_device_properties(0), "gcnArchName", "?"),
           "cus": torch.cuda.get_device_properties(0).multi_processor_count,
           "fp32_matmul_precision": torch.get_float32_matmul_precision()}
    import candle_fused_attn as cfa
    env["libfattn"] = cfa.version()
    (a.out / "accuracy.json").write_text(json.dumps(
        {"candidates": rows, "status": status, "env": env}, indent=1), encoding="utf-8")


def side_time(a) -> None:
    import torch
    torch.set_float32_matmul_precision("highest")
    bench = Bench(a.inputs, a.heads, a.causal)
    names = json.loads(a.names)
    rows = []

    def timed(name: str, phase: str) -> None:
        for _ in range(a.warmup):
            bench.call(name, phase)
        ms = []
        for _ in range(a.samples):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(a.calls):
                bench.call(name, phase)
            torch.cuda.synchronize()
            ms.append((time.perf_counter() - t0) * 1e3 / a.calls)
        rows.append({"name": name, "phase": phase, "ms": ms})

    for name in rotate(names, a.round):
        with backend_context(name):
            timed(name, "fwd")
            timed(name, "train")
    timed("head", "head")
    (a.out / f"time_r{a.round}.json").write_text(json.dumps(rows), encoding="utf-8")


def side_kernels(a) -> None:
    import torch
    torch.set_float32_matmul_precision("highest")
    bench = Bench(a.inputs, a.heads, a.causal)
    with backend_context(a.only):
        for _ in range(a.calls):
            bench.call(a.only, a.phase)
        torch.cuda.synchronize()


# --- the orchestration (parent; no GPU use) ----------------------------------------------------

def log(msg: str) -> None:
    print(f"[{time.strftime('%H:%M:%S')}] {msg}", flush=True)


def make_inputs(path: Path, b: int, h: int, s: int, seed: int) -> None:
    import torch
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(seed)
    hd = h * HEAD_DIM
    save_file({"qkv": torch.randn(b, s, 3 * hd, generator=g),
               "dout": torch.randn(b, s, hd, generator=g)}, str(path))


def score(out: Path, names: list[str], heads: int, causal: bool) -> dict[str, dict]:
    """Every candidate's o, dq, dk, dv against an fp64 CPU recompute; plus the fp32 floor."""
    import torch
    from safetensors.torch import load_file
    t = load_file(str(out / "data" / "inputs.safetensors"))
    qkv = t["qkv"].double().requires_grad_(True)
    o = composed(qkv, heads, 1.0 / HEAD_DIM ** 0.5, causal)
    (o * t["dout"].double()).sum().backward()

    def parts(o_, g_):
        dq, dk, dv = g_.chunk(3, dim=-1)
        return {"o": o_, "dq": dq, "dk": dk, "dv": dv}

    ref = parts(o.detach(), qkv.grad)

    def errors(got):
        res = {}
        for p in PARTS:
            diff = got[p].double() - ref[p]
            res[p] = {"max_abs": diff.abs().max().item(),
                      "rel_fro": (diff.norm() / ref[p].norm()).item()}
        return res

    scores = {"fp64_rounded_to_fp32": errors({p: ref[p].float() for p in PARTS})}
    for name in names:
        c = load_file(str(out / "data" / f"{name}.safetensors"))
        scores[name] = errors(parts(c["o"], c["dqkv"]))
    return scores


def collect_wall(out: Path, rounds: int) -> dict:
    """wall[name][phase] = round medians (ms per call); net = train - head within a round."""
    wall: dict = {}
    for r in range(rounds):
        rows = json.loads((out / f"time_r{r}.json").read_text(encoding="utf-8"))
        med = {(x["name"], x["phase"]): statistics.median(x["ms"]) for x in rows}
        head = med[("head", "head")]
        for (name, phase), m in med.items():
            w = wall.setdefault(name, {})
            w.setdefault(phase, []).append(m)
            if phase == "train":
                w.setdefault("net", []).append(m - head)
    return wall


def run(a) -> None:
    out = a.out.resolve()
    out.mkdir(parents=True, exist_ok=True)
    log(f"output: {out}")
    (out / "data").mkdir(exist_ok=True)
    inputs = out / "data" / "inputs.safetensors"
    make_inputs(inputs, a.batch, a.heads, a.seq, a.seed)
    me = [sys.executable, "-m", "candle_fused_attn.compare", "side"]
    common = ["--inputs", str(inputs), "--out", str(out), "--heads", str(a.heads)]
    common += ["--causal"] if a.causal else []
    env = dict(os.environ)
    pkg = str(Path(__file__).resolve().parent.parent)
    env["PYTHONPATH"] = pkg + os.pathsep + env.get("PYTHONPATH", "")

    log("accuracy + determinism (GPU)")
    subprocess.run(me + ["accuracy"] + common, check=True, env=env, timeout=600)
    acc = json.loads((out / "accuracy.json").read_text(encoding="utf-8"))
    names = [r["name"] for r in acc["candidates"]]
    scores = score(out, names, a.heads, a.causal)

    for r in range(a.rounds):
        log(f"round {r + 1}/{a.rounds} (GPU)")
        subprocess.run(me + ["time"] + common + [
            "--round", str(r), "--samples", str(a.samples), "--calls", str(a.calls),
            "--warmup", str(a.warmup), "--names", json.dumps(names)], check=True, env=env,
            timeout=900)
    wall = collect_wall(out, a.rounds)

    kernels: dict = {}
    prof = shutil.which("rocprofv3") if a.kernels else None
    if a.kernels and not prof:
        log("kernel pass SKIPPED: no rocprofv3 on PATH")
    if prof:
        jobs = [(n, p) for n in names for p in ("fwd", "train")] + [("head", "head")]
        for i, (name, phase) in enumerate(jobs):
            log(f"rocprofv3 {i + 1}/{len(jobs)}: {name} {phase} (GPU)")
            d = out / f"prof_{name}_{phase}"
            cmd = [prof, "--kernel-trace", "--stats", "--output-format", "csv", "-d", str(d),
                   "-o", "run", "--", sys.executable, "-m", "candle_fused_attn.compare", "side",
                   "kernels"] + common + ["--only", name, "--phase", phase,
                                          "--calls", str(a.kernel_calls)]
            subprocess.run(cmd, check=True, env=env, capture_output=True, timeout=600)
            stats = next(d.rglob("run_kernel_stats.csv")).read_text(encoding="utf-8")
            kernels[f"{name}:{phase}"] = per_call(kernel_rows(stats), a.kernel_calls)

    report = {"env": {"date": time.strftime("%Y-%m-%d %H:%M:%S"),
                      "shape": [a.batch, a.heads, a.seq, HEAD_DIM], "causal": a.causal,
                      "seed": a.seed, "timing": {"rounds": a.rounds, "samples": a.samples,
                                                  "calls": a.calls, "warmup": a.warmup,
                                                  "kernel_calls": a.kernel_calls}},
              "device": acc["env"], "status": acc["status"],
              "deterministic": {r["name"]: r["deterministic"] for r in acc["candidates"]},
              "accuracy": scores, "wall": wall, "kernels": kernels}
    (out / "report.json").write_text(json.dumps(report, indent=1), encoding="utf-8")
    md = render(report, names)
    (out / "report.md").write_text(md, encoding="utf-8")
    if not a.keep_data:
        shutil.rmtree(out / "data", ignore_errors=True)
    print(md)


def render(rep: dict, names: list[str]) -> str:
    """The Markdown report."""
    e, d = rep["env"], rep["device"]
    lines = [f"# fused attention vs PyTorch-ROCm fp32 attention — {e['date']}", "",
             f"{d['gpu']} ({d['arch']}, {d['cus']} CUs); torch {d['torch']} (HIP {d['hip']}), "
             f"fp32 matmul precision `{d['fp32_matmul_precision']}`; {d.get('libfattn', '')}. "
             f"Shape b·h·s·d = {' · '.join(map(str, e['shape']))}, causal {e['causal']}, "
             f"seed {e['seed']}. Timing: {e['timing']}.", "",
             "## Candidates on these inputs (forward + backward once)", ""]
    lines += [f"- `{k}`: {v}" for k, v in rep["status"].items()]
    lines += ["", "## Accuracy against fp64 (normwise relative error; max-abs in brackets)", "",
              "| candidate | o | dq | dk | dv | 2 runs bitwise equal |",
              "|---|---|---|---|---|---|"]
    for name, s in rep["accuracy"].items():
        cells = [f"{s[p]['rel_fro']:.2e} [{s[p]['max_abs']:.1e}]" for p in PARTS]
        lines.append(f"| {name} | " + " | ".join(cells) +
                     f" | {rep['deterministic'].get(name, '—')} |")
    lines += ["", "## Wall time, ms per call: median of round medians [min–max over rounds]", "",
              "| candidate | fwd | train | net = train − head |", "|---|---|---|---|"]
    for name in names:
        w = rep["wall"][name]
        lines.append(f"| {name} | " + " | ".join(fmt_range(w.get(p, [])) for p in PHASES) + " |")
    lines.append(f"| (head) | | {fmt_range(rep['wall']['head']['head'])} | |")
    ours = names[0]
    lines += ["", f"Decision rule against `{ours}` (worst round of one < best round of the "
              "other):", ""]
    for name in names[1:]:
        cells = [f"{p}: {verdict(ours, rep['wall'][ours][p], name, rep['wall'][name][p])}"
                 for p in PHASES]
        lines.append(f"- vs `{name}` — " + "; ".join(cells))
    k = rep["kernels"]
    if k:
        lines += ["", "## Kernel time (rocprofv3), ms per call", "",
                  "| candidate | fwd | train | net = train − head | irregular kernels |",
                  "|---|---|---|---|---|"]
        for name in names:
            f, t = k[f"{name}:fwd"], k[f"{name}:train"]
            net = t["ms"] - k["head:head"]["ms"]
            irr = sorted(set(f["irregular"]) | set(t["irregular"]))
            lines.append(f"| {name} | {f['ms']:.3f} | {t['ms']:.3f} | {net:.3f} | "
                         f"{', '.join(short_name(x)[:60] for x in irr) or '—'} |")
        lines += ["", "Kernels per train call (launches per call × µs per call):", ""]
        for name in names:
            ks = sorted(k[f"{name}:train"]["kernels"], key=lambda x: -x["us_per_call"])
            lines.append(f"- `{name}`: " + "; ".join(
                f"{short_name(x['name'])[:70]} ×{x['per_call']:g} {x['us_per_call']:.1f}"
                for x in ks))
    return "\n".join(lines) + "\n"


def main(argv=None) -> None:
    p = argparse.ArgumentParser(description=__doc__,
                                formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("command", choices=["run", "side"])
    p.add_argument("mode", nargs="?", choices=["accuracy", "time", "kernels"], help="side only")
    p.add_argument("--batch", type=int, default=64)
    p.add_argument("--heads", type=int, default=6)
    p.add_argument("--seq", type=int, default=240)
    p.add_argument("--causal", action="store_true")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--rounds", type=int, default=3)
    p.add_argument("--samples", type=int, default=15)
    p.add_argument("--calls", type=int, default=10, help="back-to-back calls per sample")
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--kernels", action="store_true", help="also the rocprofv3 kernel pass")
    p.add_argument("--kernel-calls", type=int, default=20)
    p.add_argument("--out", type=Path, default=Path("gpurun_out/compare"))
    p.add_argument("--keep-data", action="store_true", help="keep the inputs and outputs")
    # The child's arguments.
    p.add_argument("--inputs", type=Path)
    p.add_argument("--round", type=int, default=0)
    p.add_argument("--names", type=str, default="[]")
    p.add_argument("--only", type=str)
    p.add_argument("--phase", type=str)
    a = p.parse_args(argv)
    if a.command == "run":
        run(a)
    else:
        {"accuracy": side_accuracy, "time": side_time, "kernels": side_kernels}[a.mode](a)


if __name__ == "__main__":
    main()
