"""bench.py's kernel-trace summary (`--trace-from`) on a synthetic rocprofv3 kernel trace: it must
pick the headline's windows out of a run that also launches configs 3-5 and the other head dims
with kernels of the same names (CPU only; no GPU, no rocprofv3)."""
import csv
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402

PREFIX = "void fattn::(anonymous namespace)::"
FWD, MAIN, DQ = (bench.KERNEL_NAMES[k] for k in ("fwd", "bwd_main", "bwd_dq"))
CAUSAL_FWD = "fwd_kernel<64, 64, 32, 3>"
D32_FWD = "fwd_kernel<32, 128, 64, 3>"


def write_trace(path, w, k):
    """The dispatch sequence of `bench.py --warmup w --steps k` with distinct durations per
    window: idle steps (fwd 60, main 160), config 3 (other forward), the headline's timed steps
    (fwd 54, main 136), forwards (53), kernel-level steps (fwd 52, main 135, dq 4), backwards
    (main 137), then config 2 at d 32."""
    b, h, s = bench.CONFIGS[2][2], bench.CONFIGS[2][3], bench.CONFIGS[2][4]
    grid = ((s + 127) // 128) * b * h
    seq = []
    seq += [(FWD, grid, 60.0), (MAIN, 1536, 160.0)] * (w + k)          # from idle
    seq += [(CAUSAL_FWD, 1536, 40.0), (MAIN, 1536, 95.0)] * 30          # config 3
    seq += [(FWD, grid, 70.0), (MAIN, 1536, 170.0)] * w                 # warm-up
    seq += [(FWD, grid, 54.0), (MAIN, 1536, 136.0)] * k                 # timed
    seq += [(FWD, grid, 53.0)] * k                                      # forwards
    seq += [(FWD, grid, 52.0), (MAIN, 1536, 135.0), (DQ, 256, 4.0)] * k  # kernel-level
    seq += [(MAIN, 1536, 137.0)] * k                                    # backwards
    seq += [(D32_FWD, grid, 30.0), (MAIN, 1536, 80.0)] * 30             # d 32
    t = 1_000_000
    with open(path, "w", newline="") as f:
        wr = csv.DictWriter(f, fieldnames=["Kernel_Name", "Grid_Size_X", "Workgroup_Size_X",
                                           "Start_Timestamp", "End_Timestamp"])
        wr.writeheader()
        for name, wgs, us in seq:
            wr.writerow({"Kernel_Name": f"{PREFIX}{name}(fattn::Args)",
                         "Grid_Size_X": wgs * 256, "Workgroup_Size_X": 256,
                         "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000)})
            t += int(us * 1000) + 2000


def tables(text):
    """{title: {kernel: (calls, average)}} from the summary's markdown."""
    out, cur = {}, None
    for line in text.splitlines():
        if line.startswith("The "):
            cur = out.setdefault(line, {})
        elif line.startswith("| `") and cur is not None:
            cells = [c.strip() for c in line.strip("|").split("|")]
            cur[cells[0].strip("`")] = (int(cells[1]), float(cells[2]))
    return out


def test_trace_windows(tmp_path):
    w, k = 5, 20
    trace = tmp_path / "kernel_trace.csv"
    write_trace(trace, w, k)
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--trace-from", str(trace),
                        "--warmup", str(w), "--steps", str(k)],
                       capture_output=True, text=True, check=True)
    t = tables(r.stdout)
    by = {title.split(" (")[0]: rows for title, rows in t.items()}
    assert by[f"The {k} timed forward+backward steps"] == {MAIN: (k, 136.0), FWD: (k, 54.0)}
    assert by[f"The {k} op-level forwards"] == {FWD: (k, 53.0)}
    assert by[f"The {k} op-level backwards"] == {MAIN: (k, 137.0)}
    assert by[f"The {k} kernel-level steps"] == {MAIN: (k, 135.0), FWD: (k, 52.0), DQ: (k, 4.0)}
    assert by[f"The first {k} steps from idle"] == {MAIN: (k, 160.0), FWD: (k, 60.0)}
