"""bench.py's profile summaries on synthetic rocprofv3 files (CPU only; no GPU, no rocprofv3):
the kernel-trace summary (`--trace-from`) must pick the headline's windows out of a run that also
launches configs 3-5 and the other head dims with kernels of the same names, and the traffic
summary (`--traffic-from`) must scale the counters by the copy's and go stale with the library."""
import csv
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
import pytest  # noqa: E402

PREFIX = "void fattn::(anonymous namespace)::"
FWD, MAIN, DQ = (bench.KERNEL_NAMES[k] for k in ("fwd", "bwd_main", "bwd_dq"))
CAUSAL_FWD = bench.CAUSAL_FWD_NAME
D32_FWD = "fwd_kernel<32, 128, 64, 3, false>"


def write_trace(path, w, k, cfg=2):
    """The dispatch sequence of `bench.py --warmup w --steps k` (config `cfg` as the headline)
    with distinct durations per window: idle steps (fwd 60, main 160), another config (another
    forward), the headline's timed steps (fwd 54, main 136), forwards (53), kernel-level steps
    (fwd 52, main 135, dq 4), backwards (main 137), then config 2 at d 32."""
    b, h, s = bench.CONFIGS[2][2], bench.CONFIGS[2][3], bench.CONFIGS[2][4]
    grid = ((s + 127) // 128) * b * h
    head, other = (FWD, grid), (CAUSAL_FWD, ((s + 63) // 64) * b * h)
    if cfg == 3:  # config 3 as the headline (bench.py --causal); config 2 is then the other
        head, other = other, head
    FWD_, grid = head
    seq = []
    seq += [(FWD_, grid, 60.0), (MAIN, 1536, 160.0)] * (w + k)          # from idle
    seq += [(other[0], other[1], 40.0), (MAIN, 1536, 95.0)] * 30        # another config
    seq += [(FWD_, grid, 70.0), (MAIN, 1536, 170.0)] * w                 # warm-up
    seq += [(FWD_, grid, 54.0), (MAIN, 1536, 136.0)] * k                 # timed
    seq += [(FWD_, grid, 53.0)] * k                                      # forwards
    seq += [(FWD_, grid, 52.0), (MAIN, 1536, 135.0), (DQ, 256, 4.0)] * k  # kernel-level
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


@pytest.mark.parametrize("cfg", [2, 3])
def test_trace_windows(tmp_path, cfg):
    w, k = 5, 20
    trace = tmp_path / "kernel_trace.csv"
    write_trace(trace, w, k, cfg)
    fwd = CAUSAL_FWD if cfg == 3 else FWD
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--trace-from", str(trace),
                        "--warmup", str(w), "--steps", str(k)]
                       + (["--causal"] if cfg == 3 else []),
                       capture_output=True, text=True, check=True)
    t = tables(r.stdout)
    by = {title.split(" (")[0]: rows for title, rows in t.items()}
    assert by[f"The {k} timed forward+backward steps"] == {MAIN: (k, 136.0), fwd: (k, 54.0)}
    assert by[f"The {k} op-level forwards"] == {fwd: (k, 53.0)}
    assert by[f"The {k} op-level backwards"] == {MAIN: (k, 137.0)}
    assert by[f"The {k} kernel-level steps"] == {MAIN: (k, 135.0), fwd: (k, 52.0), DQ: (k, 4.0)}
    assert by[f"The first {k} steps from idle"] == {MAIN: (k, 160.0), fwd: (k, 60.0)}


def write_counters(path, counter, rows):
    with open(path, "w", newline="") as f:
        wr = csv.DictWriter(f, fieldnames=["Kernel_Name", "Counter_Name", "Counter_Value"])
        wr.writeheader()
        for name, value in rows:
            wr.writerow({"Kernel_Name": name, "Counter_Name": counter, "Counter_Value": value})


def test_traffic_summary_and_staleness(tmp_path, monkeypatch):
    """`--traffic-from`: each kernel's mean counter, scaled by what the counter reads for the
    256 MiB copy (FETCH_SIZE half the copied bytes: factor 2; WRITE_SIZE whole: factor 1); the
    bench line reports the step-2 bytes only while the measured library is the loaded one."""
    copy = "__amd_rocclr_copyBuffer"
    main = f"{PREFIX}{MAIN}(fattn::BwdArgs)"
    fwd = f"{PREFIX}{FWD}(fattn::FwdArgs)"
    fetch, write = tmp_path / "fetch.csv", tmp_path / "write.csv"
    write_counters(fetch, "FETCH_SIZE", [(copy, 131072.0), (fwd, 46000.0), (fwd, 46400.0),
                                         (main, 100000.0), (main, 100002.0)])
    write_counters(write, "WRITE_SIZE", [(copy, 262144.0), (fwd, 23000.0), (fwd, 23000.0),
                                         (main, 200000.0), (main, 200000.0)])
    monkeypatch.setattr(bench, "TRAFFIC", tmp_path / "traffic.json")
    monkeypatch.setattr(bench, "lib_sha256", lambda: "aaaa")
    assert bench.summarize_traffic(str(fetch), str(write)) == 0
    t = bench.json.loads((tmp_path / "traffic.json").read_text())
    assert (t["scale_fetch"], t["scale_write"]) == (2.0, 1.0)
    assert t["fwd"]["fetch_bytes"] == 46200 * 1024 * 2 and t["fwd"]["write_bytes"] == 23000 * 1024
    assert t["bwd_main_bytes"] == 100001 * 1024 * 2 + 200000 * 1024
    assert t["lib_sha256"] == "aaaa"
    assert bench.traffic_entry()["traffic"] == t["bwd_main_bytes"]
    monkeypatch.setattr(bench, "lib_sha256", lambda: "bbbb")  # another library: stale
    e = bench.traffic_entry()
    assert e["traffic"] is None and e["traffic_stale_bytes"] == t["bwd_main_bytes"]


def write_counter_run(path, w, k, counters):
    """A counter file of `bench.py --no-extra --warmup w --steps k` (config 2): the dispatch
    sequence of one run (idle W + K steps, W warm-up, K timed, K forwards, K kernel-level steps, K
    backwards), each dispatch with `counters(window, kernel)` -> {counter: value}, one row per
    counter, as rocprofv3 --pmc writes them."""
    b, h, s = bench.CONFIGS[2][2], bench.CONFIGS[2][3], bench.CONFIGS[2][4]
    grid = ((s + 127) // 128) * b * h
    seq = []
    for win, n, kinds in (("idle", w + k, (FWD, MAIN)), ("warm", w, (FWD, MAIN)),
                          ("timed", k, (FWD, MAIN)), ("fwds", k, (FWD,)),
                          ("kern", k, (FWD, MAIN, DQ)), ("bwds", k, (MAIN,))):
        for _ in range(n):
            seq += [(win, kind) for kind in kinds]
    fields = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Workgroup_Size", "Counter_Name",
              "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    t = 1_000_000
    with open(path, "w", newline="") as f:
        wr = csv.DictWriter(f, fieldnames=fields)
        wr.writeheader()
        for i, (win, kind) in enumerate(seq):
            wgs = grid if kind == FWD else (1536 if kind == MAIN else 256)
            for name, value in counters(win, kind).items():
                wr.writerow({"Dispatch_Id": i + 1, "Kernel_Name": f"{PREFIX}{kind}(fattn::Args)",
                             "Grid_Size": wgs * 256, "Workgroup_Size": 256, "Counter_Name": name,
                             "Counter_Value": value, "Start_Timestamp": t,
                             "End_Timestamp": t + 100_000})
            t += 102_000


def test_counter_summary_uses_the_timed_window(tmp_path):
    """`--counters-from`: only the K timed steps' dispatches count (other windows carry other
    values), passes are merged per kernel, and GRBM_GUI_ACTIVE (summed over the 8 XCDs) is divided
    by 8: step 2 with 1000 MFMAs (32 cycles each) over 400 GPU-busy cycles x 8 XCDs reads MFMA busy
    = 32000 / (400 x 1024 SIMDs) = 7.8125 %, 3 other VALU per MFMA, waves per SIMD = 4 x 51200 /
    (400 x 1024) = 0.5."""
    w, k = 5, 20

    def pass_a(win, kind):
        timed = win == "timed"
        return {"GRBM_GUI_ACTIVE": 3200.0 if timed else 99.0,
                "SQ_VALU_MFMA_BUSY_CYCLES": 32000.0 if timed else 7.0,
                "SQ_WAVE_CYCLES": 51200.0 if timed else 5.0}

    def pass_b(win, kind):
        timed = win == "timed"
        return {"GRBM_GUI_ACTIVE": 3200.0 if timed else 99.0,
                "SQ_INSTS_MFMA": 1000.0 if timed else 3.0,
                "SQ_INSTS_VALU": 4000.0 if timed else 3.0}

    a, b = tmp_path / "a.csv", tmp_path / "b.csv"
    write_counter_run(a, w, k, pass_a)
    write_counter_run(b, w, k, pass_b)
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--counters-from", str(a), str(b),
                        "--warmup", str(w), "--steps", str(k)],
                       capture_output=True, text=True, check=True)
    rows = {}
    for line in r.stdout.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if line.startswith("| ") and len(cells) == 3:
            rows[cells[0]] = cells[1:]
    assert rows["dispatches per run"] == [str(k), str(k)]
    main, fwd = rows["MFMA busy (% of SIMD cycles)"]
    assert float(main) == pytest.approx(7.8125, rel=1e-3) and float(fwd) == pytest.approx(7.8125,
                                                                                        rel=1e-3)
    assert float(rows["other VALU per MFMA"][0]) == pytest.approx(3.0)
    assert float(rows["waves per SIMD (average)"][0]) == pytest.approx(0.5)
    assert float(rows["MFMA instruction cycles / MFMA busy cycles"][0]) == pytest.approx(1.0)
