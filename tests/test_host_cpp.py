"""The C++ op layer (candle-fused-attn_amd/host/, libcandle_fused_attn.so) through its test program
tests/cpp/parity_host, which mirrors the reference's integration tests (tests/parity.rs) in C++.

`--cpu` covers the layer's views, alignment predicates, the errors it raises before any launch and
empty inputs (nothing allocated or launched); `--gpu` the parity cases on the device: both entry
points against the fp32 oracle at the reference's band (5e-6 max-abs, tests/parity.rs:209-220),
the merged-heads layout, backward twice over one node, eight bit-identical reruns, copy fallbacks
equal to aligned operands bit for bit, the strided gather against the host, and the C ABI's
errors. The program is built by
__graft_entry__.build(); a missing build is a failure, not a skip.
"""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "cpp" / "parity_host"


def _run(mode: str, timeout: float) -> None:
    if not BIN.exists():
        pytest.fail(f"{BIN} is not built: run __graft_entry__.build()")
    print(f"running {BIN.name} {mode}", flush=True)
    res = subprocess.run([str(BIN), mode], capture_output=True, text=True, timeout=timeout)
    print(res.stdout, res.stderr, sep="\n", flush=True)
    assert res.returncode == 0, f"{BIN.name} {mode} exited {res.returncode}:\n{res.stdout[-3000:]}"
    assert " passed" in res.stdout and "FAIL" not in res.stdout


def test_host_layer_without_a_device():
    _run("--cpu", 60)


@pytest.mark.gpu
def test_host_layer_on_the_device():
    _run("--gpu", 100)
