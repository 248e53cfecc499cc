"""The copy-on-write and continuous-batching configurations on the GPU, at
reduced sizes, through their C++ drivers (qwenvl-paged_amd/host/bench): the
device allocator's decisions and bytes equal the host allocator's, copied
frames equal their sources, sampled decodes match float64 attention, and a
scheduler trace with preemption and swap drains completely."""

from __future__ import annotations

import json
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BENCH = ROOT / "build" / "bench"


def run(name: str, *args: str) -> dict:
    exe = BENCH / name
    assert exe.exists(), f"{exe} is missing: run __graft_entry__.build() first"
    print(f"running {name} {' '.join(args)}", flush=True)
    proc = subprocess.run([str(exe), *args], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=100)
    print(proc.stdout, proc.stderr)
    assert proc.returncode == 0, proc.stderr + proc.stdout
    return json.loads(proc.stdout.strip().splitlines()[-1])


@pytest.mark.gpu
def test_copy_on_write_configuration_small():
    r = run("cow_bench", "--prompts", "4", "--branches", "8", "--reps", "3")
    assert r["cow_pairs"] == 32
    assert r["pending_before_flush"] == 32
    assert r["copy_launches"] == 1
    assert r["frames_equal_host_allocator"] and r["copies_equal_source"]
    assert r["decode_within_tolerance"] and r["checked_elements"] > 0


@pytest.mark.gpu
def test_continuous_batching_trace_small():
    r = run("trace_bench", "--requests", "24", "--seed", "7")
    assert r["finished"] == 24 and r["drained"]
    assert r["decode_tokens"] == r["expected_decode_tokens"]
    assert r["preemptions"] > 0 and r["resumes"] > 0
    assert r["swapped_out_blocks"] > 0 and r["swapped_in_blocks"] > 0
