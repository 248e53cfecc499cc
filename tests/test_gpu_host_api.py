"""The C++ host API on device-placed frames (HBM block pool, pinned swap arena,
batched copy/gather/scatter launches, GPU decode behind
paged_attention_decode<T> and PagedAttentionBatch), against the specification
suites in tests/cpp/{DeviceAllocator,PagedAttention,EndToEnd}.test.cpp."""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BINARY = ROOT / "build" / "tests" / "device_tests"

SUITES = ["DeviceAllocatorTest", "PagedAttentionTest", "PagedAttentionBatchTest", "EngineTest", "KVAppendTest", "PrefillTest", "MRopeTest"]


@pytest.mark.gpu
@pytest.mark.parametrize("suite", SUITES)
def test_device_suite(suite):
    assert BINARY.exists(), f"{BINARY} is missing: run __graft_entry__.build() first"
    print(f"running {BINARY.name} {suite}", flush=True)
    proc = subprocess.run([str(BINARY), suite], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                          timeout=100)
    print(proc.stdout[-3000:])
    assert proc.returncode == 0, proc.stdout[-4000:]
    assert "[       OK ]" in proc.stdout
