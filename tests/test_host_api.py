"""The C++ host API (Block, BlockTable, CacheLayout, MemoryAllocator,
SwapBackend, KVCacheManager, Scheduler) against its specification suites on
host-placed frames: no GPU needed. Each suite is one test here; the binary is
tests/cpp/*.test.cpp built by qwenvl-paged_amd/host/build_host.py."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
BINARY = ROOT / "build" / "tests" / "host_tests"

SUITES = [
    "BlockShapeTest", "LogicalBlockTest", "PhysicalBlockTest", "BlockTableTest", "KVBlockLayoutTest",
    "CacheViewStaticTest", "CacheViewTest", "MemoryAllocatorTest", "MemoryAllocatorSwapTest",
    "MemoryAllocatorEvictionTest", "HostSwapBackendTest", "KVCacheManagerTest", "KVCacheSwapTest",
    "KVCacheSwapSingleFrameTest", "SchedulerTest", "SchedulerPressureTest", "SchedulerWatermarkTest",
    "SchedulerTraceTest", "ElementTypeTest",
]


@pytest.fixture(scope="module")
def host_binary() -> Path:
    if not BINARY.exists():
        # Built by __graft_entry__.build(); build it here only if it is missing.
        subprocess.run([sys.executable, str(ROOT / "qwenvl-paged_amd" / "build.py")], check=True)
    assert BINARY.exists(), f"{BINARY} was not built"
    return BINARY


def run_suite(binary: Path, suite: str) -> str:
    proc = subprocess.run([str(binary), suite], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                          timeout=120)
    assert proc.returncode == 0, proc.stdout[-4000:]
    return proc.stdout


@pytest.mark.parametrize("suite", SUITES)
def test_host_suite(host_binary, suite):
    out = run_suite(host_binary, suite)
    assert "[       OK ]" in out, f"suite {suite} ran no test"


def test_every_suite_is_listed(host_binary):
    out = run_suite(host_binary, "NoSuchSuite")
    assert "0 tests ran" in out
    full = subprocess.run([str(host_binary)], stdout=subprocess.PIPE, text=True, timeout=120).stdout
    ran = {line.split()[3].split(".")[0] for line in full.splitlines() if line.startswith("[ RUN")}
    assert ran == set(SUITES)
