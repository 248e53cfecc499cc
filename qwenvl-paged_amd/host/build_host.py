"""Builds the C++17 host library (the reference's public API over libqvp) and
the specification test binaries, in-tree.

Outputs (git-ignored, shipped with the tree):
  qwenvl-paged_amd/libqvp_host.so   host API: Block, BlockTable, CacheLayout,
                                    MemoryAllocator, SwapBackend, KVCacheManager,
                                    Scheduler, PagedAttention (links libqvp.so)
  build/tests/host_tests            suites that run on host-placed frames (no GPU)
  build/tests/device_tests          suites that run on device-placed frames (GPU)
  build/bench/cow_bench             copy-on-write configuration driver (GPU)
  build/bench/trace_bench           continuous-batching trace driver (GPU)
  build/bench/config3_bench         long-context multimodal decode driver (GPU)
  build/bench/engine_bench          config2 decode through PagedAttentionBatch over CacheViews (GPU)

libqvp.so must be built first (qwenvl-paged_amd/build.py does both).
"""

from __future__ import annotations

import concurrent.futures
import os
import shlex
import subprocess
from pathlib import Path

HOST = Path(__file__).resolve().parent
PKG = HOST.parent
ROOT = PKG.parent
BUILD = ROOT / "build"
CXX = os.environ.get("CXX", "g++")
ROCM_LIB = "/opt/rocm/lib"

CXXFLAGS = [
    "-std=c++17",
    "-O2",
    "-fPIC",
    "-Wall",
    "-Wextra",
    "-Wno-unused-parameter",
    f"-I{HOST / 'include'}",
    f"-I{ROOT / 'include'}",
]
SOURCES = sorted((HOST / "src").glob("*.cpp"))
# Test binary -> specification suites it holds (tests/cpp/*.test.cpp).
TEST_BINARIES = {
    "host_tests": [
        "Block.test.cpp",
        "BlockTable.test.cpp",
        "CacheView.test.cpp",
        "MemoryAllocator.test.cpp",
        "SwapBackend.test.cpp",
        "KVCacheManager.test.cpp",
        "Scheduler.test.cpp",
        "SchedulerTrace.test.cpp",
        "ElementType.test.cpp",
    ],
    "device_tests": [
        "DeviceAllocator.test.cpp",
        "PagedAttention.test.cpp",
        "EndToEnd.test.cpp",
        "KVAppend.test.cpp",
        "Prefill.test.cpp",
        "MRope.test.cpp",
    ],
}


# Benchmark drivers of the copy-on-write and continuous-batching configurations.
BENCH_BINARIES = {"cow_bench": "cow_bench.cpp", "trace_bench": "trace_bench.cpp", "config3_bench": "config3_bench.cpp",
                  "engine_bench": "engine_bench.cpp"}


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {shlex.join(cmd)}\n{proc.stdout}")
    if proc.stdout.strip():
        print(proc.stdout)


def _compile(src: Path, obj: Path, extra: list[str] | None = None) -> None:
    obj.parent.mkdir(parents=True, exist_ok=True)
    _run([CXX, *CXXFLAGS, *(extra or []), "-c", str(src), "-o", str(obj)])


def build() -> None:
    lib_qvp = PKG / "libqvp.so"
    if not lib_qvp.exists():
        raise RuntimeError(f"{lib_qvp} is missing: build the HIP library first")
    obj_dir = BUILD / "host"
    test_src = ROOT / "tests" / "cpp"
    jobs = [(s, obj_dir / (s.stem + ".o"), None) for s in SOURCES]
    for names in TEST_BINARIES.values():
        for n in names:
            src = test_src / n
            if src.exists():
                jobs.append((src, BUILD / "tests" / "obj" / (src.stem + ".o"), [f"-I{test_src}"]))
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        list(ex.map(lambda j: _compile(*j), jobs))

    rpath = [f"-Wl,-rpath,{PKG}", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM_LIB}"]
    host_lib = PKG / "libqvp_host.so"
    tmp = host_lib.with_suffix(".so.tmp")
    _run([CXX, "-shared", "-o", str(tmp), *[str(obj_dir / (s.stem + ".o")) for s in SOURCES],
          f"-L{PKG}", "-lqvp", *rpath])
    os.replace(tmp, host_lib)

    bench_rpath = [f"-Wl,-rpath,$ORIGIN/../../{PKG.name}", f"-Wl,-rpath,{PKG}", f"-Wl,-rpath,{ROCM_LIB}"]
    (BUILD / "bench").mkdir(parents=True, exist_ok=True)
    for binary, src in BENCH_BINARIES.items():
        _run([CXX, *CXXFLAGS, "-o", str(BUILD / "bench" / binary), str(HOST / "bench" / src), f"-L{PKG}",
              "-lqvp_host", "-lqvp", *bench_rpath])

    # Test binaries find both libraries through the package directory, given
    # both as an absolute path (this tree) and relative to the binary (a copy
    # of the tree elsewhere).
    test_rpath = [f"-Wl,-rpath,$ORIGIN/../../{PKG.name}", f"-Wl,-rpath,{PKG}", f"-Wl,-rpath,{ROCM_LIB}"]
    for binary, names in TEST_BINARIES.items():
        objs = [str(BUILD / "tests" / "obj" / (Path(n).stem + ".o")) for n in names if (test_src / n).exists()]
        if not objs:
            continue
        out = BUILD / "tests" / binary
        _run([CXX, "-o", str(out), str(test_src / "main.cpp"), f"-I{test_src}", *CXXFLAGS, *objs,
              f"-L{PKG}", "-lqvp_host", "-lqvp", "-lpthread", "-lz", *test_rpath])


if __name__ == "__main__":
    build()
    print("built host library and test binaries")
