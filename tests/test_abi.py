"""The drop-in boundary without a GPU: libqvp.so loads and exports every
function include/qvp.h declares, the ctypes binding covers each of them, the
host library exports the C++ API, and the host-only entry points answer
without touching a device."""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

import qvp

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "qvp.h"
HOST_LIB = ROOT / "qwenvl-paged_amd" / "libqvp_host.so"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    names = re.findall(r"\b(qvp_[a-z0-9_]+)\s*\(", text)
    return sorted(set(n for n in names if not n.endswith("_t")))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("qvp_paged_decode", "qvp_pack", "qvp_copy_blocks", "qvp_swap_gather", "qvp_swap_scatter",
                     "qvp_pool_create", "qvp_decode_workspace_bytes", "qvp_batch_view"):
        assert required in names
    assert len(names) >= 40


def test_library_exports_every_declared_function():
    lib = qvp.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_exports_are_plain_c_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", str(qvp.LIB_PATH)], stdout=subprocess.PIPE, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for name in declared_functions():
        assert name in exported, f"{name} is not an unmangled export"


def test_binding_covers_the_header():
    assert set(qvp.SIGNATURES) == set(declared_functions())


def test_host_only_entry_points():
    lib = qvp.load()
    assert lib.qvp_version() >= 1
    assert lib.qvp_status_name(0) == b"QVP_OK"
    for code in range(1, 6):
        assert lib.qvp_status_name(code).startswith(b"QVP_ERR_")
    assert lib.qvp_status_name(99) is not None


def test_status_codes_match_the_header():
    text = HEADER.read_text()
    for name, value in (("QVP_OK", 0), ("QVP_ERR_INVALID_ARGUMENT", 1), ("QVP_ERR_UNMAPPED", 2),
                        ("QVP_ERR_OUT_OF_MEMORY", 3), ("QVP_ERR_CAPACITY", 4), ("QVP_ERR_DEVICE", 5)):
        assert re.search(rf"\b{name}\s*=\s*{value}\b", text), name
        assert getattr(qvp, name.replace("QVP_", "")) == value


@pytest.mark.skipif(not HOST_LIB.exists(), reason="host library not built")
def test_host_library_exports_the_cpp_api():
    out = subprocess.run(["nm", "-DC", "--defined-only", str(HOST_LIB)], stdout=subprocess.PIPE, text=True,
                         check=True).stdout
    for symbol in ("qwenvl_paged::MemoryAllocator::allocate()", "qwenvl_paged::KVCacheManager::fork_sequence",
                   "qwenvl_paged::Scheduler::schedule_next()", "qwenvl_paged::PinnedSwapBackend::store",
                   "qwenvl_paged::PagedAttentionBatch::decode", "qwenvl_paged::paged_attention_decode<float>",
                   "qwenvl_paged::paged_attention_decode<qwenvl_paged::bf16>", "qwenvl_paged::KVBlockLayout"):
        assert symbol in out, symbol
