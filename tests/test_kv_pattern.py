"""The numpy restatement of the verifying driver's seeded K/V and query rows
(tests/kv_pattern.py) against the C++ header the driver compiles
(qwenvl-paged_amd/host/bench/kv_pattern.h): a small g++ program prints rows of
the header and every element must agree. Runs on the CPU."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import kv_pattern as P

ROOT = Path(__file__).resolve().parents[1]
HEADER_DIR = ROOT / "qwenvl-paged_amd" / "host" / "bench"

PROGRAM = r"""
#include "kv_pattern.h"
#include <cstdio>
#include <initializer_list>
int main() {
    const unsigned long long cases[][3] = {{1, 0, 0}, {1, 0, 1}, {200, 9215, 0}, {77, 4096, 1}, {0xFFFFFFFFull, 123456, 0}};
    std::uint16_t row[512];
    for (const auto& c : cases) {
        kv_pattern::kv_row(c[0], c[1], static_cast<std::uint32_t>(c[2]), row, 512);
        for (int e = 0; e < 512; ++e) std::printf("%u%c", row[e], e == 511 ? '\n' : ' ');
    }
    std::uint16_t q[3584];
    for (unsigned r : {0u, 1u, 255u}) {
        kv_pattern::query_row(r, q, 3584);
        for (int e = 0; e < 3584; ++e) std::printf("%u%c", q[e], e == 3583 ? '\n' : ' ');
    }
    return 0;
}
"""


@pytest.fixture(scope="module")
def header_rows(tmp_path_factory) -> list[np.ndarray]:
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ is not installed")
    d = tmp_path_factory.mktemp("kv_pattern")
    src, exe = d / "p.cpp", d / "p"
    src.write_text(PROGRAM)
    subprocess.run([cxx, "-std=c++17", "-O1", f"-I{HEADER_DIR}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True, check=True).stdout
    return [np.array(line.split(), dtype=np.uint16) for line in out.splitlines()]


def test_kv_rows_equal_the_header(header_rows):
    cases = [(1, 0, 0), (1, 0, 1), (200, 9215, 0), (77, 4096, 1), (0xFFFFFFFF, 123456, 0)]
    for k, (seq, pos, stream) in enumerate(cases):
        got = P.kv_rows([seq], [pos], stream, 512)[0]
        assert np.array_equal(got, header_rows[k]), f"kv row {seq}/{pos}/{stream}"


def test_query_rows_equal_the_header(header_rows):
    got = P.query_rows([0, 1, 255], 3584)
    for k in range(3):
        assert np.array_equal(got[k], header_rows[5 + k]), f"query row {k}"


def test_rows_are_finite_bf16_in_their_ranges_and_distinct():
    kv = P.kv_rows(np.arange(64), np.arange(64) * 97, 0, 512)
    q = P.query_rows(np.arange(64), 3584)
    kv_exp = (kv >> 7) & 0xFF
    q_exp = (q >> 7) & 0xFF
    assert set(np.unique(kv_exp)) == {124, 125, 126}
    assert set(np.unique(q_exp)) == {125, 126, 127}
    # K and V of one token differ, and so do neighbouring positions.
    assert not np.array_equal(P.kv_rows([5], [10], 0, 512), P.kv_rows([5], [10], 1, 512))
    assert not np.array_equal(P.kv_rows([5], [10], 0, 512), P.kv_rows([5], [11], 0, 512))
    assert len({r.tobytes() for r in kv}) == 64
