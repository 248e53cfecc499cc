"""The M-RoPE oracle (oracle.c orc_mrope_positions) pinned on the CPU.

QwenVL-Paged carries the span metadata (include/qwenvl_paged/
KVCacheManager.h:23-78) but never materialises positions; the rule comes from
the model's published implementation, Qwen2-VL / Qwen2.5-VL get_rope_index in
transformers 5.15.0, whose outputs are committed as fixtures
(tests/golden/make_mrope_golden.py). Checks: every fixture position and the
decode continuation p + rope_delta; uncovered text equals explicit text where
the continuation rule and get_rope_index's `cur += max(h, w)` agree, and
differs where a video's temporal extent reaches further; closed forms of a
single span; refusals.
"""

from __future__ import annotations

import numpy as np
import pytest

import mrope_cases as M
import pyoracle as O

CASES = M.golden_cases()


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_oracle_reproduces_transformers_positions(case):
    want = np.array(case["positions"], np.int64)
    n = want.shape[1]
    got = O.mrope_positions(M.spans_of(case), 0, n)
    assert got is not None
    assert np.array_equal(got, want)
    # Decode tokens after the prompt: position_ids = p + rope_delta on all
    # three axes (transformers' incremental-generation branch).
    dec = O.mrope_positions(M.spans_of(case), n, n + 7)
    expect = np.arange(n, n + 7, dtype=np.int64) + case["rope_delta"]
    assert np.array_equal(dec, np.stack([expect] * 3))
    # A window in the middle equals the same columns of the whole prompt.
    assert np.array_equal(O.mrope_positions(M.spans_of(case), n // 3, n - 1), want[:, n // 3:n - 1])


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_uncovered_text_continues_from_the_running_maximum(case):
    want = np.array(case["positions"], np.int64)
    got = O.mrope_positions(M.spans_of(case, explicit_text=False), 0, want.shape[1])
    if M.continuation_agrees(case):
        assert np.array_equal(got, want)
    else:
        # get_rope_index resumes text at cur + max(h, w) / m, below the video's
        # last temporal position; the continuation rule resumes above it.
        assert not np.array_equal(got, want)
        assert got[:, -1].min() > want[:, -1].max()


def test_fixtures_exercise_both_rules():
    agree = [M.continuation_agrees(c) for c in CASES]
    assert any(agree) and not all(agree)


def test_transposed_grid_is_caught_by_the_fixtures():
    # A planted mistake in the span construction (h and w swapped for every
    # non-square image) must change the positions of some fixture.
    caught = 0
    for case in CASES:
        spans = M.spans_of(case)
        bad = spans.copy()
        for s in bad:
            if s["kind"] != M.TEXT and s["grid"][1] != s["grid"][2]:
                s["grid"][1], s["grid"][2] = s["grid"][2], s["grid"][1]
        if not np.array_equal(bad["grid"], spans["grid"]):
            n = len(case["positions"][0])
            caught += not np.array_equal(O.mrope_positions(bad, 0, n), np.array(case["positions"]))
    assert caught >= 5


def test_single_span_closed_forms():
    video = np.array([(3, 24, M.VIDEO, 0, (100, -7, 5), (10, 2, -3), (2, 3, 4))], M.SPAN)
    got = O.mrope_positions(video, 0, 30)
    # Before the span: 0, 1, 2. Inside: origin + (i // 12, (i // 4) % 3, i % 4) * stride.
    i = np.arange(24)
    assert np.array_equal(got[:, :3], np.stack([np.arange(3)] * 3))
    assert np.array_equal(got[0, 3:27], 100 + 10 * (i // 12))
    assert np.array_equal(got[1, 3:27], -7 + 2 * ((i // 4) % 3))
    assert np.array_equal(got[2, 3:27], 5 - 3 * (i % 4))
    # After it: 1 + the largest position so far (the temporal 110).
    assert np.array_equal(got[:, 27:], np.stack([np.arange(111, 114)] * 3))
    text = np.array([(0, 5, M.TEXT, 0, (4, 9, -2), (2, 0, -1), (0, 0, 0))], M.SPAN)
    got = O.mrope_positions(text, 0, 6)
    assert np.array_equal(got[:, :5], np.array([[4, 6, 8, 10, 12], [9] * 5, [-2, -3, -4, -5, -6]]))
    assert np.array_equal(got[:, 5], [13, 13, 13])
    assert np.array_equal(O.mrope_positions(np.zeros(0, M.SPAN), 5, 9), np.stack([np.arange(5, 9)] * 3))


@pytest.mark.parametrize("bad", [
    "overlap", "unsorted", "empty", "kind", "grid product", "image t", "origin", "stride", "range"])
def test_refusals(bad):
    spans = np.array([(0, 6, M.IMAGE, 0, (0, 0, 0), (1, 1, 1), (1, 2, 3)),
                      (8, 4, M.TEXT, 0, (9, 9, 9), (1, 1, 1), (0, 0, 0))], M.SPAN)
    begin, end = 0, 20
    if bad == "overlap":
        spans[1]["start_token"] = 5
    elif bad == "unsorted":
        spans = spans[::-1].copy()
    elif bad == "empty":
        spans[1]["token_count"] = 0
    elif bad == "kind":
        spans[1]["kind"] = 3
    elif bad == "grid product":
        spans[0]["grid"] = (1, 2, 2)
    elif bad == "image t":
        spans[0]["grid"] = (2, 1, 3)
    elif bad == "origin":
        spans[1]["origin"] = ((1 << 24) + 1, 0, 0)
    elif bad == "stride":
        spans[0]["stride"] = (1, -(1 << 24) - 1, 1)
    elif bad == "range":
        begin, end = 10, 9
    assert O.mrope_positions(spans, begin, end) is None
