"""GPU parity: M-RoPE position materialisation (qvp_mrope_positions) through
the C ABI, bit-exact against the transformers fixtures (Qwen2-VL / Qwen2.5-VL
get_rope_index, tests/golden/mrope_positions.json) and against the oracle
(oracle.c orc_mrope_positions) on seeded random span layouts."""

from __future__ import annotations

import numpy as np
import pytest

import mrope_cases as M
import pyoracle as O
import qvp

pytestmark = pytest.mark.gpu


def _gpu(spans_per_seq, begin, end, mr=None):
    """Runs one packed call; returns [3][rows] int64."""
    mr = mr or qvp.MRope()
    spans = np.concatenate(spans_per_seq) if spans_per_seq else np.zeros(0, M.SPAN)
    cu = np.concatenate([[0], np.cumsum([len(s) for s in spans_per_seq])]).astype(np.uint32)
    total = int(sum(int(e) - int(b) for b, e in zip(begin, end)))
    out = qvp.DeviceBuffer(max(total, 1) * 3 * 8)
    out.fill(0xA5)
    mr.positions(spans, cu, begin, end, out.ptr, total)
    qvp.synchronize()
    return out.download(np.int64, (3, total)) if total else np.zeros((3, 0), np.int64)


def _oracle(spans_per_seq, begin, end):
    cols = [O.mrope_positions(s, int(b), int(e)) for s, b, e in zip(spans_per_seq, begin, end)]
    assert all(c is not None for c in cols)
    return np.concatenate(cols, axis=1) if cols else np.zeros((3, 0), np.int64)


def test_transformers_fixtures_in_one_batch():
    print("case: mrope fixtures, one packed call with decode tails", flush=True)
    cases = M.golden_cases()
    spans = [M.spans_of(c) for c in cases]
    n = [len(c["positions"][0]) for c in cases]
    got = _gpu(spans, [0] * len(cases), [x + 5 for x in n])
    col = 0
    for c, length in zip(cases, n):
        want = np.array(c["positions"], np.int64)
        assert np.array_equal(got[:, col:col + length], want), c["name"]
        tail = np.arange(length, length + 5) + c["rope_delta"]
        assert np.array_equal(got[:, col + length:col + length + 5], np.stack([tail] * 3)), c["name"]
        col += length + 5


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_layouts_match_the_oracle(seed):
    print(f"case: mrope random layouts seed={seed}", flush=True)
    rng = np.random.default_rng(seed)
    spans, begin, end = [], [], []
    for _ in range(64):
        length = int(rng.integers(1, 700))
        spans.append(M.random_spans(rng, length))
        b = int(rng.integers(0, length + 1))
        e = int(rng.integers(b, length + 40))
        if rng.integers(0, 5) == 0:
            e = b  # an empty window
        begin.append(b)
        end.append(e)
    assert np.array_equal(_gpu(spans, begin, end), _oracle(spans, begin, end))


def test_a_64_x_8192_token_batch():
    print("case: mrope 64 x 8192 tokens, image and video spans", flush=True)
    rng = np.random.default_rng(7)
    spans = []
    for b in range(64):
        rows, tok, cur = [], 0, 0
        while True:
            text = int(rng.integers(5, 200))
            gh, gw = int(rng.integers(4, 40)), int(rng.integers(4, 40))
            gt = 1 if rng.integers(0, 2) == 0 else int(rng.integers(2, 6))
            n = gt * gh * gw
            if tok + text + n > 8192:
                break
            rows.append((tok, text, M.TEXT, 0, (cur,) * 3, (1, 1, 1), (0, 0, 0)))
            tok, cur = tok + text, cur + text
            rows.append((tok, n, M.VIDEO if gt > 1 else M.IMAGE, 0, (cur,) * 3, (int(rng.integers(1, 9)), 1, 1),
                         (gt, gh, gw)))
            tok, cur = tok + n, cur + max(gh, gw)
        spans.append(np.array(rows, M.SPAN))
    begin, end = [0] * 64, [8192] * 64
    assert np.array_equal(_gpu(spans, begin, end), _oracle(spans, begin, end))


def test_one_token_spans_fill_a_whole_window():
    print("case: mrope 600 one-token spans (257-span windows)", flush=True)
    rng = np.random.default_rng(5)
    rows = [(k, 1, int(rng.integers(0, 2)) * 0, 0, tuple(int(x) for x in rng.integers(-100, 100, 3)),
             (1, 1, 1), (0, 0, 0)) for k in range(600)]
    spans = [np.array(rows, M.SPAN), np.array(rows[:5], M.SPAN)]
    begin, end = [0, 3], [700, 300]
    assert np.array_equal(_gpu(spans, begin, end), _oracle(spans, begin, end))


def test_decode_step_and_object_reuse():
    print("case: mrope decode rows and buffer growth on one object", flush=True)
    rng = np.random.default_rng(11)
    mr = qvp.MRope()
    for batch in (3, 200, 17):
        spans = [M.random_spans(rng, 400, max_spans=6) for _ in range(batch)]
        ctx = [int(rng.integers(1, 500)) for _ in range(batch)]
        # One decode row per sequence: position ctx (the token being generated).
        got = _gpu(spans, ctx, [c + 1 for c in ctx], mr)
        assert np.array_equal(got, _oracle(spans, ctx, [c + 1 for c in ctx]))
    mr.destroy()


def test_refused_calls_write_nothing():
    print("case: mrope refusals", flush=True)
    mr = qvp.MRope()
    good = np.array([(0, 6, M.IMAGE, 0, (0, 0, 0), (1, 1, 1), (1, 2, 3)),
                     (8, 4, M.TEXT, 0, (9, 9, 9), (1, 1, 1), (0, 0, 0))], M.SPAN)
    out = qvp.DeviceBuffer(3 * 20 * 8)
    out.fill(0x5A)
    qvp.synchronize()
    before = out.download(np.uint8, (out.nbytes,))
    cu = np.array([0, 2], np.uint32)
    for what in ("overlap", "grid", "kind", "origin", "window", "rows"):
        s = good.copy()
        b, e, total = [0], [20], 20
        if what == "overlap":
            s[1]["start_token"] = 3
        elif what == "grid":
            s[0]["grid"] = (1, 3, 3)
        elif what == "kind":
            s[0]["kind"] = 7
        elif what == "origin":
            s[1]["origin"] = (0, -(1 << 25), 0)
        elif what == "window":
            b, e = [15], [14]
        elif what == "rows":
            total = 19
        with pytest.raises(qvp.QvpError) as err:
            mr.positions(s, cu, b, e, out.ptr, total)
        assert err.value.status == qvp.ERR_INVALID_ARGUMENT, what
    qvp.synchronize()
    assert np.array_equal(out.download(np.uint8, (out.nbytes,)), before)
    # The same object still works after refusals.
    assert np.array_equal(_gpu([good], [0], [20], mr), _oracle([good], [0], [20]))
