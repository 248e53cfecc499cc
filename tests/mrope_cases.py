"""M-RoPE test inputs: the committed transformers fixtures
(tests/golden/mrope_positions.json) as PositionalEncodingSpan lists, and
seeded random span layouts.

A prompt's runs become spans the way Qwen2-VL's get_rope_index
(transformers 5.15.0) walks them: a text run of n tokens at running position
`cur` is a Text1D span with origin (cur, cur, cur) and stride 1, then cur +=
n; an image / video of (t, h, w) patches is an Image2D / Video3D span of
t * (h/m) * (w/m) tokens with origin (cur, cur, cur), grid (t, h/m, w/m) and
stride (interval, 1, 1) -- interval 1, or tokens_per_second * seconds per grid
for Qwen2.5-VL videos -- then cur += max(h, w) / m.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden" / "mrope_positions.json"

SPAN = np.dtype([("start_token", "<u4"), ("token_count", "<u4"), ("kind", "<u4"), ("reserved", "<u4"),
                 ("origin", "<i8", 3), ("stride", "<i8", 3), ("grid", "<i8", 3)])
TEXT, IMAGE, VIDEO = 0, 1, 2


def golden_cases() -> list[dict]:
    return json.loads(GOLDEN.read_text())["cases"]


def spans_of(case: dict, explicit_text: bool = True) -> np.ndarray:
    """The case's spans; explicit_text=False leaves text runs uncovered."""
    m, tps = case["spatial_merge"], case["tokens_per_second"]
    rows, tok, cur = [], 0, 0
    for run in case["runs"]:
        if run[0] == "text":
            n = run[1]
            if explicit_text:
                rows.append((tok, n, TEXT, 0, (cur,) * 3, (1, 1, 1), (0, 0, 0)))
            tok += n
            cur += n
            continue
        t, h, w = run[1:4]
        grid = (t, h // m, w // m)
        n = grid[0] * grid[1] * grid[2]
        interval = 1
        if run[0] == "video" and case["model"] == "qwen2_5vl":
            interval = tps * int(run[4])
        rows.append((tok, n, IMAGE if run[0] == "image" else VIDEO, 0, (cur,) * 3, (interval, 1, 1), grid))
        tok += n
        cur += max(h, w) // m
    return np.array(rows, SPAN)


def continuation_agrees(case: dict) -> bool:
    """True when leaving text runs uncovered gives transformers' positions:
    every vision span's largest position is cur + max(H, W) - 1, i.e. its
    temporal extent does not reach past its spatial one."""
    m, tps = case["spatial_merge"], case["tokens_per_second"]
    for run in case["runs"]:
        if run[0] == "text":
            continue
        t, h, w = run[1:4]
        interval = tps * int(run[4]) if run[0] == "video" and case["model"] == "qwen2_5vl" else 1
        if (t - 1) * interval > max(h, w) // m - 1:
            return False
    return True


def random_spans(rng: np.random.Generator, length: int, max_spans: int = 12) -> np.ndarray:
    """Sorted, non-overlapping spans with gaps, all three kinds, any origins and
    strides (negative included) inside [0, length)."""
    rows, tok = [], int(rng.integers(0, 4))
    for _ in range(int(rng.integers(0, max_spans + 1))):
        if tok >= length:
            break
        kind = int(rng.integers(0, 3))
        if kind == TEXT:
            n = int(rng.integers(1, 40))
            grid = (0, 0, 0)
        else:
            t = 1 if kind == IMAGE else int(rng.integers(1, 5))
            grid = (t, int(rng.integers(1, 9)), int(rng.integers(1, 9)))
            n = grid[0] * grid[1] * grid[2]
        if tok + n > length:
            break
        origin = tuple(int(x) for x in rng.integers(-50, 3000, 3))
        stride = tuple(int(x) for x in rng.integers(-3, 30, 3))
        rows.append((tok, n, kind, 0, origin, stride, grid))
        tok += n + int(rng.integers(0, 3)) * int(rng.integers(0, 20))
    return np.array(rows, SPAN)
