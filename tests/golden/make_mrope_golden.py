"""Writes tests/golden/mrope_positions.json: M-RoPE position ids of
Qwen2-VL / Qwen2.5-VL prompts as computed by the published implementation in
Hugging Face transformers (pinned: 5.15.0, the version in this image):
`Qwen2VLModel.get_rope_index` (models/qwen2_vl/modeling_qwen2_vl.py) and
`Qwen2_5_VLModel.get_rope_index` (models/qwen2_5_vl/modeling_qwen2_5_vl.py).

QwenVL-Paged carries the metadata these ids are built from (a
PositionalEncodingSpan per text / image / video span, include/qwenvl_paged/
KVCacheManager.h:41-60) but implements no materialisation, so the fixtures
come from the model's own library. Run from the repository root:

    python tests/golden/make_mrope_golden.py

Each case stores its inputs (the prompt as runs of text tokens and vision
items, the merge size, tokens_per_second and per-video seconds per grid) and
transformers' outputs (position ids [3][L], rope delta). Only the token types
and grids matter to get_rope_index; the token ids are placeholders.
"""

from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import torch
import transformers
from transformers.models.qwen2_5_vl.modeling_qwen2_5_vl import Qwen2_5_VLModel
from transformers.models.qwen2_vl.modeling_qwen2_vl import Qwen2VLModel

HERE = Path(__file__).resolve().parent

# (name, model, spatial merge, tokens_per_second, runs); a run is
# ("text", n) | ("image", t, h, w) | ("video", t, h, w, seconds_per_grid),
# grids in vision-encoder patches (before the spatial merge).
CASES = [
    ("qwen2vl text-image-text", "qwen2vl", 2, 0, [("text", 5), ("image", 1, 4, 6), ("text", 4)]),
    ("qwen2vl two images", "qwen2vl", 2, 0,
     [("text", 3), ("image", 1, 8, 4), ("text", 2), ("image", 1, 2, 10), ("text", 7)]),
    ("qwen2vl image first", "qwen2vl", 2, 0, [("image", 1, 6, 6), ("text", 9)]),
    ("qwen2vl 14x20 image", "qwen2vl", 2, 0, [("text", 20), ("image", 1, 28, 40), ("text", 10)]),
    ("qwen2vl video longer than wide", "qwen2vl", 2, 0, [("text", 4), ("video", 4, 6, 6, 1), ("text", 6)]),
    ("qwen2vl image then video", "qwen2vl", 2, 0,
     [("text", 2), ("image", 1, 4, 4), ("text", 1), ("video", 2, 4, 8, 1), ("text", 3)]),
    ("qwen2.5vl video, 2 s per grid", "qwen2_5vl", 2, 2, [("text", 3), ("video", 2, 4, 4, 2), ("text", 5)]),
    ("qwen2.5vl image and video", "qwen2_5vl", 2, 25,
     [("text", 6), ("image", 1, 10, 4), ("text", 2), ("video", 3, 6, 4, 1), ("text", 4)]),
    ("qwen2.5vl images with one-token separators", "qwen2_5vl", 2, 2,
     [("image", 1, 4, 2), ("text", 1), ("image", 1, 2, 4), ("text", 3)]),
]


class _Model:
    """The attributes get_rope_index reads from the model: its vision config and
    get_vision_position_ids (bound to this object)."""

    def __init__(self, cls, spatial_merge: int, tokens_per_second: int):
        self._cls = cls
        self.config = SimpleNamespace(vision_config=SimpleNamespace(spatial_merge_size=spatial_merge,
                                                                    tokens_per_second=tokens_per_second))

    def get_vision_position_ids(self, *args, **kwargs):
        return self._cls.get_vision_position_ids(self, *args, **kwargs)

    def get_rope_index(self, *args, **kwargs):
        return self._cls.get_rope_index(self, *args, **kwargs)


def run_case(model: str, merge: int, tps: int, runs) -> tuple[list[list[int]], int]:
    types, images, videos, seconds = [], [], [], []
    for r in runs:
        if r[0] == "text":
            types += [0] * r[1]
        else:
            t, h, w = r[1:4]
            n = t * (h // merge) * (w // merge)
            types += [1 if r[0] == "image" else 2] * n
            (images if r[0] == "image" else videos).append([t, h, w])
            if r[0] == "video":
                seconds.append(r[4])
    ids = torch.zeros(1, len(types), dtype=torch.long)
    tt = torch.tensor([types], dtype=torch.int32)
    kw = dict(image_grid_thw=torch.tensor(images, dtype=torch.long) if images else None,
              video_grid_thw=torch.tensor(videos, dtype=torch.long) if videos else None)
    if model == "qwen2vl":
        m = _Model(Qwen2VLModel, merge, tps)
    else:
        m = _Model(Qwen2_5_VLModel, merge, tps)
        kw["second_per_grid_ts"] = torch.tensor(seconds, dtype=torch.float) if seconds else None
    pos, delta = m.get_rope_index(ids, tt, **kw)
    return pos[:, 0, :].tolist(), int(delta.reshape(-1)[0])


def main() -> None:
    out = {"generator": "tests/golden/make_mrope_golden.py", "transformers": transformers.__version__, "cases": []}
    for name, model, merge, tps, runs in CASES:
        pos, delta = run_case(model, merge, tps, runs)
        out["cases"].append({"name": name, "model": model, "spatial_merge": merge, "tokens_per_second": tps,
                             "runs": [list(r) for r in runs], "positions": pos, "rope_delta": delta})
    path = HERE / "mrope_positions.json"
    path.write_text(json.dumps(out, separators=(",", ":")) + "\n")
    print(f"wrote {path} ({len(out['cases'])} cases)")


if __name__ == "__main__":
    main()
