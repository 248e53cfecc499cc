"""GPU parity: the persistent decode's work plan reused across decode steps.

A decode loop packs its batch every step (PagedAttention.h:53-58 is called per
view after each step's bookkeeping), and a sequence usually gains one token
from one step to the next. The planner then keeps the previous step's plan and
rewrites only the context lengths stored in it when every sequence's tile count
and the shared-prefix groups are unchanged, and plans afresh otherwise. Either
way the decode must equal a decode planned from scratch -- bit for bit, since
the plan fixes the order of every sum -- and the oracle at the bf16 bar.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest

import qvp
import workloads as W
from helpers import GpuRun, assert_close_bf16, oracle_decode

pytestmark = pytest.mark.gpu


def _decode(run: GpuRun, batch: qvp.Batch, lens: np.ndarray) -> np.ndarray:
    w = run.w
    n = w.num_seqs * w.num_query_heads * w.head_dim
    out = qvp.DeviceBuffer(n * 4)
    out.fill(0xFF)
    args = qvp.decode_args(query=run.q.ptr, out=out.ptr, kv_base=run.pool.base, block_stride=run.pool.stride,
                           batch=batch, kv_dtype=w.kv_dtype, out_dtype=qvp.DTYPE_F32, layer=w.layer,
                           num_layers=w.num_layers, num_query_heads=w.num_query_heads, num_kv_heads=w.num_kv_heads,
                           head_dim=w.head_dim, tokens_per_block=w.tokens_per_block, scale=w.scale,
                           strides=w.strides)
    batch.pack(w.ids, w.cu_blocks, lens, w.tokens_per_block, w.num_pool_blocks, w.split_tokens, decode=args)
    qvp.paged_decode(args)
    return out.download(np.float32, (w.num_seqs, w.num_query_heads, w.head_dim))


def _steps(w: W.Workload, lens_steps, oracle_steps, expect_groups: int = 0):
    # The tables hold the frames for the largest lengths; each step decodes a
    # prefix of every table.
    run = GpuRun(w)
    reused = qvp.Batch()
    for i, lens in enumerate(lens_steps):
        lens = np.asarray(lens, dtype=np.uint32)
        print(f"case: plan reuse {w.name} step {i}", flush=True)
        got = _decode(run, reused, lens)
        plan = reused.decode_plan()
        assert plan["kernel"] == "mfma" and plan["shared_prefix_groups"] == expect_groups, plan
        fresh = _decode(run, qvp.Batch(), lens)
        assert np.array_equal(got.view(np.uint32), fresh.view(np.uint32)), f"step {i}: reused plan differs"
        if i in oracle_steps:
            _, ref32 = oracle_decode(dataclasses.replace(w, context_lens=lens), run.image, run.query)
            assert_close_bf16(got, ref32, f"{w.name} step {i}")


def test_growing_contexts_reuse_and_replan():
    # 24 sequences at the 7B shape, one token per step; steps 0 -> 1 -> 2 keep
    # every tile count (reuse), some sequences cross 16- and 32-token
    # boundaries later (a new frame, a new tile: a fresh plan).
    rng = np.random.default_rng(3)
    base = rng.integers(200, 3000, size=24)
    base[:4] = [31, 32, 63, 95]  # at tile edges
    w = W.custom(base + 40, 28, 4, 128, seed=4)
    steps = [base + d for d in (0, 1, 2, 3, 17, 18, 33, 40)]
    _steps(w, steps, oracle_steps={0, 2, 5, 7})


def test_forked_branches_reuse_the_shared_prefix_plan():
    # Three prompts forked into 8, 3 and 2 branches: the shared-prefix items
    # are reused while the branches' private tails grow inside their tiles.
    branches = [8, 3, 2]
    extra = [[40] * n for n in branches]
    w = W.forked([1000, 2100, 333], branches, extra, 28, 4, solo_lens=[700])
    full = w.context_lens.astype(np.int64)
    steps = [full - d for d in (39, 38, 37, 20, 19, 1, 0)]
    _steps(w, steps, oracle_steps={0, 1, 6}, expect_groups=3)


@pytest.mark.parametrize("split", [512])
def test_split_partitions_reuse(split):
    # config3-like split-K partitions: the reuse keeps the partition cuts.
    rng = np.random.default_rng(8)
    base = rng.integers(2000, 9000, size=6)
    w = dataclasses.replace(W.custom(base + 8, 64, 8, 128, seed=9), split_tokens=split)
    steps = [base + d for d in (0, 1, 5, 8)]
    _steps(w, steps, oracle_steps={0, 3})
