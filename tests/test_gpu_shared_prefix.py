"""GPU parity of the shared-prefix decode: sequences forked from one prompt
share the prompt's frames (the page-table state KVCacheManager::fork leaves,
reference src/KVCacheManager.cpp fork), and the persistent decode reads those
frames once for the whole group (a launch before the main one) while every
sequence's own tail runs as ordinary pieces. The result must equal the
reference's per-sequence decode (PagedAttention.h:53-127) at the bf16 bar;
the oracle decodes each sequence over its own block list, so sharing is
invisible to it."""

from __future__ import annotations

import numpy as np
import pytest

import qvp
import workloads as W
from helpers import GpuRun, assert_close_16bit, assert_close_bf16, oracle_decode, tiled_pool_image

pytestmark = pytest.mark.gpu


def _extra(seed: int, branches, lo: int = 1, hi: int = 120):
    rng = np.random.default_rng(seed)
    return [list(rng.integers(lo, hi, size=n)) for n in branches]


def _check(w: W.Workload, expect_groups: int | None = None):
    run = GpuRun(w)
    _, ref32 = oracle_decode(w, run.image, run.query)
    got32 = run.decode(out_dtype=qvp.DTYPE_F32)
    plan = run.batch.decode_plan()
    assert plan["kernel"] == "mfma"
    if expect_groups is not None:
        assert plan["shared_prefix_groups"] == expect_groups, plan
        assert plan["shared_prefix_items"] >= expect_groups * w.num_kv_heads, plan
    stats = assert_close_bf16(got32, ref32, f"{w.name} fp32 out")
    got16 = run.decode(out_dtype=qvp.DTYPE_BF16)
    assert_close_16bit(got16, ref32, qvp.DTYPE_BF16, f"{w.name} bf16 out")
    return run, got32, stats


def test_forks_of_three_prompts_at_the_7b_shape():
    # Group of 8 (the most a query group of 7 fits: four column blocks of two
    # sequences), of 3 and of 2, beside two unshared sequences.
    branches = [8, 3, 2]
    w = W.forked([1000, 2100, 333], branches, _extra(1, branches), 28, 4, solo_lens=[700, 50])
    _check(w, expect_groups=3)


@pytest.mark.parametrize("hq,hkv,per_group", [(4, 4, 8), (16, 4, 8), (64, 4, 4), (32, 8, 8)])
def test_query_group_sizes_set_the_group_capacity(hq, hkv, per_group):
    # 16 // G sequences per column block, four blocks, at most eight: a fork of
    # ten splits into groups of per_group and the rest (a lone rest is left
    # to the main launch).
    branches = [10]
    w = W.forked([1500], branches, _extra(2, branches), hq, hkv)
    full, rest = divmod(10, per_group)
    _check(w, expect_groups=full + (1 if rest >= 2 else 0))


def test_prefix_shorter_than_the_minimum_is_decoded_per_sequence():
    branches = [4]
    w = W.forked([100], branches, _extra(3, branches), 28, 4)  # 6 shared blocks = 3 tiles
    _check(w, expect_groups=0)


def test_branch_ending_inside_the_shared_tail_block():
    # Branches of one token past a prompt that ends mid-block: each branch's
    # last block is its own copy, so the shared frames stop one block early.
    branches = [5]
    w = W.forked([1031], branches, [[1, 1, 2, 1, 3]], 28, 4)
    _check(w, expect_groups=1)


def test_config4_shape_matches_the_oracle_and_repeats_bit_for_bit():
    # The copy-on-write configuration's decode: 16 prompts of 2048 tokens x 8
    # branches, each one token into its own tail block (ctx 2049).
    branches = [8] * 16
    w = W.forked([2048] * 16, branches, [[1] * 8] * 16, 28, 4)
    run, got, _ = _check(w, expect_groups=16)
    for _ in range(3):
        again = run.decode(out_dtype=qvp.DTYPE_F32)
        assert np.array_equal(again, got), "shared-prefix decode is not deterministic"


@pytest.mark.parametrize("tpb", [32, 64])
def test_larger_blocks(tpb):
    # A 32-token tile is one block (tpb 32) or half of one (tpb 64); the
    # prefix launch resolves its frames through the table's tpb shift.
    branches = [6, 3]
    w = W.forked([1500, 700], branches, _extra(5, branches), 28, 4, tokens_per_block=tpb, solo_lens=[900])
    _check(w, expect_groups=2)


def test_captured_decode_with_shared_prefixes_replays_bit_for_bit():
    # Both launches (prefix, then the private tails that complete the
    # merges) in one graph: the counters the prefix launch raises are reset by
    # the merging workgroups, so every replay starts from zero.
    branches = [8, 4]
    w = W.forked([1200, 2600], branches, _extra(6, branches), 28, 4, solo_lens=[333])
    stream = qvp.Stream()
    run = GpuRun(w)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, w.tokens_per_block, w.num_pool_blocks, 0, stream)
    ws = qvp.DeviceBuffer(run.batch.workspace_bytes(w.num_query_heads, w.head_dim))
    n = w.num_seqs * w.num_query_heads * w.head_dim
    out = qvp.DeviceBuffer(n * 4)
    args = qvp.decode_args(query=run.q.ptr, out=out.ptr, kv_base=run.pool.base, block_stride=run.pool.stride,
                           batch=run.batch, kv_dtype=w.kv_dtype, out_dtype=qvp.DTYPE_F32, layer=w.layer,
                           num_layers=w.num_layers, num_query_heads=w.num_query_heads,
                           num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, tokens_per_block=w.tokens_per_block,
                           scale=w.scale, strides=w.strides, workspace=ws.ptr, workspace_bytes=ws.nbytes)
    qvp.paged_decode(args, stream)
    eager = out.download(np.float32, (n,), stream)
    assert run.batch.decode_plan()["shared_prefix_groups"] == 2
    _, ref32 = oracle_decode(w, run.image, run.query)
    assert_close_bf16(eager.reshape(ref32.shape), ref32, "eager")
    other = GpuRun(W.forked([900], [5], _extra(7, [5]), 28, 4, seed=12))
    with qvp.Graph.capture(stream) as graph:
        qvp.paged_decode(args, stream)
    for replay in range(4):
        out.fill(0xFF, stream)
        graph.launch(stream)
        stream.synchronize()
        assert np.array_equal(out.download(np.float32, (n,), stream), eager), f"replay {replay}"
        other.decode(stream=stream)
    graph.destroy()


def test_allocation_free_entry_point_with_shared_prefixes():
    branches = [8]
    w = W.forked([1800], branches, _extra(8, branches), 28, 4, solo_lens=[64, 2000])
    run = GpuRun(w)
    stream = qvp.Stream()
    _, ref32 = oracle_decode(w, run.image, run.query)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, w.tokens_per_block, w.num_pool_blocks, 0, stream)
    n = w.num_seqs * w.num_query_heads * w.head_dim
    out = qvp.DeviceBuffer(n * 4)
    args = qvp.decode_args(query=run.q.ptr, out=out.ptr, kv_base=run.pool.base, block_stride=run.pool.stride,
                           batch=run.batch, kv_dtype=w.kv_dtype, out_dtype=qvp.DTYPE_F32, layer=w.layer,
                           num_layers=w.num_layers, num_query_heads=w.num_query_heads,
                           num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, tokens_per_block=w.tokens_per_block,
                           scale=w.scale, strides=w.strides)
    # The schedule is built by a first (allocating) decode; the allocation-free
    # call then runs on the library's scratch array.
    qvp.paged_decode(args, stream)
    first = out.download(np.float32, (n,), stream)
    out.fill(0xFF, stream)
    qvp.paged_decode_noalloc(args, stream)
    got = out.download(np.float32, (n,), stream)
    assert run.batch.decode_plan()["shared_prefix_groups"] == 1
    assert np.array_equal(got, first)
    assert_close_bf16(got.reshape(ref32.shape), ref32, "no-alloc")


def test_long_and_short_private_tails_in_one_batch():
    # Branches with tails of at most four tiles are finished by the prefix
    # launch; longer tails (up to 900 tokens here) are pieces of the
    # persistent decode, which completes and merges those segments.
    branches = [6, 4]
    extra = [[1, 3, 500, 40, 900, 127], [2, 640, 5, 96]]
    w = W.forked([1400, 2050], branches, extra, 28, 4, solo_lens=[1200])
    run, got32, _ = _check(w, expect_groups=2)
    plan = run.batch.decode_plan()
    assert plan["workgroups"] > 0, plan  # the long tails need the persistent decode


def test_half_precision_output_from_the_prefix_launch():
    branches = [8]
    w = W.forked([2048], branches, [[1] * 8], 28, 4)
    run = GpuRun(w)
    _, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F16)
    assert run.batch.decode_plan()["workgroups"] == 0  # every tail was short: one launch
    assert_close_16bit(got, ref32, qvp.DTYPE_F16, "f16 out")


@pytest.mark.parametrize("prompts,grouped", [(40, True), (900, False)], ids=["few-forks", "many-tiny-forks"])
def test_many_tiny_forks_are_planned_without_shared_prefixes(prompts, grouped):
    # Prompts of 4 shared tiles forked 8 ways, each branch 5 private tiles
    # past them (too long for the prefix launch), 3 kv heads (one per
    # segment: 85 ranges per head). With 40 prompts the prefix groups are
    # used; with 900 (7,200 branches) every range would hold ~85 partial
    # private tails, more than the 64 merges a workgroup tracks in LDS, so the
    # planner drops the shared prefixes and the plain per-sequence schedule
    # decodes the batch.
    branches = [8] * prompts
    extra = _extra(9, branches, lo=129, hi=161)
    w = W.forked([128] * prompts, branches, extra, 3, 3)
    run = GpuRun(w, image=tiled_pool_image(w))
    print(f"case: {prompts} prompts x 8 branches, grouped={grouped}", flush=True)
    _, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    plan = run.batch.decode_plan()
    assert plan["kernel"] == "mfma"
    if grouped:
        assert plan["shared_prefix_groups"] == prompts, plan
    else:
        assert plan["shared_prefix_groups"] == 0, plan
    assert_close_bf16(got, ref32, f"{prompts} prompts")
