"""GPU parity: paged decode through the C ABI against the CPU oracle.

Mirrors tests/PagedAttention.test.cpp of the reference (numeric cases and
refusals) at batch scale, plus the BASELINE configurations. The oracle is the
C restatement of paged_attention_decode<T> (oracle/oracle.c), itself pinned
bit-for-bit to the compiled reference in tests/test_oracle.py.
"""

from __future__ import annotations

import numpy as np
import pytest

import qvp
import workloads as W
from helpers import F32_ABS_TOL, GpuRun, assert_close_16bit, assert_close_bf16, oracle_decode, tiled_pool_image, to_f32

pytestmark = pytest.mark.gpu


def _parity(w: W.Workload, out_dtypes=(None,), split_tokens=None):
    run = GpuRun(w)
    ref_out, ref32 = oracle_decode(w, run.image, run.query)
    results = {}
    for od in out_dtypes:
        od = w.kv_dtype if od is None else od
        raw = run.decode(out_dtype=od, split_tokens=split_tokens)
        if w.kv_dtype == qvp.DTYPE_F32 and od == qvp.DTYPE_F32:
            err = float(np.abs(raw - ref32).max())
            assert err <= F32_ABS_TOL, f"fp32 max abs {err:.3e}"
            results[od] = {"max_abs": err}
        elif od == qvp.DTYPE_F32:
            results[od] = assert_close_bf16(raw, ref32, f"{w.name} fp32 out")
        else:
            results[od] = assert_close_16bit(raw, ref32, od, f"{w.name} 16-bit out")
            if od == w.kv_dtype:
                # The oracle's own T output (PagedAttention.h:120-123) obeys the same bound.
                assert_close_16bit(raw, to_f32(ref_out, od), od, f"{w.name} vs oracle T out")
    return results


def test_config1_fp32_matches_oracle():
    print("case: config1 fp32", flush=True)
    _parity(W.config1())


# Hq, Hkv, D for the GQA-folded split kernel: groups of 1 .. 16 (register
# widths 1, 2, 4, 8 and 16), head dims below, at and above its 256 threads.
FOLDED_SHAPES = [(8, 2, 64), (28, 4, 80), (12, 4, 256), (10, 5, 32), (48, 3, 96), (4, 2, 320), (8, 8, 64)]


@pytest.mark.parametrize("kv_dtype", [qvp.DTYPE_F32, qvp.DTYPE_BF16, qvp.DTYPE_F16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", FOLDED_SHAPES, ids=[f"hq{a}-hkv{b}-d{c}" for a, b, c in FOLDED_SHAPES])
def test_gqa_folded_split_kernel_matches_the_oracle(shape, kv_dtype):
    """Head dims other than 128 (and the element types the reference template
    takes) run one workgroup per (split, kv head) for the whole query group:
    each K/V element is read once per group. Same bars as every decode."""
    hq, hkv, d = shape
    print(f"case: folded split decode hq={hq} hkv={hkv} d={d} kv_dtype={kv_dtype}", flush=True)
    w = W.custom([37, 300, 777, 1025], hq, hkv, d, kv_dtype=kv_dtype, seed=hq + d)
    run = GpuRun(w)
    _, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    plan = run.batch.decode_plan()
    # At head_dim 64 the matrix-core split kernels take over: fp32 and 16-bit.
    expect = "grouped" if d != 64 else "f32_grouped" if kv_dtype == qvp.DTYPE_F32 else "split_mfma"
    assert plan["kernel"] == expect, plan
    assert plan["workgroups"] == plan["pieces"] * hkv, plan
    if kv_dtype == qvp.DTYPE_F32:
        err = float(np.abs(got - ref32).max())
        assert err <= F32_ABS_TOL, f"fp32 max abs {err:.3e}"
    else:
        assert_close_bf16(got, ref32, f"folded {shape} fp32 out")
        got16 = run.decode(out_dtype=kv_dtype)
        assert_close_16bit(got16, ref32, kv_dtype, f"folded {shape} 16-bit out")


@pytest.mark.parametrize("tpb", [8, 12, 32])
def test_gqa_folded_split_kernel_with_other_block_sizes(tpb):
    # Frames are found per token (tok / tpb, tok % tpb), so blocks smaller
    # than, not a power of two, or larger than 16 tokens read the same rows.
    print(f"case: folded split decode tpb={tpb}", flush=True)
    w = W.custom([37, 300, 777, 1025], 28, 4, 80, tokens_per_block=tpb, seed=tpb)
    run = GpuRun(w)
    _, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    assert run.batch.decode_plan()["kernel"] == "grouped"
    assert_close_bf16(got, ref32, f"folded tpb={tpb}")


@pytest.mark.parametrize("hq,hkv,d", [(34, 2, 64), (28, 4, 66)], ids=["group-17", "head-dim-66"])
def test_other_split_shapes_run_the_per_head_split_kernel(hq, hkv, d):
    # A group above 16, or rows that four-element loads cannot read (head_dim
    # 66: 132-byte bf16 rows), take the per-query-head kernel.
    print(f"case: per-head split decode hq={hq} hkv={hkv} d={d}", flush=True)
    w = W.custom([90, 600, 1300], hq, hkv, d, seed=hq + d)
    run = GpuRun(w)
    _, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    plan = run.batch.decode_plan()
    assert plan["kernel"] == "generic", plan
    assert plan["workgroups"] == plan["pieces"] * hq, plan
    assert_close_bf16(got, ref32, f"per-head hq={hq} hkv={hkv}")


def test_config2_bf16_matches_oracle_fp32_and_bf16_outputs():
    print("case: config2 bf16 B=64", flush=True)
    _parity(W.config2(), out_dtypes=(qvp.DTYPE_F32, qvp.DTYPE_BF16))


@pytest.mark.parametrize("split", [128, 256, 512, 1024, 4096])
@pytest.mark.parametrize("kv_dtype", [qvp.DTYPE_F32, qvp.DTYPE_F16], ids=["f32-grouped", "split-f16"])
def test_split_kernels_follow_the_split_size(kv_dtype, split):
    """The split kernels partition each sequence into split_tokens pieces and
    merge them; every partition size gives the oracle's result (the fp16 case,
    group 7 at head_dim 64, on the 16-bit matrix-core split kernel)."""
    print(f"case: split kernels dtype={kv_dtype} split={split}", flush=True)
    lens = [37, 600, 1500, 4096, 129, 2049]
    if kv_dtype == qvp.DTYPE_F32:
        # A negative scale: fp32 caches with a positive one run the persistent
        # kernel (tests/test_gpu_decode_f32.py).
        w = W.custom(lens, 28, 4, 128, kv_dtype=qvp.DTYPE_F32, seed=11, kv_sigma=1.0, scale=-0.05)
        run = GpuRun(w)
    else:
        # head_dim 64: fp16 caches with head_dim 128 run the persistent MFMA
        # kernel (tests/test_gpu_decode_f16.py).
        w = W.custom(lens, 28, 4, 64, kv_dtype=qvp.DTYPE_F16, seed=11)
        w32 = W.custom(lens, 28, 4, 64, kv_dtype=qvp.DTYPE_F32, seed=11, kv_sigma=0.5)
        image = w32.pool_image().view(np.float32).astype(np.float16).view(np.uint8)
        run = GpuRun(w, image=image, query=w32.query().astype(np.float16).view(np.uint16))
    _, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32, split_tokens=split)
    plan = run.batch.decode_plan()
    assert plan["kernel"] == ("f32_grouped" if kv_dtype == qvp.DTYPE_F32 else "split_mfma"), plan
    assert plan["split_tokens"] == split, plan
    expect_splits = int(sum(-(-int(n) // split) for n in lens))
    assert plan["pieces"] == expect_splits, plan
    if kv_dtype == qvp.DTYPE_F32:
        err = float(np.abs(got - ref32).max())
        assert err <= F32_ABS_TOL, f"fp32 max abs {err:.3e}"
    else:
        assert_close_bf16(got, ref32, f"fp16 split={split}")


def test_mfma_path_holds_its_cuts_to_the_split_partition():
    """Without split_tokens the bf16 MFMA kernel cuts the batch into tile
    ranges by cost alone; with one, every range starts and ends on a
    split_tokens partition boundary of its sequence. Each range of one kv-head
    group is then a run of whole partitions, so a group holds at most one
    piece per partition -- far fewer than the cost cuts make on one long
    sequence -- and the results stay within the bf16 bound of the oracle."""
    w = W.custom([4096, 1500, 700, 129], 28, 4, 128, seed=11)
    run = GpuRun(w)
    _, ref32 = oracle_decode(w, run.image, run.query)
    print("case: mfma path, cost cuts", flush=True)
    free = run.decode(out_dtype=qvp.DTYPE_F32, split_tokens=0)
    plan0 = run.batch.decode_plan()
    assert plan0["kernel"] == "mfma" and plan0["split_tokens"] == 0, plan0
    assert_close_bf16(free, ref32, "mfma cost cuts")
    lens = w.context_lens
    for split in (128, 512, 4096):
        print(f"case: mfma path split={split}", flush=True)
        got = run.decode(out_dtype=qvp.DTYPE_F32, split_tokens=split)
        plan = run.batch.decode_plan()
        assert plan["kernel"] == "mfma" and plan["split_tokens"] == split, plan
        groups = 4 // plan["kv_heads_per_segment"]
        partitions = sum(-(-int(n) // split) for n in lens)
        assert plan["pieces"] <= groups * partitions, (plan, partitions)
        assert_close_bf16(got, ref32, f"mfma split {split}")
        again = run.decode(out_dtype=qvp.DTYPE_F32, split_tokens=split)
        assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), f"split {split} not deterministic"
    # One partition per sequence: one piece per sequence and group, as many as
    # the free cuts would make only if they never split a sequence.
    assert plan["pieces"] == groups * len(lens), plan
    assert plan0["pieces"] > groups * len(lens), plan0


def test_merge_state_carries_nothing_between_launches():
    """Each launch leaves the in-kernel merge's state (segment counters, split
    slots) ready for the next: decoding two queries in turn on one packed
    batch -- with a differently shaped batch decoded on the same batch object
    in between -- gives each query's output bit for bit as a fresh batch
    decodes it."""
    w = W.config2(seed=21, num_seqs=16)
    qa = w.query()
    qb = W.config2(seed=22, num_seqs=16).query()
    image = w.pool_image()
    fresh = {}
    for key, q in (("a", qa), ("b", qb)):
        print(f"case: fresh batch, query {key}", flush=True)
        fresh[key] = GpuRun(w, image=image, query=q).decode(out_dtype=qvp.DTYPE_F32)
    run = GpuRun(w, image=image, query=qa)
    qbuf = {"a": run.q, "b": qvp.DeviceBuffer.from_array(qb)}
    short = W.custom([100, 900, 3000, 4000], 28, 4, 128, seed=5)
    run_s = GpuRun(short)
    _, ref_s = oracle_decode(short, run_s.image, run_s.query)
    for i, key in enumerate("ababba"):
        print(f"case: launch {i} query {key}", flush=True)
        run.q = qbuf[key]
        got = run.decode(out_dtype=qvp.DTYPE_F32)
        assert run.batch.decode_plan()["slots"] > 0
        assert np.array_equal(got.view(np.uint32), fresh[key].view(np.uint32)), f"launch {i} (query {key}) differs"
        if i == 2:
            run_s.batch = run.batch
            got_s = run_s.decode(out_dtype=qvp.DTYPE_F32)
            assert run.batch.decode_plan()["kernel"] == "mfma"
            assert_close_bf16(got_s, ref_s, "other batch on the same batch object")


EDGE_LENGTHS = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 511, 512, 513, 1000]


@pytest.mark.parametrize("kv_dtype", [qvp.DTYPE_BF16, qvp.DTYPE_F32])
def test_ragged_lengths_across_block_and_split_edges(kv_dtype):
    print(f"case: edge lengths dtype={kv_dtype}", flush=True)
    w = W.custom(EDGE_LENGTHS, 28, 4, 128, kv_dtype=kv_dtype, seed=5)
    _parity(w, out_dtypes=(qvp.DTYPE_F32,))


@pytest.mark.parametrize("scale", [0.0, -0.05, 0.004], ids=["zero", "negative", "small-positive"])
def test_any_softmax_scale(scale):
    """The persistent kernel takes its running maximum on raw scores, which
    holds for scale > 0; a zero or negative scale (uniform weights, reversed
    order of the scores) runs on a split kernel (the GQA-folded one for this
    group of 7). Both match the oracle."""
    print(f"case: scale {scale}", flush=True)
    w = W.custom([70, 300, 513, 2000], 28, 4, 128, seed=19, scale=scale)
    run = GpuRun(w)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    assert run.batch.decode_plan()["kernel"] == ("mfma" if scale > 0 else "grouped")
    _, ref32 = oracle_decode(w, run.image, run.query)
    assert_close_bf16(got, ref32, f"scale {scale}")


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 4), (28, 4), (32, 4), (64, 4), (16, 1), (12, 2)])
def test_grouped_query_head_shapes(hq, hkv):
    print(f"case: gqa hq={hq} hkv={hkv}", flush=True)
    w = W.custom([70, 300, 513], hq, hkv, 128, seed=hq * 31 + hkv)
    _parity(w, out_dtypes=(qvp.DTYPE_F32,))


@pytest.mark.parametrize(
    "lens",
    [
        [1],                                   # one token: one tile, one piece
        [32768],                               # one long segment cut across every workgroup
        list(range(1, 301)),                   # many tiny segments: several pieces per workgroup
        [4096] * 3 + [1] * 50 + [777] * 7,     # mixed
        [1 + (i * 37) % 64 for i in range(4000)],  # dozens of pieces per range: LDS state sets reused
    ],
    ids=["single-token", "one-long", "many-tiny", "mixed", "many-short"],
)
def test_balanced_schedule_shapes(lens):
    print(f"case: schedule shape with {len(lens)} sequences", flush=True)
    w = W.custom(lens, 28, 4, 128, seed=len(lens))
    _parity(w, out_dtypes=(qvp.DTYPE_F32, qvp.DTYPE_BF16))


def test_pool_base_off_the_kib_grid_takes_equal_head_weights():
    """The schedule gives kv heads whose bytes sit at offsets 256..511 of each
    KiB more workgroups only when the pool base keeps those offsets fixed; a
    base 256 bytes off a KiB boundary takes the equal-weight path. Both
    schedules must decode to the oracle's result."""
    print("case: pool base off the KiB grid", flush=True)
    w = W.custom([700, 2000, 3100, 513, 1500, 2600], 28, 4, 128, seed=91)
    run = GpuRun(w)
    _, ref32 = oracle_decode(w, run.image, run.query)
    assert_close_bf16(run.decode(out_dtype=qvp.DTYPE_F32), ref32, "KiB-aligned pool base")

    buf = qvp.DeviceBuffer(run.image.nbytes + 2048)
    off = (256 - buf.ptr % 1024) % 1024
    assert (buf.ptr + off) % 1024 == 256
    buf.upload(run.image, offset=off)
    batch = qvp.Batch()
    batch.pack(w.ids, w.cu_blocks, w.context_lens, w.tokens_per_block, w.num_pool_blocks, w.split_tokens)
    out = qvp.DeviceBuffer(w.num_seqs * w.num_query_heads * w.head_dim * 4)
    out.fill(0xFF)
    args = qvp.decode_args(query=run.q.ptr, out=out.ptr, kv_base=buf.ptr + off, block_stride=w.block_stride,
                           batch=batch, kv_dtype=w.kv_dtype, out_dtype=qvp.DTYPE_F32, layer=w.layer,
                           num_layers=w.num_layers, num_query_heads=w.num_query_heads,
                           num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
                           tokens_per_block=w.tokens_per_block, scale=w.scale, strides=w.strides)
    qvp.paged_decode(args)
    got = out.download(np.float32, (w.num_seqs, w.num_query_heads, w.head_dim))
    assert_close_bf16(got, ref32, "pool base 256 bytes off the KiB grid")


def test_config3_subset_72b_shape():
    print("case: config3 shape, 2 sequences", flush=True)
    _parity(W.config3(num_seqs=2), out_dtypes=(qvp.DTYPE_F32,))


def test_config3_full_batch_matches_oracle():
    """The whole 72B batch (B=32, ctx U[8192, 32768], Hq 64 / Hkv 8): with
    this many tiles per resident wave the schedule decodes four kv heads side
    by side with GQA group 8 (32 rows per segment in the LDS merge, the
    deferred piece results and the final slot merge), the path its benchmark
    figure runs. Compared with the oracle on every output element, fp32 and
    bf16 outputs (tests/PagedAttention.test.cpp:460-495 at batch scale)."""
    w = W.config3()
    print(f"case: config3 full batch B={w.num_seqs} total tokens {int(w.context_lens.sum())}", flush=True)
    run = GpuRun(w, image=tiled_pool_image(w))
    ref_out, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    plan = run.batch.decode_plan()
    print(f"plan: {plan}", flush=True)
    assert plan["kernel"] == "mfma" and plan["kv_heads_per_segment"] == 4 and plan["query_group"] == 8, plan
    assert plan["slots"] > 0, plan
    assert_close_bf16(got, ref32, "config3 fp32 out")
    got16 = run.decode(out_dtype=qvp.DTYPE_BF16)
    assert_close_16bit(got16, ref32, qvp.DTYPE_BF16, "config3 bf16 out")
    assert_close_16bit(got16, to_f32(ref_out, qvp.DTYPE_BF16), qvp.DTYPE_BF16, "config3 vs oracle T out")


@pytest.mark.parametrize(
    "hq,hkv,total_tokens",
    [
        (64, 8, 300_000),    # four kv heads per segment, GQA group 8
        (28, 4, 560_000),    # four kv heads per segment, GQA group 7 (the 7B shape, long contexts)
        (42, 6, 380_000),    # two kv heads per segment, GQA group 7
        (16, 2, 1_080_000),  # two kv heads per segment, GQA group 8
    ],
    ids=["hps4-g8", "hps4-g7", "hps2-g7", "hps2-g8"],
)
def test_kv_head_groups_with_gqa_groups(hq, hkv, total_tokens):
    """kv heads side by side (>= 32 tiles per resident wave) with a GQA group
    above one: each segment carries hps x G query rows through the per-piece
    LDS merge, the deferred results and the split merge."""
    rng = np.random.default_rng(hq * 1000 + hkv)
    cuts = np.sort(rng.choice(np.arange(1, total_tokens), size=9, replace=False))
    lens = [int(x) for x in np.diff(np.concatenate([[0], cuts, [total_tokens]]))]
    lens.insert(4, 37)  # a short sequence among long ones stays one whole segment
    print(f"case: kv head groups hq={hq} hkv={hkv} lens={lens}", flush=True)
    w = W.custom(lens, hq, hkv, 128, seed=hq + hkv, spare=0.02)
    run = GpuRun(w, image=tiled_pool_image(w))
    _, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    plan = run.batch.decode_plan()
    print(f"plan: {plan}", flush=True)
    assert plan["kernel"] == "mfma" and plan["query_group"] == hq // hkv, plan
    assert plan["kv_heads_per_segment"] == (4 if hkv % 4 == 0 else 2), plan
    assert_close_bf16(got, ref32, f"kv head groups hq={hq} hkv={hkv}")


def test_one_packed_batch_decoded_with_two_query_group_sizes():
    """One pack, decoded first with 4 query heads on 4 kv heads and then with
    32 on the same 4 kv heads, without repacking: the cached work schedule
    sizes its per-piece LDS and slots by the GQA group, so the second decode
    must not reuse the first one's."""
    lens = [100, 2000, 513, 3000, 64, 1500, 2600, 700]
    results = {}
    w_small = W.custom(lens, 4, 4, 128, seed=77)
    w_big = W.custom(lens, 32, 4, 128, seed=77)
    assert np.array_equal(w_small.ids, w_big.ids)
    run = GpuRun(w_small)
    run.batch.pack(w_small.ids, w_small.cu_blocks, w_small.context_lens, 16, w_small.num_pool_blocks)
    for w in (w_small, w_big, w_small):
        print(f"case: same pack, hq={w.num_query_heads} hkv={w.num_kv_heads}", flush=True)
        q = qvp.DeviceBuffer.from_array(w.query())
        out = qvp.DeviceBuffer(w.num_seqs * w.num_query_heads * w.head_dim * 4)
        out.fill(0xFF)
        args = qvp.decode_args(query=q.ptr, out=out.ptr, kv_base=run.pool.base, block_stride=run.pool.stride,
                               batch=run.batch, kv_dtype=w.kv_dtype, out_dtype=qvp.DTYPE_F32, layer=0,
                               num_layers=1, num_query_heads=w.num_query_heads, num_kv_heads=w.num_kv_heads,
                               head_dim=128, tokens_per_block=16, scale=w.scale, strides=w.strides)
        qvp.paged_decode(args)
        got = out.download(np.float32, (w.num_seqs, w.num_query_heads, w.head_dim))
        _, ref32 = oracle_decode(w, run.image, w.query())
        results[w.num_query_heads] = assert_close_bf16(got, ref32, f"same pack hq={w.num_query_heads}")


@pytest.mark.parametrize("hkv", [16, 6])
def test_kv_heads_side_by_side_on_long_contexts(hkv):
    """With >= 32 tiles per resident wave the schedule decodes kv heads side by
    side (4 per workgroup for 16 kv heads, 2 per workgroup and two tile lanes
    each for 6): every long sequence is cut into many pieces, and a short
    sequence in the middle stays a whole segment written directly."""
    total_tokens = 65536 * 32 // hkv + 8192
    rng = np.random.default_rng(hkv)
    cuts = np.sort(rng.choice(np.arange(1, total_tokens), size=5, replace=False))
    lens = list(np.diff(np.concatenate([[0], cuts, [total_tokens]])))
    lens.insert(3, 100)
    print(f"case: head groups hkv={hkv} lens={lens}", flush=True)
    w = W.custom(lens, hkv, hkv, 128, seed=hkv, spare=0.02)
    run = GpuRun(w, image=tiled_pool_image(w))
    ref_out, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    assert_close_bf16(got, ref32, f"head groups hkv={hkv}")


def test_repeated_decodes_are_bitwise_identical():
    # Split segments are merged by whichever workgroup finishes them last; the
    # merge order is fixed, so every run must give the same bits. A visibility
    # race between workgroups (on different XCDs) would show up here.
    print("case: determinism over 25 decodes", flush=True)
    w = W.config2(seed=13, num_seqs=32)
    run = GpuRun(w)
    first = run.decode(out_dtype=qvp.DTYPE_F32)
    for i in range(24):
        again = run.decode(out_dtype=qvp.DTYPE_F32)
        assert np.array_equal(first.view(np.uint32), again.view(np.uint32)), f"run {i + 1} differs"
    _, ref32 = oracle_decode(w, run.image, run.query)
    assert_close_bf16(first, ref32, "determinism")


def test_repeated_decodes_reuse_the_cached_schedule_and_repack_invalidates_it():
    w1 = W.custom([100, 2000, 513], 28, 4, 128, seed=21)
    run = GpuRun(w1)
    _, ref1 = oracle_decode(w1, run.image, run.query)
    for _ in range(3):
        got = run.decode(out_dtype=qvp.DTYPE_F32)
        assert_close_bf16(got, ref1, "repeat")
    # Same pool, different lengths: the schedule must follow the new pack.
    w2 = W.custom([100, 2000, 513], 28, 4, 128, seed=21)
    w2.context_lens = np.array([37, 1500, 513], dtype=np.uint32)
    run.w = w2
    _, ref2 = oracle_decode(w2, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    assert_close_bf16(got, ref2, "repacked")


@pytest.mark.parametrize("d", [4, 64, 80, 256])
def test_other_head_dims_use_the_generic_kernel(d):
    print(f"case: head_dim={d}", flush=True)
    w = W.custom([9, 40, 77], 8, 2, d, seed=d)
    _parity(w, out_dtypes=(qvp.DTYPE_F32,))


@pytest.mark.parametrize("tpb", [4, 8, 32, 64])
def test_other_block_sizes(tpb):
    print(f"case: tokens_per_block={tpb}", flush=True)
    w = W.custom([5, 129, 600], 28, 4, 128, tokens_per_block=tpb, seed=tpb)
    _parity(w, out_dtypes=(qvp.DTYPE_F32,))


def test_multi_layer_frames_read_only_the_requested_layer():
    # Each layer holds different data (tests/PagedAttention.test.cpp:481-494).
    for layer in (0, 1, 2):
        print(f"case: 3-layer frames, layer {layer}", flush=True)
        w = W.custom([33, 200], 28, 4, 128, num_layers=3, layer=layer, seed=9)
        _parity(w, out_dtypes=(qvp.DTYPE_F32,))


def test_fp16_cache_folded_split_path():
    print("case: fp16 cache, head_dim 96 (GQA-folded split kernel)", flush=True)
    w = W.custom([50, 130], 8, 2, 96, kv_dtype=qvp.DTYPE_F16, seed=3)
    # fp16 pool: reinterpret the fp32 draws rounded to fp16.
    image32 = W.custom([50, 130], 8, 2, 96, kv_dtype=qvp.DTYPE_F32, seed=3)
    raw = image32.pool_image().view(np.float32)
    image = raw.astype(np.float16).view(np.uint8)
    q = image32.query().astype(np.float16).view(np.uint16)
    run = GpuRun(w, image=image, query=q)
    _, ref32 = oracle_decode(w, image, q)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    assert run.batch.decode_plan()["kernel"] == "grouped"
    assert_close_bf16(got, ref32, "fp16 cache")


def test_uniform_keys_average_the_values_on_the_mfma_path():
    # Closed form (tests/PagedAttention.test.cpp:380-411): equal keys make the
    # softmax uniform, so the output is the plain mean of the cached values.
    w = W.custom([16 * 5 + 3], 7, 1, 128, seed=1)
    image = w.pool_image()
    frames = image.reshape(w.num_pool_blocks, w.block_stride)
    ctx = int(w.context_lens[0])
    st = w.strides
    values = []
    for t in range(ctx):
        blk = int(w.ids[t // 16])
        k_off = ((t % 16) * st["token_stride"]) * 2
        v_off = (st["stream_stride"] + (t % 16) * st["token_stride"]) * 2
        frames[blk, k_off:k_off + 256] = W.f32_to_bf16_bits(np.full(128, 0.25, np.float32)).view(np.uint8)
        val = np.float32(t % 11 - 5) / np.float32(4.0)
        values.append(val)
        frames[blk, v_off:v_off + 256] = W.f32_to_bf16_bits(np.full(128, val, np.float32)).view(np.uint8)
    run = GpuRun(w, image=image)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    expected = np.float64(np.mean(values))
    assert np.abs(got - expected).max() <= 1e-5


def test_one_hot_keys_select_each_logical_token_in_order():
    # tests/PagedAttention.test.cpp:413-458 at the Qwen shape: token t's key is
    # one-hot in dim t and a sharp query picks exactly that logical token out of
    # scattered frames.
    ctx = 100
    w = W.custom([ctx], 1, 1, 128, seed=4, scale=50.0)
    image = w.pool_image()
    frames = image.reshape(w.num_pool_blocks, w.block_stride)
    st = w.strides
    for t in range(ctx):
        blk = int(w.ids[t // 16])
        k_off = ((t % 16) * st["token_stride"]) * 2
        v_off = (st["stream_stride"] + (t % 16) * st["token_stride"]) * 2
        key = np.zeros(128, np.float32)
        key[t] = 1.0
        frames[blk, k_off:k_off + 256] = W.f32_to_bf16_bits(key).view(np.uint8)
        frames[blk, v_off:v_off + 256] = W.f32_to_bf16_bits(np.full(128, t + 1, np.float32)).view(np.uint8)
    run = GpuRun(w, image=image)
    for target in (0, 15, 16, 17, 63, 64, 99):
        q = np.zeros((1, 1, 128), np.float32)
        q[0, 0, target] = 1.0
        run.q.upload(W.f32_to_bf16_bits(q))
        got = run.decode(out_dtype=qvp.DTYPE_F32)
        assert np.abs(got - (target + 1)).max() <= 1e-3 * (target + 1), f"target {target}"


# --------------------------------------------------------------------------
# Refusals: nothing is written when the call is refused
# (tests/PagedAttention.test.cpp:255-376).
# --------------------------------------------------------------------------


def _prepared(w):
    run = GpuRun(w)
    out = qvp.DeviceBuffer(w.num_seqs * w.num_query_heads * w.head_dim * 4)
    out.fill(0x7F)
    return run, out


def _args(run, out, **over):
    w = run.w
    kw = dict(query=run.q.ptr, out=out.ptr, kv_base=run.pool.base, block_stride=run.pool.stride, batch=run.batch,
              kv_dtype=w.kv_dtype, out_dtype=qvp.DTYPE_F32, layer=0, num_layers=w.num_layers,
              num_query_heads=w.num_query_heads, num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
              tokens_per_block=w.tokens_per_block, scale=w.scale)
    kw.update(over)
    return qvp.decode_args(**kw)


def _untouched(out):
    return bool(np.all(out.download(np.uint8, out.nbytes) == 0x7F))


def test_swapped_out_block_refuses_the_whole_batch_without_writing():
    w = W.custom([40, 64], 28, 4, 128, seed=2)
    run, out = _prepared(w)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks)
    ids = w.ids.copy()
    ids[4] = qvp.UNMAPPED_BLOCK  # second sequence's first block is swapped out
    with pytest.raises(qvp.QvpError) as e:
        run.batch.pack(ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks)
    assert e.value.status == qvp.ERR_UNMAPPED
    # The batch keeps its previous contents, and no decode ran.
    assert _untouched(out)


def test_pack_refuses_context_longer_than_the_mapped_blocks_and_zero_context():
    w = W.custom([40], 4, 4, 128, seed=2)
    batch = qvp.Batch()
    with pytest.raises(qvp.QvpError) as e:
        batch.pack(w.ids, w.cu_blocks, [49], 16, w.num_pool_blocks)
    assert e.value.status == qvp.ERR_INVALID_ARGUMENT
    with pytest.raises(qvp.QvpError) as e:
        batch.pack(w.ids, w.cu_blocks, [0], 16, w.num_pool_blocks)
    assert e.value.status == qvp.ERR_INVALID_ARGUMENT
    with pytest.raises(qvp.QvpError) as e:
        batch.pack(w.ids, w.cu_blocks, [40], 16, int(w.ids.max()))  # an id outside the pool
    assert e.value.status == qvp.ERR_UNMAPPED


@pytest.mark.parametrize(
    "over",
    [
        {"num_query_heads": 27},     # does not group onto 4 kv heads
        {"num_query_heads": 0},
        {"layer": 1},                # beyond the block shape
        {"head_dim": 256},           # layout would address past the frame
        {"tokens_per_block": 8},     # batch was packed for 16
        {"kv_dtype": 7},
    ],
)
def test_invalid_decode_arguments_are_refused_before_launch(over):
    w = W.custom([40, 64], 28, 4, 128, seed=2)
    run, out = _prepared(w)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks)
    with pytest.raises(qvp.QvpError) as e:
        qvp.paged_decode(_args(run, out, **over))
    assert e.value.status == qvp.ERR_INVALID_ARGUMENT
    assert _untouched(out)


def test_caller_workspace_too_small_is_refused_and_the_reported_size_works():
    w = W.custom([300, 700], 28, 4, 128, seed=8)
    run, out = _prepared(w)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks)
    small = qvp.DeviceBuffer(256)
    with pytest.raises(qvp.QvpError) as e:
        qvp.paged_decode(_args(run, out, workspace=small.ptr, workspace_bytes=small.nbytes))
    assert e.value.status == qvp.ERR_CAPACITY
    assert _untouched(out)
    # qvp_decode_workspace_bytes is an upper bound that serves either kernel.
    ws = qvp.DeviceBuffer(run.batch.workspace_bytes(28, 128))
    got = run.decode(out_dtype=qvp.DTYPE_F32, workspace=ws)
    _, ref32 = oracle_decode(w, run.image, run.query)
    assert_close_bf16(got, ref32, "caller workspace")
