"""GPU parity: ragged-batch packing, copy-on-write copies and swap
gather/scatter through the C ABI. All three are integer/byte work and must be
bit-exact (memcmp) against the oracle."""

from __future__ import annotations

import numpy as np
import pytest

import pyoracle as O
import qvp
import workloads as W

pytestmark = pytest.mark.gpu


def _byte_pattern(n: int, seed: int) -> np.ndarray:
    # (i + seed) % 251, the reference tests' byte pattern
    # (tests/MemoryAllocator.test.cpp:162-178, tests/SwapBackend.test.cpp:37-41).
    return ((np.arange(n, dtype=np.int64) + seed) % 251).astype(np.uint8)


@pytest.mark.parametrize("which", ["config1", "config2", "config3", "edge"])
def test_pack_is_bit_exact_against_the_block_tables(which):
    print(f"case: pack {which}", flush=True)
    if which == "config1":
        w = W.config1()
    elif which == "config2":
        w = W.config2()
    elif which == "config3":
        w = W.config3()
    else:
        w = W.custom([1, 16, 17, 511, 512, 513, 4097], 28, 4, 128, seed=1)
    batch = qvp.Batch()
    for split in (128, 512, 0, 8192):
        batch.pack(w.ids, w.cu_blocks, w.context_lens, w.tokens_per_block, w.num_pool_blocks, split)
        got = batch.download()
        exp = O.pack(w.ids, w.cu_blocks, w.context_lens, w.tokens_per_block, w.num_pool_blocks, split)
        for k in exp:
            assert np.array_equal(got[k], exp[k]), f"{k} split {split}"
        # Row b of the table lists the sequence's frames in logical order.
        for b in range(w.num_seqs):
            nb = (int(w.context_lens[b]) + w.tokens_per_block - 1) // w.tokens_per_block
            assert np.array_equal(got["block_tables"][b, :nb], w.ids[w.cu_blocks[b]:w.cu_blocks[b] + nb])
            assert np.all(got["block_tables"][b, nb:] == -1)


def test_pack_double_buffering_keeps_each_call_consistent():
    # Consecutive packs of different batches alternate staging buffers; each
    # download must equal its own inputs.
    batch = qvp.Batch()
    stream = qvp.Stream()
    for seed in range(6):
        w = W.custom(W.randint(seed, 5 + seed, 1, 3000), 28, 4, 128, seed=seed)
        batch.pack(w.ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks, 256, stream)
        stream.synchronize()
        got = batch.download()
        exp = O.pack(w.ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks, 256)
        for k in exp:
            assert np.array_equal(got[k], exp[k]), f"seed {seed} {k}"


@pytest.mark.parametrize("block_bytes", [32768, 16384 + 100, 917504])
def test_copy_blocks_is_memcpy_exact_and_leaves_other_frames_alone(block_bytes):
    print(f"case: copy_blocks {block_bytes}", flush=True)
    nblocks = 300 if block_bytes < 100000 else 40
    pool = qvp.BlockPool(nblocks, block_bytes)
    image = _byte_pattern(nblocks * pool.stride, 3)
    pool.upload_all(image)
    rng_src = W.permutation(17, nblocks)
    npairs = min(128, nblocks // 3)
    src = rng_src[:npairs].astype(np.uint32)
    dst = rng_src[npairs:2 * npairs].astype(np.uint32)
    qvp.copy_blocks(pool.base, pool.stride, nblocks, src, dst, block_bytes)
    got = pool.download_all()
    expected = image.copy()
    for s, d in zip(src, dst):
        O.oracle().orc_copy_block(expected.ctypes.data, pool.stride, nblocks, int(s), int(d), block_bytes)
    assert np.array_equal(got, expected)


def test_copy_blocks_more_pairs_than_one_launch_carries():
    nblocks = 1200
    pool = qvp.BlockPool(nblocks, 4096)
    image = _byte_pattern(nblocks * pool.stride, 9)
    pool.upload_all(image)
    perm = W.permutation(5, nblocks)
    src, dst = perm[:500].astype(np.uint32), perm[500:1000].astype(np.uint32)
    qvp.copy_blocks(pool.base, pool.stride, nblocks, src, dst, pool.stride)
    expected = image.reshape(nblocks, pool.stride).copy()
    expected[dst] = expected[src]
    assert np.array_equal(pool.download_all(), expected.reshape(-1))


@pytest.mark.parametrize(
    "src,dst,status",
    [
        ([1, 2], [3, 3], qvp.ERR_INVALID_ARGUMENT),   # repeated destination
        ([1, 2], [2, 4], qvp.ERR_INVALID_ARGUMENT),   # destination is another pair's source
        ([1, 99], [3, 4], qvp.ERR_UNMAPPED),          # source outside the pool
        ([1, 2], [3, 50], qvp.ERR_UNMAPPED),          # destination outside the pool
    ],
)
def test_copy_blocks_refusals_write_nothing(src, dst, status):
    pool = qvp.BlockPool(50, 1024)
    image = _byte_pattern(50 * pool.stride, 1)
    pool.upload_all(image)
    with pytest.raises(qvp.QvpError) as e:
        qvp.copy_blocks(pool.base, pool.stride, 50, src, dst, 1024)
    assert e.value.status == status
    assert np.array_equal(pool.download_all(), image)


def test_copy_blocks_self_pair_is_a_no_op():
    pool = qvp.BlockPool(8, 1024)
    image = _byte_pattern(8 * pool.stride, 2)
    pool.upload_all(image)
    qvp.copy_blocks(pool.base, pool.stride, 8, [3], [3], 1024)
    assert np.array_equal(pool.download_all(), image)


@pytest.mark.parametrize("count", [1, 37, 128, 300])
def test_swap_round_trip_is_bit_exact(count):
    print(f"case: swap round trip {count}", flush=True)
    nblocks = 400
    block_bytes = 32768
    pool = qvp.BlockPool(nblocks, block_bytes)
    image = _byte_pattern(nblocks * pool.stride, 7)
    pool.upload_all(image)
    frames = W.permutation(23, nblocks)[:count].astype(np.uint32)
    arena = qvp.PinnedBuffer(count * block_bytes + 4096)
    arena.array[:] = 0
    offsets = (W.permutation(29, count) * block_bytes).astype(np.uint64)
    side = qvp.Stream()
    qvp.swap_gather(pool.base, pool.stride, nblocks, frames, offsets, arena, block_bytes, side)
    side.synchronize()
    frames2d = image.reshape(nblocks, pool.stride)
    for f, o in zip(frames, offsets):
        assert np.array_equal(arena.array[int(o):int(o) + block_bytes], frames2d[f, :block_bytes]), f"gather {f}"
    # Scatter into different frames (swap-in lands in a fresh frame).
    targets = W.permutation(31, nblocks)[:count].astype(np.uint32)
    pool.upload_all(np.zeros_like(image))
    qvp.swap_scatter(pool.base, pool.stride, nblocks, targets, offsets, arena, block_bytes, side)
    side.synchronize()
    got = pool.download_all().reshape(nblocks, pool.stride)
    expected = np.zeros_like(frames2d)
    for f, t in zip(frames, targets):
        expected[t, :block_bytes] = frames2d[f, :block_bytes]
    assert np.array_equal(got, expected)


def test_swap_refusals():
    pool = qvp.BlockPool(10, 4096)
    arena = qvp.PinnedBuffer(4 * 4096)
    with pytest.raises(qvp.QvpError) as e:  # overlapping arena ranges
        qvp.swap_gather(pool.base, pool.stride, 10, [1, 2], [0, 2048], arena, 4096)
    assert e.value.status == qvp.ERR_INVALID_ARGUMENT
    with pytest.raises(qvp.QvpError) as e:  # past the arena
        qvp.swap_gather(pool.base, pool.stride, 10, [1], [4 * 4096 - 16], arena, 4096)
    assert e.value.status == qvp.ERR_CAPACITY
    with pytest.raises(qvp.QvpError) as e:  # frame outside the pool
        qvp.swap_scatter(pool.base, pool.stride, 10, [10], [0], arena, 4096)
    assert e.value.status == qvp.ERR_UNMAPPED
    with pytest.raises(qvp.QvpError) as e:  # repeated destination frame
        qvp.swap_scatter(pool.base, pool.stride, 10, [3, 3], [0, 4096], arena, 4096)
    assert e.value.status == qvp.ERR_INVALID_ARGUMENT
