"""GPU parity: K/V append (qvp_append_kv) through the C ABI.

The writes of one step, as the reference's harnesses make them after
KVCacheManager::ensure_token_writable (tests/PagedAttention.test.cpp:97-127,
tests/EndToEnd.test.cpp:157-179), are byte work and must be bit-exact: the whole
pool image after the launch equals the oracle's image (oracle/oracle.c
orc_append_kv, itself checked against the layout's closed-form offsets in
tests/test_oracle.py). A decode after the append then sees the new tokens.
"""

from __future__ import annotations

import numpy as np
import pytest

import pyoracle as O
import qvp
import workloads as W
from helpers import GpuRun, assert_close_bf16, oracle_decode

pytestmark = pytest.mark.gpu

DTYPE_BYTES = {qvp.DTYPE_F32: 4, qvp.DTYPE_BF16: 2, qvp.DTYPE_F16: 2}


def _run(tpb, layers, hkv, d, dtype, first_layer, layer_count, tokens, nframes, seed, strides=None,
         stride_pad=0):
    bpe = DTYPE_BYTES[dtype]
    rng = np.random.default_rng(seed)
    block_bytes = tpb * layers * hkv * d * bpe * 2 + stride_pad
    pool = qvp.BlockPool(nframes, block_bytes)
    image = rng.integers(0, 256, nframes * pool.stride, dtype=np.uint8)
    pool.upload_all(image)
    pairs = rng.choice(nframes * tpb, size=tokens, replace=False)
    frames, slots = (pairs // tpb).astype(np.uint32), (pairs % tpb).astype(np.uint32)
    nbytes = tokens * layer_count * hkv * d * bpe
    k = rng.integers(0, 256, nbytes, dtype=np.uint8)
    v = rng.integers(0, 256, nbytes, dtype=np.uint8)
    dk, dv = qvp.DeviceBuffer.from_array(k), qvp.DeviceBuffer.from_array(v)
    args = qvp.append_args(kv_base=pool.base, block_stride=pool.stride, num_blocks=nframes, kv_dtype=dtype,
                           num_layers=layers, first_layer=first_layer, layer_count=layer_count, num_kv_heads=hkv,
                           head_dim=d, tokens_per_block=tpb, k=dk.ptr, v=dv.ptr, strides=strides)
    qvp.append_kv(args, frames, slots)
    qvp.synchronize()
    got = pool.download_all()
    exp = image.copy()
    assert O.append_kv(exp, pool.stride, nframes, bpe, tpb, layers, hkv, d, first_layer, layer_count, frames,
                       slots, k, v) == 0
    return got, exp, (pool, image, args, frames, slots, dk, dv)


CASES = [
    # tpb, layers, hkv, d, dtype, first_layer, layer_count, tokens, frames
    (16, 1, 2, 64, qvp.DTYPE_F32, 0, 1, 4, 8),           # config1 shape
    (16, 1, 4, 128, qvp.DTYPE_BF16, 0, 1, 64, 200),      # config2 shape, one step of B=64
    (16, 1, 8, 128, qvp.DTYPE_BF16, 0, 1, 32, 100),      # config3 shape
    (16, 28, 4, 128, qvp.DTYPE_BF16, 0, 28, 16, 24),     # all 28 layers of a Qwen2-VL-7B frame
    (16, 28, 4, 128, qvp.DTYPE_BF16, 5, 3, 16, 24),      # a layer range
    (16, 1, 4, 128, qvp.DTYPE_BF16, 0, 1, 128, 20),      # offsets in the kernel arguments, at the limit
    (16, 1, 4, 128, qvp.DTYPE_BF16, 0, 1, 129, 20),      # one past: offsets uploaded to the device
    (16, 1, 4, 128, qvp.DTYPE_F16, 0, 1, 300, 40),       # uploaded offsets
    (16, 1, 4, 128, qvp.DTYPE_BF16, 0, 1, 6000, 400),    # a prompt's rows in one launch
    (16, 28, 4, 128, qvp.DTYPE_BF16, 0, 28, 700, 50),    # a prompt's rows, all 28 layers
    (8, 2, 3, 4, qvp.DTYPE_F16, 1, 1, 9, 5),             # 8-byte rows: the byte-copy path
    (8, 2, 3, 4, qvp.DTYPE_F16, 0, 2, 200, 40),          # byte-copy path with uploaded offsets
    (4, 3, 1, 5, qvp.DTYPE_F32, 0, 3, 7, 3),             # odd head_dim
]


@pytest.mark.parametrize("case", CASES)
def test_append_is_bit_exact_against_the_oracle(case):
    print(f"case: append {case}", flush=True)
    got, exp, _ = _run(*case, seed=sum(case))
    assert np.array_equal(got, exp)


def test_append_with_padded_frame_stride():
    # A frame stride above the layout's size (alignment padding) leaves the
    # padding alone.
    print("case: append padded stride", flush=True)
    got, exp, _ = _run(16, 1, 4, 128, qvp.DTYPE_BF16, 0, 1, 20, 30, seed=3, stride_pad=256 + 32)
    assert np.array_equal(got, exp)


def test_back_to_back_uploaded_appends_keep_their_offsets():
    # Calls of the uploaded-offset path enqueued without waiting in between
    # (growing staging, reusing both staging slots, the kernel-argument path
    # between them) each write their own rows.
    print("case: append back to back", flush=True)
    tpb, layers, hkv, d = 16, 1, 4, 128
    nframes = 600
    rng = np.random.default_rng(11)
    pool = qvp.BlockPool(nframes, tpb * layers * hkv * d * 2 * 2)
    image = rng.integers(0, 256, nframes * pool.stride, dtype=np.uint8)
    pool.upload_all(image)
    stream = qvp.Stream()
    exp = image.copy()
    pairs = rng.permutation(nframes * tpb)
    used = 0
    keep = []
    for count in (200, 5000, 40, 300, 9000, 129):
        sel = pairs[used:used + count]
        used += count
        frames, slots = (sel // tpb).astype(np.uint32), (sel % tpb).astype(np.uint32)
        k = rng.integers(0, 256, count * hkv * d * 2, dtype=np.uint8)
        v = rng.integers(0, 256, count * hkv * d * 2, dtype=np.uint8)
        dk, dv = qvp.DeviceBuffer.from_array(k), qvp.DeviceBuffer.from_array(v)
        keep.append((dk, dv))
        args = qvp.append_args(kv_base=pool.base, block_stride=pool.stride, num_blocks=nframes,
                               kv_dtype=qvp.DTYPE_BF16, num_layers=layers, first_layer=0, layer_count=layers,
                               num_kv_heads=hkv, head_dim=d, tokens_per_block=tpb, k=dk.ptr, v=dv.ptr)
        qvp.append_kv(args, frames, slots, stream)
        # The host arrays may be reused at once: the call staged the offsets.
        frames[:] = 0
        slots[:] = 0
        assert O.append_kv(exp, pool.stride, nframes, 2, tpb, layers, hkv, d, 0, layers,
                           (sel // tpb).astype(np.uint32), (sel % tpb).astype(np.uint32), k, v) == 0
    stream.synchronize()
    assert np.array_equal(pool.download_all(), exp)


def test_refused_appends_write_nothing():
    print("case: append refusals", flush=True)
    got, exp, (pool, image, args, frames, slots, dk, dv) = _run(16, 2, 4, 128, qvp.DTYPE_BF16, 0, 2, 10, 12,
                                                                  seed=9)
    assert np.array_equal(got, exp)
    pool.upload_all(image)
    bad = [
        (np.r_[frames[:-1], 12], slots, qvp.ERR_UNMAPPED),                 # frame outside the pool
        (frames, np.r_[slots[:-1], 16], qvp.ERR_INVALID_ARGUMENT),         # slot past the block
        (np.r_[frames, frames[0]], np.r_[slots, slots[0]], qvp.ERR_INVALID_ARGUMENT),  # pair twice
    ]
    for f, s, status in bad:
        with pytest.raises(qvp.QvpError) as e:
            qvp.append_kv(args, f, s)
        assert e.value.status == status
    for field, value in (("first_layer", 1), ("layer_count", 0), ("kv_dtype", 7), ("head_stride", 64),
                         ("block_stride", args.block_stride - 16)):
        a2 = qvp.append_args(kv_base=args.kv_base, block_stride=args.block_stride, num_blocks=args.num_blocks,
                             kv_dtype=args.kv_dtype, num_layers=args.num_layers, first_layer=args.first_layer,
                             layer_count=args.layer_count, num_kv_heads=args.num_kv_heads, head_dim=args.head_dim,
                             tokens_per_block=args.tokens_per_block, k=args.k, v=args.v)
        setattr(a2, field, value)
        with pytest.raises(qvp.QvpError) as e:
            qvp.append_kv(a2, frames, slots)
        assert e.value.status == qvp.ERR_INVALID_ARGUMENT, field
    qvp.synchronize()
    assert np.array_equal(pool.download_all(), image)


def test_decode_after_append_sees_the_new_tokens():
    """One engine step: append token ctx_b of every sequence, then decode with
    context ctx_b + 1; the result equals the oracle decode of the updated pool."""
    print("case: append then decode", flush=True)
    w = W.config2(seed=21, num_seqs=16)
    run = GpuRun(w)
    rng = np.random.default_rng(5)
    tpb = w.tokens_per_block
    new_lens = w.context_lens.astype(np.int64) + 1
    # Sequences whose next token starts a new block get one of the pool's
    # unused frames.
    ids = []
    cu = [0]
    unused = sorted(set(range(w.num_pool_blocks)) - set(int(x) for x in w.ids))
    frames, slots = [], []
    for b in range(w.num_seqs):
        row = [int(x) for x in w.ids[w.cu_blocks[b]:w.cu_blocks[b + 1]]]
        pos = int(w.context_lens[b])
        if pos // tpb >= len(row):
            row.append(unused.pop())
        frames.append(row[pos // tpb])
        slots.append(pos % tpb)
        ids += row
        cu.append(len(ids))
    hkv, d = w.num_kv_heads, w.head_dim
    k = W.f32_to_bf16_bits(rng.normal(0, 0.5, (w.num_seqs, 1, hkv, d)).astype(np.float32))
    v = W.f32_to_bf16_bits(rng.normal(0, 0.5, (w.num_seqs, 1, hkv, d)).astype(np.float32))
    dk, dv = qvp.DeviceBuffer.from_array(k), qvp.DeviceBuffer.from_array(v)
    args = qvp.append_args(kv_base=run.pool.base, block_stride=run.pool.stride, num_blocks=w.num_pool_blocks,
                           kv_dtype=w.kv_dtype, num_layers=w.num_layers, first_layer=w.layer, layer_count=1,
                           num_kv_heads=hkv, head_dim=d, tokens_per_block=tpb, k=dk.ptr, v=dv.ptr)
    qvp.append_kv(args, np.array(frames, np.uint32), np.array(slots, np.uint32))
    image = run.image.copy()
    assert O.append_kv(image, run.pool.stride, w.num_pool_blocks, 2, tpb, w.num_layers, hkv, d, w.layer, 1,
                       np.array(frames, np.uint32), np.array(slots, np.uint32), k, v) == 0
    qvp.synchronize()
    assert np.array_equal(run.pool.download_all(), image)
    w2 = W.Workload(**{**w.__dict__, "ids": np.array(ids, np.uint32), "cu_blocks": np.array(cu, np.uint32),
                       "context_lens": new_lens.astype(np.uint32)})
    run.w = w2
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    _, ref32 = oracle_decode(w2, image, run.query)
    assert_close_bf16(got, ref32, "decode after append")
