"""GPU parity: causal paged prefill (qvp_paged_prefill) through the C ABI.

The reference defines prefill as paged_attention_decode<T> applied per prompt
position p with context_len = p + 1 (include/qwenvl_paged/PagedAttention.h:43-44,
tests/EndToEnd.test.cpp:252-256). The expected output of every new position is
therefore the oracle's decode of that position (oracle/oracle.c, bit-equal to
the compiled reference in tests/test_oracle.py), run here as one virtual
sequence per position over the same frames. Tolerances are the decode's.
"""

from __future__ import annotations

import numpy as np
import pytest

import pyoracle as O
import qvp
import workloads as W
from helpers import GpuRun, assert_close_16bit, assert_close_bf16, oracle_dtype, to_f32

pytestmark = pytest.mark.gpu


def _oracle_prefill(w: W.Workload, image: np.ndarray, queries: np.ndarray, q_start):
    ids, cu, ctx = [], [0], []
    for b in range(w.num_seqs):
        row = w.ids[w.cu_blocks[b]:w.cu_blocks[b + 1]]
        for p in range(int(q_start[b]), int(w.context_lens[b])):
            nb = (p + w.tokens_per_block) // w.tokens_per_block
            ids.extend(row[:nb])
            cu.append(len(ids))
            ctx.append(p + 1)
    refused, out, out32 = O.decode_batch(image, w.block_stride, w.num_pool_blocks, np.array(ids, np.uint32),
                                         np.array(cu, np.uint32), np.array(ctx, np.uint32),
                                         oracle_dtype(w.kv_dtype), queries, w.layer, w.num_layers,
                                         w.num_query_heads, w.num_kv_heads, w.head_dim, w.tokens_per_block,
                                         w.scale, threads=min(O.host_threads(), 8))
    assert refused == 0
    return out, out32


def _queries(w: W.Workload, total: int, seed: int) -> np.ndarray:
    q = np.random.default_rng(seed).normal(0.0, 1.0, (total, w.num_query_heads, w.head_dim)).astype(np.float32)
    return q if w.kv_dtype == qvp.DTYPE_F32 else W.f32_to_bf16_bits(q)


def _run(w: W.Workload, q_start, out_dtype: int, seed: int = 1, image=None, queries=None, out_offset: int = 0):
    run = GpuRun(w, image=image)
    q_start = np.asarray(q_start, np.uint32)
    total = int((w.context_lens.astype(np.int64) - q_start).sum())
    if queries is None:
        queries = _queries(w, total, seed)
    dq = qvp.DeviceBuffer.from_array(queries)
    n = total * w.num_query_heads * w.head_dim
    nbytes = n * qvp.DTYPE_BYTES[out_dtype]
    # out_offset > 0: the output starts that many bytes into a larger buffer
    # whose other bytes must stay 0xFF.
    out = qvp.DeviceBuffer(nbytes + (2 * out_offset if out_offset else 0))
    out.fill(0xFF)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, w.tokens_per_block, w.num_pool_blocks, w.split_tokens)
    args = qvp.prefill_args(query=dq.ptr, out=out.ptr + out_offset, kv_base=run.pool.base,
                            block_stride=run.pool.stride, batch=run.batch, q_start=q_start, kv_dtype=w.kv_dtype,
                            out_dtype=out_dtype, layer=w.layer, num_layers=w.num_layers,
                            num_query_heads=w.num_query_heads, num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
                            tokens_per_block=w.tokens_per_block, scale=w.scale, strides=w.strides)
    qvp.paged_prefill(args)
    np_dtype = np.float32 if out_dtype == qvp.DTYPE_F32 else np.uint16
    if out_offset:
        raw = out.download(np.uint8, (out.nbytes,))
        assert (raw[:out_offset] == 0xFF).all() and (raw[out_offset + nbytes:] == 0xFF).all(), \
            "bytes outside the output were written"
        got = raw[out_offset:out_offset + nbytes].copy().view(np_dtype).reshape(total, w.num_query_heads, w.head_dim)
    else:
        got = out.download(np_dtype, (total, w.num_query_heads, w.head_dim))
    ref_out, ref32 = _oracle_prefill(w, run.image, queries, q_start)
    return got, ref_out, ref32, (run, args, out, dq)


def _check(w, got, ref_out, ref32, out_dtype, what):
    if w.kv_dtype == qvp.DTYPE_F32 and out_dtype == qvp.DTYPE_F32:
        err = float(np.abs(got - ref32).max())
        assert err <= 1e-5, f"{what}: fp32 max abs {err:.3e}"
    elif out_dtype == qvp.DTYPE_F32:
        assert_close_bf16(got, ref32, what)
    else:
        assert_close_16bit(got, ref32, out_dtype, what)
        if out_dtype == w.kv_dtype:
            assert_close_16bit(got, to_f32(ref_out, out_dtype), out_dtype, what + " vs oracle T out")


CASES = [
    # name, context lens, first new positions, Hq, Hkv
    ("7B full, chunked and one-token prefill", [37, 300, 1030, 17], [0, 100, 1000, 16], 28, 4),
    ("72B shape, group 8", [64, 513], [0, 200], 64, 8),
    ("group 16", [129, 40], [0, 7], 16, 1),
    ("group 12: two head sets", [90, 33], [5, 0], 12, 1),
    ("multi-head groups of 1", [70], [0], 4, 4),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("out_dtype", [qvp.DTYPE_F32, qvp.DTYPE_BF16])
def test_prefill_matches_the_decode_of_every_position(case, out_dtype):
    name, lens, q_start, hq, hkv = case
    print(f"case: prefill {name} out={out_dtype}", flush=True)
    w = W.custom(lens, hq, hkv, 128, seed=len(lens) + hq)
    got, ref_out, ref32, _ = _run(w, q_start, out_dtype)
    _check(w, got, ref_out, ref32, out_dtype, name)


def test_prefill_of_a_1024_token_prompt():
    print("case: prefill 1024-token prompt, 7B shape", flush=True)
    w = W.custom([1024, 700], 28, 4, 128, seed=3)
    got, ref_out, ref32, _ = _run(w, [0, 0], qvp.DTYPE_F32)
    _check(w, got, ref_out, ref32, qvp.DTYPE_F32, "1024-token prefill")


@pytest.mark.parametrize("out_dtype", [qvp.DTYPE_F32, qvp.DTYPE_BF16])
def test_scores_far_above_the_first_tile_move_the_running_maximum(out_dtype):
    # The MFMA prefill's running maximum moves lazily: only when a tile's
    # maximum exceeds it by more than 2^8 in weight, and O and l are then
    # rescaled. Here every query shares a direction (entries 1 + N(0, 0.3^2))
    # and one token per sequence has K = 3.0 along it: its score is ~384
    # (scaled: ~49 in log2 units) against ~15 at most in the first tile, so
    # every position from that token on moves its maximum by far more than the
    # lazy threshold and rescales O by ~2^-47. Every row must equal the oracle.
    print(f"case: prefill, scores far above the first tile, out={out_dtype}", flush=True)
    w = W.custom([300, 130], 28, 4, 128, seed=21)
    image = w.pool_image()
    st = w.strides
    bright = W.f32_to_bf16_bits(np.full(128, 3.0, np.float32)).view(np.uint8)
    for b, tok in ((0, 200), (1, 100)):
        blk = int(w.ids[w.cu_blocks[b] + tok // w.tokens_per_block])
        for g in range(w.num_kv_heads):
            off = blk * w.block_stride + 2 * ((tok % w.tokens_per_block) * st["token_stride"] + g * st["head_stride"])
            image[off:off + 256] = bright
    total = int(w.context_lens.sum())
    rng = np.random.default_rng(22)
    queries = W.f32_to_bf16_bits((1.0 + rng.normal(0.0, 0.3, (total, 28, 128))).astype(np.float32))
    got, ref_out, ref32, _ = _run(w, [0, 0], out_dtype, image=image, queries=queries)
    _check(w, got, ref_out, ref32, out_dtype, "scores far above the first tile")


@pytest.mark.parametrize("shape", [(8, 2, 64, qvp.DTYPE_F32), (8, 2, 128, qvp.DTYPE_F32), (4, 2, 80, qvp.DTYPE_BF16)])
def test_other_shapes_use_the_decode_path(shape):
    hq, hkv, d, dtype = shape
    print(f"case: prefill fallback hq={hq} hkv={hkv} d={d} dtype={dtype}", flush=True)
    w = W.custom([37, 128, 250], hq, hkv, d, kv_dtype=dtype, seed=d)
    got, ref_out, ref32, _ = _run(w, [0, 64, 249], qvp.DTYPE_F32)
    _check(w, got, ref_out, ref32, qvp.DTYPE_F32, f"fallback {shape}")


@pytest.mark.parametrize("out_dtype", [qvp.DTYPE_F32, qvp.DTYPE_BF16])
def test_output_off_a_16_byte_boundary_takes_the_decode_path(out_dtype):
    # The tile kernel stores each lane's outputs as 16-byte (fp32) or 8-byte
    # (bf16) vectors; an output pointer 4 bytes past a 16-byte boundary goes to
    # the decode-kernel path, which must write the same rows and nothing else.
    print(f"case: prefill with out 4 bytes off alignment, out={out_dtype}", flush=True)
    w = W.custom([37, 300], 28, 4, 128, seed=4)
    got, ref_out, ref32, _ = _run(w, [0, 100], out_dtype, out_offset=4)
    _check(w, got, ref_out, ref32, out_dtype, "unaligned output")


def test_decode_path_runs_long_prompts_in_chunks():
    # The decode-kernel path packs one virtual sequence per position, at most
    # 2^20 block ids per pack: a 6000-token prompt (about 1.1M ids) and a
    # second sequence starting at position 1000 take two chunks, the second
    # starting mid-sequence, and every row must land in its own place.
    print("case: prefill decode path, chunked virtual batches", flush=True)
    w = W.custom([6000, 3000], 4, 2, 64, kv_dtype=qvp.DTYPE_F32, seed=12)
    got, ref_out, ref32, _ = _run(w, [0, 1000], qvp.DTYPE_F32)
    _check(w, got, ref_out, ref32, qvp.DTYPE_F32, "chunked decode path")


def test_refused_prefill_writes_nothing():
    print("case: prefill refusals", flush=True)
    w = W.custom([40, 20], 28, 4, 128, seed=9)
    got, ref_out, ref32, (run, args, out, dq) = _run(w, [0, 0], qvp.DTYPE_BF16)
    out.fill(0x5A)
    qvp.synchronize()
    before = out.download(np.uint8, (out.nbytes,))
    for bad_start in ([40, 0], [0, 25]):
        a2 = qvp.prefill_args(query=dq.ptr, out=out.ptr, kv_base=run.pool.base, block_stride=run.pool.stride,
                              batch=run.batch, q_start=bad_start, kv_dtype=w.kv_dtype, out_dtype=qvp.DTYPE_BF16,
                              layer=0, num_layers=1, num_query_heads=28, num_kv_heads=4, head_dim=128,
                              tokens_per_block=16, scale=w.scale)
        with pytest.raises(qvp.QvpError) as e:
            qvp.paged_prefill(a2)
        assert e.value.status == qvp.ERR_INVALID_ARGUMENT
    for field, value in (("layer", 1), ("num_query_heads", 30), ("block_stride", 1024)):
        a2 = qvp.prefill_args(query=dq.ptr, out=out.ptr, kv_base=run.pool.base, block_stride=run.pool.stride,
                              batch=run.batch, q_start=[0, 0], kv_dtype=w.kv_dtype, out_dtype=qvp.DTYPE_BF16,
                              layer=0, num_layers=1, num_query_heads=28, num_kv_heads=4, head_dim=128,
                              tokens_per_block=16, scale=w.scale)
        setattr(a2, field, value)
        with pytest.raises(qvp.QvpError):
            qvp.paged_prefill(a2)
    qvp.synchronize()
    assert np.array_equal(out.download(np.uint8, (out.nbytes,)), before)
