"""GPU: the path under HIP graph capture (qvp_graph_*).

A decode step (MFMA and generic paths) and a step's block work (K/V append
plus copy-on-write copies) are captured once and replayed several times, with
eager work of the program between the replays; every replay must give the
eager result bit for bit. The decode kernel resets its own merge counters, so
replays need no memset nodes (none is recorded)."""

from __future__ import annotations

import numpy as np
import pytest

import pyoracle as O
import qvp
import workloads as W
from helpers import GpuRun

pytestmark = pytest.mark.gpu


def _decode_args(run: GpuRun, out: qvp.DeviceBuffer, ws: qvp.DeviceBuffer, od: int):
    w = run.w
    return qvp.decode_args(query=run.q.ptr, out=out.ptr, kv_base=run.pool.base, block_stride=run.pool.stride,
                           batch=run.batch, kv_dtype=w.kv_dtype, out_dtype=od, layer=w.layer,
                           num_layers=w.num_layers, num_query_heads=w.num_query_heads,
                           num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, tokens_per_block=w.tokens_per_block,
                           scale=w.scale, strides=w.strides, workspace=ws.ptr, workspace_bytes=ws.nbytes)


@pytest.mark.parametrize("shape", ["mfma", "generic"])
def test_captured_decode_replays_match_eager_decodes(shape):
    print(f"case: graph decode {shape}", flush=True)
    if shape == "mfma":
        w = W.custom([300, 2000, 513, 77, 1], 28, 4, 128, seed=31)
        od = qvp.DTYPE_BF16
        other = W.custom([700, 90], 28, 4, 128, seed=32)
    else:
        w = W.config1()
        od = qvp.DTYPE_F32
        other = W.custom([40, 9], 8, 2, 64, kv_dtype=qvp.DTYPE_F32, seed=33)
    stream = qvp.Stream()
    run = GpuRun(w)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, w.tokens_per_block, w.num_pool_blocks, w.split_tokens, stream)
    ws = qvp.DeviceBuffer(max(run.batch.workspace_bytes(w.num_query_heads, w.head_dim), 256))
    n = w.num_seqs * w.num_query_heads * w.head_dim
    out = qvp.DeviceBuffer(n * qvp.DTYPE_BYTES[od])
    args = _decode_args(run, out, ws, od)
    np_dtype = np.float32 if od == qvp.DTYPE_F32 else np.uint16
    # Eager decode first: it caches the schedule, so the captured call
    # enqueues kernels only.
    qvp.paged_decode(args, stream)
    eager = out.download(np_dtype, (n,), stream)
    with qvp.Graph.capture(stream) as graph:
        qvp.paged_decode(args, stream)
    other_run = GpuRun(other)
    for replay in range(4):
        out.fill(0xFF, stream)
        graph.launch(stream)
        stream.synchronize()
        got = out.download(np_dtype, (n,), stream)
        assert np.array_equal(got, eager), f"replay {replay}"
        # Eager work of the program between replays (another batch's decode).
        other_run.decode(stream=stream)
    # The graph reads the buffers it was captured with: a new query there
    # gives the new query's decode.
    rng = np.random.default_rng(7)
    new_q = rng.normal(0, 1, run.query.shape).astype(np.float32)
    if w.kv_dtype != qvp.DTYPE_F32:
        new_q = W.f32_to_bf16_bits(new_q)
    run.q.upload(new_q, stream)
    graph.launch(stream)
    stream.synchronize()
    replayed = out.download(np_dtype, (n,), stream)
    qvp.paged_decode(args, stream)
    assert np.array_equal(replayed, out.download(np_dtype, (n,), stream))
    assert not np.array_equal(replayed, eager)
    graph.destroy()


def test_captured_append_and_copies_replay_like_eager_calls():
    print("case: graph append + copy_blocks", flush=True)
    tpb, layers, hkv, d = 16, 2, 4, 128
    strides = qvp.layout_strides(tpb, layers, hkv, d)
    block_bytes = 2 * layers * tpb * hkv * d * 2
    nblocks = 64
    rng = np.random.default_rng(5)
    image = rng.integers(0, 256, nblocks * block_bytes, dtype=np.uint8)
    count = 24
    frames = rng.choice(nblocks // 2, count, replace=False).astype(np.uint32)
    slots = rng.integers(0, tpb, count).astype(np.uint32)
    rows = rng.integers(0, 256, count * layers * hkv * d * 2, dtype=np.uint8)
    dk = qvp.DeviceBuffer.from_array(rows)
    dv = qvp.DeviceBuffer.from_array(rows[::-1].copy())
    src = np.arange(0, 20, dtype=np.uint32)
    dst = np.arange(40, 60, dtype=np.uint32)
    stream = qvp.Stream()

    def fresh_pool():
        pool = qvp.BlockPool(nblocks, block_bytes)
        pool.upload_all(image)
        return pool

    def enqueue(pool):
        a = qvp.append_args(kv_base=pool.base, block_stride=pool.stride, num_blocks=nblocks, kv_dtype=qvp.DTYPE_BF16,
                            num_layers=layers, first_layer=0, layer_count=layers, num_kv_heads=hkv, head_dim=d,
                            tokens_per_block=tpb, k=dk.ptr, v=dv.ptr, strides=strides)
        qvp.append_kv(a, frames, slots, stream)
        qvp.copy_blocks(pool.base, pool.stride, nblocks, src, dst, block_bytes, stream)

    eager_pool = fresh_pool()
    enqueue(eager_pool)
    stream.synchronize()
    eager = eager_pool.download_all()
    # The expected bytes also follow from the oracle: append, then copy.
    expected = image.copy()
    assert O.append_kv(expected, block_bytes, nblocks, 2, tpb, layers, hkv, d, 0, layers, frames, slots,
                       rows, rows[::-1].copy()) == 0
    exp2 = expected.reshape(nblocks, block_bytes)
    exp2[dst] = exp2[src]
    assert np.array_equal(eager, expected)

    pool = fresh_pool()
    with qvp.Graph.capture(stream) as graph:
        enqueue(pool)
    for replay in range(3):
        pool.upload_all(image)
        graph.launch(stream)
        stream.synchronize()
        assert np.array_equal(pool.download_all(), expected), f"replay {replay}"
    graph.destroy()


def test_capture_needs_a_created_stream():
    with pytest.raises(qvp.QvpError):
        with qvp.Graph.capture(None):
            pass


def test_capture_neither_carries_nor_replays_a_pending_pack_ahead_upload():
    """A decode captured while another batch's qvp_pack_ahead upload is
    pending on the stream does not take it into the graph (replays would copy
    whatever the staging holds then): the upload stays pending and the other
    batch's own decode enqueues it. A decode of a batch whose own upload is
    pending is refused under capture."""
    w = W.custom([300, 2000, 513, 77, 1], 28, 4, 128, seed=31)
    stream = qvp.Stream()
    run = GpuRun(w)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, w.tokens_per_block, w.num_pool_blocks, 0, stream)
    ws = qvp.DeviceBuffer(max(run.batch.workspace_bytes(w.num_query_heads, w.head_dim), 256))
    n = w.num_seqs * w.num_query_heads * w.head_dim
    out = qvp.DeviceBuffer(n * 2)
    args = _decode_args(run, out, ws, qvp.DTYPE_BF16)
    qvp.paged_decode(args, stream)
    eager = out.download(np.uint16, (n,), stream)

    other = qvp.Batch()
    lens = np.maximum(w.context_lens.astype(np.int64) - 50, 1).astype(np.uint32)
    out2 = qvp.DeviceBuffer(n * 2)
    args2 = qvp.decode_args(query=run.q.ptr, out=out2.ptr, kv_base=run.pool.base, block_stride=run.pool.stride,
                            batch=other, kv_dtype=w.kv_dtype, out_dtype=qvp.DTYPE_BF16, layer=w.layer,
                            num_layers=w.num_layers, num_query_heads=w.num_query_heads,
                            num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, tokens_per_block=w.tokens_per_block,
                            scale=w.scale, strides=w.strides)
    other.pack(w.ids, w.cu_blocks, lens, w.tokens_per_block, w.num_pool_blocks, 0, stream, decode=args2, ahead=True)
    print("case: capture beside a pending upload", flush=True)
    with qvp.Graph.capture(stream) as graph:
        qvp.paged_decode(args, stream)
    for replay in range(3):
        out.fill(0xFF, stream)
        graph.launch(stream)
        stream.synchronize()
        assert np.array_equal(out.download(np.uint16, (n,), stream), eager), f"replay {replay}"
    graph.destroy()
    # Still pending: the other batch's own decode uploads it first.
    qvp.paged_decode(args2, stream)
    got2 = out2.download(np.uint16, (n,), stream)
    fresh = qvp.Batch()
    out3 = qvp.DeviceBuffer(n * 2)
    args3 = qvp.decode_args(query=run.q.ptr, out=out3.ptr, kv_base=run.pool.base, block_stride=run.pool.stride,
                            batch=fresh, kv_dtype=w.kv_dtype, out_dtype=qvp.DTYPE_BF16, layer=w.layer,
                            num_layers=w.num_layers, num_query_heads=w.num_query_heads,
                            num_kv_heads=w.num_kv_heads, head_dim=w.head_dim, tokens_per_block=w.tokens_per_block,
                            scale=w.scale, strides=w.strides)
    fresh.pack(w.ids, w.cu_blocks, lens, w.tokens_per_block, w.num_pool_blocks, 0, stream, decode=args3)
    qvp.paged_decode(args3, stream)
    assert np.array_equal(got2, out3.download(np.uint16, (n,), stream))

    print("case: capture of a batch with its own upload pending is refused", flush=True)
    other.pack(w.ids, w.cu_blocks, lens, w.tokens_per_block, w.num_pool_blocks, 0, stream, decode=args2, ahead=True)
    with pytest.raises(qvp.QvpError) as e:
        with qvp.Graph.capture(stream):
            qvp.paged_decode(args2, stream)
    assert e.value.status == qvp.ERR_INVALID_ARGUMENT
    other.upload(stream)
    qvp.paged_decode(args2, stream)
    assert np.array_equal(out2.download(np.uint16, (n,), stream), got2)
