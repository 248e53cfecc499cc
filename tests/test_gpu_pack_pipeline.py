"""GPU parity of the one-upload pack (qvp_pack_for_decode: packed arrays and
the decode's work schedule in a single upload) and of packs pipelined on a
second stream against decodes still running (packs alternate between two
device buffers). Every decode is compared with the oracle."""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest

import qvp
import workloads as W
from helpers import GpuRun, assert_close_bf16, oracle_decode

pytestmark = pytest.mark.gpu


def _args(run: GpuRun, w: W.Workload, q: qvp.DeviceBuffer, out: qvp.DeviceBuffer, batch: qvp.Batch,
          out_dtype=qvp.DTYPE_F32):
    return qvp.decode_args(query=q.ptr, out=out.ptr, kv_base=run.pool.base, block_stride=run.pool.stride,
                           batch=batch, kv_dtype=w.kv_dtype, out_dtype=out_dtype, layer=w.layer,
                           num_layers=w.num_layers, num_query_heads=w.num_query_heads, num_kv_heads=w.num_kv_heads,
                           head_dim=w.head_dim, tokens_per_block=w.tokens_per_block, scale=w.scale,
                           strides=w.strides)


def test_pack_for_decode_carries_the_schedule_and_matches_the_plain_pack():
    """A decode after qvp_pack_for_decode runs the schedule uploaded with the
    pack: same plan and the same bits as pack-then-decode, oracle result."""
    w = W.config2(seed=5, num_seqs=24)
    run = GpuRun(w)
    out = qvp.DeviceBuffer(w.num_seqs * w.num_query_heads * w.head_dim * 4)
    args = _args(run, w, run.q, out, run.batch)
    print("case: plain pack then decode", flush=True)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks)
    qvp.paged_decode(args)
    plain = out.download(np.float32, (w.num_seqs, w.num_query_heads, w.head_dim))
    plain_plan = run.batch.decode_plan()
    print("case: pack for decode then decode", flush=True)
    out.fill(0xFF)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks, decode=args)
    assert run.batch.decode_plan()["kernel"] == "none"
    qvp.paged_decode(args)
    hinted = out.download(np.float32, (w.num_seqs, w.num_query_heads, w.head_dim))
    assert run.batch.decode_plan() == plain_plan
    assert np.array_equal(plain.view(np.uint32), hinted.view(np.uint32))
    _, ref32 = oracle_decode(w, run.image, run.query)
    assert_close_bf16(hinted, ref32, "pack for decode")


def test_decode_with_other_heads_than_the_pack_named_builds_its_own_schedule():
    lens = [100, 2000, 513, 3000, 64, 1500]
    w_named = W.custom(lens, 28, 4, 128, seed=12)
    w_other = W.custom(lens, 8, 4, 128, seed=12)
    run = GpuRun(w_named)
    q_other = qvp.DeviceBuffer.from_array(w_other.query())
    out_named = qvp.DeviceBuffer(w_named.num_seqs * 28 * 128 * 4)
    out_other = qvp.DeviceBuffer(w_other.num_seqs * 8 * 128 * 4)
    a_named = _args(run, w_named, run.q, out_named, run.batch)
    a_other = _args(run, w_other, q_other, out_other, run.batch)
    run.batch.pack(w_named.ids, w_named.cu_blocks, w_named.context_lens, 16, w_named.num_pool_blocks,
                   decode=a_named)
    for w, a, out, q in ((w_other, a_other, out_other, w_other.query()),
                         (w_named, a_named, out_named, w_named.query())):
        print(f"case: pack named hq=28, decode hq={w.num_query_heads}", flush=True)
        qvp.paged_decode(a)
        assert run.batch.decode_plan()["query_group"] == w.group
        got = out.download(np.float32, (w.num_seqs, w.num_query_heads, 128))
        _, ref32 = oracle_decode(w, run.image, q)
        assert_close_bf16(got, ref32, f"hq={w.num_query_heads}")


def test_pack_refuses_invalid_decode_arguments_and_keeps_the_previous_pack():
    w = W.custom([40, 64], 28, 4, 128, seed=2)
    run = GpuRun(w)
    out = qvp.DeviceBuffer(w.num_seqs * 28 * 128 * 4)
    good = _args(run, w, run.q, out, run.batch)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks, decode=good)
    bad = _args(run, w, run.q, out, run.batch)
    bad.num_query_heads = 27
    lens2 = np.array([41, 64], np.uint32)
    with pytest.raises(qvp.QvpError) as e:
        run.batch.pack(w.ids, w.cu_blocks, lens2, 16, w.num_pool_blocks, decode=bad)
    assert e.value.status == qvp.ERR_INVALID_ARGUMENT
    assert run.batch.view().max_seq_len == 64 and run.batch.download()["seq_lens"].tolist() == [40, 64]
    qvp.paged_decode(good)
    got = out.download(np.float32, (w.num_seqs, 28, 128))
    _, ref32 = oracle_decode(w, run.image, run.query)
    assert_close_bf16(got, ref32, "previous pack after a refused one")


@pytest.mark.parametrize("hinted", [True, False], ids=["pack-for-decode", "plain-pack"])
def test_packs_on_a_second_stream_overlap_running_decodes(hinted):
    """Steps alternate between two batches of different lengths over one
    pool; each step packs on stream P (while the previous step's decode may
    still run on stream D), D waits for the pack, decodes into its own output
    buffer. Every output equals the oracle's: a pack never overwrote arrays a
    running decode still read."""
    lens_a = [700, 2000, 3100, 513, 1500, 2600, 90, 4000]
    lens_b = [650, 1999, 3300, 77, 1600, 2100, 4096, 31]
    w_a = W.custom(lens_a, 28, 4, 128, seed=33, spare=0.3)
    w_b = W.custom(lens_a, 28, 4, 128, seed=33, spare=0.3)
    # Same pool and tables (w_b uses at most as many blocks as w_a maps).
    w_b.context_lens = np.minimum(np.array(lens_b, np.uint32),
                                  np.diff(w_a.cu_blocks).astype(np.uint32) * 16).astype(np.uint32)
    run = GpuRun(w_a)
    P, D = qvp.Stream(), qvp.Stream()
    ev = qvp.Event()
    steps = 8
    outs = [qvp.DeviceBuffer(w_a.num_seqs * 28 * 128 * 4) for _ in range(steps)]
    for i in range(steps):
        w = w_a if i % 2 == 0 else w_b
        a = _args(run, w, run.q, outs[i], run.batch)
        run.batch.pack(w.ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks, stream=P,
                       decode=a if hinted else None)
        ev.record(P)
        D.wait(ev)
        qvp.paged_decode(a, D)
    D.synchronize()
    refs = {}
    for i in range(steps):
        w = w_a if i % 2 == 0 else w_b
        if i % 2 not in refs:
            refs[i % 2] = oracle_decode(w, run.image, run.query)[1]
        print(f"case: pipelined step {i} hinted={hinted}", flush=True)
        got = outs[i].download(np.float32, (w.num_seqs, 28, 128))
        assert_close_bf16(got, refs[i % 2], f"pipelined step {i}")


def _plain_decode(run: GpuRun, w: W.Workload, lens: np.ndarray) -> np.ndarray:
    """A fresh batch, packed with its upload and decoded: the reference bits."""
    batch = qvp.Batch()
    out = qvp.DeviceBuffer(w.num_seqs * w.num_query_heads * w.head_dim * 4)
    a = _args(run, w, run.q, out, batch)
    batch.pack(w.ids, w.cu_blocks, lens, 16, w.num_pool_blocks, decode=a)
    qvp.paged_decode(a)
    return out.download(np.float32, (w.num_seqs, w.num_query_heads, w.head_dim))


def test_pack_ahead_upload_rides_in_the_other_batchs_decode():
    """Two batch objects in turn, the pattern qvp_pack_ahead is for: step i + 1
    is packed ahead on one while step i decodes from the other. The decode of
    step i carries step i + 1's upload in the tail of its launch -- once it has
    run, the other batch's device arrays hold step i + 1's lengths, before any
    decode of that batch -- and every step's output equals, bit for bit, a
    plain pack-then-decode of the same step (and the oracle for one step)."""
    w = W.config2(seed=41, num_seqs=16)
    run = GpuRun(w)
    batches = [qvp.Batch(), qvp.Batch()]
    steps = 6
    lens = [np.maximum(w.context_lens.astype(np.int64) - 40 * i, 1).astype(np.uint32) for i in range(steps)]
    outs = [qvp.DeviceBuffer(w.num_seqs * w.num_query_heads * w.head_dim * 4) for _ in range(steps)]
    args = [_args(run, w, run.q, outs[i], batches[i % 2]) for i in range(steps)]
    s = qvp.Stream()
    batches[0].pack(w.ids, w.cu_blocks, lens[0], 16, w.num_pool_blocks, stream=s, decode=args[0])
    for i in range(steps):
        print(f"case: pack-ahead step {i}", flush=True)
        if i + 1 < steps:
            batches[(i + 1) % 2].pack(w.ids, w.cu_blocks, lens[i + 1], 16, w.num_pool_blocks, stream=s,
                                      decode=args[i + 1], ahead=True)
        qvp.paged_decode(args[i], s)
        assert batches[i % 2].decode_plan()["kernel"] == "mfma"
        if i + 1 < steps:
            s.synchronize()
            assert batches[(i + 1) % 2].download()["seq_lens"].tolist() == lens[i + 1].astype(np.int64).tolist()
    s.synchronize()
    for i in range(steps):
        got = outs[i].download(np.float32, (w.num_seqs, w.num_query_heads, w.head_dim))
        ref = _plain_decode(run, w, lens[i])
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"step {i} differs from a plain pack"
    w_last = dataclasses.replace(w, context_lens=lens[-1])
    _, ref32 = oracle_decode(w_last, run.image, run.query)
    got = outs[-1].download(np.float32, (w.num_seqs, w.num_query_heads, w.head_dim))
    assert_close_bf16(got, ref32, "last pack-ahead step")


def test_pack_ahead_without_a_carrier():
    """A pending upload that no other decode carries: the batch's own decode
    enqueues it first; qvp_batch_upload enqueues it on request; a later pack
    of the batch discards it; a split-kernel decode of another batch leaves
    it pending; destroying the batch with it pending is safe."""
    w = W.config2(seed=43, num_seqs=12)
    run = GpuRun(w)
    s = qvp.Stream()
    lens1 = np.maximum(w.context_lens.astype(np.int64) - 100, 1).astype(np.uint32)
    lens2 = np.maximum(w.context_lens.astype(np.int64) - 300, 1).astype(np.uint32)
    b = qvp.Batch()
    out = qvp.DeviceBuffer(w.num_seqs * w.num_query_heads * w.head_dim * 4)
    a = _args(run, w, run.q, out, b)

    print("case: own decode after pack-ahead", flush=True)
    b.pack(w.ids, w.cu_blocks, lens1, 16, w.num_pool_blocks, stream=s, decode=a, ahead=True)
    qvp.paged_decode(a, s)
    got = out.download(np.float32, (w.num_seqs, w.num_query_heads, w.head_dim), s)
    assert np.array_equal(got.view(np.uint32), _plain_decode(run, w, lens1).view(np.uint32))

    print("case: upload on request", flush=True)
    b.pack(w.ids, w.cu_blocks, lens2, 16, w.num_pool_blocks, stream=s, decode=a, ahead=True)
    b.upload(s)
    s.synchronize()
    assert b.download()["seq_lens"].tolist() == lens2.astype(np.int64).tolist()

    print("case: pack-ahead superseded by a plain pack", flush=True)
    b.pack(w.ids, w.cu_blocks, lens1, 16, w.num_pool_blocks, stream=s, decode=a, ahead=True)
    b.pack(w.ids, w.cu_blocks, lens2, 16, w.num_pool_blocks, stream=s, decode=a)
    qvp.paged_decode(a, s)
    got = out.download(np.float32, (w.num_seqs, w.num_query_heads, w.head_dim), s)
    assert np.array_equal(got.view(np.uint32), _plain_decode(run, w, lens2).view(np.uint32))

    print("case: a split-kernel decode of another batch leaves it pending", flush=True)
    w64 = W.custom([300, 700, 1200], 28, 4, 64, seed=8)
    run64 = GpuRun(w64)
    b.pack(w.ids, w.cu_blocks, lens1, 16, w.num_pool_blocks, stream=s, decode=a, ahead=True)
    run64.decode(out_dtype=qvp.DTYPE_F32, stream=s)
    assert run64.batch.decode_plan()["kernel"] == "split_mfma"
    qvp.paged_decode(a, s)
    got = out.download(np.float32, (w.num_seqs, w.num_query_heads, w.head_dim), s)
    assert np.array_equal(got.view(np.uint32), _plain_decode(run, w, lens1).view(np.uint32))

    print("case: destroy with a pending upload", flush=True)
    c = qvp.Batch()
    c.pack(w.ids, w.cu_blocks, lens1, 16, w.num_pool_blocks, stream=s, decode=a, ahead=True)
    c.destroy()
    qvp.paged_decode(a, s)  # no pending upload of a destroyed batch is carried
    s.synchronize()


@pytest.mark.parametrize("enqueue", ["upload", "decode"])
def test_pack_ahead_upload_on_another_stream_waits_for_the_slots_last_decode(enqueue):
    """Steps 0 and 1 are packed and decoded on stream P, step 0's decode
    queued behind a dozen decodes of another batch; step 2 is packed ahead on
    P into step 0's buffer and its upload enqueued on stream D (by
    qvp_batch_upload, or by the batch's own decode on D). The upload has to
    wait for step 0's decode on P: every step's output equals a plain
    pack-then-decode of its lengths, bit for bit."""
    w = W.config2(seed=47, num_seqs=64)
    run = GpuRun(w)
    P, D = qvp.Stream(), qvp.Stream()
    lens = [np.maximum(w.context_lens.astype(np.int64) - d, 1).astype(np.uint32) for d in (0, 150, 400)]
    b = qvp.Batch()
    outs = [qvp.DeviceBuffer(w.num_seqs * w.num_query_heads * w.head_dim * 4) for _ in range(3)]
    args = [_args(run, w, run.q, outs[i], b) for i in range(3)]
    busy_out = qvp.DeviceBuffer(w.num_seqs * w.num_query_heads * w.head_dim * 4)
    busy = _args(run, w, run.q, busy_out, run.batch)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks, stream=P, decode=busy)
    print(f"case: pack-ahead upload on a second stream via {enqueue}", flush=True)
    b.pack(w.ids, w.cu_blocks, lens[0], 16, w.num_pool_blocks, stream=P, decode=args[0])
    for _ in range(12):
        qvp.paged_decode(busy, P)
    qvp.paged_decode(args[0], P)
    b.pack(w.ids, w.cu_blocks, lens[1], 16, w.num_pool_blocks, stream=P, decode=args[1])
    qvp.paged_decode(args[1], P)
    b.pack(w.ids, w.cu_blocks, lens[2], 16, w.num_pool_blocks, stream=P, decode=args[2], ahead=True)
    if enqueue == "upload":
        b.upload(D)
    qvp.paged_decode(args[2], D)
    D.synchronize()
    P.synchronize()
    for i in range(3):
        got = outs[i].download(np.float32, (w.num_seqs, w.num_query_heads, w.head_dim))
        ref = _plain_decode(run, w, lens[i])
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"step {i} differs from a plain pack"
