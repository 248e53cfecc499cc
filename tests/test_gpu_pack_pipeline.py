"""GPU parity of the one-upload pack (qvp_pack_for_decode: packed arrays and
the decode's work schedule in a single upload) and of packs pipelined on a
second stream against decodes still running (packs alternate between two
device buffers). Every decode is compared with the oracle."""

from __future__ import annotations

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
