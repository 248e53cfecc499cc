"""The long-context multimodal (config3), copy-on-write (config4) and
continuous-batching (config5) configurations on the GPU at their full sizes,
through their C++ drivers
(qwenvl-paged_amd/host/bench): the device allocator's decisions and bytes
equal the host allocator's, copied frames equal their sources, sampled
decodes match float64 attention, the 200-request trace writes the event log
the reference's own Scheduler / KVCacheManager / MemoryAllocator wrote for the
same requests (tests/golden/scheduler_trace_config5.txt.gz) and drains
completely. A config4-shaped step through the C ABI is compared with the
oracle element by element."""

from __future__ import annotations

import gzip
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import kv_pattern as KP
import qvp
import workloads as W
from helpers import assert_close_16bit, assert_close_bf16, oracle_decode, to_f32

ROOT = Path(__file__).resolve().parents[1]
BENCH = ROOT / "build" / "bench"
GOLDEN = ROOT / "tests" / "golden"


def run(name: str, *args: str) -> dict:
    exe = BENCH / name
    assert exe.exists(), f"{exe} is missing: run __graft_entry__.build() first"
    print(f"running {name} {' '.join(args)}", flush=True)
    proc = subprocess.run([str(exe), *args], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=110)
    print(proc.stdout, proc.stderr)
    assert proc.returncode == 0, proc.stderr + proc.stdout
    return json.loads(proc.stdout.strip().splitlines()[-1])


@pytest.mark.gpu
@pytest.mark.parametrize("layers", [1, 28])
def test_copy_on_write_configuration_full_size(layers):
    """config4 as specified: 16 prompts x 8 branches, 128 copy-on-write pairs
    and the branches' 128 new tokens in one launch (KVAppendBatch), decode over
    the 128 branches; with one layer per frame and with whole 28-layer
    Qwen2-VL-7B frames (917,504 B copies). The device pool after the step
    equals the host-placement allocator's (memcpy copies, then memcpy rows)
    byte for byte."""
    r = run("cow_bench", "--layers", str(layers), "--reps", "5")
    assert r["layers"] == layers and r["cow_pairs"] == 128
    assert r["pending_after_append"] == 0
    assert r["copy_launches"] == 1
    assert r["frames_equal_host_allocator"] and r["copies_equal_source_plus_rows"]
    assert r["decode_within_tolerance"] and r["checked_elements"] > 0


def _reference_config5_log() -> str:
    return gzip.decompress((GOLDEN / "scheduler_trace_config5.txt.gz").read_bytes()).decode()


def _first_difference(a: str, b: str) -> str:
    for k, (x, y) in enumerate(zip(a.splitlines(), b.splitlines())):
        if x != y:
            return f"line {k + 1}:\n  expected {y[:300]}\n  actual   {x[:300]}"
    return f"lengths differ: {len(a.splitlines())} vs {len(b.splitlines())} lines"


@pytest.mark.gpu
@pytest.mark.parametrize("engine", ["0", "1"], ids=["decode-only", "full-engine-step"])
def test_continuous_batching_trace_full_size_matches_the_reference(tmp_path, engine):
    """config5 as specified: 200 requests, pool 60 % of demand, watermark 64.
    The step log (admissions, preemptions, resumes, completions, frame and
    swap-slot ids hashed per step) equals the reference's; every request
    finishes and the pool and the swap arena drain. With the full engine step
    (append, prefill, M-RoPE, decode) the decisions are the same."""
    log = tmp_path / "trace.log"
    r = run("trace_bench", "--requests", "200", "--seed", "5", "--engine", engine, "--log", str(log))
    assert r["finished"] == 200 and r["drained"]
    assert r["decode_tokens"] == r["expected_decode_tokens"]
    assert r["preemptions"] > 0 and r["resumes"] > 0
    assert r["swapped_out_blocks"] > 0 and r["swapped_in_blocks"] > 0
    got, expected = log.read_text(), _reference_config5_log()
    assert got == expected, _first_difference(got, expected)


# One record of trace_bench's --verify-dump: step, sequence, batch row,
# context length, then the sequence's decode output (28 heads x 128, bf16).
_DUMP_RECORD = np.dtype([("step", "<u4"), ("seq", "<u4"), ("row", "<u4"), ("len", "<u4"), ("out", "<u2", (28 * 128,))])


def _oracle_check_dump(path: Path) -> int:
    """Rebuilds each dumped sequence's K/V from the seeded pattern (one frame
    per logical block, layer 0, K rows then V rows) and its query from the
    batch row, decodes them with the oracle and compares with the dumped bf16
    outputs. Returns the number of records checked."""
    recs = np.fromfile(path, dtype=_DUMP_RECORD)
    assert len(recs) > 0, "empty verify dump"
    tpb, hkv, hq, d = 16, 4, 28, 128
    for chunk in np.array_split(recs, -(-len(recs) // 12)):
        lens = chunk["len"].astype(np.int64)
        nb = (lens + tpb - 1) // tpb
        cu = np.zeros(len(chunk) + 1, np.uint32)
        cu[1:] = np.cumsum(nb)
        total = int(cu[-1])
        frames = np.zeros((total, 2, tpb, hkv * d), np.uint16)
        for r, rec in enumerate(chunk):
            pos = np.arange(int(rec["len"]), dtype=np.int64)
            f = int(cu[r]) + pos // tpb
            for st in (0, 1):
                frames[f, st, pos % tpb] = KP.kv_rows(int(rec["seq"]), pos, st, hkv * d)
        w = W.Workload("config5_checks", tpb, 1, hq, hkv, d, qvp.DTYPE_BF16, 1.0 / np.sqrt(d),
                       chunk["len"].astype(np.uint32), np.arange(total, dtype=np.uint32), cu, total, seed=0)
        query = KP.query_rows(chunk["row"], hq * d).reshape(len(chunk), hq, d)
        _, ref32 = oracle_decode(w, frames.reshape(-1).view(np.uint8), query)
        got = chunk["out"].reshape(len(chunk), hq, d)
        assert_close_16bit(got, ref32, qvp.DTYPE_BF16,
                           f"config5 decode at steps {chunk['step'].min()}..{chunk['step'].max()}")
    return len(recs)


@pytest.mark.gpu
@pytest.mark.parametrize("engine,in_flight", [("0", "2"), ("1", "2"), ("0", "1")],
                         ids=["decode-only", "full-engine-step", "one-step-at-a-time"])
def test_continuous_batching_trace_full_size_bytes(tmp_path, engine, in_flight):
    """config5 at full size with the bytes checked, not only the decisions
    (reference tests/EndToEnd.test.cpp:311-351: a preempted request resumes
    with an intact cache; swap semantics src/MemoryAllocator.cpp:105-152).
    Every K/V row is a seeded function of (sequence, position), written by
    the append kernel; swap gathers and scatters run on the side stream beside
    the engine's appends and decodes with two steps in flight. After every
    resume, and for four sequences every 40 steps, the driver copies the
    sequence's frames behind its decode and compares every row below its
    length with the pattern (no mismatch allowed), and the decode outputs it
    dumps equal the oracle's decode of the same rows at the bf16 bar. The
    decisions still equal the reference's log."""
    log, dump = tmp_path / "trace.log", tmp_path / "checks.bin"
    r = run("trace_bench", "--requests", "200", "--seed", "5", "--engine", engine, "--in-flight", in_flight,
            "--verify", "1", "--check-every", "40", "--verify-dump", str(dump), "--log", str(log))
    assert r["verify"] and r["finished"] == 200 and r["drained"]
    assert r["row_mismatches"] == 0, r["first_mismatch"]
    assert r["resumes"] > 0 and r["resume_checks"] == r["resumes"] and r["unchecked_resumes"] == 0
    assert r["sequence_checks"] > r["resume_checks"] and r["rows_checked"] > 500_000
    got, expected = log.read_text(), _reference_config5_log()
    assert got == expected, _first_difference(got, expected)
    assert _oracle_check_dump(dump) == r["decode_records"] == r["sequence_checks"]


@pytest.mark.gpu
def test_continuous_batching_trace_with_whole_28_layer_frames(tmp_path):
    """The config5 trace with every frame holding all 28 layers (917,504 B):
    the same decisions and ids as the reference's log (frame size changes no
    decision), 39.5 GB swapped out and back in, and everything drains."""
    log = tmp_path / "trace28.log"
    r = run("trace_bench", "--requests", "200", "--seed", "5", "--layers", "28", "--log", str(log))
    assert r["layers"] == 28 and r["finished"] == 200 and r["drained"]
    assert r["swap_bytes"] == (r["swapped_out_blocks"] + r["swapped_in_blocks"]) * 917504
    got, expected = log.read_text(), _reference_config5_log()
    assert got == expected, _first_difference(got, expected)


@pytest.mark.gpu
def test_long_context_multimodal_configuration_full_size():
    """config3 as specified, through the host API: 32 Qwen2-VL-72B-shaped
    sequences with contexts on [8192, 32768], each created with an image span
    over its first quarter (MultimodalSpan + Image2D positional span on a
    patch grid, then a Text1D span). metadata() returns what was given, the
    M-RoPE positions of every token equal the closed form, the decode over the
    tagged sequences equals the decode over untagged forks bit for bit, and
    sampled heads match float64 attention. The decode runs with config3's
    split-K partitions of 512 tokens (the plan reports them)."""
    r = run("config3_bench")
    assert r["sequences"] == 32 and r["image_tokens"] > 0
    assert r["metadata_roundtrip"] and r["positions_match_closed_form"]
    assert r["tagged_equals_untagged_bitwise"]
    assert r["decode_within_tolerance"] and r["checked_elements"] == 4 * 8 * 128
    assert r["plan"]["query_group"] == 8 and r["plan"]["split_tokens"] == 512


@pytest.mark.gpu
def test_config4_step_through_the_abi_matches_the_oracle():
    """The config4 step on the C ABI at full size: 16 prompts of 2048 tokens
    (2049 slots reserved, so logical block 128 is a partly filled tail), 8
    branches each sharing the 128 full blocks; one qvp_copy_blocks gives every
    branch a private copy of its prompt's tail (128 pairs, checked byte for
    byte), each branch writes its first decode token into the copy, and one
    decode runs over the 128 branches (context 2049) -- compared with the
    oracle on every output element."""
    prompts, branches, full = 16, 8, 128
    w_shape = W.custom([16], 28, 4, 128)
    block = w_shape.block_bytes
    frames = prompts * (full + 1) + prompts * branches
    rng = np.random.default_rng(44)
    image = W.f32_to_bf16_bits(rng.normal(0.0, 0.5, frames * block // 2).astype(np.float32)).view(np.uint8)
    pool = qvp.BlockPool(frames, block)
    pool.upload_all(image)
    prompt_frames = np.arange(prompts * (full + 1), dtype=np.uint32).reshape(prompts, full + 1)
    branch_tail = np.arange(prompts * (full + 1), frames, dtype=np.uint32).reshape(prompts, branches)
    src = np.repeat(prompt_frames[:, full], branches)
    dst = branch_tail.reshape(-1)
    print("case: config4 copy of 128 shared tails", flush=True)
    qvp.copy_blocks(pool.base, pool.stride, frames, src, dst, pool.stride)
    # Each branch's first decode token: position 2048, slot 0 of its tail copy.
    st = qvp.layout_strides(16, 1, 4, 128)
    k_new = W.f32_to_bf16_bits(rng.normal(0.0, 0.5, (prompts * branches, 4 * 128)).astype(np.float32))
    v_new = W.f32_to_bf16_bits(rng.normal(0.0, 0.5, (prompts * branches, 4 * 128)).astype(np.float32))
    for i, f in enumerate(dst):
        pool.write(int(f), k_new[i].view(np.uint8), offset=0)
        pool.write(int(f), v_new[i].view(np.uint8), offset=st["stream_stride"] * 2)
    qvp.synchronize()
    got_image = pool.download_all()
    expect = image.reshape(frames, block).copy()
    expect[dst] = expect[src]
    for i, f in enumerate(dst):
        expect[f, : 4 * 128 * 2] = k_new[i].view(np.uint8)
        off = st["stream_stride"] * 2
        expect[f, off: off + 4 * 128 * 2] = v_new[i].view(np.uint8)
    assert np.array_equal(got_image.reshape(frames, block), expect), "copy-on-write frames differ"
    ids = np.concatenate([np.concatenate([prompt_frames[p, :full], [branch_tail[p, b]]])
                          for p in range(prompts) for b in range(branches)]).astype(np.uint32)
    cu = np.arange(0, (full + 1) * prompts * branches + 1, full + 1, dtype=np.uint32)
    w = W.custom([2049] * (prompts * branches), 28, 4, 128, seed=45)
    w.ids, w.cu_blocks, w.num_pool_blocks = ids, cu, frames
    query = w.query()
    q = qvp.DeviceBuffer.from_array(query)
    batch = qvp.Batch()
    batch.pack(ids, cu, w.context_lens, 16, frames)
    outs = {}
    for od in (qvp.DTYPE_F32, qvp.DTYPE_BF16):
        out = qvp.DeviceBuffer(w.num_seqs * 28 * 128 * qvp.DTYPE_BYTES[od])
        args = qvp.decode_args(query=q.ptr, out=out.ptr, kv_base=pool.base, block_stride=pool.stride, batch=batch,
                               kv_dtype=qvp.DTYPE_BF16, out_dtype=od, layer=0, num_layers=1, num_query_heads=28,
                               num_kv_heads=4, head_dim=128, tokens_per_block=16, scale=w.scale, strides=st)
        print(f"case: config4 decode over 128 branches, out dtype {od}", flush=True)
        qvp.paged_decode(args)
        outs[od] = out.download(np.float32 if od == qvp.DTYPE_F32 else np.uint16, (w.num_seqs, 28, 128))
    ref_out, ref32 = oracle_decode(w, got_image, query)
    assert_close_bf16(outs[qvp.DTYPE_F32], ref32, "config4 fp32 out")
    assert_close_16bit(outs[qvp.DTYPE_BF16], ref32, qvp.DTYPE_BF16, "config4 bf16 out")
    assert_close_16bit(outs[qvp.DTYPE_BF16], to_f32(ref_out, qvp.DTYPE_BF16), qvp.DTYPE_BF16, "config4 vs oracle T")
