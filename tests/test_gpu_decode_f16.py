"""GPU parity of fp16 caches on the persistent MFMA decode: the reference
template runs with any two-byte element type (PagedAttention.h:53-64), and an
IEEE binary16 cache with head_dim 128 now runs the same GQA-folded persistent
schedule as bf16 (v_mfma_f32_16x16x32_f16 tiles, weights scaled by 2^15 so
the hi + lo fp16 split keeps ~22 bits). Every result is compared with the
oracle's fp16 decode (pinned bit for bit against the compiled reference with
an F16C half) at the bf16 bar, and 16-bit outputs within one rounding of the
oracle's fp32 result."""

from __future__ import annotations

import numpy as np
import pytest

import qvp
import workloads as W
from helpers import GpuRun, assert_close_16bit, assert_close_bf16, oracle_decode

pytestmark = pytest.mark.gpu


def _f16_run(lens, hq: int, hkv: int, seed: int, tpb: int = 16, spare: float = 0.25) -> tuple[W.Workload, GpuRun]:
    w = W.custom(lens, hq, hkv, 128, kv_dtype=qvp.DTYPE_F16, seed=seed, tokens_per_block=tpb, spare=spare)
    return w, GpuRun(w)


def test_config2_shaped_fp16_batch_runs_the_persistent_kernel():
    lens = W.config2().context_lens
    print(f"case: config2 lengths, fp16 cache ({len(lens)} sequences)", flush=True)
    w, run = _f16_run(lens, 28, 4, seed=21, spare=0.1)
    _, ref32 = oracle_decode(w, run.image, run.query)
    for od in (qvp.DTYPE_F32, qvp.DTYPE_BF16, qvp.DTYPE_F16):
        got = run.decode(out_dtype=od)
        plan = run.batch.decode_plan()
        assert plan["kernel"] == "mfma" and plan["tile_engine"] == "matrix", plan
        if od == qvp.DTYPE_F32:
            assert_close_bf16(got, ref32, "fp16 cache, fp32 out")
        else:
            assert_close_16bit(got, ref32, od, f"fp16 cache, {od} out")


@pytest.mark.parametrize("hq,hkv", [(28, 4), (8, 8), (64, 4), (32, 8), (16, 1)])
def test_ragged_lengths_and_query_groups(hq, hkv):
    lens = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 129, 1000, 2049, 4096]
    print(f"case: fp16 ragged hq={hq} hkv={hkv}", flush=True)
    w, run = _f16_run(lens, hq, hkv, seed=hq + hkv)
    _, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    assert run.batch.decode_plan()["kernel"] == "mfma"
    assert_close_bf16(got, ref32, f"fp16 hq={hq} hkv={hkv}")


@pytest.mark.parametrize("tpb", [16, 32, 64])
def test_block_sizes_and_split_partitions(tpb):
    lens = [700, 2000, 3100, 513, 90]
    print(f"case: fp16 tpb={tpb}", flush=True)
    w, run = _f16_run(lens, 28, 4, seed=tpb, tpb=tpb)
    _, ref32 = oracle_decode(w, run.image, run.query)
    for split in (0, 512):
        got = run.decode(out_dtype=qvp.DTYPE_F32, split_tokens=split)
        plan = run.batch.decode_plan()
        assert plan["kernel"] == "mfma" and plan["split_tokens"] == split, plan
        assert_close_bf16(got, ref32, f"fp16 tpb={tpb} split={split}")


def test_large_values_stay_finite_and_accurate():
    """fp16 caches with large elements: keys and values ~N(0, 300^2) (up to
    ~1500), queries small, so scores spread over ~30 and the weights (scaled
    by 2^15 in fp16) multiply values of hundreds -- nothing overflows and the
    output matches. Outputs here are sums of terms of ~300 that cancel, so
    fp32 summation order alone moves a small output by ~1e-5 of the terms'
    size (the oracle and the kernel sum in different orders): the bar is the
    absolute and norm-wise one scaled to the values, not a per-element
    relative one."""
    lens = [300, 1700]
    w = W.custom(lens, 28, 4, 128, kv_dtype=qvp.DTYPE_F16, seed=5, kv_sigma=300.0, q_sigma=0.05)
    run = GpuRun(w)
    _, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    assert np.all(np.isfinite(got))
    err = np.abs(got.astype(np.float64) - ref32)
    assert float(err.max()) <= 2e-3 * 300.0, float(err.max())
    assert float(err.max() / np.abs(ref32).max()) <= 1e-4, float(err.max() / np.abs(ref32).max())


def test_repeated_decodes_are_bitwise_identical_and_vector_tiles_are_refused():
    lens = [100, 2500, 777]
    w, run = _f16_run(lens, 28, 4, seed=9)
    first = run.decode(out_dtype=qvp.DTYPE_F32)
    for _ in range(5):
        assert np.array_equal(run.decode(out_dtype=qvp.DTYPE_F32), first)
    with pytest.raises(qvp.QvpError) as e:
        run.decode(out_dtype=qvp.DTYPE_F32, tile_engine=qvp.TILE_VECTOR)
    assert e.value.status == qvp.ERR_INVALID_ARGUMENT


def test_forked_sequences_decode_without_shared_prefixes():
    # The shared-prefix launch reads bf16 caches: forks of an fp16 prompt run
    # as ordinary sequences of the persistent decode.
    branches = [8]
    w = W.forked([2048], branches, [[1] * 8], 28, 4, kv_dtype=qvp.DTYPE_F16)
    run = GpuRun(w)
    _, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32)
    plan = run.batch.decode_plan()
    assert plan["kernel"] == "mfma" and plan["shared_prefix_groups"] == 0, plan
    assert_close_bf16(got, ref32, "fp16 forks")
