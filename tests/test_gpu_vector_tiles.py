"""GPU parity of the persistent bf16 decode with vector-ALU tiles
(QVP_TILE_VECTOR: the GQA group folded into each lane's fp32 dot products,
groups of one or two query heads per kv head) against the CPU oracle, on the
schedules the matrix-core tiles run: one kv head per workgroup, kv heads side
by side on long contexts, ragged edges at the block and tile boundaries, and
every output type. The engine is a call argument; the automatic choice is
reported by the decode plan."""

from __future__ import annotations

import numpy as np
import pytest

import qvp
import workloads as W
from helpers import GpuRun, assert_close_16bit, assert_close_bf16, oracle_decode, tiled_pool_image

pytestmark = pytest.mark.gpu

EDGE_LENS = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 1000, 4096, 2049]


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 4), (2, 1), (28, 14)], ids=["g1", "g2", "g2-hkv1", "g2-hkv14"])
def test_vector_tiles_match_the_oracle_on_ragged_lengths(hq, hkv):
    w = W.custom(EDGE_LENS, hq, hkv, 128, seed=hq * 31 + hkv)
    print(f"case: vector tiles hq={hq} hkv={hkv} lens={EDGE_LENS}", flush=True)
    run = GpuRun(w)
    ref_out, ref32 = oracle_decode(w, run.image, run.query)
    got32 = run.decode(out_dtype=qvp.DTYPE_F32, tile_engine=qvp.TILE_VECTOR)
    plan = run.batch.decode_plan()
    assert plan["kernel"] == "mfma" and plan["tile_engine"] == "vector", plan
    assert_close_bf16(got32, ref32, f"vector tiles hq={hq} hkv={hkv} fp32 out")
    for od in (qvp.DTYPE_BF16, qvp.DTYPE_F16):
        got16 = run.decode(out_dtype=od, tile_engine=qvp.TILE_VECTOR)
        assert_close_16bit(got16, ref32, od, f"vector tiles hq={hq} hkv={hkv} out dtype {od}")


@pytest.mark.parametrize("hq,hkv", [(16, 16), (32, 16), (6, 6)], ids=["hps4-g1", "hps4-g2", "hps2-g1"])
def test_vector_tiles_with_kv_heads_side_by_side(hq, hkv):
    """Long contexts (>= 32 tiles per resident wave): kv heads side by side in
    a workgroup, each with its own staged query, many split segments."""
    total_tokens = 65536 * 32 // hkv + 8192
    rng = np.random.default_rng(hkv + hq)
    cuts = np.sort(rng.choice(np.arange(1, total_tokens), size=5, replace=False))
    lens = [int(x) for x in np.diff(np.concatenate([[0], cuts, [total_tokens]]))]
    lens.insert(3, 100)
    print(f"case: vector tiles side by side hq={hq} hkv={hkv} lens={lens}", flush=True)
    w = W.custom(lens, hq, hkv, 128, seed=hq + hkv, spare=0.02)
    run = GpuRun(w, image=tiled_pool_image(w))
    _, ref32 = oracle_decode(w, run.image, run.query)
    got = run.decode(out_dtype=qvp.DTYPE_F32, tile_engine=qvp.TILE_VECTOR)
    plan = run.batch.decode_plan()
    print(f"plan: {plan}", flush=True)
    assert plan["tile_engine"] == "vector" and plan["kv_heads_per_segment"] == (4 if hkv % 4 == 0 else 2), plan
    assert_close_bf16(got, ref32, f"vector tiles side by side hq={hq} hkv={hkv}")


def test_engines_agree_and_switching_rebuilds_the_schedule():
    """The same pack decoded with matrix, vector and matrix tiles again: the
    cached schedule is keyed by the engine (its LDS budget differs), and the
    two engines' results agree to the bf16 bar."""
    lens = [300, 2000, 77, 4096, 1234, 513]
    w = W.custom(lens, 8, 4, 128, seed=5)
    run = GpuRun(w)
    _, ref32 = oracle_decode(w, run.image, run.query)
    outs = {}
    for engine in (qvp.TILE_MATRIX, qvp.TILE_VECTOR, qvp.TILE_MATRIX):
        print(f"case: engine {engine}", flush=True)
        outs.setdefault(engine, []).append(run.decode(out_dtype=qvp.DTYPE_F32, tile_engine=engine))
        assert run.batch.decode_plan()["tile_engine"] == qvp.TILE_ENGINES[engine]
        assert_close_bf16(outs[engine][-1], ref32, f"engine {engine}")
    assert np.array_equal(outs[qvp.TILE_MATRIX][0], outs[qvp.TILE_MATRIX][1])
    assert_close_bf16(outs[qvp.TILE_VECTOR][0], outs[qvp.TILE_MATRIX][0].astype(np.float64), "vector vs matrix")


def test_automatic_choice_and_refusals():
    w7 = W.custom([700, 64], 28, 4, 128, seed=3)
    run = GpuRun(w7)
    run.decode(out_dtype=qvp.DTYPE_F32)
    assert run.batch.decode_plan()["tile_engine"] == "matrix"
    with pytest.raises(qvp.QvpError, match="vector tiles take query groups of at most 2"):
        run.decode(out_dtype=qvp.DTYPE_F32, tile_engine=qvp.TILE_VECTOR)
    with pytest.raises(qvp.QvpError, match="unknown tile engine"):
        run.decode(out_dtype=qvp.DTYPE_F32, tile_engine=7)
