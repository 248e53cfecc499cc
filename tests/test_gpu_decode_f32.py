"""GPU parity: fp32 caches with head_dim 128 on the fp32 matrix cores against
the CPU oracle -- the reference's paged_attention_decode<float>
(include/qwenvl_paged/PagedAttention.h:53-127), whose fp32 arithmetic the
oracle restates bit for bit (tests/test_oracle.py). With a positive softmax
scale the persistent decode runs them (csrc/f32_tile.h: 16-token fp32 half
tiles on the GQA-folded schedule, merges fused); a zero or negative scale
takes the split kernel (csrc/decode_f32.hip) and its separate merge.
Tolerance: fp32, 1e-5 absolute."""

from __future__ import annotations

import numpy as np
import pytest

import qvp
import workloads as W
from helpers import F32_ABS_TOL, GpuRun, assert_close_16bit, oracle_decode, tiled_pool_image

pytestmark = pytest.mark.gpu

EDGES = [1, 2, 15, 16, 17, 31, 32, 33, 511, 512, 513, 1000, 1024, 2049]


def _check(w: W.Workload, split_tokens=None, out_dtypes=(qvp.DTYPE_F32,), image=None, kernel="mfma"):
    run = GpuRun(w, image=image)
    _, ref32 = oracle_decode(w, run.image, run.query)
    for od in out_dtypes:
        got = run.decode(out_dtype=od, split_tokens=split_tokens)
        plan = run.batch.decode_plan()
        assert plan["kernel"] == kernel, plan
        if od == qvp.DTYPE_F32:
            err = float(np.abs(got - ref32).max())
            assert err <= F32_ABS_TOL, f"fp32 max abs {err:.3e}"
        else:
            assert_close_16bit(got, ref32, od, f"{w.name} 16-bit out")


@pytest.mark.parametrize("hq,hkv", [(28, 4), (64, 8), (16, 1), (4, 4), (12, 2)])
def test_group_shapes_and_block_edges(hq, hkv):
    print(f"case: fp32 persistent hq={hq} hkv={hkv}", flush=True)
    w = W.custom(EDGES, hq, hkv, 128, kv_dtype=qvp.DTYPE_F32, seed=hq + hkv)
    _check(w, out_dtypes=(qvp.DTYPE_F32, qvp.DTYPE_BF16))


@pytest.mark.parametrize("tpb", [16, 32, 64])
def test_block_sizes(tpb):
    print(f"case: fp32 persistent tpb={tpb}", flush=True)
    w = W.custom([5, 129, 600, 2000], 28, 4, 128, kv_dtype=qvp.DTYPE_F32, tokens_per_block=tpb, seed=tpb)
    _check(w)


@pytest.mark.parametrize("split", [16, 64, 512, 2048, 100])
def test_split_sizes(split):
    # The persistent decode holds its range cuts to the partition (rounded up
    # to 128 tokens by the packer).
    print(f"case: fp32 persistent split={split}", flush=True)
    w = W.custom([1, 77, 513, 1500], 28, 4, 128, kv_dtype=qvp.DTYPE_F32, seed=split)
    _check(w, split_tokens=split)


@pytest.mark.parametrize("scale", [0.0, -0.0625])
@pytest.mark.parametrize("split", [16, 512, 100])
def test_non_positive_scales_take_the_split_kernel(scale, split):
    # 100 is not a multiple of 16: the packer rounds it to 128, which the
    # split kernel takes too.
    print(f"case: fp32 split kernel scale={scale} split={split}", flush=True)
    w = W.custom([1, 77, 513, 1500], 28, 4, 128, kv_dtype=qvp.DTYPE_F32, seed=split, scale=scale)
    _check(w, split_tokens=split, kernel="f32_grouped")


def test_multi_layer_frames():
    print("case: fp32 persistent, layer 2 of 3", flush=True)
    w = W.custom([33, 200, 700], 28, 4, 128, kv_dtype=qvp.DTYPE_F32, num_layers=3, layer=2, seed=4)
    _check(w)


def test_config2_shape_in_fp32():
    print("case: fp32 persistent, config2 shape (64 sequences, 145K tokens)", flush=True)
    c2 = W.config2()
    w = W.custom(list(c2.context_lens), 28, 4, 128, kv_dtype=qvp.DTYPE_F32, seed=2, spare=0.1)
    _check(w, image=tiled_pool_image(w))


def test_repeated_decodes_are_bitwise_identical_and_vector_tiles_are_refused():
    w = W.custom([100, 2500, 777, 16], 28, 4, 128, kv_dtype=qvp.DTYPE_F32, seed=31)
    run = GpuRun(w)
    first = run.decode(out_dtype=qvp.DTYPE_F32)
    for _ in range(5):
        assert np.array_equal(run.decode(out_dtype=qvp.DTYPE_F32), first)
    with pytest.raises(qvp.QvpError) as e:
        run.decode(out_dtype=qvp.DTYPE_F32, tile_engine=qvp.TILE_VECTOR)
    assert e.value.status == qvp.ERR_INVALID_ARGUMENT
