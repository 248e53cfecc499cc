"""qvp_paged_decode_noalloc (the decode on the library's fixed device scratch
array, for callers that cannot allocate) against qvp_paged_decode: the same
bits on two calls in a row, the second with a smaller batch, on the bf16 MFMA
kernel and on the split kernels (fp32 and generic); refusals leave the output
untouched; the calls change no device memory accounting."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import qvp
import workloads as W
from helpers import GpuRun, assert_close_bf16, oracle_decode

pytestmark = pytest.mark.gpu


def _args(run: GpuRun, out: qvp.DeviceBuffer, w: W.Workload | None = None, **over):
    w = w or run.w
    kw = dict(query=run.q.ptr, out=out.ptr, kv_base=run.pool.base, block_stride=run.pool.stride, batch=run.batch,
              kv_dtype=w.kv_dtype, out_dtype=qvp.DTYPE_F32, layer=w.layer, num_layers=w.num_layers,
              num_query_heads=w.num_query_heads, num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
              tokens_per_block=w.tokens_per_block, scale=w.scale, strides=w.strides)
    kw.update(over)
    return qvp.decode_args(**kw)


def _device_free_bytes() -> int:
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


_SCRATCH_READY = False


def _set_up_scratch() -> None:
    """The first call on a device takes the scratch array's device address
    (the runtime places the library's device variables then); later calls
    must leave device memory use unchanged. One small decode does it."""
    global _SCRATCH_READY
    if _SCRATCH_READY:
        return
    run = GpuRun(W.custom([33, 70], 8, 2, 64, kv_dtype=qvp.DTYPE_F32, seed=1))
    out = qvp.DeviceBuffer(2 * 8 * 64 * 4)
    run.batch.pack(run.w.ids, run.w.cu_blocks, run.w.context_lens, 16, run.w.num_pool_blocks)
    qvp.paged_decode_noalloc(_args(run, out))
    qvp.synchronize()
    _SCRATCH_READY = True


def _both(run: GpuRun, hinted: bool):
    """Decodes run's batch with both entry points into two outputs."""
    _set_up_scratch()
    w = run.w
    n = w.num_seqs * w.num_query_heads * w.head_dim
    out_ref, out_na = qvp.DeviceBuffer(n * 4), qvp.DeviceBuffer(n * 4)
    out_ref.fill(0xFF)
    out_na.fill(0xFF)
    a_ref, a_na = _args(run, out_ref), _args(run, out_na)
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, w.tokens_per_block, w.num_pool_blocks, w.split_tokens,
                   decode=a_na if hinted else None)
    if not hinted:
        qvp.paged_decode(a_ref)
    qvp.synchronize()
    before = _device_free_bytes()
    qvp.paged_decode_noalloc(a_na)
    qvp.synchronize()
    assert _device_free_bytes() == before, "the allocation-free decode changed device memory use"
    if hinted:
        qvp.paged_decode(a_ref)
    shape = (w.num_seqs, w.num_query_heads, w.head_dim)
    return out_ref.download(np.float32, shape), out_na.download(np.float32, shape)


def test_noalloc_matches_the_allocating_decode_on_two_calls_the_second_smaller():
    runs = [GpuRun(W.config2(seed=2)), GpuRun(W.config2(seed=9, num_seqs=8))]
    for i, run in enumerate(runs):
        print(f"case: noalloc mfma call {i + 1}, B={run.w.num_seqs}", flush=True)
        ref, got = _both(run, hinted=True)
        assert run.batch.decode_plan()["kernel"] == "mfma"
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), f"call {i + 1} differs"
        _, ref32 = oracle_decode(run.w, run.image, run.query)
        assert_close_bf16(got, ref32, f"noalloc call {i + 1}")


@pytest.mark.parametrize("kernel", ["f32_grouped", "split_mfma", "grouped", "generic"])
def test_noalloc_on_the_split_kernels_two_calls_the_second_smaller(kernel):
    # fp32 caches with a negative scale take the fp32 split kernel (the
    # persistent decode takes positive scales); bf16 at head_dim 64 the
    # 16-bit matrix-core split kernel, at 80 the GQA-folded one, and at 66
    # (rows four-element loads cannot read) the per-head generic one.
    for i, lens in enumerate(([37, 600, 1500, 4096, 129, 2049], [90, 700])):
        print(f"case: noalloc {kernel} call {i + 1}, lens={lens}", flush=True)
        if kernel == "f32_grouped":
            w = W.custom(lens, 28, 4, 128, kv_dtype=qvp.DTYPE_F32, seed=40 + i, kv_sigma=1.0, scale=-0.0625)
        elif kernel == "split_mfma":
            w = W.custom(lens, 28, 4, 64, seed=50 + i)
        elif kernel == "grouped":
            w = W.custom(lens, 28, 4, 80, seed=70 + i)
        else:
            w = W.custom(lens, 28, 4, 66, seed=60 + i)
        run = GpuRun(w)
        ref, got = _both(run, hinted=False)
        assert run.batch.decode_plan()["kernel"] == kernel
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), f"call {i + 1} differs"


def test_noalloc_refusals_write_nothing():
    w = W.custom([300, 700, 2000], 28, 4, 128, seed=8)
    run = GpuRun(w)
    out = qvp.DeviceBuffer(w.num_seqs * 28 * 128 * 4)
    out.fill(0x7F)
    # A plain pack of a fresh batch: the MFMA schedule would need buffers.
    run.batch.pack(w.ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks)
    with pytest.raises(qvp.QvpError) as e:
        qvp.paged_decode_noalloc(_args(run, out))
    assert e.value.status == qvp.ERR_CAPACITY
    # A caller workspace is not accepted.
    ws = qvp.DeviceBuffer(1 << 20)
    with pytest.raises(qvp.QvpError) as e:
        qvp.paged_decode_noalloc(_args(run, out, workspace=ws.ptr, workspace_bytes=ws.nbytes))
    assert e.value.status == qvp.ERR_INVALID_ARGUMENT
    # A workspace beyond the scratch array: 64 query heads on one kv head
    # (the generic kernel) over 640 partitions of 128 tokens need 21 MB of
    # split partials.
    big = W.custom([8192] * 10, 64, 1, 128, seed=3, spare=0.01)
    run_big = GpuRun(big, image=np.zeros(big.num_pool_blocks * big.block_stride, np.uint8),
                     query=np.zeros((big.num_seqs, 64, 128), np.uint16))
    assert run_big.batch is not None
    out_big = qvp.DeviceBuffer(big.num_seqs * 64 * 128 * 4)
    out_big.fill(0x7F)
    run_big.batch.pack(big.ids, big.cu_blocks, big.context_lens, 16, big.num_pool_blocks, 128)
    with pytest.raises(qvp.QvpError) as e:
        qvp.paged_decode_noalloc(_args(run_big, out_big))
    assert e.value.status == qvp.ERR_CAPACITY
    qvp.synchronize()
    assert np.all(out.download(np.uint8, out.nbytes) == 0x7F)
    assert np.all(out_big.download(np.uint8, out_big.nbytes) == 0x7F)
