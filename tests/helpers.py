"""Shared helpers for the parity tests: run a workload through the C ABI and
through the CPU oracle, and compare at the stated tolerances."""

from __future__ import annotations

import numpy as np

import pyoracle as O
import qvp
import workloads as W

# fp32 caches: the reference tests' tolerance (tests/PagedAttention.test.cpp:38).
F32_ABS_TOL = 1e-5
# bf16 caches: max abs <= 2e-3 and max rel <= 1e-2 over elements with
# |ref| >= 1e-3, plus a norm-wise ||diff||_inf / ||ref||_inf <= 1e-2.
BF16_ABS_TOL = 2e-3
BF16_REL_TOL = 1e-2
BF16_REL_FLOOR = 1e-3


def tiled_pool_image(w: W.Workload, chunk_elems: int = 16_777_259) -> np.ndarray:
    """A pool image for large workloads, quick to make: one seeded chunk of
    N(0, kv_sigma^2) elements of the cache type (bf16 or fp32) repeated over the
    frames. The chunk length is odd, so no two frames see the same bytes at the
    same offsets."""
    assert w.block_stride == w.block_bytes
    esz = qvp.DTYPE_BYTES[w.kv_dtype]
    total = w.num_pool_blocks * w.block_bytes // esz
    chunk = np.random.default_rng(w.seed).normal(0.0, w.kv_sigma, chunk_elems).astype(np.float32)
    chunk = W.to_elements(chunk, w.kv_dtype)
    reps = -(-total // chunk_elems)
    return np.tile(chunk, reps)[:total].view(np.uint8)


def oracle_dtype(kv_dtype: int) -> int:
    return {qvp.DTYPE_F32: O.ORC_F32, qvp.DTYPE_BF16: O.ORC_BF16, qvp.DTYPE_F16: O.ORC_F16}[kv_dtype]


def oracle_decode(w: W.Workload, image: np.ndarray, query: np.ndarray, threads: int = 0):
    threads = threads or min(O.host_threads(), 8)
    refused, out, out32 = O.decode_batch(
        image, w.block_stride, w.num_pool_blocks, w.ids, w.cu_blocks, w.context_lens, oracle_dtype(w.kv_dtype),
        query, w.layer, w.num_layers, w.num_query_heads, w.num_kv_heads, w.head_dim, w.tokens_per_block, w.scale,
        threads)
    assert refused == 0
    return out, out32


class GpuRun:
    """A workload resident on the GPU: pool, query, batch and output buffers."""

    def __init__(self, w: W.Workload, image: np.ndarray | None = None, query: np.ndarray | None = None):
        self.w = w
        self.image = w.pool_image() if image is None else image
        self.query = w.query() if query is None else query
        self.pool = qvp.BlockPool(w.num_pool_blocks, w.block_bytes)
        assert self.pool.stride == w.block_stride
        self.pool.upload_all(self.image)
        self.q = qvp.DeviceBuffer.from_array(self.query)
        self.batch = qvp.Batch()

    def decode(self, out_dtype: int | None = None, split_tokens: int | None = None, workspace=None,
               stream=None, tile_engine: int = qvp.TILE_AUTO) -> np.ndarray:
        w = self.w
        od = w.kv_dtype if out_dtype is None else out_dtype
        self.batch.pack(w.ids, w.cu_blocks, w.context_lens, w.tokens_per_block, w.num_pool_blocks,
                        w.split_tokens if split_tokens is None else split_tokens, stream)
        n = w.num_seqs * w.num_query_heads * w.head_dim
        out = qvp.DeviceBuffer(n * qvp.DTYPE_BYTES[od])
        out.fill(0xFF, stream)
        ws_ptr, ws_bytes = (workspace.ptr, workspace.nbytes) if workspace is not None else (0, 0)
        args = qvp.decode_args(query=self.q.ptr, out=out.ptr, kv_base=self.pool.base, block_stride=self.pool.stride,
                               batch=self.batch, kv_dtype=w.kv_dtype, out_dtype=od, layer=w.layer,
                               num_layers=w.num_layers, num_query_heads=w.num_query_heads,
                               num_kv_heads=w.num_kv_heads, head_dim=w.head_dim,
                               tokens_per_block=w.tokens_per_block, scale=w.scale, strides=w.strides,
                               workspace=ws_ptr, workspace_bytes=ws_bytes, tile_engine=tile_engine)
        qvp.paged_decode(args, stream)
        np_dtype = np.float32 if od == qvp.DTYPE_F32 else np.uint16
        return out.download(np_dtype, (w.num_seqs, w.num_query_heads, w.head_dim), stream)


def to_f32(arr: np.ndarray, dtype: int) -> np.ndarray:
    if dtype == qvp.DTYPE_F32:
        return arr.astype(np.float32)
    if dtype == qvp.DTYPE_BF16:
        return W.bf16_bits_to_f32(arr)
    return arr.view(np.float16).astype(np.float32)


def ulp16(x: np.ndarray, dtype: int) -> np.ndarray:
    """Spacing of the 16-bit format at |x| (bf16: 8 significant bits, fp16: 11)."""
    mant = 8 if dtype == qvp.DTYPE_BF16 else 11
    e = np.floor(np.log2(np.maximum(np.abs(x), 1e-30)))
    return np.exp2(e - (mant - 1))


def round16(x: np.ndarray, dtype: int) -> np.ndarray:
    """Round-to-nearest-even of fp32 values to the 16-bit format, as float32."""
    if dtype == qvp.DTYPE_BF16:
        return W.bf16_bits_to_f32(W.f32_to_bf16_bits(x))
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def assert_close_16bit(got16: np.ndarray, ref32: np.ndarray, dtype: int, what: str = "") -> dict:
    """A 16-bit output is the rounding of the kernel's fp32 result, so it is
    compared with the oracle's fp32 result rounded the same way: equal, or one
    unit in the last place apart where the two fp32 values straddle a rounding
    boundary, and within the bf16 absolute tolerance otherwise."""
    got = to_f32(got16, dtype).astype(np.float64)
    exp = round16(ref32, dtype).astype(np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    diff = np.abs(got - exp)
    allowed = np.maximum(BF16_ABS_TOL, ulp16(exp, dtype) * 1.0001)
    worst = float((diff / allowed).max())
    stats = {"max_abs": float(diff.max()), "exact_fraction": float((diff == 0).mean()), "worst_over_allowed": worst}
    assert worst <= 1.0, f"{what}: 16-bit output off by more than max(2e-3, 1 ulp): {stats}"
    return stats


def assert_close_bf16(got: np.ndarray, ref: np.ndarray, what: str = "") -> dict:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    diff = np.abs(got - ref)
    max_abs = float(diff.max())
    mask = np.abs(ref) >= BF16_REL_FLOOR
    max_rel = float((diff[mask] / np.abs(ref[mask])).max()) if mask.any() else 0.0
    normwise = float(diff.max() / max(np.abs(ref).max(), 1e-30))
    stats = {"max_abs": max_abs, "max_rel": max_rel, "normwise": normwise}
    assert max_abs <= BF16_ABS_TOL, f"{what}: max abs {max_abs:.3e} > {BF16_ABS_TOL} {stats}"
    assert max_rel <= BF16_REL_TOL, f"{what}: max rel {max_rel:.3e} > {BF16_REL_TOL} {stats}"
    assert normwise <= BF16_REL_TOL, f"{what}: normwise {normwise:.3e} > {BF16_REL_TOL} {stats}"
    return stats
