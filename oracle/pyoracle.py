"""ctypes access to the CPU oracle (oracle/_build/liboracle.so) and, where it was
built, the compiled reference (oracle/_ref/libqvp_ref.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_int64, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "_build" / "liboracle.so"
REF_LIB = HERE / "_ref" / "libqvp_ref.so"

ORC_F32, ORC_BF16, ORC_F16 = 0, 1, 2

_u32p = POINTER(c_uint32)
_i32p = POINTER(c_int32)

_oracle = None
_ref = None


def oracle() -> ctypes.CDLL:
    global _oracle
    if _oracle is None:
        if not ORACLE_LIB.exists():
            raise FileNotFoundError(f"{ORACLE_LIB} missing; run `make -C oracle`")
        lib = ctypes.CDLL(str(ORACLE_LIB))
        lib.orc_bf16_from_f32.restype = ctypes.c_uint16
        lib.orc_bf16_from_f32.argtypes = [c_float]
        lib.orc_f32_from_bf16.restype = c_float
        lib.orc_f32_from_bf16.argtypes = [ctypes.c_uint16]
        lib.orc_f16_from_f32.restype = ctypes.c_uint16
        lib.orc_f16_from_f32.argtypes = [c_float]
        lib.orc_f32_from_f16.restype = c_float
        lib.orc_f32_from_f16.argtypes = [ctypes.c_uint16]
        lib.orc_round_to_bf16.argtypes = [c_void_p, c_void_p, ctypes.c_size_t]
        lib.orc_round_to_f16.argtypes = [c_void_p, c_void_p, ctypes.c_size_t]
        lib.orc_block_byte_size.restype = c_uint64
        lib.orc_block_byte_size.argtypes = [c_uint32] * 5
        lib.orc_block_stride.restype = c_uint64
        lib.orc_block_stride.argtypes = [c_uint64, c_uint64]
        lib.orc_layout_strides.argtypes = [c_uint32] * 4 + [POINTER(c_uint64)]
        lib.orc_element_offset.restype = c_int64
        lib.orc_element_offset.argtypes = [c_uint32] * 8
        lib.orc_paged_attention_decode.restype = c_int
        lib.orc_paged_attention_decode.argtypes = [
            c_void_p, c_uint64, c_uint32, _u32p, c_uint32, c_int, c_void_p,
            c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_float, c_void_p, c_void_p,
        ]
        lib.orc_paged_decode_batch.restype = c_int
        lib.orc_paged_decode_batch.argtypes = [
            c_void_p, c_uint64, c_uint32, c_uint32, _u32p, _u32p, _u32p, c_int, c_void_p,
            c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_float, c_void_p, c_void_p, c_int,
        ]
        lib.orc_pack.restype = c_int
        lib.orc_pack.argtypes = [
            c_uint32, _u32p, _u32p, _u32p, c_uint32, c_uint32, c_uint32, _u32p, _u32p,
            _i32p, _i32p, _i32p, _i32p, _i32p, _i32p,
        ]
        lib.orc_copy_block.argtypes = [c_void_p, c_uint64, c_uint32, c_uint32, c_uint32, c_uint64]
        lib.orc_append_kv.restype = ctypes.c_int
        lib.orc_append_kv.argtypes = [c_void_p, c_uint64] + [c_uint32] * 8 + [_u32p, _u32p, c_uint32, c_void_p,
                                                                              c_void_p]
        lib.orc_mrope_positions.restype = ctypes.c_int
        lib.orc_mrope_positions.argtypes = [c_void_p, c_uint32, c_uint32, c_uint32, c_void_p]
        _oracle = lib
    return _oracle


def reference_available() -> bool:
    return REF_LIB.exists()


def reference() -> ctypes.CDLL:
    global _ref
    if _ref is None:
        if not REF_LIB.exists():
            raise FileNotFoundError(f"{REF_LIB} missing (reference tree not present at build time)")
        lib = ctypes.CDLL(str(REF_LIB))
        lib.ref_session_create.restype = c_void_p
        lib.ref_session_create.argtypes = [c_void_p, c_uint64, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                                           c_uint32]
        lib.ref_session_destroy.argtypes = [c_void_p]
        lib.ref_session_decode.restype = c_int
        lib.ref_session_decode.argtypes = [c_void_p, c_uint32, _u32p, _u32p, _u32p, c_int, c_void_p, c_uint32,
                                           c_uint32, c_float, c_void_p, POINTER(c_double)]
        lib.ref_session_decode_threads.restype = c_int
        lib.ref_session_decode_threads.argtypes = list(lib.ref_session_decode.argtypes) + [c_uint32]
        lib.ref_block_byte_size.restype = c_uint64
        lib.ref_block_byte_size.argtypes = [c_uint32] * 5
        lib.ref_block_size_bytes.restype = c_uint64
        lib.ref_block_size_bytes.argtypes = [c_uint32] * 5 + [c_uint64]
        lib.ref_half_from_float.restype = ctypes.c_uint16
        lib.ref_half_from_float.argtypes = [c_float]
        lib.ref_float_from_half.restype = c_float
        lib.ref_float_from_half.argtypes = [ctypes.c_uint16]
        lib.ref_element_offset.restype = c_int64
        lib.ref_element_offset.argtypes = [c_uint32] * 8
        _ref = lib
    return _ref


def _u32(a):
    arr = np.ascontiguousarray(a, dtype=np.uint32)
    if arr.size == 0:
        arr = np.zeros(1, np.uint32)
    return arr, arr.ctypes.data_as(_u32p)


def decode_batch(pool: np.ndarray, block_stride: int, num_pool_blocks: int, ids, cu_blocks, context_lens,
                 dtype: int, query: np.ndarray, layer: int, num_layers: int, hq: int, hkv: int, d: int, tpb: int,
                 scale: float, threads: int = 1) -> tuple[int, np.ndarray, np.ndarray]:
    """Oracle decode of a CSR batch. Returns (refused, out in dtype, out_f32)."""
    pool = np.ascontiguousarray(pool)
    query = np.ascontiguousarray(query)
    ids_a, ids_p = _u32(ids)
    cu_a, cu_p = _u32(cu_blocks)
    ctx_a, ctx_p = _u32(context_lens)
    B = len(np.asarray(context_lens))
    np_dtype = np.float32 if dtype == ORC_F32 else np.uint16
    out = np.zeros((B, hq, d), dtype=np_dtype)
    out_f32 = np.zeros((B, hq, d), dtype=np.float32)
    refused = oracle().orc_paged_decode_batch(
        pool.ctypes.data, block_stride, num_pool_blocks, B, ids_p, cu_p, ctx_p, dtype, query.ctypes.data,
        layer, num_layers, hq, hkv, d, tpb, scale, out.ctypes.data, out_f32.ctypes.data, threads)
    return refused, out, out_f32


def append_kv(pool: np.ndarray, block_stride: int, num_pool_blocks: int, elem_bytes: int, tpb: int,
              num_layers: int, hkv: int, d: int, first_layer: int, layer_count: int, frames, slots,
              k: np.ndarray, v: np.ndarray) -> int:
    """Applies one step's K/V writes to a host pool image in place; -1 = refused."""
    assert pool.flags["C_CONTIGUOUS"]
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    f_a, f_p = _u32(frames)
    s_a, s_p = _u32(slots)
    return oracle().orc_append_kv(pool.ctypes.data, block_stride, num_pool_blocks, elem_bytes, tpb, num_layers,
                                  hkv, d, first_layer, layer_count, f_p, s_p, len(np.atleast_1d(frames)),
                                  k.ctypes.data, v.ctypes.data)


# orc_mrope_span (oracle.h): PositionalEncodingSpan plus grid extents.
MROPE_SPAN = np.dtype([("start_token", "<u4"), ("token_count", "<u4"), ("kind", "<u4"), ("reserved", "<u4"),
                       ("origin", "<i8", 3), ("stride", "<i8", 3), ("grid", "<i8", 3)])
assert MROPE_SPAN.itemsize == 88


def mrope_positions(spans: np.ndarray, begin: int, end: int):
    """Positions [3][end - begin] (int64) of one sequence, or None when refused."""
    spans = np.ascontiguousarray(spans, dtype=MROPE_SPAN)
    out = np.zeros((3, max(end - begin, 0)), np.int64)
    rc = oracle().orc_mrope_positions(spans.ctypes.data if len(spans) else None, len(spans), begin, end,
                                      out.ctypes.data)
    return None if rc != 0 else out


def pack(ids, cu_blocks, context_lens, tpb: int, num_pool_blocks: int, split_tokens: int = 0):
    """Expected qvp_pack arrays, or None when the batch would be refused."""
    lib = oracle()
    ids_a, ids_p = _u32(ids)
    cu_a, cu_p = _u32(cu_blocks)
    ctx_a, ctx_p = _u32(context_lens)
    B = len(np.asarray(context_lens))
    max_nb = c_uint32(0)
    nspl = c_uint32(0)
    null = ctypes.cast(None, _i32p)
    if lib.orc_pack(B, ids_p, cu_p, ctx_p, tpb, num_pool_blocks, split_tokens, ctypes.byref(max_nb),
                    ctypes.byref(nspl), null, null, null, null, null, null) != 0:
        return None
    out = {
        "block_tables": np.zeros(max(B * max_nb.value, 1), np.int32),
        "seq_lens": np.zeros(max(B, 1), np.int32),
        "cu_seqlens": np.zeros(B + 1, np.int32),
        "cu_splits": np.zeros(B + 1, np.int32),
        "split_seq": np.zeros(max(nspl.value, 1), np.int32),
        "split_start": np.zeros(max(nspl.value, 1), np.int32),
    }
    ptrs = [out[k].ctypes.data_as(_i32p) for k in
            ("block_tables", "seq_lens", "cu_seqlens", "cu_splits", "split_seq", "split_start")]
    lib.orc_pack(B, ids_p, cu_p, ctx_p, tpb, num_pool_blocks, split_tokens, None, None, *ptrs)
    out["block_tables"] = out["block_tables"][: B * max_nb.value].reshape(B, max_nb.value)
    out["seq_lens"] = out["seq_lens"][:B]
    out["split_seq"] = out["split_seq"][: nspl.value]
    out["split_start"] = out["split_start"][: nspl.value]
    return out


class RefSession:
    """The compiled reference allocator holding a copy of a flat pool."""

    def __init__(self, pool: np.ndarray, stride: int, num_blocks: int, tpb: int, num_layers: int, hkv: int,
                 d: int, bpe: int):
        self._pool = np.ascontiguousarray(pool)
        self.h = reference().ref_session_create(self._pool.ctypes.data, stride, num_blocks, tpb, num_layers, hkv,
                                                d, bpe)

    def decode(self, ids, cu_blocks, context_lens, dtype: int, query: np.ndarray, layer: int, hq: int, d: int,
               scale: float, threads: int = 1) -> tuple[int, np.ndarray, float]:
        ids_a, ids_p = _u32(ids)
        cu_a, cu_p = _u32(cu_blocks)
        ctx_a, ctx_p = _u32(context_lens)
        B = len(np.asarray(context_lens))
        np_dtype = np.float32 if dtype == ORC_F32 else np.uint16
        out = np.zeros((B, hq, d), dtype=np_dtype)
        q = np.ascontiguousarray(query)
        secs = c_double(0.0)
        if threads > 1:
            refused = reference().ref_session_decode_threads(self.h, B, ids_p, cu_p, ctx_p, dtype, q.ctypes.data,
                                                             layer, hq, scale, out.ctypes.data, ctypes.byref(secs),
                                                             threads)
        else:
            refused = reference().ref_session_decode(self.h, B, ids_p, cu_p, ctx_p, dtype, q.ctypes.data, layer,
                                                     hq, scale, out.ctypes.data, ctypes.byref(secs))
        return refused, out, secs.value

    def close(self):
        if self.h:
            reference().ref_session_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def host_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1
