"""ctypes binding of libqvp.so (the C ABI declared in include/qvp.h).

This is how Python callers (the tests, bench.py) reach the HIP kernels. It adds
no compute of its own: every call below lands in the shared library, and
loading fails loudly when the library has not been built.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, byref, c_char_p, c_float, c_int, c_size_t, c_uint8, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().with_name("libqvp.so")

OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_UNMAPPED = 2
ERR_OUT_OF_MEMORY = 3
ERR_CAPACITY = 4
ERR_DEVICE = 5

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2
DTYPE_BYTES = {DTYPE_F32: 4, DTYPE_BF16: 2, DTYPE_F16: 2}

UNMAPPED_BLOCK = 0xFFFFFFFF


class QvpError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{message} [{status_name(status)}]")
        self.status = status


class PackedView(ctypes.Structure):
    _fields_ = [
        ("block_tables", c_void_p),
        ("seq_lens", c_void_p),
        ("cu_seqlens", c_void_p),
        ("cu_splits", c_void_p),
        ("split_seq", c_void_p),
        ("split_start", c_void_p),
        ("num_seqs", c_uint32),
        ("max_blocks_per_seq", c_uint32),
        ("num_splits", c_uint32),
        ("split_tokens", c_uint32),
        ("tokens_per_block", c_uint32),
        ("num_pool_blocks", c_uint32),
        ("max_seq_len", c_uint32),
        ("total_tokens", c_uint64),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("query", c_void_p),
        ("out", c_void_p),
        ("kv_base", c_void_p),
        ("block_stride", c_uint64),
        ("batch", c_void_p),
        ("kv_dtype", c_uint32),
        ("out_dtype", c_uint32),
        ("layer", c_uint32),
        ("num_layers", c_uint32),
        ("num_query_heads", c_uint32),
        ("num_kv_heads", c_uint32),
        ("head_dim", c_uint32),
        ("tokens_per_block", c_uint32),
        ("head_stride", c_uint64),
        ("token_stride", c_uint64),
        ("stream_stride", c_uint64),
        ("layer_stride", c_uint64),
        ("scale", c_float),
        ("workspace", c_void_p),
        ("workspace_bytes", c_uint64),
        ("split_event", c_void_p),
        ("tile_engine", c_uint32),
        ("shared_prefix_groups", c_uint32),
        ("shared_prefix_items", c_uint32),
    ]


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("query", c_void_p),
        ("out", c_void_p),
        ("kv_base", c_void_p),
        ("block_stride", c_uint64),
        ("batch", c_void_p),
        ("q_start", POINTER(c_uint32)),
        ("kv_dtype", c_uint32),
        ("out_dtype", c_uint32),
        ("layer", c_uint32),
        ("num_layers", c_uint32),
        ("num_query_heads", c_uint32),
        ("num_kv_heads", c_uint32),
        ("head_dim", c_uint32),
        ("tokens_per_block", c_uint32),
        ("head_stride", c_uint64),
        ("token_stride", c_uint64),
        ("stream_stride", c_uint64),
        ("layer_stride", c_uint64),
        ("scale", c_float),
    ]


class AppendArgs(ctypes.Structure):
    _fields_ = [
        ("kv_base", c_void_p),
        ("block_stride", c_uint64),
        ("num_blocks", c_uint32),
        ("kv_dtype", c_uint32),
        ("num_layers", c_uint32),
        ("first_layer", c_uint32),
        ("layer_count", c_uint32),
        ("num_kv_heads", c_uint32),
        ("head_dim", c_uint32),
        ("tokens_per_block", c_uint32),
        ("head_stride", c_uint64),
        ("token_stride", c_uint64),
        ("stream_stride", c_uint64),
        ("layer_stride", c_uint64),
        ("k", c_void_p),
        ("v", c_void_p),
    ]


class DecodePlan(ctypes.Structure):
    _fields_ = [
        ("kernel", c_uint32),
        ("workgroups", c_uint32),
        ("pieces", c_uint32),
        ("slots", c_uint32),
        ("kv_heads_per_segment", c_uint32),
        ("split_tokens", c_uint32),
        ("deferred_results", c_uint32),
        ("query_group", c_uint32),
        ("tile_engine", c_uint32),
        ("shared_prefix_groups", c_uint32),
        ("shared_prefix_items", c_uint32),
    ]


DECODE_KERNELS = {0: "none", 1: "mfma", 2: "f32_grouped", 3: "generic", 4: "grouped", 5: "split_mfma"}
# qvp_tile_engine: arithmetic of the persistent bf16 kernel's tiles.
TILE_AUTO = 0
TILE_MATRIX = 1
TILE_VECTOR = 2
TILE_ENGINES = {0: "none", 1: "matrix", 2: "vector"}

_u32p = POINTER(c_uint32)
_u64p = POINTER(c_uint64)

# name -> (restype, argtypes); every function include/qvp.h declares.
SIGNATURES = {
    "qvp_last_error": (c_char_p, []),
    "qvp_status_name": (c_char_p, [c_int]),
    "qvp_version": (c_int, []),
    "qvp_device_count": (c_int, [POINTER(c_int)]),
    "qvp_set_device": (c_int, [c_int]),
    "qvp_device_synchronize": (c_int, []),
    "qvp_malloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "qvp_free": (c_int, [c_void_p]),
    "qvp_host_alloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "qvp_host_free": (c_int, [c_void_p]),
    "qvp_host_device_pointer": (c_int, [POINTER(c_void_p), c_void_p]),
    "qvp_memcpy_htod": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "qvp_memcpy_dtoh": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "qvp_memcpy_dtod": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "qvp_fill_bytes": (c_int, [c_void_p, c_uint8, c_size_t, c_void_p]),
    "qvp_stream_create": (c_int, [POINTER(c_void_p)]),
    "qvp_stream_destroy": (c_int, [c_void_p]),
    "qvp_stream_synchronize": (c_int, [c_void_p]),
    "qvp_event_create": (c_int, [POINTER(c_void_p)]),
    "qvp_event_destroy": (c_int, [c_void_p]),
    "qvp_event_record": (c_int, [c_void_p, c_void_p]),
    "qvp_event_synchronize": (c_int, [c_void_p]),
    "qvp_stream_wait_event": (c_int, [c_void_p, c_void_p]),
    "qvp_event_query": (c_int, [c_void_p, POINTER(c_int)]),
    "qvp_event_elapsed_ms": (c_int, [POINTER(c_float), c_void_p, c_void_p]),
    "qvp_pool_create": (c_int, [c_uint32, c_size_t, c_size_t, POINTER(c_void_p)]),
    "qvp_pool_destroy": (c_int, [c_void_p]),
    "qvp_pool_base": (c_void_p, [c_void_p]),
    "qvp_pool_block_stride": (c_size_t, [c_void_p]),
    "qvp_pool_block_bytes": (c_size_t, [c_void_p]),
    "qvp_pool_num_blocks": (c_uint32, [c_void_p]),
    "qvp_pool_block_ptr": (c_void_p, [c_void_p, c_uint32]),
    "qvp_pool_write": (c_int, [c_void_p, c_uint32, c_size_t, c_void_p, c_size_t, c_void_p]),
    "qvp_pool_read": (c_int, [c_void_p, c_uint32, c_size_t, c_void_p, c_size_t, c_void_p]),
    "qvp_batch_create": (c_int, [POINTER(c_void_p)]),
    "qvp_batch_destroy": (c_int, [c_void_p]),
    "qvp_pack": (c_int, [c_void_p, c_uint32, _u32p, _u32p, _u32p, c_uint32, c_uint32, c_uint32, c_void_p]),
    "qvp_batch_view": (c_int, [c_void_p, POINTER(PackedView)]),
    "qvp_decode_workspace_bytes": (c_int, [c_void_p, c_uint32, c_uint32, _u64p]),
    "qvp_paged_decode": (c_int, [POINTER(DecodeArgs), c_void_p]),
    "qvp_decode_plan_info": (c_int, [c_void_p, POINTER(DecodePlan)]),
    "qvp_paged_decode_noalloc": (c_int, [POINTER(DecodeArgs), c_void_p]),
    "qvp_pack_for_decode": (c_int, [c_void_p, c_uint32, _u32p, _u32p, _u32p, c_uint32, c_uint32, c_uint32,
                                    c_void_p, c_void_p]),
    "qvp_pack_ahead": (c_int, [c_void_p, c_uint32, _u32p, _u32p, _u32p, c_uint32, c_uint32, c_uint32,
                                    c_void_p, c_void_p]),
    "qvp_batch_upload": (c_int, [c_void_p, c_void_p]),
    "qvp_copy_blocks": (c_int, [c_void_p, c_uint64, c_uint32, _u32p, _u32p, c_uint32, c_uint64, c_void_p]),
    "qvp_swap_gather": (
        c_int,
        [c_void_p, c_uint64, c_uint32, _u32p, _u64p, c_uint32, c_void_p, c_uint64, c_uint64, c_void_p],
    ),
    "qvp_swap_scatter": (
        c_int,
        [c_void_p, c_uint64, c_uint32, _u32p, _u64p, c_uint32, c_void_p, c_uint64, c_uint64, c_void_p],
    ),
    "qvp_append_kv": (c_int, [POINTER(AppendArgs), _u32p, _u32p, c_uint32, c_void_p]),
    "qvp_copy_append_kv": (c_int, [POINTER(AppendArgs), _u32p, _u32p, c_uint32, c_uint64, _u32p, _u32p, c_uint32,
                                   c_void_p]),
    "qvp_paged_prefill": (c_int, [POINTER(PrefillArgs), c_void_p]),
    "qvp_graph_begin_capture": (c_int, [c_void_p]),
    "qvp_graph_end_capture": (c_int, [c_void_p, POINTER(c_void_p)]),
    "qvp_graph_launch": (c_int, [c_void_p, c_void_p]),
    "qvp_graph_destroy": (c_int, [c_void_p]),
    "qvp_mrope_create": (c_int, [POINTER(c_void_p)]),
    "qvp_mrope_destroy": (c_int, [c_void_p]),
    "qvp_mrope_positions": (c_int, [c_void_p, c_void_p, _u32p, _u32p, _u32p, c_uint32, c_void_p, c_uint64,
                                    c_void_p]),
}

_lib: ctypes.CDLL | None = None


def load(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Loads libqvp.so; raises if it is missing (there is no fallback path)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is not built; run `python qwenvl-paged_amd/build.py` (the HIP library is required)"
        )
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def status_name(status: int) -> str:
    return load().qvp_status_name(status).decode()


def check(status: int) -> None:
    if status != OK:
        raise QvpError(status, load().qvp_last_error().decode())


def _u32(a) -> tuple[np.ndarray, ctypes._Pointer]:
    arr = np.ascontiguousarray(a, dtype=np.uint32)
    return arr, arr.ctypes.data_as(_u32p)


def _u64(a) -> tuple[np.ndarray, ctypes._Pointer]:
    arr = np.ascontiguousarray(a, dtype=np.uint64)
    return arr, arr.ctypes.data_as(_u64p)


# --------------------------------------------------------------------------
# Runtime plumbing
# --------------------------------------------------------------------------


def device_count() -> int:
    n = c_int(0)
    check(load().qvp_device_count(byref(n)))
    return n.value


def synchronize() -> None:
    check(load().qvp_device_synchronize())


class DeviceBuffer:
    """A device allocation owned by this object."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = c_void_p()
        check(load().qvp_malloc(byref(p), self.nbytes))
        self.ptr = p.value or 0

    @classmethod
    def from_array(cls, arr: np.ndarray, stream=None) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr, stream)
        if stream is not None:
            stream.synchronize()
        return buf

    def upload(self, arr: np.ndarray, stream=None, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError("upload exceeds buffer")
        check(load().qvp_memcpy_htod(self.ptr + offset, arr.ctypes.data, arr.nbytes, _sp(stream)))
        if stream is None:
            synchronize()

    def download(self, dtype, shape, stream=None, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download exceeds buffer")
        check(load().qvp_memcpy_dtoh(out.ctypes.data, self.ptr + offset, out.nbytes, _sp(stream)))
        if stream is None:
            synchronize()
        else:
            stream.synchronize()
        return out

    def fill(self, value: int, stream=None) -> None:
        check(load().qvp_fill_bytes(self.ptr, value, self.nbytes, _sp(stream)))

    def free(self) -> None:
        if self.ptr:
            check(load().qvp_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PinnedBuffer:
    """Pinned host memory (qvp_host_alloc) viewed as a numpy byte array."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = c_void_p()
        check(load().qvp_host_alloc(byref(p), self.nbytes))
        self.ptr = p.value or 0
        self.array = np.ctypeslib.as_array((ctypes.c_uint8 * self.nbytes).from_address(self.ptr)) if self.ptr else np.empty(0, np.uint8)

    def free(self) -> None:
        if self.ptr:
            self.array = None
            check(load().qvp_host_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _sp(stream) -> int | None:
    if stream is None:
        return None
    return stream.handle if isinstance(stream, Stream) else stream


class Stream:
    def __init__(self):
        p = c_void_p()
        check(load().qvp_stream_create(byref(p)))
        self.handle = p.value

    def synchronize(self) -> None:
        check(load().qvp_stream_synchronize(self.handle))

    def wait(self, event: "Event") -> None:
        check(load().qvp_stream_wait_event(self.handle, event.handle))

    def destroy(self) -> None:
        if self.handle:
            check(load().qvp_stream_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Event:
    def __init__(self):
        p = c_void_p()
        check(load().qvp_event_create(byref(p)))
        self.handle = p.value

    def record(self, stream=None) -> None:
        check(load().qvp_event_record(self.handle, _sp(stream)))

    def synchronize(self) -> None:
        check(load().qvp_event_synchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float(0.0)
        check(load().qvp_event_elapsed_ms(byref(ms), self.handle, end.handle))
        return ms.value

    def destroy(self) -> None:
        if self.handle:
            check(load().qvp_event_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


# --------------------------------------------------------------------------
# Pool, batch, kernels
# --------------------------------------------------------------------------


class BlockPool:
    """HBM block pool (qvp_pool_*)."""

    def __init__(self, num_blocks: int, block_bytes: int, alignment: int = 256):
        p = c_void_p()
        check(load().qvp_pool_create(num_blocks, block_bytes, alignment, byref(p)))
        self.handle = p.value
        lib = load()
        self.base = lib.qvp_pool_base(self.handle)
        self.stride = lib.qvp_pool_block_stride(self.handle)
        self.block_bytes = lib.qvp_pool_block_bytes(self.handle)
        self.num_blocks = lib.qvp_pool_num_blocks(self.handle)

    def block_ptr(self, block: int) -> int | None:
        return load().qvp_pool_block_ptr(self.handle, block)

    def write(self, block: int, data: np.ndarray, offset: int = 0, stream=None) -> None:
        data = np.ascontiguousarray(data)
        check(load().qvp_pool_write(self.handle, block, offset, data.ctypes.data, data.nbytes, _sp(stream)))
        if stream is None:
            synchronize()

    def read(self, block: int, nbytes: int | None = None, offset: int = 0) -> np.ndarray:
        n = self.stride - offset if nbytes is None else nbytes
        out = np.empty(n, dtype=np.uint8)
        check(load().qvp_pool_read(self.handle, block, offset, out.ctypes.data, n, None))
        synchronize()
        return out

    def upload_all(self, frames: np.ndarray, stream=None) -> None:
        """Copies a host image of the whole pool (num_blocks * stride bytes)."""
        frames = np.ascontiguousarray(frames).view(np.uint8).reshape(-1)
        if frames.nbytes != self.num_blocks * self.stride:
            raise ValueError(f"pool image is {frames.nbytes} bytes, pool is {self.num_blocks * self.stride}")
        check(load().qvp_memcpy_htod(self.base, frames.ctypes.data, frames.nbytes, _sp(stream)))
        if stream is None:
            synchronize()

    def download_all(self) -> np.ndarray:
        out = np.empty(self.num_blocks * self.stride, dtype=np.uint8)
        check(load().qvp_memcpy_dtoh(out.ctypes.data, self.base, out.nbytes, None))
        synchronize()
        return out

    def destroy(self) -> None:
        if self.handle:
            check(load().qvp_pool_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Batch:
    """Packed ragged batch (qvp_batch_* / qvp_pack)."""

    def __init__(self):
        p = c_void_p()
        check(load().qvp_batch_create(byref(p)))
        self.handle = p.value

    def pack(self, ids, cu_blocks, context_lens, tokens_per_block: int, num_pool_blocks: int,
             split_tokens: int = 0, stream=None, decode: "DecodeArgs | None" = None,
             ahead: bool = False) -> PackedView:
        """qvp_pack, or qvp_pack_for_decode when the decode the pack is for is
        given; with ahead=True qvp_pack_ahead (the upload left pending for the
        next decode of another batch on the stream)."""
        ids_a, ids_p = _u32(ids if len(ids) else np.zeros(1, np.uint32))
        cu_a, cu_p = _u32(cu_blocks)
        ctx_a, ctx_p = _u32(context_lens)
        num_seqs = len(ctx_a)
        if ahead:
            check(load().qvp_pack_ahead(self.handle, num_seqs, ids_p, cu_p, ctx_p, tokens_per_block,
                                        num_pool_blocks, split_tokens, byref(decode) if decode is not None else None,
                                        _sp(stream)))
        elif decode is None:
            check(load().qvp_pack(self.handle, num_seqs, ids_p, cu_p, ctx_p, tokens_per_block, num_pool_blocks,
                                  split_tokens, _sp(stream)))
        else:
            check(load().qvp_pack_for_decode(self.handle, num_seqs, ids_p, cu_p, ctx_p, tokens_per_block,
                                             num_pool_blocks, split_tokens, byref(decode), _sp(stream)))
        # The library copies from pinned staging, so the numpy inputs may go now.
        return self.view()

    def upload(self, stream=None) -> None:
        """qvp_batch_upload: enqueue a pending pack-ahead upload now."""
        check(load().qvp_batch_upload(self.handle, _sp(stream)))

    def view(self) -> PackedView:
        v = PackedView()
        check(load().qvp_batch_view(self.handle, byref(v)))
        return v

    def download(self) -> dict[str, np.ndarray]:
        """Reads the device arrays of the last pack back to the host."""
        synchronize()
        v = self.view()
        B, nb, S = v.num_seqs, v.max_blocks_per_seq, v.num_splits
        out = {}
        for name, count in (("block_tables", B * nb), ("seq_lens", B), ("cu_seqlens", B + 1),
                            ("cu_splits", B + 1), ("split_seq", S), ("split_start", S)):
            arr = np.empty(count, dtype=np.int32)
            if count:
                check(load().qvp_memcpy_dtoh(arr.ctypes.data, getattr(v, name), arr.nbytes, None))
            out[name] = arr
        synchronize()
        out["block_tables"] = out["block_tables"].reshape(B, nb)
        return out

    def decode_plan(self) -> dict:
        """The work decomposition of the last decode on this pack."""
        p = DecodePlan()
        check(load().qvp_decode_plan_info(self.handle, byref(p)))
        d = {name: int(getattr(p, name)) for name, _ in DecodePlan._fields_}
        d["kernel"] = DECODE_KERNELS.get(d["kernel"], str(d["kernel"]))
        d["tile_engine"] = TILE_ENGINES.get(d["tile_engine"], str(d["tile_engine"]))
        return d

    def workspace_bytes(self, num_query_heads: int, head_dim: int) -> int:
        n = c_uint64(0)
        check(load().qvp_decode_workspace_bytes(self.handle, num_query_heads, head_dim, byref(n)))
        return n.value

    def destroy(self) -> None:
        if self.handle:
            check(load().qvp_batch_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class Graph:
    """A captured stream (qvp_graph_*): `with Graph.capture(stream) as g:` then g.launch(stream)."""

    def __init__(self, handle: int):
        self.handle = handle

    @staticmethod
    def capture(stream: "Stream"):
        return _Capture(stream)

    def launch(self, stream=None) -> None:
        check(load().qvp_graph_launch(self.handle, _sp(stream)))

    def destroy(self) -> None:
        if self.handle:
            check(load().qvp_graph_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class _Capture:
    def __init__(self, stream):
        self.stream = stream
        self.graph = Graph(None)

    def __enter__(self) -> Graph:
        check(load().qvp_graph_begin_capture(_sp(self.stream)))
        return self.graph

    def __exit__(self, exc_type, exc, tb):
        h = c_void_p()
        rc = load().qvp_graph_end_capture(_sp(self.stream), byref(h))
        if exc_type is None:
            check(rc)
            self.graph.handle = h.value
        elif rc == 0 and h.value:
            # The capture ended because its body raised: nothing to replay.
            load().qvp_graph_destroy(h.value)
        return False


# qvp_mrope_span: PositionalEncodingSpan with grid extents.
MROPE_SPAN = np.dtype([("start_token", "<u4"), ("token_count", "<u4"), ("kind", "<u4"), ("reserved", "<u4"),
                       ("origin", "<i8", 3), ("stride", "<i8", 3), ("grid", "<i8", 3)])


class MRope:
    """M-RoPE position materialisation (qvp_mrope_*)."""

    def __init__(self):
        p = c_void_p()
        check(load().qvp_mrope_create(byref(p)))
        self.handle = p.value

    def positions(self, spans, cu_spans, begin, end, out: int, total_rows: int, stream=None) -> None:
        """Writes int64 [3][total_rows] positions to device address `out`."""
        spans = np.ascontiguousarray(spans, dtype=MROPE_SPAN)
        cu_a, cu_p = _u32(cu_spans)
        b_a, b_p = _u32(begin)
        e_a, e_p = _u32(end)
        check(load().qvp_mrope_positions(self.handle, spans.ctypes.data if len(spans) else None, cu_p, b_p, e_p,
                                         len(b_a), out, total_rows, _sp(stream)))

    def destroy(self) -> None:
        if self.handle:
            check(load().qvp_mrope_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def layout_strides(tokens_per_block: int, num_layers: int, num_kv_heads: int, head_dim: int) -> dict:
    """KVBlockLayout strides in elements (CacheLayout.cpp:5-23)."""
    head = head_dim
    token = num_kv_heads * head
    stream = tokens_per_block * token
    layer = 2 * stream
    return {"head_stride": head, "token_stride": token, "stream_stride": stream, "layer_stride": layer}


def decode_args(*, query: int, out: int, kv_base: int, block_stride: int, batch: Batch, kv_dtype: int,
                out_dtype: int, layer: int, num_layers: int, num_query_heads: int, num_kv_heads: int,
                head_dim: int, tokens_per_block: int, scale: float, strides: dict | None = None,
                workspace: int = 0, workspace_bytes: int = 0, split_event: "Event | None" = None,
                tile_engine: int = TILE_AUTO) -> DecodeArgs:
    s = strides or layout_strides(tokens_per_block, num_layers, num_kv_heads, head_dim)
    return DecodeArgs(query, out, kv_base, block_stride, batch.handle, kv_dtype, out_dtype, layer, num_layers,
                      num_query_heads, num_kv_heads, head_dim, tokens_per_block, s["head_stride"],
                      s["token_stride"], s["stream_stride"], s["layer_stride"], scale, workspace or None,
                      workspace_bytes, split_event.handle if split_event is not None else None, tile_engine)


def paged_decode(args: DecodeArgs, stream=None) -> None:
    check(load().qvp_paged_decode(byref(args), _sp(stream)))


def paged_decode_noalloc(args: DecodeArgs, stream=None) -> None:
    """qvp_paged_decode_noalloc: the decode on the library's fixed device
    scratch array, allocating nothing (args.workspace must be 0)."""
    check(load().qvp_paged_decode_noalloc(byref(args), _sp(stream)))


def copy_blocks(kv_base: int, block_stride: int, num_blocks: int, src, dst, copy_bytes: int, stream=None) -> None:
    s_a, s_p = _u32(src)
    d_a, d_p = _u32(dst)
    if len(s_a) != len(d_a):
        raise ValueError("src and dst differ in length")
    check(load().qvp_copy_blocks(kv_base, block_stride, num_blocks, s_p, d_p, len(s_a), copy_bytes, _sp(stream)))


def swap_gather(kv_base: int, block_stride: int, num_blocks: int, frames, offsets, arena: PinnedBuffer,
                copy_bytes: int, stream=None) -> None:
    f_a, f_p = _u32(frames)
    o_a, o_p = _u64(offsets)
    check(load().qvp_swap_gather(kv_base, block_stride, num_blocks, f_p, o_p, len(f_a), arena.ptr, arena.nbytes,
                                 copy_bytes, _sp(stream)))


def swap_scatter(kv_base: int, block_stride: int, num_blocks: int, frames, offsets, arena: PinnedBuffer,
                 copy_bytes: int, stream=None) -> None:
    f_a, f_p = _u32(frames)
    o_a, o_p = _u64(offsets)
    check(load().qvp_swap_scatter(kv_base, block_stride, num_blocks, f_p, o_p, len(f_a), arena.ptr, arena.nbytes,
                                  copy_bytes, _sp(stream)))


def append_args(*, kv_base: int, block_stride: int, num_blocks: int, kv_dtype: int, num_layers: int,
                first_layer: int, layer_count: int, num_kv_heads: int, head_dim: int, tokens_per_block: int,
                k: int, v: int, strides: dict | None = None) -> AppendArgs:
    s = strides or layout_strides(tokens_per_block, num_layers, num_kv_heads, head_dim)
    return AppendArgs(kv_base, block_stride, num_blocks, kv_dtype, num_layers, first_layer, layer_count,
                      num_kv_heads, head_dim, tokens_per_block, s["head_stride"], s["token_stride"],
                      s["stream_stride"], s["layer_stride"], k, v)


def append_kv(args: AppendArgs, frames, slots, stream=None) -> None:
    """Writes count tokens' K/V rows (qvp_append_kv); frames and slots are host arrays."""
    f_a, f_p = _u32(frames)
    s_a, s_p = _u32(slots)
    if len(f_a) != len(s_a):
        raise ValueError("frames and slots differ in length")
    check(load().qvp_append_kv(byref(args), f_p, s_p, len(f_a), _sp(stream)))


def copy_append_kv(args: AppendArgs, src, dst, copy_bytes: int, frames, slots, stream=None) -> None:
    """A copy-on-write step in one launch (qvp_copy_append_kv): copy_blocks(src, dst, copy_bytes) then
    append_kv(frames, slots) on the pool args describes."""
    s_a, s_p = _u32(src)
    d_a, d_p = _u32(dst)
    f_a, f_p = _u32(frames)
    t_a, t_p = _u32(slots)
    if len(s_a) != len(d_a) or len(f_a) != len(t_a):
        raise ValueError("src/dst or frames/slots differ in length")
    check(load().qvp_copy_append_kv(byref(args), s_p, d_p, len(s_a), copy_bytes, f_p, t_p, len(f_a), _sp(stream)))


def prefill_args(*, query: int, out: int, kv_base: int, block_stride: int, batch: "Batch", q_start, kv_dtype: int,
                 out_dtype: int, layer: int, num_layers: int, num_query_heads: int, num_kv_heads: int, head_dim: int,
                 tokens_per_block: int, scale: float, strides: dict | None = None) -> PrefillArgs:
    """Arguments of qvp_paged_prefill; keeps the q_start array alive on the returned object."""
    s = strides or layout_strides(tokens_per_block, num_layers, num_kv_heads, head_dim)
    qs, qs_p = _u32(q_start)
    a = PrefillArgs(query, out, kv_base, block_stride, batch.handle, qs_p, kv_dtype, out_dtype, layer, num_layers,
                    num_query_heads, num_kv_heads, head_dim, tokens_per_block, s["head_stride"], s["token_stride"],
                    s["stream_stride"], s["layer_stride"], scale)
    a._q_start = qs
    return a


def paged_prefill(args: PrefillArgs, stream=None) -> None:
    check(load().qvp_paged_prefill(byref(args), _sp(stream)))
