"""numpy restatement of qwenvl-paged_amd/host/bench/kv_pattern.h: the seeded
K/V rows (a function of sequence id and token position) and query rows (a
function of the batch row) the verifying trace driver writes, so the test
suite can rebuild what a frame held and what a decode read."""

from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
GOLDEN2 = np.uint64(0xD1B54A32D192ED03)
KV_SALT = np.uint64(0x632BE59BD9B4E019)
QUERY_SALT = np.uint64(0x8CB92BA72F3D8DD7)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def mix(z: np.ndarray) -> np.ndarray:
    z = np.asarray(z, np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _rows(keys: np.ndarray, exponent_base: int, n: int) -> np.ndarray:
    """bf16 bits [len(keys), n] of the rows with the given keys."""
    assert n % 4 == 0
    keys = np.asarray(keys, np.uint64).reshape(-1, 1)
    g = np.arange(1, n // 4 + 1, dtype=np.uint64).reshape(1, -1)
    with np.errstate(over="ignore"):
        x = mix(keys + g * GOLDEN)
    chunks = np.ascontiguousarray(x).view("<u2").reshape(len(keys), n).astype(np.uint32)
    exponent = exponent_base + ((chunks >> 7) & 0xFF) % 3
    return ((chunks & 0x8000) | (exponent << 7) | (chunks & 0x7F)).astype(np.uint16)


def kv_keys(seq, pos, stream: int) -> np.ndarray:
    seq = np.asarray(seq, np.uint64)
    pos = np.asarray(pos, np.uint64)
    with np.errstate(over="ignore"):
        return mix(seq * GOLDEN + np.uint64(2) * pos + np.uint64(stream) + KV_SALT)


def kv_rows(seq, pos, stream: int, n: int) -> np.ndarray:
    """K (stream 0) or V (stream 1) rows of tokens `pos` of sequences `seq`
    (broadcast together), n = kv heads x head_dim elements each."""
    seq, pos = np.broadcast_arrays(np.asarray(seq, np.uint64), np.asarray(pos, np.uint64))
    return _rows(kv_keys(seq.ravel(), pos.ravel(), stream), 124, n)


def query_rows(rows, n: int) -> np.ndarray:
    rows = np.asarray(rows, np.uint64).ravel()
    with np.errstate(over="ignore"):
        keys = mix(rows * GOLDEN2 + QUERY_SALT)
    return _rows(keys, 125, n)
