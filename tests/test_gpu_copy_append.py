"""GPU parity: a copy-on-write step in one launch (qvp_copy_append_kv).

The reference's order within a step is: KVCacheManager::ensure_token_writable
copies a shared block into a fresh frame (src/KVCacheManager.cpp:141-150, the
memcpy of MemoryAllocator::copy_block, src/MemoryAllocator.cpp:76-85), then the
harness stores the token's K/V rows into that frame
(tests/PagedAttention.test.cpp:97-127). Byte work, so the bar is bit-exact:
the whole pool image after the one launch equals the oracle's image after its
copies (orc_copy_block) and then its append (orc_append_kv), and equals the
image of the two separate launches (qvp_copy_blocks, qvp_append_kv).
"""

from __future__ import annotations

import numpy as np
import pytest

import pyoracle as O
import qvp

pytestmark = pytest.mark.gpu

DTYPE_BYTES = {qvp.DTYPE_F32: 4, qvp.DTYPE_BF16: 2, qvp.DTYPE_F16: 2}


def _setup(tpb, layers, hkv, d, dtype, layer_count, npairs, rows_in_copies, rows_elsewhere, nframes, seed,
           first_layer=0, self_pairs=0):
    """Random pool image; npairs copies between distinct frames; rows_in_copies
    tokens written into copy destinations and rows_elsewhere into frames that no
    copy touches; self_pairs (src == dst) no-op pairs among frames no row or
    copy touches."""
    bpe = DTYPE_BYTES[dtype]
    rng = np.random.default_rng(seed)
    block_bytes = tpb * layers * hkv * d * bpe * 2
    pool = qvp.BlockPool(nframes, block_bytes)
    image = rng.integers(0, 256, nframes * pool.stride, dtype=np.uint8)
    pool.upload_all(image)
    perm = rng.permutation(nframes)
    src = perm[:npairs].astype(np.uint32)
    dst = perm[npairs:2 * npairs].astype(np.uint32)
    others = perm[2 * npairs:]
    idle = others[:self_pairs]
    others = others[self_pairs:]
    # Rows: slots drawn without repetition per frame.
    frames, slots = [], []
    if rows_in_copies:
        cells = rng.choice(npairs * tpb, size=rows_in_copies, replace=False)
        frames += [int(dst[c // tpb]) for c in cells]
        slots += [int(c % tpb) for c in cells]
    if rows_elsewhere:
        cells = rng.choice(len(others) * tpb, size=rows_elsewhere, replace=False)
        frames += [int(others[c // tpb]) for c in cells]
        slots += [int(c % tpb) for c in cells]
    order = rng.permutation(len(frames))
    frames = np.asarray(frames, dtype=np.uint32)[order] if frames else np.zeros(0, np.uint32)
    slots = np.asarray(slots, dtype=np.uint32)[order] if slots else np.zeros(0, np.uint32)
    src = np.concatenate([src, idle.astype(np.uint32)])
    dst = np.concatenate([dst, idle.astype(np.uint32)])
    count = len(frames)
    nbytes = max(count, 1) * layer_count * hkv * d * bpe
    k = rng.integers(0, 256, nbytes, dtype=np.uint8)
    v = rng.integers(0, 256, nbytes, dtype=np.uint8)
    dk, dv = qvp.DeviceBuffer.from_array(k), qvp.DeviceBuffer.from_array(v)
    args = qvp.append_args(kv_base=pool.base, block_stride=pool.stride, num_blocks=nframes, kv_dtype=dtype,
                           num_layers=layers, first_layer=first_layer, layer_count=layer_count, num_kv_heads=hkv,
                           head_dim=d, tokens_per_block=tpb, k=dk.ptr, v=dv.ptr)
    return dict(pool=pool, image=image, src=src, dst=dst, frames=frames, slots=slots, k=k, v=v, dk=dk, dv=dv,
                args=args, bpe=bpe, geom=(tpb, layers, hkv, d, first_layer, layer_count), nframes=nframes)


def _oracle_image(c, copy_bytes):
    exp = c["image"].copy()
    pool = c["pool"]
    for s, d in zip(c["src"], c["dst"]):
        if s != d:
            O.oracle().orc_copy_block(exp.ctypes.data, pool.stride, c["nframes"], int(s), int(d), copy_bytes)
    tpb, layers, hkv, d, first_layer, layer_count = c["geom"]
    if len(c["frames"]):
        assert O.append_kv(exp, pool.stride, c["nframes"], c["bpe"], tpb, layers, hkv, d, first_layer, layer_count,
                           c["frames"], c["slots"], c["k"], c["v"]) == 0
    return exp


CASES = [
    # tpb, layers, hkv, d, dtype, layer_count, pairs, rows in copies, rows elsewhere, frames
    (16, 1, 4, 128, qvp.DTYPE_BF16, 1, 128, 128, 0, 400),    # config4: 128 branches, one row each
    (16, 1, 4, 128, qvp.DTYPE_BF16, 1, 16, 40, 60, 300),     # several rows per copied frame, rows elsewhere
    (16, 1, 2, 64, qvp.DTYPE_F32, 1, 3, 4, 2, 20),           # config1 shape
    (16, 1, 8, 128, qvp.DTYPE_BF16, 1, 32, 32, 32, 200),     # config3 shape
    (16, 28, 4, 128, qvp.DTYPE_BF16, 28, 6, 10, 5, 24),      # whole Qwen2-VL-7B frames, 112 chunks each
    (16, 1, 4, 128, qvp.DTYPE_F16, 1, 0, 0, 128, 40),        # no copies: the append alone
    (16, 1, 4, 128, qvp.DTYPE_BF16, 1, 64, 0, 0, 200),       # no rows: the copies alone
    (16, 1, 4, 128, qvp.DTYPE_BF16, 1, 128, 0, 128, 400),    # rows only in uncopied frames
]


@pytest.mark.parametrize("case", CASES)
def test_copy_append_is_bit_exact_against_copy_then_append(case):
    print(f"case: copy_append {case}", flush=True)
    c = _setup(*case, seed=sum(case))
    pool = c["pool"]
    qvp.copy_append_kv(c["args"], c["src"], c["dst"], pool.stride, c["frames"], c["slots"])
    qvp.synchronize()
    got = pool.download_all()
    assert np.array_equal(got, _oracle_image(c, pool.stride))
    # The same step as two launches gives the same bytes.
    pool.upload_all(c["image"])
    qvp.copy_blocks(pool.base, pool.stride, c["nframes"], c["src"], c["dst"], pool.stride)
    qvp.append_kv(c["args"], c["frames"], c["slots"])
    qvp.synchronize()
    assert np.array_equal(pool.download_all(), got)


def test_copy_append_layer_range_and_partial_copy():
    # Rows of layers 5..7 of 28-layer frames; only the first 100 KiB of each
    # frame is copied, so the rows land past the copied range (written all
    # the same) and the rest of the destination keeps its bytes.
    print("case: copy_append layer range, partial copy", flush=True)
    c = _setup(16, 28, 4, 128, qvp.DTYPE_BF16, 3, 5, 12, 4, 24, seed=11, first_layer=5)
    pool = c["pool"]
    copy_bytes = 100 * 1024
    qvp.copy_append_kv(c["args"], c["src"], c["dst"], copy_bytes, c["frames"], c["slots"])
    qvp.synchronize()
    assert np.array_equal(pool.download_all(), _oracle_image(c, copy_bytes))


def test_copy_append_with_padded_strides():
    # Gaps between kv heads, token rows, streams and layers, and frame padding
    # past the layout: a unit's place in the layout is found from its frame
    # offset, so the gaps must read as "not a row" and keep the copied bytes.
    # Expected image: the frame copies, then each row at its closed-form
    # offset (first_layer + l) * Ls + s * Ss + slot * Ts + h * Hs (elements).
    print("case: copy_append padded strides", flush=True)
    tpb, layers, hkv, d, bpe = 16, 3, 4, 128, 2
    st = {"head_stride": d + 8, "token_stride": hkv * (d + 8) + 16}
    st["stream_stride"] = tpb * st["token_stride"] + 64
    st["layer_stride"] = 2 * st["stream_stride"] + 128
    first_layer, layer_count, nframes = 1, 2, 40
    block_bytes = layers * st["layer_stride"] * bpe + 512
    rng = np.random.default_rng(21)
    pool = qvp.BlockPool(nframes, block_bytes)
    image = rng.integers(0, 256, nframes * pool.stride, dtype=np.uint8)
    pool.upload_all(image)
    perm = rng.permutation(nframes)
    src, dst, others = perm[:8], perm[8:16], perm[16:]
    frames = np.concatenate([dst[[0, 0, 1, 3, 7]], others[[0, 2]]]).astype(np.uint32)
    slots = np.array([0, 15, 7, 3, 9, 4, 11], dtype=np.uint32)
    n = len(frames)
    k = rng.integers(0, 256, n * layer_count * hkv * d * bpe, dtype=np.uint8)
    v = rng.integers(0, 256, n * layer_count * hkv * d * bpe, dtype=np.uint8)
    dk, dv = qvp.DeviceBuffer.from_array(k), qvp.DeviceBuffer.from_array(v)
    args = qvp.append_args(kv_base=pool.base, block_stride=pool.stride, num_blocks=nframes, kv_dtype=qvp.DTYPE_BF16,
                           num_layers=layers, first_layer=first_layer, layer_count=layer_count, num_kv_heads=hkv,
                           head_dim=d, tokens_per_block=tpb, k=dk.ptr, v=dv.ptr, strides=st)
    qvp.copy_append_kv(args, src, dst, pool.stride, frames, slots)
    qvp.synchronize()
    got = pool.download_all()
    exp = image.reshape(nframes, pool.stride).copy()
    exp[dst] = exp[src]
    exp = exp.reshape(-1)
    row = d * bpe
    for i in range(n):
        for l in range(layer_count):
            for s_, data in ((0, k), (1, v)):
                for h in range(hkv):
                    el = ((first_layer + l) * st["layer_stride"] + s_ * st["stream_stride"] +
                          int(slots[i]) * st["token_stride"] + h * st["head_stride"])
                    at = int(frames[i]) * pool.stride + el * bpe
                    src_at = ((i * layer_count + l) * hkv + h) * row
                    exp[at:at + row] = data[src_at:src_at + row]
    assert np.array_equal(got, exp)
    # And the two launches give the same bytes.
    pool.upload_all(image)
    qvp.copy_blocks(pool.base, pool.stride, nframes, src, dst, pool.stride)
    qvp.append_kv(args, frames, slots)
    qvp.synchronize()
    assert np.array_equal(pool.download_all(), got)


def test_copy_append_self_pairs_are_no_ops():
    print("case: copy_append self pairs", flush=True)
    c = _setup(16, 1, 4, 128, qvp.DTYPE_BF16, 1, 8, 8, 4, 64, seed=5, self_pairs=3)
    pool = c["pool"]
    qvp.copy_append_kv(c["args"], c["src"], c["dst"], pool.stride, c["frames"], c["slots"])
    qvp.synchronize()
    assert np.array_equal(pool.download_all(), _oracle_image(c, pool.stride))


def test_copy_append_repeated_calls_with_shrinking_lists():
    # Consecutive steps reuse nothing of each other's lists.
    print("case: copy_append consecutive steps", flush=True)
    for seed, (pairs, rows_in, rows_out) in enumerate([(100, 100, 20), (7, 3, 1), (1, 1, 0)]):
        c = _setup(16, 1, 4, 128, qvp.DTYPE_BF16, 1, pairs, rows_in, rows_out, 300, seed=40 + seed)
        pool = c["pool"]
        qvp.copy_append_kv(c["args"], c["src"], c["dst"], pool.stride, c["frames"], c["slots"])
        qvp.synchronize()
        assert np.array_equal(pool.download_all(), _oracle_image(c, pool.stride)), f"step {seed}"


@pytest.mark.parametrize(
    "what",
    ["row_in_source", "dst_repeats", "dst_is_source", "too_many_pairs", "too_many_rows", "copy_not_16",
     "src_outside", "frame_outside", "slot_twice"],
)
def test_copy_append_refusals_write_nothing(what):
    c = _setup(16, 1, 4, 128, qvp.DTYPE_BF16, 1, 4, 4, 2, 300, seed=3)
    pool = c["pool"]
    src, dst = list(c["src"]), list(c["dst"])
    frames, slots = list(c["frames"]), list(c["slots"])
    copy_bytes = pool.stride
    status = qvp.ERR_INVALID_ARGUMENT
    if what == "row_in_source":
        frames[0] = src[1]
    elif what == "dst_repeats":
        dst[1] = dst[0]
    elif what == "dst_is_source":
        dst[1] = src[0]
    elif what == "too_many_pairs":
        used = set(frames)
        free = [f for f in range(300) if f not in used]
        src, dst = free[:129], free[129:258]
    elif what == "too_many_rows":
        frames = list(range(150, 279))
        slots = [0] * 129
    elif what == "copy_not_16":
        copy_bytes = pool.stride - 8
    elif what == "src_outside":
        src[0] = 300
        status = qvp.ERR_UNMAPPED
    elif what == "frame_outside":
        frames[0] = 300
        status = qvp.ERR_UNMAPPED
    elif what == "slot_twice":
        frames[1], slots[1] = frames[0], slots[0]
    with pytest.raises(qvp.QvpError) as e:
        qvp.copy_append_kv(c["args"], src, dst, copy_bytes, frames, slots)
    assert e.value.status == status
    qvp.synchronize()
    assert np.array_equal(pool.download_all(), c["image"])
