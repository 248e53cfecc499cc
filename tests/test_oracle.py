"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker of
the GPU path. No GPU needed.

What pins each oracle function:
  decode    bitwise equality with the reference's own paged_attention_decode<T>
            for T = float, bf16 and fp16 (committed fixture
            tests/golden/decode_goldens.npz, and the live compiled reference
            oracle/_ref where it was built); the closed-form
            cases of the reference suite (tests/PagedAttention.test.cpp:380-566:
            equal keys -> mean of values, one-hot keys -> exact selection, GQA
            head mapping, layer isolation, copy-on-write branches); float64
            textbook attention on random inputs; the refusal rules.
  layout    closed forms of byte_size / stride / strides / element_offset and
            the injectivity of the offset map, plus equality with the reference
  pack      block tables equal the CSR ids (BlockTable::entries() order),
            lengths and prefix sums by construction, split bookkeeping
  copy      memcpy identity, other frames untouched
  fp16/bf16 conversions: numpy's float16 on every half bit pattern and on
            edge and random floats (ties, overflow, subnormals); bf16 on ties,
            infinities, NaN and random floats
A planted mistake (in a Python restatement, on the CPU) shows the closed-form
checks reject plausible errors: swapped K/V, a dropped scale, a wrong GQA map.
"""

from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import pytest

import pyoracle as O
import workloads as W

GOLDEN = Path(__file__).resolve().parent / "golden"
F32_TOL = 1e-5


# ---------------------------------------------------------------------------
# Small pool builder: frames laid out [layer][K|V][token][kv_head][dim]
# ---------------------------------------------------------------------------

class Pool:
    def __init__(self, frames: int, tpb: int, layers: int, hkv: int, d: int, dtype=np.float32):
        self.tpb, self.layers, self.hkv, self.d = tpb, layers, hkv, d
        self.dtype = dtype
        self.elems = tpb * layers * hkv * d * 2
        self.bpe = np.dtype(dtype).itemsize
        self.stride = (self.elems * self.bpe + 255) // 256 * 256
        self.image = np.zeros(frames * self.stride, np.uint8)
        self.frames = frames

    def frame(self, f: int) -> np.ndarray:
        return self.image[f * self.stride: f * self.stride + self.elems * self.bpe].view(self.dtype).reshape(
            self.layers, 2, self.tpb, self.hkv, self.d)

    def put(self, table, layer, stream, token, head, vec):
        f = table[token // self.tpb]
        self.frame(f)[layer, stream, token % self.tpb, head, :] = vec

    def decode(self, table, ctx, query, layer, hq, scale, orc_dtype=O.ORC_F32):
        refused, out, out32 = O.decode_batch(self.image, self.stride, self.frames, np.asarray(table, np.uint32),
                                             np.array([0, len(table)], np.uint32), np.array([ctx], np.uint32),
                                             orc_dtype, np.asarray(query)[None], layer, self.layers, hq, self.hkv,
                                             self.d, self.tpb, scale)
        return refused, out[0], out32[0]


def textbook(q, K, V, scale, group):
    """float64 softmax attention; q [Hq][D], K/V [T][Hkv][D]."""
    hq = q.shape[0]
    out = np.zeros(q.shape, np.float64)
    for h in range(hq):
        kh = h // group
        s = (K[:, kh, :].astype(np.float64) @ q[h].astype(np.float64)) * scale
        w = np.exp(s - s.max())
        out[h] = (w[:, None] * V[:, kh, :].astype(np.float64)).sum(0) / w.sum()
    return out


# ---------------------------------------------------------------------------
# Decode against the reference itself
# ---------------------------------------------------------------------------

ORC_DTYPE = {W.DTYPE_F32: O.ORC_F32, W.DTYPE_BF16: O.ORC_BF16, W.DTYPE_F16: O.ORC_F16}


def _oracle_out(w: W.Workload):
    dtype = ORC_DTYPE[w.kv_dtype]
    refused, out, _ = O.decode_batch(w.pool_image(), w.block_stride, w.num_pool_blocks, w.ids, w.cu_blocks,
                                     w.context_lens, dtype, w.query(), w.layer, w.num_layers, w.num_query_heads,
                                     w.num_kv_heads, w.head_dim, w.tokens_per_block, w.scale, 4)
    assert refused == 0
    return out


def _golden_workloads():
    import sys
    sys.path.insert(0, str(GOLDEN))
    import make_golden
    return make_golden.golden_workloads(), make_golden.input_digest


@pytest.mark.parametrize("name", ["config1", "bf16_gqa7", "bf16_tpb32", "f16_gqa4"])
def test_oracle_matches_reference_goldens_bitwise(name):
    workloads, digest = _golden_workloads()
    w = workloads[name]
    g = np.load(GOLDEN / "decode_goldens.npz")
    # The input generators still produce the inputs the fixture was made from.
    assert digest(w) == bytes(g[f"{name}_digest"]).hex()
    out = _oracle_out(w)
    expect = g[f"{name}_out"]
    assert out.dtype == expect.dtype and out.shape == expect.shape
    assert np.array_equal(out.view(np.uint8), expect.view(np.uint8))


@pytest.mark.skipif(not O.reference_available(), reason="oracle/_ref not built (reference tree absent)")
@pytest.mark.parametrize("case", [
    dict(ctx=[1, 2, 15, 16, 17, 31, 32, 33], hq=8, hkv=8, d=64, dtype=W.DTYPE_F32),
    dict(ctx=[5, 129, 1000], hq=28, hkv=4, d=128, dtype=W.DTYPE_BF16),
    dict(ctx=[7, 64, 257], hq=16, hkv=1, d=96, dtype=W.DTYPE_BF16, tpb=8),
    dict(ctx=[100, 3], hq=12, hkv=3, d=40, dtype=W.DTYPE_F32, tpb=5, layers=3, layer=2),
    dict(ctx=[1, 33, 500, 129], hq=28, hkv=4, d=128, dtype=W.DTYPE_F16),
    dict(ctx=[9, 70], hq=6, hkv=2, d=40, dtype=W.DTYPE_F16, tpb=8, layers=2, layer=1),
])
def test_oracle_matches_live_reference_bitwise(case):
    w = W.custom(case["ctx"], case["hq"], case["hkv"], case["d"], case["dtype"], tokens_per_block=case.get("tpb", 16),
                 num_layers=case.get("layers", 1), layer=case.get("layer", 0), seed=31)
    dtype = ORC_DTYPE[w.kv_dtype]
    sess = O.RefSession(w.pool_image(), w.block_stride, w.num_pool_blocks, w.tokens_per_block, w.num_layers,
                        w.num_kv_heads, w.head_dim, w.elem_bytes)
    refused, ref, _ = sess.decode(w.ids, w.cu_blocks, w.context_lens, dtype, w.query(), w.layer, w.num_query_heads,
                                  w.head_dim, w.scale)
    sess.close()
    assert refused == 0
    assert np.array_equal(_oracle_out(w).view(np.uint8), ref.view(np.uint8))


@pytest.mark.skipif(not O.reference_available(), reason="oracle/_ref not built (reference tree absent)")
def test_live_reference_reproduces_the_committed_fixtures():
    workloads, _ = _golden_workloads()
    import make_golden
    g = np.load(GOLDEN / "decode_goldens.npz")
    for name, w in workloads.items():
        assert np.array_equal(make_golden.reference_decode(w).view(np.uint8), g[f"{name}_out"].view(np.uint8))
    for fname, t in make_golden.TRACES.items():
        assert make_golden.reference_trace(t["requests"], t["seed"], t["pool_percent"], t["watermark"]) == \
            (GOLDEN / fname).read_text()
    import gzip
    assert make_golden.reference_trace_config(make_golden.CONFIG5_PARAMS, make_golden.CONFIG5_SEED) == \
        gzip.decompress((GOLDEN / make_golden.CONFIG5_TRACE).read_bytes()).decode()


# ---------------------------------------------------------------------------
# Closed forms (tests/PagedAttention.test.cpp:380-566 of the reference)
# ---------------------------------------------------------------------------

def test_equal_keys_give_the_mean_of_the_values():
    p = Pool(8, 4, 1, 1, 4)
    table = [5, 2]
    for t in range(8):
        p.put(table, 0, 0, t, 0, np.ones(4))
        p.put(table, 0, 1, t, 0, np.full(4, t + 1.0))
    for ctx in (1, 3, 8):
        refused, out, _ = p.decode(table, ctx, np.full((1, 4), 0.5, np.float32), 0, 1, 1.0)
        assert refused == 0
        np.testing.assert_allclose(out, np.full((1, 4), (ctx + 1) / 2.0), atol=F32_TOL, rtol=0)


def test_one_hot_keys_select_each_logical_token():
    p = Pool(8, 4, 1, 1, 8)
    table = [6, 1]  # scattered frames
    for t in range(8):
        k = np.zeros(8)
        k[t] = 1.0
        p.put(table, 0, 0, t, 0, k)
        p.put(table, 0, 1, t, 0, np.full(8, 10.0 * (t + 1)))
    for target in range(8):
        q = np.zeros((1, 8), np.float32)
        q[0, target] = 1.0
        _, out, _ = p.decode(table, 8, q, 0, 1, 50.0)
        np.testing.assert_allclose(out, np.full((1, 8), 10.0 * (target + 1)), atol=1e-3, rtol=0)


def test_query_heads_read_their_own_kv_head():
    p = Pool(4, 4, 1, 2, 4)
    table = [3]
    for kh, val in ((0, 100.0), (1, 200.0)):
        for t in range(4):
            p.put(table, 0, 0, t, kh, np.ones(4))
            p.put(table, 0, 1, t, kh, np.full(4, val))
    _, out, _ = p.decode(table, 4, np.ones((4, 4), np.float32), 0, 4, 1.0)
    np.testing.assert_allclose(out, np.array([[100.0] * 4, [100.0] * 4, [200.0] * 4, [200.0] * 4]), atol=F32_TOL)


def test_layers_are_isolated_and_match_textbook_attention():
    rng = np.random.default_rng(3)
    p = Pool(16, 4, 2, 2, 4)
    table = [9, 2, 14]  # three blocks, the last partial
    K = rng.uniform(-1, 1, (2, 10, 2, 4)).astype(np.float32)
    V = rng.uniform(-1, 1, (2, 10, 2, 4)).astype(np.float32)
    for layer in range(2):
        for t in range(10):
            for h in range(2):
                p.put(table, layer, 0, t, h, K[layer, t, h])
                p.put(table, layer, 1, t, h, V[layer, t, h])
    q = rng.uniform(-1, 1, (4, 4)).astype(np.float32)
    for layer in range(2):
        for ctx in (1, 5, 10):
            _, out, _ = p.decode(table, ctx, q, layer, 4, 0.5)
            np.testing.assert_allclose(out, textbook(q, K[layer, :ctx], V[layer, :ctx], 0.5, 2), atol=F32_TOL, rtol=0)


def test_copy_on_write_branches_see_their_own_values():
    p = Pool(4, 4, 1, 1, 4)
    parent, child = [0], [1]
    for t in range(4):
        p.put(parent, 0, 0, t, 0, np.ones(4))
        p.put(parent, 0, 1, t, 0, np.full(4, 5.0))
    O.oracle().orc_copy_block(p.image.ctypes.data, p.stride, p.frames, 0, 1, p.stride)
    for t in range(4):
        p.put(child, 0, 1, t, 0, np.full(4, 9.0))
    q = np.full((1, 4), 0.5, np.float32)
    np.testing.assert_allclose(p.decode(parent, 4, q, 0, 1, 1.0)[1], np.full((1, 4), 5.0), atol=F32_TOL)
    np.testing.assert_allclose(p.decode(child, 4, q, 0, 1, 1.0)[1], np.full((1, 4), 9.0), atol=F32_TOL)


@pytest.mark.parametrize("seed", range(6))
def test_random_shapes_match_float64_textbook(seed):
    rng = np.random.default_rng(100 + seed)
    tpb = int(rng.choice([1, 3, 4, 16]))
    hkv = int(rng.choice([1, 2, 3]))
    group = int(rng.choice([1, 2, 4]))
    d = int(rng.choice([4, 8, 64]))
    ctx = int(rng.integers(1, 70))
    nb = (ctx + tpb - 1) // tpb
    frames = nb + 5
    p = Pool(frames, tpb, 1, hkv, d)
    table = list(rng.permutation(frames)[:nb])
    K = rng.normal(size=(ctx, hkv, d)).astype(np.float32)
    V = rng.normal(size=(ctx, hkv, d)).astype(np.float32)
    for t in range(ctx):
        for h in range(hkv):
            p.put(table, 0, 0, t, h, K[t, h])
            p.put(table, 0, 1, t, h, V[t, h])
    q = rng.normal(size=(hkv * group, d)).astype(np.float32)
    scale = float(1.0 / np.sqrt(d))
    _, out, _ = p.decode(table, ctx, q, 0, hkv * group, scale)
    np.testing.assert_allclose(out, textbook(q, K, V, scale, group), atol=F32_TOL, rtol=0)


def test_refusals_leave_the_output_untouched():
    p = Pool(4, 4, 2, 2, 4)
    q = np.ones((4, 4), np.float32)
    assert p.decode([0, 1], 8, q, 0, 4, 1.0)[0] == 0
    assert p.decode([0, 1], 0, q, 0, 4, 1.0)[0] == 1              # context_len 0
    assert p.decode([0, 1], 9, q, 0, 4, 1.0)[0] == 1              # past the table
    assert p.decode([0, 0xFFFFFFFF], 8, q, 0, 4, 1.0)[0] == 1     # unmapped / swapped block
    assert p.decode([0, 4], 8, q, 0, 4, 1.0)[0] == 1              # frame outside the pool
    assert p.decode([0, 1], 8, q, 2, 4, 1.0)[0] == 1              # layer outside the shape
    assert p.decode([0, 1], 8, np.ones((3, 4), np.float32), 0, 3, 1.0)[0] == 1  # 3 heads onto 2
    # Only the blocks the context needs are checked.
    assert p.decode([0, 0xFFFFFFFF], 4, q, 0, 4, 1.0)[0] == 0


# ---------------------------------------------------------------------------
# A planted mistake must fail the closed-form checks
# ---------------------------------------------------------------------------

def _mutant(q, K, V, scale, group, mistake):
    if mistake == "swap_kv":
        K, V = V, K
    if mistake == "drop_scale":
        scale = 1.0
    if mistake == "gqa_modulo":
        hkv = K.shape[1]
        out = np.zeros(q.shape)
        for h in range(q.shape[0]):
            out[h] = textbook(q[h:h + 1], K[:, [h % hkv]], V[:, [h % hkv]], scale, 1)[0]
        return out
    return textbook(q, K, V, scale, group)


@pytest.mark.parametrize("mistake", ["swap_kv", "drop_scale", "gqa_modulo"])
def test_checks_reject_a_planted_mistake(mistake):
    rng = np.random.default_rng(9)
    p = Pool(8, 4, 1, 2, 8)
    table = [4, 0, 6]
    K = rng.normal(size=(12, 2, 8)).astype(np.float32)
    V = rng.normal(size=(12, 2, 8)).astype(np.float32)
    for t in range(12):
        for h in range(2):
            p.put(table, 0, 0, t, h, K[t, h])
            p.put(table, 0, 1, t, h, V[t, h])
    q = rng.normal(size=(4, 8)).astype(np.float32)
    _, out, _ = p.decode(table, 12, q, 0, 4, 0.35)
    np.testing.assert_allclose(out, _mutant(q, K, V, 0.35, 2, None), atol=F32_TOL)
    assert not np.allclose(out, _mutant(q, K, V, 0.35, 2, mistake), atol=F32_TOL)


# ---------------------------------------------------------------------------
# Layout, pack and copy
# ---------------------------------------------------------------------------

SHAPES = [(16, 1, 2, 64, 4), (16, 1, 4, 128, 2), (16, 1, 8, 128, 2), (16, 28, 4, 128, 2), (3, 2, 3, 5, 2),
          (1, 1, 1, 1, 4)]


@pytest.mark.parametrize("shape", SHAPES)
def test_layout_closed_forms(shape):
    tpb, layers, hkv, d, bpe = shape
    lib = O.oracle()
    assert lib.orc_block_byte_size(tpb, layers, hkv, d, bpe) == tpb * layers * hkv * d * bpe * 2
    strides = (O.c_uint64 * 5)()
    lib.orc_layout_strides(tpb, layers, hkv, d, strides)
    assert list(strides) == [d, hkv * d, tpb * hkv * d, 2 * tpb * hkv * d, layers * 2 * tpb * hkv * d]
    seen = np.zeros(layers * 2 * tpb * hkv * d, np.int32)
    for layer in range(layers):
        for s in range(2):
            for t in range(tpb):
                for h in range(hkv):
                    off = lib.orc_element_offset(tpb, layers, hkv, d, layer, s, t, h)
                    assert off == ((layer * 2 + s) * tpb + t) * hkv * d + h * d
                    seen[off:off + d] += 1
    assert (seen == 1).all()
    assert lib.orc_element_offset(tpb, layers, hkv, d, layers, 0, 0, 0) == -1
    assert lib.orc_element_offset(tpb, layers, hkv, d, 0, 0, tpb, 0) == -1
    assert lib.orc_element_offset(tpb, layers, hkv, d, 0, 0, 0, hkv) == -1


def test_block_stride_rounding():
    lib = O.oracle()
    assert lib.orc_block_stride(192, 256) == 256
    assert lib.orc_block_stride(256, 256) == 256
    assert lib.orc_block_stride(320, 256) == 512
    assert lib.orc_block_stride(100, 0) == 256      # 0 selects the default alignment
    assert lib.orc_block_stride(0, 256) == 256      # never zero bytes
    assert lib.orc_block_stride(5000, 4096) == 8192


@pytest.mark.skipif(not O.reference_available(), reason="oracle/_ref not built (reference tree absent)")
@pytest.mark.parametrize("shape", SHAPES)
def test_layout_equals_the_reference(shape):
    tpb, layers, hkv, d, bpe = shape
    lib, ref = O.oracle(), O.reference()
    assert lib.orc_block_byte_size(*shape) == ref.ref_block_byte_size(*shape)
    for align in (0, 64, 256, 4096):
        assert lib.orc_block_stride(lib.orc_block_byte_size(*shape), align) == ref.ref_block_size_bytes(*shape, align)
    for layer in range(layers + 1):
        for s in range(2):
            for t in (0, tpb - 1, tpb):
                for h in (0, hkv - 1, hkv):
                    assert lib.orc_element_offset(tpb, layers, hkv, d, layer, s, t, h) == \
                        ref.ref_element_offset(tpb, layers, hkv, d, layer, s, t, h)


def test_pack_flattens_the_tables_in_logical_order():
    w = W.config2(seed=2, num_seqs=16)
    out = O.pack(w.ids, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks, 512)
    assert out is not None
    nb = np.diff(w.cu_blocks.astype(np.int64))
    assert out["block_tables"].shape == (16, nb.max())
    for b in range(16):
        row = out["block_tables"][b]
        assert np.array_equal(row[: nb[b]], w.ids[w.cu_blocks[b]: w.cu_blocks[b + 1]].astype(np.int32))
    assert np.array_equal(out["seq_lens"], w.context_lens.astype(np.int32))
    assert np.array_equal(out["cu_seqlens"], np.concatenate([[0], np.cumsum(w.context_lens)]).astype(np.int32))
    splits = (w.context_lens.astype(np.int64) + 511) // 512
    assert np.array_equal(out["cu_splits"], np.concatenate([[0], np.cumsum(splits)]).astype(np.int32))
    for b in range(16):
        for s in range(splits[b]):
            i = out["cu_splits"][b] + s
            assert out["split_seq"][i] == b and out["split_start"][i] == s * 512
    # Refused: an unmapped block inside the context, a frame outside the pool,
    # a zero context, and a table shorter than the context.
    bad = w.ids.copy()
    bad[3] = 0xFFFFFFFF
    assert O.pack(bad, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks) is None
    bad[3] = w.num_pool_blocks
    assert O.pack(bad, w.cu_blocks, w.context_lens, 16, w.num_pool_blocks) is None
    ctx = w.context_lens.copy()
    ctx[0] = 0
    assert O.pack(w.ids, w.cu_blocks, ctx, 16, w.num_pool_blocks) is None
    ctx[0] = nb[0] * 16 + 1
    assert O.pack(w.ids, w.cu_blocks, ctx, 16, w.num_pool_blocks) is None


def test_copy_block_is_memcpy_identity():
    frames, stride = 9, 512
    rng = np.random.default_rng(4)
    image = rng.integers(0, 256, frames * stride, dtype=np.uint8)
    before = image.copy()
    O.oracle().orc_copy_block(image.ctypes.data, stride, frames, 2, 7, stride)
    view, orig = image.reshape(frames, stride), before.reshape(frames, stride)
    assert np.array_equal(view[7], orig[2])
    others = [i for i in range(frames) if i != 7]
    assert np.array_equal(view[others], orig[others])


# K/V append: every written head row lands at the closed-form offset of the
# layout ((layer * 2 + stream) * tpb + slot) * Hkv * D + h * D (pinned against
# the compiled reference above), and no other byte of the pool changes.
APPEND_CASES = [
    # tpb, layers, hkv, d, bpe, first_layer, layer_count, tokens, frames
    (16, 1, 2, 64, 4, 0, 1, 4, 8),
    (16, 1, 4, 128, 2, 0, 1, 40, 64),
    (16, 3, 3, 8, 2, 1, 2, 20, 6),
    (4, 2, 1, 5, 4, 0, 2, 7, 3),
]


def _append_expected_rows(shape, frames, slots, first_layer, layer_count):
    tpb, layers, hkv, d, bpe = shape
    for i, (f, t) in enumerate(zip(frames, slots)):
        for l in range(layer_count):
            for s in range(2):
                for h in range(hkv):
                    off = (((first_layer + l) * 2 + s) * tpb + t) * hkv * d + h * d
                    yield i, l, s, h, f, off * bpe


def _append_case(case, seed):
    tpb, layers, hkv, d, bpe, first_layer, layer_count, tokens, nframes = case
    shape = (tpb, layers, hkv, d, bpe)
    rng = np.random.default_rng(seed)
    stride = O.oracle().orc_block_stride(O.oracle().orc_block_byte_size(*shape), 256)
    pool = rng.integers(0, 256, nframes * stride, dtype=np.uint8)
    pairs = rng.choice(nframes * tpb, size=tokens, replace=False)
    frames, slots = (pairs // tpb).astype(np.uint32), (pairs % tpb).astype(np.uint32)
    k = rng.integers(0, 256, tokens * layer_count * hkv * d * bpe, dtype=np.uint8)
    v = rng.integers(0, 256, tokens * layer_count * hkv * d * bpe, dtype=np.uint8)
    return shape, stride, pool, frames, slots, k, v


def _check_append(case, stride, before, after, frames, slots, k, v):
    tpb, layers, hkv, d, bpe, first_layer, layer_count, tokens, nframes = case
    shape = (tpb, layers, hkv, d, bpe)
    row = d * bpe
    written = np.zeros(before.size, bool)
    for i, l, s, h, f, off in _append_expected_rows(shape, frames, slots, first_layer, layer_count):
        src = (k if s == 0 else v)[((i * layer_count + l) * hkv + h) * row:][:row]
        at = f * stride + off
        if not np.array_equal(after[at:at + row], src):
            return False
        written[at:at + row] = True
    return np.array_equal(after[~written], before[~written])


@pytest.mark.parametrize("case", APPEND_CASES)
def test_append_writes_rows_at_the_layout_offsets(case):
    shape, stride, pool, frames, slots, k, v = _append_case(case, seed=7)
    before = pool.copy()
    tpb, layers, hkv, d, bpe, first_layer, layer_count, tokens, nframes = case
    assert O.append_kv(pool, stride, nframes, bpe, tpb, layers, hkv, d, first_layer, layer_count, frames, slots,
                       k, v) == 0
    assert _check_append(case, stride, before, pool, frames, slots, k, v)
    # Refusals write nothing: a frame outside the pool, a slot past the block,
    # layers past num_layers.
    for f2, s2, fl, lc in ((nframes, 0, first_layer, layer_count), (0, tpb, first_layer, layer_count),
                           (0, 0, layers - layer_count + 1, layer_count)):
        img = before.copy()
        bad_f, bad_s = frames.copy(), slots.copy()
        bad_f[-1], bad_s[-1] = (f2, s2) if (f2, s2) != (0, 0) else (bad_f[-1], bad_s[-1])
        assert O.append_kv(img, stride, nframes, bpe, tpb, layers, hkv, d, fl, lc, bad_f, bad_s, k, v) == -1
        assert np.array_equal(img, before)


def test_append_check_rejects_a_planted_mistake():
    """The read-back check fails for an oracle call with K and V swapped."""
    case = APPEND_CASES[1]
    shape, stride, pool, frames, slots, k, v = _append_case(case, seed=8)
    before = pool.copy()
    tpb, layers, hkv, d, bpe, first_layer, layer_count, tokens, nframes = case
    assert O.append_kv(pool, stride, nframes, bpe, tpb, layers, hkv, d, first_layer, layer_count, frames, slots,
                       v, k) == 0
    assert not _check_append(case, stride, before, pool, frames, slots, k, v)


def test_bf16_conversion_rounds_to_nearest_even():
    lib = O.oracle()
    assert lib.orc_bf16_from_f32(1.0) == 0x3F80
    assert lib.orc_bf16_from_f32(np.float32(1.0 + 2 ** -8)) == 0x3F80       # tie -> even
    assert lib.orc_bf16_from_f32(np.float32(1.0 + 3 * 2 ** -8)) == 0x3F82   # tie -> even (up)
    assert lib.orc_bf16_from_f32(np.float32(1.0 + 2 ** -8 + 2 ** -20)) == 0x3F81
    assert lib.orc_bf16_from_f32(float("inf")) == 0x7F80
    assert lib.orc_bf16_from_f32(float("nan")) & 0x7FC0 == 0x7FC0
    x = np.random.default_rng(0).normal(size=4096).astype(np.float32)
    bits = W.f32_to_bf16_bits(x)
    assert np.array_equal(bits, np.array([lib.orc_bf16_from_f32(float(v)) for v in x], np.uint16))


def _f16_edge_and_random_f32(n_random: int = 1_000_000) -> np.ndarray:
    """float32 values that exercise every branch of a float -> half rounding:
    ties to even in the normal range, the overflow threshold, subnormal ties,
    the smallest normal, signed zeros and infinities, plus random bit patterns
    over the whole exponent range and random normals."""
    ulp = lambda e: 2.0 ** (e - 10)  # noqa: E731 - half spacing at exponent e
    edges = [0.0, -0.0, 1.0, -1.0, 1 + ulp(0) / 2, 1 + 3 * ulp(0) / 2, 1 + ulp(0) / 2 + 2 ** -20,
             2.0 - ulp(0) / 4, 65504.0, 65504.0 + 8.0, 65519.99, 65520.0, 65536.0, 1e9, -65520.0,
             2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 2.0 ** -14 - 2.0 ** -26, 2.0 ** -24, 2.0 ** -25,
             3 * 2.0 ** -25, 5 * 2.0 ** -25, 2.0 ** -25 + 2.0 ** -40, 2.0 ** -26, 1e-30, -2.0 ** -25,
             float("inf"), float("-inf"), 3.14159, -2.71828, 1000.5, 1001.5, 2048.0 + 1.0, 2048.0 + 3.0]
    rng = np.random.default_rng(16)
    bits = rng.integers(0, 2 ** 32, n_random // 2, dtype=np.uint64).astype(np.uint32)
    rand_bits = bits.view(np.float32)
    rand_bits = rand_bits[~np.isnan(rand_bits)]
    normals = (rng.normal(size=n_random // 2) * rng.choice([1e-6, 1e-3, 1.0, 1e3, 3e4], n_random // 2)).astype(
        np.float32)
    return np.concatenate([np.array(edges, np.float32), rand_bits, normals])


def test_f16_to_f32_matches_numpy_on_every_bit_pattern():
    """orc_f32_from_f16 (oracle.c) against numpy's float16 -> float32 for all
    65,536 half bit patterns: bitwise, except NaNs, which must stay NaNs of the
    same sign (a float crossing ctypes may be quieted)."""
    lib = O.oracle()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expect = h.view(np.float16).astype(np.float32)
    got = np.array([lib.orc_f32_from_f16(int(x)) for x in h], np.float32)
    nan = np.isnan(expect)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), expect[~nan].view(np.uint32))
    assert np.array_equal(np.signbit(got[nan]), np.signbit(expect[nan]))


def test_f32_to_f16_matches_numpy_rounding():
    """orc_f16_from_f32 / orc_round_to_f16 (oracle.c) against numpy's
    float32 -> float16 (round to nearest, ties to even; overflow to infinity;
    gradual underflow) on edge values and ~10^6 random floats, bitwise; a NaN
    stays a NaN of the same sign."""
    lib = O.oracle()
    x = _f16_edge_and_random_f32()
    with np.errstate(over="ignore"):
        expect = x.astype(np.float16).view(np.uint16)
    got = np.zeros(x.size, np.uint16)
    lib.orc_round_to_f16(x.ctypes.data, got.ctypes.data, x.size)
    assert np.array_equal(got, expect), np.flatnonzero(got != expect)[:10]
    # The scalar entry point agrees with the array one.
    for v, e in zip(x[:64], expect[:64]):
        assert lib.orc_f16_from_f32(float(v)) == e
    for nan in (float("nan"), -float("nan")):
        h = lib.orc_f16_from_f32(nan)
        assert (h & 0x7C00) == 0x7C00 and (h & 0x3FF) != 0 and (h >> 15) == int(np.signbit(nan))


@pytest.mark.skipif(not O.reference_available(), reason="oracle/_ref not built (reference tree absent)")
def test_reference_half_type_converts_like_numpy():
    """The reference decode's fp16 element type (oracle/ref_shim.cpp, x86 F16C
    conversions) rounds like numpy, so its decode is an independent check of
    the oracle's fp16 path."""
    ref = O.reference()
    x = _f16_edge_and_random_f32(20_000)
    with np.errstate(over="ignore"):
        expect = x.astype(np.float16).view(np.uint16)
    got = np.array([ref.ref_half_from_float(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, expect)
    h = np.arange(0, 65536, 7, dtype=np.uint32).astype(np.uint16)
    e32 = h.view(np.float16).astype(np.float32)
    g32 = np.array([ref.ref_float_from_half(int(v)) for v in h], np.float32)
    ok = ~np.isnan(e32)
    assert np.array_equal(g32[ok].view(np.uint32), e32[ok].view(np.uint32))
    assert np.array_equal(np.isnan(g32), ~ok)


def test_workload_generators_are_deterministic():
    a, b = W.config2(seed=2, num_seqs=8), W.config2(seed=2, num_seqs=8)
    assert np.array_equal(a.ids, b.ids) and np.array_equal(a.context_lens, b.context_lens)
    assert hashlib.sha256(a.query().tobytes()).digest() == hashlib.sha256(b.query().tobytes()).digest()
    assert len(set(a.ids.tolist())) == len(a.ids)          # no frame used twice
    assert a.ids.max() < a.num_pool_blocks
    c1 = W.config1()
    assert c1.context_lens.tolist() == [37, 128, 250, 509] and c1.block_bytes == 16384
