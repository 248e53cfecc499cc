"""Deterministic synthetic workloads for the paged-decode hot path.

The five configurations are the ones the benchmark and the parity tests are
quoted on (Qwen2-VL-7B / 72B KV shapes, block size 16). Every random draw comes
from an explicit counter-based SplitMix64 stream, Box-Muller normals and a
Fisher-Yates shuffle written here, so the same seed gives the same bits on any
machine and in any process.

Block tables follow the reference allocator's order exactly: the pool starts
with free list [0, 1, ..., N-1], allocate() pops the back
(src/MemoryAllocator.cpp:13-25,28-40) and release() pushes to the back (:52-57).
"Shuffled" pools allocate every frame and release them in a seeded
permutation, after which each sequence reserves its blocks in batch order.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from qvp import DTYPE_BF16, DTYPE_F16, DTYPE_F32, layout_strides

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Outputs offset .. offset+n-1 of the SplitMix64 stream started at `seed`."""
    with np.errstate(over="ignore"):
        idx = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform01(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Doubles in [0, 1) with 53 random bits."""
    return (splitmix64(seed, n, offset) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def randint(seed: int, n: int, lo: int, hi: int, offset: int = 0) -> np.ndarray:
    """Integers uniform on [lo, hi] (inclusive)."""
    u = uniform01(seed, n, offset)
    return (lo + np.floor(u * (hi - lo + 1))).astype(np.int64)


def normal(seed: int, n: int, sigma: float = 1.0, offset: int = 0) -> np.ndarray:
    """float32 normals N(0, sigma^2) by Box-Muller over pairs of uniforms."""
    m = (n + 1) // 2
    u = uniform01(seed, 2 * m, 2 * offset)
    u1 = 1.0 - u[0::2]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * math.pi * u2
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(t)
    z[1::2] = r * np.sin(t)
    return (z[:n] * sigma).astype(np.float32)


def permutation(seed: int, n: int) -> np.ndarray:
    """Fisher-Yates shuffle of 0..n-1 (j drawn uniform on [0, i])."""
    perm = np.arange(n, dtype=np.int64)
    u = uniform01(seed, max(n - 1, 0))
    for k, i in enumerate(range(n - 1, 0, -1)):
        j = int(u[k] * (i + 1))
        perm[i], perm[j] = perm[j], perm[i]
    return perm


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    with np.errstate(over="ignore"):
        r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    r[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def to_elements(x: np.ndarray, kv_dtype: int) -> np.ndarray:
    """float32 draws in the cache element type: fp32 as is, bf16 and fp16 as
    round-to-nearest-even bit patterns (fp16 through numpy's float16)."""
    if kv_dtype == DTYPE_F32:
        return np.asarray(x, np.float32)
    if kv_dtype == DTYPE_BF16:
        return f32_to_bf16_bits(x)
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def shuffled_allocation_order(num_blocks: int, seed: int) -> np.ndarray:
    """Frame ids in the order allocate() returns them after allocate-all and a
    release in seeded permutation order."""
    perm = permutation(seed, num_blocks)
    return perm[::-1].astype(np.uint32)


@dataclass
class Workload:
    name: str
    tokens_per_block: int
    num_layers: int
    num_query_heads: int
    num_kv_heads: int
    head_dim: int
    kv_dtype: int
    scale: float
    context_lens: np.ndarray          # uint32 [B]
    ids: np.ndarray                   # uint32 CSR block ids
    cu_blocks: np.ndarray             # uint32 [B + 1]
    num_pool_blocks: int
    seed: int
    layer: int = 0
    # 0: the library default (512-token partitions for the split kernels,
    # free cost-balanced cuts for the persistent kernel).
    split_tokens: int = 0
    q_sigma: float = 1.0
    kv_sigma: float = 1.0
    notes: dict = field(default_factory=dict)

    @property
    def num_seqs(self) -> int:
        return len(self.context_lens)

    @property
    def elem_bytes(self) -> int:
        return 4 if self.kv_dtype == DTYPE_F32 else 2

    @property
    def block_bytes(self) -> int:
        # BlockShape::byte_size (src/Block.cpp:8-13)
        return self.tokens_per_block * self.num_layers * self.num_kv_heads * self.head_dim * self.elem_bytes * 2

    @property
    def block_stride(self) -> int:
        return (self.block_bytes + 255) // 256 * 256

    @property
    def strides(self) -> dict:
        return layout_strides(self.tokens_per_block, self.num_layers, self.num_kv_heads, self.head_dim)

    @property
    def group(self) -> int:
        return self.num_query_heads // self.num_kv_heads

    def query(self) -> np.ndarray:
        """Query [B][Hq][D] in the cache element type (fp32, or bf16 / fp16 bits)."""
        n = self.num_seqs * self.num_query_heads * self.head_dim
        q = normal(self.seed ^ 0x5151, n, self.q_sigma).reshape(self.num_seqs, self.num_query_heads, self.head_dim)
        return to_elements(q, self.kv_dtype)

    def pool_image(self, chunk_elems: int = 1 << 24) -> np.ndarray:
        """Host image of the whole pool (num_pool_blocks * block_stride bytes):
        every element of every frame drawn N(0, kv_sigma^2) (fp32, or rounded
        to bf16 / fp16), padding bytes zero."""
        per_frame = self.block_bytes // self.elem_bytes
        total = per_frame * self.num_pool_blocks
        np_dtype = np.float32 if self.kv_dtype == DTYPE_F32 else np.uint16
        elems = np.empty(total, dtype=np_dtype)
        for off in range(0, total, chunk_elems):
            n = min(chunk_elems, total - off)
            v = normal(self.seed ^ 0xCAC4E, n, self.kv_sigma, offset=off // 2)
            elems[off:off + n] = to_elements(v, self.kv_dtype)
        frames = elems.view(np.uint8).reshape(self.num_pool_blocks, self.block_bytes)
        if self.block_stride == self.block_bytes:
            return frames.reshape(-1)
        image = np.zeros((self.num_pool_blocks, self.block_stride), dtype=np.uint8)
        image[:, : self.block_bytes] = frames
        return image.reshape(-1)

    def algorithmic_bytes(self) -> int:
        """KV + q + out + block ids + lengths read/written by one decode step."""
        kv = int(self.context_lens.astype(np.int64).sum()) * self.num_kv_heads * self.head_dim * 2 * self.elem_bytes
        qo = self.num_seqs * self.num_query_heads * self.head_dim * 2 * self.elem_bytes
        nb = int(((self.context_lens.astype(np.int64) + self.tokens_per_block - 1) // self.tokens_per_block).sum())
        return kv + qo + nb * 4 + self.num_seqs * 4

    def kv_bytes(self) -> int:
        return int(self.context_lens.astype(np.int64).sum()) * self.num_kv_heads * self.head_dim * 2 * self.elem_bytes


def _tables_from_order(order: np.ndarray, context_lens: np.ndarray, tpb: int) -> tuple[np.ndarray, np.ndarray]:
    nb = (context_lens.astype(np.int64) + tpb - 1) // tpb
    cu = np.zeros(len(context_lens) + 1, dtype=np.uint32)
    cu[1:] = np.cumsum(nb)
    ids = order[: int(cu[-1])].astype(np.uint32)
    return ids, cu


def config1(seed: int = 0) -> Workload:
    """Small fp32 case the reference CPU kernel runs: B=4, ctx {37,128,250,509},
    Hq 8 / Hkv 2 / D 64, block 16, 256-block pool shuffled with seed 0."""
    ctx = np.array([37, 128, 250, 509], dtype=np.uint32)
    order = shuffled_allocation_order(256, seed)
    ids, cu = _tables_from_order(order, ctx, 16)
    return Workload("config1", 16, 1, 8, 2, 64, DTYPE_F32, 1.0 / 8.0, ctx, ids, cu, 256, seed)


def config2(seed: int = 2, num_seqs: int = 64) -> Workload:
    """Qwen2-VL-7B single-layer decode: Hq 28 / Hkv 4 / D 128, block 16, bf16,
    B=64, ctx uniform on [512, 4096], pool = batch blocks + 10% free."""
    ctx = randint(seed, num_seqs, 512, 4096).astype(np.uint32)
    need = int(((ctx.astype(np.int64) + 15) // 16).sum())
    pool = int(math.ceil(need * 1.1))
    order = shuffled_allocation_order(pool, seed)
    ids, cu = _tables_from_order(order, ctx, 16)
    return Workload("config2", 16, 1, 28, 4, 128, DTYPE_BF16, 1.0 / math.sqrt(128.0), ctx, ids, cu, pool, seed,
                    q_sigma=1.0, kv_sigma=0.5)


def config3(seed: int = 3, num_seqs: int = 32, ctx_lo: int = 8192, ctx_hi: int = 32768) -> Workload:
    """Qwen2-VL-72B layer: Hq 64 / Hkv 8 / D 128, block 16, bf16, B=32, ctx
    uniform on [8192, 32768], split partitions of 512 tokens; the first 25% of
    each context is an image span (metadata only, no effect on attention)."""
    ctx = randint(seed, num_seqs, ctx_lo, ctx_hi).astype(np.uint32)
    need = int(((ctx.astype(np.int64) + 15) // 16).sum())
    pool = int(math.ceil(need * 1.1))
    order = shuffled_allocation_order(pool, seed)
    ids, cu = _tables_from_order(order, ctx, 16)
    w = Workload("config3", 16, 1, 64, 8, 128, DTYPE_BF16, 1.0 / math.sqrt(128.0), ctx, ids, cu, pool, seed,
                 q_sigma=1.0, kv_sigma=0.5, split_tokens=512)
    w.notes["image_spans"] = [(0, int(c) // 4) for c in ctx]
    return w


def custom(context_lens, num_query_heads: int, num_kv_heads: int, head_dim: int, kv_dtype: int = DTYPE_BF16,
           tokens_per_block: int = 16, num_layers: int = 1, seed: int = 7, spare: float = 0.25,
           scale: float | None = None, layer: int = 0, q_sigma: float = 1.0, kv_sigma: float = 0.5,
           split_tokens: int = 0) -> Workload:
    """Any shape, with a shuffled pool holding `spare` extra free frames."""
    ctx = np.asarray(context_lens, dtype=np.uint32)
    need = int(((ctx.astype(np.int64) + tokens_per_block - 1) // tokens_per_block).sum())
    pool = max(int(math.ceil(need * (1.0 + spare))), need + 1)
    order = shuffled_allocation_order(pool, seed)
    ids, cu = _tables_from_order(order, ctx, tokens_per_block)
    return Workload("custom", tokens_per_block, num_layers, num_query_heads, num_kv_heads, head_dim, kv_dtype,
                    scale if scale is not None else 1.0 / math.sqrt(head_dim), ctx, ids, cu, pool, seed,
                    layer=layer, split_tokens=split_tokens, q_sigma=q_sigma, kv_sigma=kv_sigma)


def forked(prompt_lens, branches, extra_tokens, num_query_heads: int, num_kv_heads: int, head_dim: int = 128,
           kv_dtype: int = DTYPE_BF16, tokens_per_block: int = 16, seed: int = 11, solo_lens=(),
           spare: float = 0.1) -> Workload:
    """Parallel-sampling batch: prompt p (prompt_lens[p] tokens) forked into
    branches[p] sequences that share the prompt's whole blocks (the same frame
    ids, as KVCacheManager::fork leaves them), each with its own copy of the
    prompt's partial tail block and its own later blocks; branch k of prompt p
    holds extra_tokens[p][k] tokens past the prompt. `solo_lens` adds
    unshared sequences. Frames come from a seeded shuffled pool."""
    tpb = tokens_per_block
    ctx: list[int] = []
    shared_of: list[int] = []
    for p, (plen, nb) in enumerate(zip(prompt_lens, branches)):
        for k in range(nb):
            ctx.append(int(plen) + int(extra_tokens[p][k]))
            shared_of.append(p)
    for n in solo_lens:
        ctx.append(int(n))
        shared_of.append(-1)
    shared_blocks = [int(plen) // tpb for plen in prompt_lens]
    need = sum(shared_blocks) + sum((c + tpb - 1) // tpb - (shared_blocks[s] if s >= 0 else 0)
                                    for c, s in zip(ctx, shared_of))
    pool = max(int(math.ceil(need * (1.0 + spare))), need + 1)
    order = list(shuffled_allocation_order(pool, seed))
    prompt_frames = []
    for n in shared_blocks:
        prompt_frames.append(order[:n])
        order = order[n:]
    ids: list[int] = []
    cu = [0]
    for c, s in zip(ctx, shared_of):
        nb = (c + tpb - 1) // tpb
        own = shared_blocks[s] if s >= 0 else 0
        ids.extend(prompt_frames[s] if s >= 0 else [])
        ids.extend(order[: nb - own])
        order = order[nb - own:]
        cu.append(len(ids))
    ctx_a = np.asarray(ctx, dtype=np.uint32)
    return Workload("forked", tpb, 1, num_query_heads, num_kv_heads, head_dim, kv_dtype,
                    1.0 / math.sqrt(head_dim), ctx_a, np.asarray(ids, dtype=np.uint32),
                    np.asarray(cu, dtype=np.uint32), pool, seed, q_sigma=1.0, kv_sigma=0.5)
