"""Seeded synthetic workloads at Qwen3-ASR decoder attention shapes.

Five configurations (c1..c5) of the paged-KV path: the metadata (context
lengths, block tables, slot mappings) is drawn with numpy from a seed, the
tensor data on the device with a seeded torch generator. Shapes follow the
Qwen3-ASR decoder attention: 16 query heads, 8 kv heads, head_dim 128.

The slot/context relation is the reference's decode rule: the token appended
at a step sits at position ``context_len - 1`` and its slot is
``block_table[pos // bs] * bs + pos % bs``
(``vasr-paged-attn/src/paged_kv_cache.rs:74-103, 985-1017``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List

import numpy as np

NUM_HEADS = 16
NUM_KV_HEADS = 8
HEAD_DIM = 128
BLOCK_SIZE = 16
NUM_LAYERS = 28


@dataclass
class DecodeLayer:
    """Metadata of one layer's decode step."""

    num_blocks: int                 # pool size of this layer
    block_tables: np.ndarray        # [B, cols] uint32
    slot_mapping: np.ndarray        # [B] int64: slot of position context_len-1


@dataclass
class DecodeWorkload:
    name: str
    dtype: str                      # "f32" | "bf16" | "f16"
    context_lens: np.ndarray        # [B] uint32, after the append
    layers: List[DecodeLayer]
    seed: int
    num_heads: int = NUM_HEADS
    num_kv_heads: int = NUM_KV_HEADS
    head_dim: int = HEAD_DIM
    block_size: int = BLOCK_SIZE
    shared_pool: bool = False       # all layers view one pool (c5)
    notes: str = ""

    @property
    def num_seqs(self) -> int:
        return int(self.context_lens.shape[0])

    @property
    def max_context_len(self) -> int:
        return int(self.context_lens.max()) if self.num_seqs else 0

    @property
    def elem_bytes(self) -> int:
        return 4 if self.dtype == "f32" else 2

    def kv_bytes_per_token(self) -> int:
        """kvb = 2 * KVH * D * sizeof: K+V bytes of one token of one layer."""
        return 2 * self.num_kv_heads * self.head_dim * self.elem_bytes

    def decode_bytes_per_layer(self) -> int:
        """Algorithmic HBM bytes of one layer's paged_attention:
        sum_s L_s*kvb + 2*H*D*sizeof (q, out) + 4*ceil(L_s/BS) + 4 (block ids, length)."""
        L = self.context_lens.astype(np.int64)
        kvb = self.kv_bytes_per_token()
        per = (L * kvb + 2 * self.num_heads * self.head_dim * self.elem_bytes
               + 4 * ((L + self.block_size - 1) // self.block_size) + 4)
        return int(per.sum())

    def decode_flops_per_layer(self) -> int:
        return int(4 * self.num_heads * self.head_dim * self.context_lens.astype(np.int64).sum())

    def append_bytes_per_layer(self) -> int:
        """Algorithmic bytes of one layer's reshape_and_cache: T*kvb read +
        T*kvb written + 8*T slot ids."""
        t = self.num_seqs
        return 2 * t * self.kv_bytes_per_token() + 8 * t


def _tables_from_pool(rng: np.random.Generator, lens: np.ndarray, num_blocks: int, bs: int,
                      first_free: int = 1) -> np.ndarray:
    """Assign each sequence ceil(L/bs) distinct physical blocks drawn at random
    from ids first_free..num_blocks-1 (block 0 is the reserved null block,
    paged_cache_runtime.rs:270-273). Unused columns are 0."""
    need = (lens.astype(np.int64) + bs - 1) // bs
    cols = int(need.max()) if len(need) else 1
    total = int(need.sum())
    ids = rng.permutation(np.arange(first_free, num_blocks, dtype=np.int64))[:total]
    if ids.shape[0] < total:
        raise ValueError(f"pool of {num_blocks} blocks too small for {total} blocks")
    bt = np.zeros((len(lens), max(cols, 1)), dtype=np.uint32)
    off = 0
    for i, n in enumerate(need):
        bt[i, :n] = ids[off:off + n]
        off += n
    return bt


def _tables_with_replacement(rng: np.random.Generator, lens: np.ndarray, num_blocks: int,
                             bs: int) -> np.ndarray:
    """Block tables drawn independently from a huge pool (c5): ids are random in
    1..num_blocks-1, distinct within a sequence; different sequences may share
    blocks (layers alias physical blocks anyway)."""
    need = (lens.astype(np.int64) + bs - 1) // bs
    cols = int(need.max())
    bt = np.zeros((len(lens), cols), dtype=np.uint32)
    for i, n in enumerate(need):
        bt[i, :n] = rng.choice(num_blocks - 1, size=int(n), replace=False) + 1
    return bt


def _slots(bt: np.ndarray, lens: np.ndarray, bs: int) -> np.ndarray:
    pos = lens.astype(np.int64) - 1
    blk = bt[np.arange(len(lens)), pos // bs].astype(np.int64)
    return blk * bs + pos % bs


def compact_tables(block_tables: np.ndarray, lens: np.ndarray, bs: int,
                   slots: np.ndarray | None = None):
    """The blocks a set of sequences reads and their tables renumbered over
    those blocks alone, so that a sample of a pool too large for host memory
    (c5) can be copied out and handed to a CPU restatement.

    Returns (blocks, tables, slots): `blocks` is the sorted int64 array of
    physical ids read, block 0 (the null block) always first; `tables[i, c]`
    is the index into `blocks` of block_tables[i, c] for the columns a
    context of lens[i] tokens uses (0 elsewhere); `slots`, when given, is
    renumbered the same way (PAD -1 kept)."""
    lens = np.asarray(lens, dtype=np.int64)
    need = (lens + bs - 1) // bs
    used = [block_tables[i, :n].astype(np.int64) for i, n in enumerate(need)]
    blocks = np.unique(np.concatenate([np.zeros(1, np.int64)] + used))
    tables = np.zeros((len(lens), max(int(need.max()) if len(need) else 1, 1)), np.uint32)
    for i, ids in enumerate(used):
        tables[i, :len(ids)] = np.searchsorted(blocks, ids)
    new_slots = None
    if slots is not None:
        slots = np.asarray(slots, dtype=np.int64)
        blk = slots // bs
        idx = np.searchsorted(blocks, np.where(slots >= 0, blk, 0))
        if np.any((slots >= 0) & (blocks[np.minimum(idx, len(blocks) - 1)] != blk)):
            raise ValueError("a slot lies in a block the tables do not read")
        new_slots = np.where(slots >= 0, idx * bs + slots % bs, -1)
    return blocks, tables, new_slots


def c1(seed: int = 1) -> DecodeWorkload:
    """f32, B=1, L=512 (511 prefilled + 1 appended), 32 blocks taken from a
    seeded permutation of a 64-block pool, one layer."""
    rng = np.random.default_rng(seed)
    lens = np.array([512], dtype=np.uint32)
    bt = rng.permutation(64)[:32].astype(np.uint32)[None, :]
    layer = DecodeLayer(64, bt, _slots(bt, lens, BLOCK_SIZE))
    return DecodeWorkload("c1", "f32", lens, [layer], seed,
                          notes="prefill positions 0..510, append at 511")


def c2(seed: int = 2) -> DecodeWorkload:
    """bf16, B=32, L~U[100,1500], pool = 1.25x the blocks needed, shuffled, one layer."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(100, 1500, size=32, endpoint=True).astype(np.uint32)
    need = int(((lens.astype(np.int64) + BLOCK_SIZE - 1) // BLOCK_SIZE).sum())
    nb = int(math.ceil(1.25 * need)) + 1
    bt = _tables_from_pool(rng, lens, nb, BLOCK_SIZE)
    return DecodeWorkload("c2", "bf16", lens, [DecodeLayer(nb, bt, _slots(bt, lens, BLOCK_SIZE))],
                          seed)


def c3(seed: int = 3, num_layers: int = NUM_LAYERS, batch: int = 256) -> DecodeWorkload:
    """bf16, B=256, L = clip(Geom(p=1/800), 16, 4096), 28 layers each with its
    own pool and seeded random block allocation."""
    rng = np.random.default_rng(seed)
    lens = np.clip(rng.geometric(1.0 / 800.0, size=batch), 16, 4096).astype(np.uint32)
    need = int(((lens.astype(np.int64) + BLOCK_SIZE - 1) // BLOCK_SIZE).sum())
    nb = need + 1 + need // 8   # null block + 12.5% slack
    layers = []
    for _ in range(num_layers):
        bt = _tables_from_pool(rng, lens, nb, BLOCK_SIZE)
        layers.append(DecodeLayer(nb, bt, _slots(bt, lens, BLOCK_SIZE)))
    return DecodeWorkload("c3", "bf16", lens, layers, seed)


def c5(seed: int = 5, num_layers: int = NUM_LAYERS, batch: int = 1024,
       pool_bytes: int = int(0.6 * 288e9)) -> DecodeWorkload:
    """bf16, B=1024, L~U[256,8192], 28 layers over ONE pool of ~60% of HBM.

    As stated (28 separate pools) the config needs ~496 GB; here every layer's
    cache is the same pool and each layer draws independent block tables from
    all of it, so gathers stay scattered and cache-cold."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(256, 8192, size=batch, endpoint=True).astype(np.uint32)
    block_bytes = 2 * NUM_KV_HEADS * HEAD_DIM * BLOCK_SIZE * 2
    nb = pool_bytes // block_bytes
    layers = []
    for _ in range(num_layers):
        bt = _tables_with_replacement(rng, lens, nb, BLOCK_SIZE)
        layers.append(DecodeLayer(nb, bt, _slots(bt, lens, BLOCK_SIZE)))
    return DecodeWorkload("c5", "bf16", lens, layers, seed, shared_pool=True,
                          notes="layers alias one pool")


@dataclass
class PrefillWorkload:
    """c4: chunked prefill of N new tokens per sequence over P prior tokens."""

    name: str
    dtype: str
    prior_lens: np.ndarray          # [B] P_s
    query_lens: np.ndarray          # [B] N_s
    num_blocks: int
    block_tables: np.ndarray        # [B, cols] uint32
    seed: int
    num_heads: int = NUM_HEADS
    num_kv_heads: int = NUM_KV_HEADS
    head_dim: int = HEAD_DIM
    block_size: int = BLOCK_SIZE
    notes: str = ""

    @property
    def context_lens(self) -> np.ndarray:
        return (self.prior_lens + self.query_lens).astype(np.uint32)

    @property
    def cu_seqlens_q(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.query_lens)]).astype(np.uint32)

    def slot_mapping(self) -> np.ndarray:
        bs = self.block_size
        out = []
        for s in range(len(self.prior_lens)):
            pos = np.arange(self.prior_lens[s], self.prior_lens[s] + self.query_lens[s],
                            dtype=np.int64)
            out.append(self.block_tables[s, pos // bs].astype(np.int64) * bs + pos % bs)
        return np.concatenate(out)

    def flops(self) -> int:
        n = self.query_lens.astype(np.int64)
        p = self.prior_lens.astype(np.int64)
        return int((4 * self.num_heads * self.head_dim * (n * p + n * (n + 1) // 2)).sum())


def c4(seed: int = 4, batch: int = 64, new_tokens: int = 512) -> PrefillWorkload:
    """bf16, 64 seqs x 512 new tokens over U[0,1024] prior tokens in a
    fragmented (shuffled) 16-token-block pool."""
    rng = np.random.default_rng(seed)
    prior = rng.integers(0, 1024, size=batch, endpoint=True).astype(np.uint32)
    q = np.full(batch, new_tokens, dtype=np.uint32)
    lens = prior + q
    need = int(((lens.astype(np.int64) + BLOCK_SIZE - 1) // BLOCK_SIZE).sum())
    nb = need + 1 + need // 4
    bt = _tables_from_pool(rng, lens, nb, BLOCK_SIZE)
    return PrefillWorkload("c4", "bf16", prior, q, nb, bt, seed)


CONFIGS = {"c1": c1, "c2": c2, "c3": c3, "c4": c4, "c5": c5}
