"""Host-side paged-cache bookkeeping over libvpa's C ABI (include/vpa_host.h).

Mirrors vasr-paged-attn's Rust host code with the same names and meaning:

* pool sizing — ``bytes_per_paged_block`` and ``resolve_num_blocks``
  (``paged_cache_runtime.rs:46-201``);
* ``BlockManager`` — ``PagedBlockManager`` (``paged_cache_runtime.rs:217-380``);
* metadata builders — ``input_metadata_from_block_tables``,
  ``input_metadata_from_attention_masks``, ``input_metadata_from_query_lens``,
  ``decode_metadata_for_batch_steps`` (``paged_kv_cache.rs:547-1044``);
* decode-graph padding — ``cuda_graph_batch_bucket``,
  ``cuda_graph_batch_buckets``, ``bucket_block_table_cols``,
  ``pad_decode_batch_to_max`` (``cuda_graph.rs:28-81, 373-486``).

Every computation runs in the C++ of libvpa; this module converts lists and
numpy arrays. Metadata comes back as numpy arrays in a ``dict`` keyed like
the fields of ``PagedInputMetadata`` (``paged_kv_cache.rs:23-38``).
"""

from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import _lib
from ._lib import VpaError, check

PAD_SLOT_ID = -1
_DTYPE = {"f32": _lib.DTYPE_F32, "f16": _lib.DTYPE_F16, "bf16": _lib.DTYPE_BF16}


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _dtype_code(dtype) -> int:
    if isinstance(dtype, int):
        return dtype
    return _DTYPE[str(dtype).replace("torch.", "").replace("bfloat16", "bf16")
                  .replace("float16", "f16").replace("float32", "f32")]


# ------------------------------------------------------------------ sizing

def bytes_per_paged_block(num_layers: int, num_kv_heads: int, head_dim: int, block_size: int,
                          dtype="bf16") -> int:
    out = ctypes.c_uint64()
    check(_lib.load().vpa_bytes_per_paged_block(num_layers, num_kv_heads, head_dim, block_size,
                                                _dtype_code(dtype), ctypes.byref(out)))
    return out.value


def blocks_for_byte_budget(byte_budget: int, bytes_per_block: int) -> int:
    out = ctypes.c_int64()
    check(_lib.load().vpa_pool_blocks_for_byte_budget(byte_budget, bytes_per_block,
                                                      ctypes.byref(out)))
    return out.value


def resolve_num_blocks(memory: str, value, num_layers: int, num_kv_heads: int, head_dim: int,
                       block_size: int, dtype="bf16") -> int:
    """PagedCacheMemory: ``("context", tokens)``, ``("blocks", n)`` or
    ``("fraction", f)`` of the current GPU's memory (hipMemGetInfo)."""
    lib = _lib.load()
    out = ctypes.c_int64()
    if memory == "context":
        check(lib.vpa_pool_blocks_for_context(int(value), block_size, ctypes.byref(out)))
        return out.value
    if memory == "blocks":
        return int(value)
    if memory == "fraction":
        bpb = bytes_per_paged_block(num_layers, num_kv_heads, head_dim, block_size, dtype)
        check(lib.vpa_pool_blocks_for_memory_fraction(float(value), bpb, ctypes.byref(out)))
        return out.value
    raise VpaError(_lib.VPA_ERR_INVALID_ARGUMENT, f"unknown paged cache memory kind {memory!r}")


# ------------------------------------------------------------ block manager

class BlockManager:
    """``PagedBlockManager``: FIFO free list over block ids 1..num_blocks-1
    (block 0 is reserved for padded batches), per-request block lists."""

    def __init__(self, num_blocks: int, block_size: int):
        self._lib = _lib.load()
        h = ctypes.c_void_p()
        check(self._lib.vpa_block_manager_create(num_blocks, block_size, ctypes.byref(h)))
        self._h = h
        self.block_size = block_size

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            self._lib.vpa_block_manager_destroy(h)
            self._h = None

    @staticmethod
    def allocatable_block_capacity(num_blocks: int) -> int:
        return max(num_blocks - 1, 0)

    def free_blocks(self) -> int:
        return self._lib.vpa_block_manager_free_blocks(self._h)

    def blocks_for_request(self, request_id: int) -> int:
        return self._lib.vpa_block_manager_blocks_for_request(self._h, request_id)

    def total_allocated_blocks(self) -> int:
        return self._lib.vpa_block_manager_total_allocated_blocks(self._h)

    def slots_available_for(self, request_id: int, num_tokens: int) -> bool:
        return bool(self._lib.vpa_block_manager_slots_available(self._h, request_id, num_tokens))

    def try_allocate_slots(self, request_id: int, num_tokens: int) -> bool:
        ok = ctypes.c_int32()
        check(self._lib.vpa_block_manager_try_allocate(self._h, request_id, num_tokens,
                                                       ctypes.byref(ok)))
        return bool(ok.value)

    def allocate_slots(self, request_id: int, num_tokens: int) -> None:
        check(self._lib.vpa_block_manager_allocate(self._h, request_id, num_tokens))

    def trim_request_to_num_tokens(self, request_id: int, num_tokens: int) -> None:
        check(self._lib.vpa_block_manager_trim(self._h, request_id, num_tokens))

    def free_request(self, request_id: int) -> None:
        check(self._lib.vpa_block_manager_free_request(self._h, request_id))

    def free_many(self, request_ids: Sequence[int]) -> None:
        for r in request_ids:
            self.free_request(r)

    def block_ids(self, request_id: int) -> List[int]:
        n = self.blocks_for_request(request_id)
        ids = np.zeros(max(n, 1), dtype=np.uint32)
        count = ctypes.c_int64()
        check(self._lib.vpa_block_manager_block_ids(self._h, request_id, _ptr(ids), n,
                                                    ctypes.byref(count)))
        return ids[:count.value].tolist()

    def block_tables_for(self, request_ids: Sequence[int]) -> List[List[int]]:
        if not request_ids:
            return []
        rids = np.ascontiguousarray(request_ids, dtype=np.uint64)
        cols = max(max(self.blocks_for_request(r) for r in request_ids), 1)
        tables = np.zeros((len(rids), cols), dtype=np.uint32)
        lens = np.zeros(len(rids), dtype=np.int32)
        check(self._lib.vpa_block_manager_block_tables(self._h, _ptr(rids), len(rids), cols,
                                                       _ptr(tables), _ptr(lens)))
        return [tables[i, :lens[i]].tolist() for i in range(len(rids))]


# -------------------------------------------------------- metadata builders

def _ragged(block_tables: Sequence[Sequence[int]]):
    lens = np.array([len(t) for t in block_tables], dtype=np.int32)
    stride = max(int(lens.max()) if len(lens) else 0, 1)
    arr = np.zeros((max(len(block_tables), 1), stride), dtype=np.uint32)
    for i, t in enumerate(block_tables):
        arr[i, :len(t)] = np.asarray(t, dtype=np.uint32)
    return arr, stride, lens


def _meta(batch: int, tokens: int, cols: int):
    arrays = dict(
        slot_mapping=np.zeros(max(tokens, 1), dtype=np.int64),
        block_tables=np.zeros((max(batch, 1), max(cols, 1)), dtype=np.uint32),
        context_lens=np.zeros(max(batch, 1), dtype=np.uint32),
        cu_seqlens_q=np.zeros(batch + 1, dtype=np.uint32),
        cu_seqlens_kv=np.zeros(batch + 1, dtype=np.uint32),
    )
    m = _lib.PagedMetadata()
    for k, a in arrays.items():
        setattr(m, k, a.ctypes.data)
    m.cols = max(cols, 1)
    return m, arrays


def _result(m, arrays, batch: int, cols: int, query_lens, kv_lens, masks=None) -> Dict:
    return {
        "slot_mapping": arrays["slot_mapping"][:m.num_tokens].copy(),
        "block_tables": arrays["block_tables"][:batch, :cols].copy(),
        "context_lens": arrays["context_lens"][:batch].copy(),
        "max_context_len": int(m.max_context_len),
        "token_attention_mask": masks,
        "prefill_causal_only": bool(m.causal_only),
        "query_lens": list(query_lens),
        "kv_lens": list(kv_lens),
        "cu_seqlens_q": arrays["cu_seqlens_q"].copy(),
        "cu_seqlens_kv": arrays["cu_seqlens_kv"].copy(),
        "max_query_len": int(m.max_query_len),
        "max_kv_len": int(m.max_kv_len),
    }


def input_metadata_from_block_tables(block_tables: Sequence[Sequence[int]], starts: Sequence[int],
                                     length: int, context_lens: Sequence[int], block_size: int,
                                     num_blocks: int) -> Dict:
    tables, stride, lens = _ragged(block_tables)
    batch = len(block_tables)
    cols = int(lens.max()) if batch else 0
    m, arrays = _meta(batch, batch * length, cols)
    st = np.ascontiguousarray(starts, dtype=np.int64)
    cl = np.ascontiguousarray(context_lens, dtype=np.int64)
    check(_lib.load().vpa_metadata_from_block_tables(
        _ptr(tables), stride, _ptr(lens), batch, _ptr(st), length, _ptr(cl), block_size,
        num_blocks, ctypes.byref(m)))
    return _result(m, arrays, batch, cols, [length] * batch, list(context_lens))


def input_metadata_from_attention_masks(block_tables: Sequence[Sequence[int]],
                                        attention_masks: Sequence[Sequence[int]], block_size: int,
                                        num_blocks: int) -> Dict:
    tables, stride, lens = _ragged(block_tables)
    masks = np.ascontiguousarray(attention_masks, dtype=np.uint32)
    batch = len(attention_masks)
    seq_len = masks.shape[1] if masks.ndim == 2 else 0
    cols = int(lens.max()) if len(lens) else 0
    m, arrays = _meta(batch, batch * seq_len, cols)
    check(_lib.load().vpa_metadata_from_attention_masks(
        _ptr(tables), stride, _ptr(lens), batch, _ptr(masks), seq_len, block_size, num_blocks,
        ctypes.byref(m)))
    q = arrays["context_lens"][:batch].astype(np.int64).tolist()
    return _result(m, arrays, batch, cols, q, q, masks.copy())


def input_metadata_from_query_lens(block_tables: Sequence[Sequence[int]],
                                   query_lens: Sequence[int], block_size: int,
                                   num_blocks: int) -> Dict:
    tables, stride, lens = _ragged(block_tables)
    batch = len(query_lens)
    cols = int(lens.max()) if len(lens) else 0
    ql = np.ascontiguousarray(query_lens, dtype=np.int64)
    m, arrays = _meta(batch, int(ql.sum()) if batch else 0, cols)
    check(_lib.load().vpa_metadata_from_query_lens(
        _ptr(tables), stride, _ptr(lens), batch, _ptr(ql), block_size, num_blocks,
        ctypes.byref(m)))
    return _result(m, arrays, batch, cols, list(query_lens), list(query_lens))


def decode_metadata_for_batch_steps(block_tables: Sequence[Sequence[int]],
                                    prompt_lens: Sequence[int], steps: int, block_size: int,
                                    num_blocks: int, max_tokens_per_sequence: int,
                                    graph_buckets: bool = False) -> List[Dict]:
    """One metadata dict per decode step; the block tables are shared and
    padded to the bucketed width when ``graph_buckets`` (the cuda-graph
    build, ``paged_kv_cache.rs:948-952``)."""
    tables, stride, lens = _ragged(block_tables)
    batch = len(block_tables)
    raw = int(lens.max()) if batch else 0
    cols = bucket_block_table_cols(raw, block_size) if graph_buckets else raw
    pl = np.ascontiguousarray(prompt_lens, dtype=np.int64)
    slots = np.zeros((max(steps, 1), max(batch, 1)), dtype=np.int64)
    ctx = np.zeros((max(steps, 1), max(batch, 1)), dtype=np.uint32)
    mx = np.zeros(max(steps, 1), dtype=np.int64)
    bt = np.zeros((max(batch, 1), max(cols, 1)), dtype=np.uint32)
    check(_lib.load().vpa_decode_metadata_for_batch_steps(
        _ptr(tables), stride, _ptr(lens), batch, _ptr(pl), steps, block_size, num_blocks,
        max_tokens_per_sequence, int(bool(graph_buckets)), max(cols, 1), _ptr(slots), _ptr(ctx),
        _ptr(mx), _ptr(bt)))
    out = []
    for t in range(steps):
        out.append({
            "slot_mapping": slots[t, :batch].copy(),
            "block_tables": bt[:batch, :cols].copy(),
            "context_lens": ctx[t, :batch].copy(),
            "max_context_len": int(mx[t]),
            "cu_seqlens_q": None,
            "cu_seqlens_kv": None,
        })
    return out


def slot_for_block_table_position(table: Sequence[int], block_size: int, num_blocks: int,
                                  position: int) -> int:
    t = np.ascontiguousarray(table if len(table) else [0], dtype=np.uint32)
    out = ctypes.c_int64()
    check(_lib.load().vpa_slot_for_block_table_position(_ptr(t), len(table), block_size,
                                                        num_blocks, position, ctypes.byref(out)))
    return out.value


def cumulative_seqlens(lengths: Sequence[int]) -> np.ndarray:
    ln = np.ascontiguousarray(lengths if len(lengths) else [0], dtype=np.int64)
    cu = np.zeros(len(lengths) + 1, dtype=np.uint32)
    check(_lib.load().vpa_cumulative_seqlens(_ptr(ln), len(lengths), _ptr(cu)))
    return cu


class ContiguousCache:
    """Slot arithmetic of a ``PagedKvCache::new_batched`` cache, whose
    sequence s owns blocks s*bps .. s*bps+bps-1 (``paged_kv_cache.rs:171-200,
    352-468``)."""

    def __init__(self, block_size: int, batch_size: int, max_tokens_per_sequence: int):
        self.block_size = block_size
        self.batch_size = batch_size
        self.max_tokens_per_sequence = max_tokens_per_sequence
        self.num_blocks_per_sequence = -(-max_tokens_per_sequence // block_size)
        self.num_blocks = batch_size * self.num_blocks_per_sequence
        self.max_tokens = self.num_blocks * block_size

    def block_table_host(self) -> List[int]:
        return list(range(self.num_blocks))

    def slot_for_sequence_position(self, sequence: int, position: int) -> int:
        out = ctypes.c_int64()
        check(_lib.load().vpa_contiguous_slot(sequence, position, self.batch_size,
                                              self.num_blocks_per_sequence, self.block_size,
                                              self.max_tokens_per_sequence, ctypes.byref(out)))
        return out.value

    def slot_for_position(self, position: int) -> int:
        return self.slot_for_sequence_position(0, position)

    def slot_mapping_for_range(self, start: int, length: int) -> np.ndarray:
        if start + length > self.max_tokens:
            raise VpaError(_lib.VPA_ERR_INVALID_ARGUMENT,
                           f"slot range exceeds paged kv cache capacity: start={start} "
                           f"len={length} max_tokens={self.max_tokens}")
        return np.array([self.slot_for_position(p) for p in range(start, start + length)],
                        dtype=np.int64)

    def block_tables_for_batch(self, batch: int) -> List[List[int]]:
        n = self.num_blocks_per_sequence
        return [list(range(s * n, (s + 1) * n)) for s in range(batch)]

    def decode_metadata_for_steps(self, prompt_len: int, steps: int) -> List[Dict]:
        """Single-sequence decode steps: slot of position prompt_len + t,
        context prompt_len + t + 1 (``paged_kv_cache.rs:871-922``,
        ``generation.rs:1475-1483``)."""
        if prompt_len + steps > self.max_tokens:
            raise VpaError(_lib.VPA_ERR_INVALID_ARGUMENT,
                           "decode metadata range exceeds paged kv cache capacity")
        return [{"slot_mapping": np.array([self.slot_for_position(prompt_len + t)], np.int64),
                 "block_tables": np.array([self.block_table_host()], np.uint32),
                 "context_lens": np.array([prompt_len + t + 1], np.uint32),
                 "max_context_len": prompt_len + t + 1}
                for t in range(steps)]


# ------------------------------------------------------ decode-graph padding

def cuda_graph_batch_bucket(actual_batch: int, max_batch: int) -> Optional[int]:
    b = _lib.load().vpa_graph_batch_bucket(actual_batch, max_batch)
    return None if b == 0 else b


def cuda_graph_batch_buckets(max_batch: int) -> List[int]:
    out = np.zeros(64, dtype=np.int32)
    n = ctypes.c_int32()
    check(_lib.load().vpa_graph_batch_buckets(max_batch, _ptr(out), len(out), ctypes.byref(n)))
    return out[:n.value].tolist()


def bucket_block_table_cols(blocks: int, block_size: int) -> int:
    return int(_lib.load().vpa_bucket_block_table_cols(blocks, block_size))


def pad_decode_batch_to_max(max_batch: int, input_ids, slot_mapping, context_lens, block_tables,
                            block_table_cols: int):
    """Pad the decode batch to ``max_batch`` rows (ids 0, slot 0, context 1,
    table 0) and the tables to ``block_table_cols`` columns (repeating each
    row's last column). Returns (ids, slots, context_lens, block_tables)."""
    ids = np.ascontiguousarray(input_ids, dtype=np.uint32).reshape(-1)
    slots = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    ctx = np.ascontiguousarray(context_lens, dtype=np.uint32)
    bt = np.ascontiguousarray(block_tables, dtype=np.uint32)
    actual = len(ids)
    cols_in = bt.shape[1] if bt.ndim == 2 else 0
    o_ids = np.zeros(max(max_batch, 1), dtype=np.uint32)
    o_slots = np.zeros(max(max_batch, 1), dtype=np.int64)
    o_ctx = np.zeros(max(max_batch, 1), dtype=np.uint32)
    o_bt = np.zeros((max(max_batch, 1), max(block_table_cols, 1)), dtype=np.uint32)
    check(_lib.load().vpa_pad_decode_batch(max_batch, actual, _ptr(ids), _ptr(slots), _ptr(ctx),
                                           _ptr(bt), cols_in, block_table_cols, _ptr(o_ids),
                                           _ptr(o_slots), _ptr(o_ctx), _ptr(o_bt)))
    return (o_ids[:max_batch], o_slots[:max_batch], o_ctx[:max_batch],
            o_bt[:max_batch, :block_table_cols])
