"""TEST INFRASTRUCTURE ONLY — numpy/ctypes face of the CPU oracle.

Wraps ``oracle/libvpa_oracle.so`` (built from ``oracle/vpa_oracle.c``) for
numpy arrays. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module; the product path never does.

The restated reference semantics and their file:line sources are listed in
the header of ``vpa_oracle.c``. In short: the paged cache layout of
``vasr-paged-attn/src/paged_kv_cache.rs:263-294``, slot mapping with
``PAD_SLOT_ID`` skip (``paged_kv_cache.rs:7, 74-103, 697-700``), GQA
``repeat_kv`` (``vasr-models/src/model/attention.rs:12-21``), eager softmax
attention (``attention.rs:243-286``), cached causal mask
(``attention.rs:78-149``) and the ``+1e-6`` softmax denominator of the paged
sibling kernel (``prefill_paged_attn.metal:1300``). FP8 (E4M3FN) caches:
decode as ``prefill_paged_attn.metal:698-722``, dequantisation
``(float)byte * scale`` rounded to the query type (``:764-769``), and the
published quantising rule of the un-vendored kernels, round-to-nearest-even
of ``x / scale`` saturating at 448.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

F32, F16, BF16, FP8 = 0, 1, 2, 3

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libvpa_oracle.so")
_lib = None

_p = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_dbl = ctypes.c_double
_flt = ctypes.c_float


def build() -> None:
    """Compile libvpa_oracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-B", "-C", _HERE], check=True, capture_output=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_reshape_and_cache.argtypes = [_i32, _p, _p, _i64, _i64, _p, _p, _p, _i64, _i32,
                                               _i32, _i32, _i64, _i64, _i64]
        L.oracle_reshape_and_cache.restype = None
        L.oracle_gather_kv_cache.argtypes = [_i32, _p, _p, _p, _p, _p, _i32, _p, _i32, _i32, _i32,
                                             _i32, _i64, _i64, _i64]
        L.oracle_gather_kv_cache.restype = None
        L.oracle_paged_attention_f64.argtypes = [_i32, _p, _p, _p, _p, _p, _i32, _p, _i32, _dbl,
                                                 _i32, _i32, _i32, _i32, _i32, _i64, _i64, _i64]
        L.oracle_paged_attention_f64.restype = None
        L.oracle_fp8_to_f32_array.argtypes = [_p, _p, _i64]
        L.oracle_fp8_to_f32_array.restype = None
        L.oracle_fp8_from_f32_array.argtypes = [_p, _p, _i64]
        L.oracle_fp8_from_f32_array.restype = None
        L.oracle_reshape_and_cache_fp8.argtypes = [_i32, _p, _p, _i64, _i64, _p, _p, _p, _i64,
                                                   _i32, _i32, _i32, _i64, _i64, _i64, _flt,
                                                   _flt]
        L.oracle_reshape_and_cache_fp8.restype = None
        L.oracle_gather_kv_cache_fp8.argtypes = [_i32, _p, _p, _p, _p, _p, _i32, _p, _i32, _i32,
                                                 _i32, _i32, _i64, _i64, _i64, _flt, _flt]
        L.oracle_gather_kv_cache_fp8.restype = None
        L.oracle_paged_attention_kv_f64.argtypes = [_i32, _i32, _flt, _flt, _p, _p, _p, _p, _p,
                                                    _i32, _p, _i32, _dbl, _i32, _i32, _i32, _i32,
                                                    _i32, _i64, _i64, _i64]
        L.oracle_paged_attention_kv_f64.restype = None
        L.oracle_prefill_attention_kv_f64.argtypes = [_i32, _i32, _flt, _flt, _p, _p, _p, _p, _p,
                                                      _i32, _p, _p, _i32, _i32, _dbl, _i32, _i32,
                                                      _i32, _i32, _i64, _i64, _i64, _dbl]
        L.oracle_prefill_attention_kv_f64.restype = None
        L.oracle_argmax_rows.argtypes = [_i32, _p, _i64, _i32, _i32, _p]
        L.oracle_argmax_rows.restype = None
        L.oracle_decode_consume_tokens.argtypes = [_p, _p, _p, _p, _p, _i32, _p, _i32,
                                                   ctypes.c_uint32, _p, _p, _i32]
        L.oracle_decode_consume_tokens.restype = None
        L.oracle_prefill_attention_f64.argtypes = [_i32, _p, _p, _p, _p, _p, _i32, _p, _p, _i32,
                                                   _i32, _dbl, _i32, _i32, _i32, _i32, _i64,
                                                   _i64, _i64, _dbl]
        L.oracle_prefill_attention_f64.restype = None
        L.cpu_baseline_decode_step.argtypes = [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _i32, _p,
                                               _flt, _i32, _i32, _i32, _i32, _i32, _i64, _i64,
                                               _i64]
        L.cpu_baseline_decode_step.restype = _i32
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def dtype_code(a: np.ndarray, code: int | None = None) -> int:
    """16-bit data travels as uint16 words; the caller names bf16 vs f16."""
    if code is not None:
        return code
    if a.dtype == np.float32:
        return F32
    raise ValueError("16-bit arrays need an explicit dtype code (F16 or BF16)")


def _cache_geom(key_cache: np.ndarray):
    nb, kvh, dx, bs, x = key_cache.shape
    return nb, kvh, dx * x, bs, kvh * dx * bs * x, dx * bs * x


def reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, dtype=None):
    """In-place append of key/value rows [T, KVH, D] into the caches."""
    code = dtype_code(key, dtype)
    nb, kvh, d, bs, bstride, hstride = _cache_geom(key_cache)
    t = key.shape[0]
    slot_mapping = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    lib().oracle_reshape_and_cache(code, _ptr(key), _ptr(value), kvh * d, kvh * d,
                                   _ptr(key_cache), _ptr(value_cache), _ptr(slot_mapping), t,
                                   kvh, d, bs, nb, bstride, hstride)


def gather_kv_cache(key_cache, value_cache, block_tables, cu_seqlens, dtype=None):
    code = dtype_code(key_cache, dtype)
    nb, kvh, d, bs, bstride, hstride = _cache_geom(key_cache)
    block_tables = np.ascontiguousarray(block_tables, dtype=np.uint32)
    cu_seqlens = np.ascontiguousarray(cu_seqlens, dtype=np.uint32)
    rows = int(cu_seqlens[-1])
    ok = np.zeros((rows, kvh, d), dtype=key_cache.dtype)
    ov = np.zeros((rows, kvh, d), dtype=key_cache.dtype)
    lib().oracle_gather_kv_cache(code, _ptr(ok), _ptr(ov), _ptr(key_cache), _ptr(value_cache),
                                 _ptr(block_tables), block_tables.shape[1], _ptr(cu_seqlens),
                                 block_tables.shape[0], kvh, d, bs, nb, bstride, hstride)
    return ok, ov


def paged_attention(q, key_cache, value_cache, block_tables, context_lens, max_context_len,
                    scale, dtype=None, kv_dtype=None, k_scale=1.0, v_scale=1.0) -> np.ndarray:
    """Decode attention, float64 result [B, H, D]. ``kv_dtype=FP8`` reads an
    fp8 cache (uint8 arrays) dequantised with ``k_scale`` / ``v_scale``."""
    code = dtype_code(q, dtype)
    kv = code if kv_dtype is None else kv_dtype
    nb, kvh, d, bs, bstride, hstride = _cache_geom(key_cache)
    b, h, _ = q.shape
    block_tables = np.ascontiguousarray(block_tables, dtype=np.uint32)
    context_lens = np.ascontiguousarray(context_lens, dtype=np.uint32)
    out = np.zeros((b, h, d), dtype=np.float64)
    lib().oracle_paged_attention_kv_f64(code, kv, float(k_scale), float(v_scale), _ptr(out),
                                        _ptr(q), _ptr(key_cache), _ptr(value_cache),
                                        _ptr(block_tables), block_tables.shape[1],
                                        _ptr(context_lens), int(max_context_len), float(scale), b,
                                        h, kvh, d, bs, nb, bstride, hstride)
    return out


def prefill_attention(q, key_cache, value_cache, block_tables, context_lens, cu_seqlens_q, scale,
                      causal=True, dtype=None, eps=0.0, kv_dtype=None, k_scale=1.0,
                      v_scale=1.0) -> np.ndarray:
    """Chunked prefill attention over the paged cache, float64 [total_q, H, D].

    ``eps`` is added to the softmax denominator: 0.0 is the flash varlen path
    (attention.rs:554-664), 1e-6 the Metal prefill kernel
    (prefill_paged_attn.metal:1300)."""
    code = dtype_code(q, dtype)
    nb, kvh, d, bs, bstride, hstride = _cache_geom(key_cache)
    tq, h, _ = q.shape
    block_tables = np.ascontiguousarray(block_tables, dtype=np.uint32)
    context_lens = np.ascontiguousarray(context_lens, dtype=np.uint32)
    cu_seqlens_q = np.ascontiguousarray(cu_seqlens_q, dtype=np.uint32)
    out = np.zeros((tq, h, d), dtype=np.float64)
    kv = code if kv_dtype is None else kv_dtype
    lib().oracle_prefill_attention_kv_f64(code, kv, float(k_scale), float(v_scale), _ptr(out),
                                          _ptr(q), _ptr(key_cache), _ptr(value_cache),
                                          _ptr(block_tables), block_tables.shape[1],
                                          _ptr(context_lens), _ptr(cu_seqlens_q),
                                          block_tables.shape[0], int(bool(causal)), float(scale),
                                          h, kvh, d, bs, nb, bstride, hstride, float(eps))
    return out


def fp8_to_f32(b: np.ndarray) -> np.ndarray:
    """E4M3FN bytes -> float32 (exact)."""
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(b.shape, dtype=np.float32)
    lib().oracle_fp8_to_f32_array(_ptr(b), _ptr(out), b.size)
    return out


def fp8_from_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> E4M3FN bytes (round to nearest even, saturate at 448)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().oracle_fp8_from_f32_array(_ptr(x), _ptr(out), x.size)
    return out


def reshape_and_cache_fp8(key, value, key_cache, value_cache, slot_mapping, dtype, k_scale,
                          v_scale):
    """In-place append of key/value rows [T, KVH, D] (dtype code ``dtype``)
    into uint8 fp8 caches [NB, KVH, D/16, BS, 16] / [NB, KVH, D, BS]."""
    nb, kvh, d, bs, bstride, hstride = _cache_geom(key_cache)
    t = key.shape[0]
    slot_mapping = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    lib().oracle_reshape_and_cache_fp8(dtype, _ptr(key), _ptr(value), kvh * d, kvh * d,
                                       _ptr(key_cache), _ptr(value_cache), _ptr(slot_mapping), t,
                                       kvh, d, bs, nb, bstride, hstride, float(k_scale),
                                       float(v_scale))


def gather_kv_cache_fp8(key_cache, value_cache, block_tables, cu_seqlens, out_dtype, k_scale,
                        v_scale):
    """Packed dequantised rows [rows, KVH, D] of ``out_dtype`` (code) from fp8 caches."""
    nb, kvh, d, bs, bstride, hstride = _cache_geom(key_cache)
    block_tables = np.ascontiguousarray(block_tables, dtype=np.uint32)
    cu_seqlens = np.ascontiguousarray(cu_seqlens, dtype=np.uint32)
    rows = int(cu_seqlens[-1])
    npdt = np.float32 if out_dtype == F32 else np.uint16
    ok = np.zeros((rows, kvh, d), dtype=npdt)
    ov = np.zeros((rows, kvh, d), dtype=npdt)
    lib().oracle_gather_kv_cache_fp8(out_dtype, _ptr(ok), _ptr(ov), _ptr(key_cache),
                                     _ptr(value_cache), _ptr(block_tables), block_tables.shape[1],
                                     _ptr(cu_seqlens), block_tables.shape[0], kvh, d, bs, nb,
                                     bstride, hstride, float(k_scale), float(v_scale))
    return ok, ov


def cpu_baseline_decode_step(q, new_key, new_value, slot_mapping, key_cache, value_cache,
                             block_tables, context_lens, scale, dtype=None):
    """The reference's CPU decode path (append + gather + eager attention) in f32.

    Returns (out [B, H, D] float32, threads used)."""
    code = dtype_code(q, dtype)
    nb, kvh, d, bs, bstride, hstride = _cache_geom(key_cache)
    b, h, _ = q.shape
    out = np.zeros((b, h, d), dtype=np.float32)
    slot_mapping = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    block_tables = np.ascontiguousarray(block_tables, dtype=np.uint32)
    context_lens = np.ascontiguousarray(context_lens, dtype=np.uint32)
    threads = lib().cpu_baseline_decode_step(code, _ptr(out), _ptr(q), _ptr(new_key),
                                             _ptr(new_value), _ptr(slot_mapping), _ptr(key_cache),
                                             _ptr(value_cache), _ptr(block_tables),
                                             block_tables.shape[1], _ptr(context_lens),
                                             float(scale), b, h, kvh, d, bs, nb, bstride, hstride)
    return out, threads


# ---- element conversions used by tests to build inputs -------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 words (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def to_f32(a: np.ndarray, code: int) -> np.ndarray:
    if code == F32:
        return np.asarray(a, dtype=np.float32)
    return bf16_bits_to_f32(a) if code == BF16 else f16_bits_to_f32(a)


def from_f32(a: np.ndarray, code: int) -> np.ndarray:
    if code == F32:
        return np.ascontiguousarray(a, dtype=np.float32)
    return f32_to_bf16_bits(a) if code == BF16 else f32_to_f16_bits(a)


def argmax_rows(logits: np.ndarray, dtype=None) -> np.ndarray:
    """u32 next-token ids of logits [B, V] (candle's argmax scan)."""
    code = dtype_code(logits, dtype)
    logits = np.ascontiguousarray(logits)
    b, v = logits.shape
    out = np.zeros(b, dtype=np.uint32)
    lib().oracle_argmax_rows(code, _ptr(logits), v, v, b, _ptr(out))
    return out


def decode_consume_tokens(next_ids, finished, generated, gen_len, eos_ids, eos_fill_id,
                          prev_slots=None, input_ids=None):
    """In-place step-start bookkeeping; returns (input_ids, active_count).
    ``prev_slots``: the previous step's slot_mapping (rows with a negative
    slot did not run and feed ``input_ids`` again); ``input_ids``: the
    previous step's input ids (read for those rows)."""
    b, cap = generated.shape
    eos = np.ascontiguousarray(eos_ids, dtype=np.uint32)
    inp = (np.zeros(b, dtype=np.uint32) if input_ids is None
           else np.array(input_ids, dtype=np.uint32, copy=True))
    cnt = np.zeros(1, dtype=np.uint32)
    prev = None if prev_slots is None else np.ascontiguousarray(prev_slots, dtype=np.int64)
    lib().oracle_decode_consume_tokens(_ptr(np.ascontiguousarray(next_ids, dtype=np.uint32)),
                                       _ptr(finished), None if prev is None else _ptr(prev),
                                       _ptr(generated), _ptr(gen_len), cap,
                                       _ptr(eos), eos.size, int(eos_fill_id), _ptr(inp),
                                       _ptr(cnt), b)
    return inp, int(cnt[0])



# ------------------------------------------------------------------ block manager
class OracleError(RuntimeError):
    """An error the reference's block manager raises (same message)."""


class BlockManager:
    """Pure-Python restatement of PagedBlockManager
    (vasr-paged-attn/src/paged_cache_runtime.rs:217-371): a FIFO free list of
    the block ids 1 .. num_blocks - 1 (block 0 is kept for padded batch rows,
    :224-231, :271-274), per-request block lists grown by try_allocate_slots
    (:287-316: take `ceil(tokens / block_size) - held` ids from the front,
    nothing when the pool has fewer), shrunk by trim_request_to_num_tokens
    (:322-337) and released by free_request (:350-359), both handing the
    removed blocks back to the end of the free list last block first."""

    def __init__(self, num_blocks: int, block_size: int):
        from collections import deque

        self.block_size = int(block_size)
        self.free = deque(range(1, int(num_blocks)))
        self.requests: dict[int, list[int]] = {}

    @staticmethod
    def allocatable_block_capacity(num_blocks: int) -> int:
        return max(int(num_blocks) - 1, 0)

    def free_blocks(self) -> int:
        return len(self.free)

    def _needed(self, request_id: int, num_tokens: int) -> int:
        required = -(-int(num_tokens) // self.block_size)
        return max(required - len(self.requests.get(request_id, [])), 0)

    def slots_available_for(self, request_id: int, num_tokens: int) -> bool:
        return self._needed(request_id, num_tokens) <= len(self.free)

    def blocks_for_request(self, request_id: int) -> int:
        return len(self.requests.get(request_id, []))

    def total_allocated_blocks(self) -> int:
        return sum(len(b) for b in self.requests.values())

    def try_allocate_slots(self, request_id: int, num_tokens: int) -> bool:
        needed = self._needed(request_id, num_tokens)
        if needed == 0:
            return True
        if needed > len(self.free):
            return False
        ids = self.requests.setdefault(request_id, [])
        for _ in range(needed):
            ids.append(self.free.popleft())
        return True

    def allocate_slots(self, request_id: int, num_tokens: int) -> None:
        if not self.try_allocate_slots(request_id, num_tokens):
            raise OracleError(f"paged KV cache exhausted: request_id={request_id} "
                              f"num_tokens={num_tokens} free_blocks={len(self.free)}")

    def trim_request_to_num_tokens(self, request_id: int, num_tokens: int) -> None:
        keep = -(-int(num_tokens) // self.block_size)
        ids = self.requests.get(request_id)
        if ids is None or keep >= len(ids):
            return
        removed = ids[keep:]
        del ids[keep:]
        for b in reversed(removed):
            if b != 0:
                self.free.append(b)

    def block_ids(self, request_id: int) -> list[int]:
        if request_id not in self.requests:
            raise OracleError("paged KV request has no allocated blocks: "
                              f"request_id={request_id}")
        return list(self.requests[request_id])

    def free_request(self, request_id: int) -> None:
        ids = self.requests.pop(request_id, None)
        if ids is None:
            return
        for b in reversed(ids):
            if b != 0:
                self.free.append(b)

    def free_many(self, request_ids) -> None:
        for r in request_ids:
            self.free_request(r)

    def block_tables_for(self, request_ids) -> list[list[int]]:
        return [self.block_ids(r) for r in request_ids]


def slot_for_position(table, block_size: int, num_blocks: int, position: int) -> int:
    """slot = table[position / block_size] * block_size + position % block_size
    (vasr-paged-attn/src/paged_kv_cache.rs:74-103); a position past the
    table, or a block id past the pool, is the reference's error."""
    idx = int(position) // int(block_size)
    if idx >= len(table):
        raise OracleError(f"missing block table entry: block_idx={idx} position={position}")
    block = int(table[idx])
    if block >= int(num_blocks):
        raise OracleError(f"block id exceeds paged cache capacity: block_id={block} "
                          f"num_blocks={num_blocks}")
    return block * int(block_size) + int(position) % int(block_size)
