"""ctypes binding of libvpa.so (the C ABI declared in include/vpa.h).

The library is built in-tree by ``__graft_entry__.build()`` (or
``make -C qwen3asr.rs_amd/csrc``) and must be present: there is no fallback
path, a missing library raises immediately.
"""

from __future__ import annotations

import ctypes
import os

# VPA_LIBRARY may point at another build of the same library.
LIB_PATH = os.environ.get("VPA_LIBRARY") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "libvpa.so")

VPA_OK = 0
VPA_ERR_INVALID_ARGUMENT = 1
VPA_ERR_UNSUPPORTED = 2
VPA_ERR_WORKSPACE = 3
VPA_ERR_HIP = 4
VPA_ERR_CAPACITY = 5
VPA_ERR_NOT_FOUND = 6

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2
DTYPE_FP8_E4M3 = 3  # cache element only (OCP E4M3FN bytes)

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_f32 = ctypes.c_float
_sz = ctypes.c_size_t
_cstr = ctypes.c_char_p

# name -> (restype, argtypes); mirrors include/vpa.h
SIGNATURES = {
    "vpa_last_error": (_cstr, []),
    "vpa_version": (_cstr, []),
    "vpa_cache_layout": (ctypes.c_int, [_i32, _i32, _i32, _i64, _i32, _p, _p]),
    "vpa_reshape_and_cache": (ctypes.c_int, [_p, _p, _i64, _i64, _p, _p, _p, _p, _p, _i64, _i32,
                                             _i32, _i32, _i64, _i64, _i64, _i32, _i32, _p]),
    "vpa_paged_attention_workspace_size": (_sz, [_i32, _i32, _i32, _i32]),
    "vpa_paged_attention": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _i32, _f32,
                                           _f32, _p, _i32, _i32, _i32, _i32, _i32, _i64, _i64,
                                           _i64, _i32, _i32, _p, _sz, _p]),
    "vpa_paged_attention_plan": (ctypes.c_int, [_p, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                                _i32, _p, _sz, _p]),
    "vpa_paged_attention_planned": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _i32,
                                                   _f32, _f32, _p, _i32, _i32, _i32, _i32, _i32,
                                                   _i64, _i64, _i64, _i32, _i32, _p, _sz, _p]),
    "vpa_reshape_and_cache_paged_attention": (ctypes.c_int, [
        _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _i32, _p, _i32, _f32, _i32, _i32, _i32,
        _i32, _i32, _i64, _i64, _i64, _i32, _i32, _p, _sz, _p]),
    "vpa_reshape_and_cache_paged_attention_planned": (ctypes.c_int, [
        _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _i32, _p, _i32, _f32, _i32, _i32, _i32,
        _i32, _i32, _i64, _i64, _i64, _i32, _i32, _p, _sz, _p]),
    "vpa_paged_attention_noalloc": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _i32,
                                                   _f32, _f32, _p, _i32, _i32, _i32, _i32, _i32,
                                                   _i64, _i64, _i64, _i32, _i32, _p]),
    "vpa_paged_cache_read": (ctypes.c_int, [_p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                            _i64, _i64, _i64, _i32, _p, _sz, _u32, _p, _p]),
    "vpa_gather_kv_cache": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i32, _p, _i32, _i64, _i32,
                                           _i32, _i32, _i64, _i64, _i64, _i32, _i32, _p]),
    "vpa_chunked_prefill_paged_attention": (ctypes.c_int, [
        _p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _i32, _i32, _i32, _i64, _f32, _f32, _i32,
        _i32, _i32, _i32, _i32, _i64, _i64, _i64, _i32, _i32, _p]),
    "vpa_argmax_rows": (ctypes.c_int, [_p, _i64, _i32, _i32, _i32, _p, _p]),
    "vpa_decode_consume_tokens": (ctypes.c_int, [
        _p, _p, _p, _p, _p, _i32, _p, _i32, _u32, _p, _p, _i32, _p]),
    "vpa_allocate_rows": (ctypes.c_int, [_p, _i32, _p, _p, _p, _p, _p, _i32, _i32, _i32, _p]),
    "vpa_decode_step_metadata": (ctypes.c_int, [
        _p, _i32, _p, _p, _p, _p, _p, _i32, _i32, _p, _p, _p, _i32, _p]),
    "vpa_release_blocks": (ctypes.c_int, [_p, _i32, _p, _p, _p, _p, _i32, _i32, _p]),
    # include/vpa_host.h
    "vpa_bytes_per_paged_block": (ctypes.c_int, [_i32, _i32, _i32, _i32, _i32, _p]),
    "vpa_pool_blocks_for_context": (ctypes.c_int, [_i64, _i32, _p]),
    "vpa_pool_blocks_for_byte_budget": (ctypes.c_int, [_u64, _u64, _p]),
    "vpa_pool_blocks_for_memory_fraction": (ctypes.c_int, [_f32, _u64, _p]),
    "vpa_block_manager_create": (ctypes.c_int, [_i64, _i32, _p]),
    "vpa_block_manager_destroy": (None, [_p]),
    "vpa_block_manager_free_blocks": (_i64, [_p]),
    "vpa_block_manager_blocks_for_request": (_i64, [_p, _u64]),
    "vpa_block_manager_total_allocated_blocks": (_i64, [_p]),
    "vpa_block_manager_slots_available": (ctypes.c_int, [_p, _u64, _i64]),
    "vpa_block_manager_try_allocate": (ctypes.c_int, [_p, _u64, _i64, _p]),
    "vpa_block_manager_allocate": (ctypes.c_int, [_p, _u64, _i64]),
    "vpa_block_manager_trim": (ctypes.c_int, [_p, _u64, _i64]),
    "vpa_block_manager_free_request": (ctypes.c_int, [_p, _u64]),
    "vpa_block_manager_block_ids": (ctypes.c_int, [_p, _u64, _p, _i64, _p]),
    "vpa_block_manager_block_tables": (ctypes.c_int, [_p, _p, _i32, _i32, _p, _p]),
    "vpa_slot_for_block_table_position": (ctypes.c_int, [_p, _i32, _i32, _i64, _i64, _p]),
    "vpa_cumulative_seqlens": (ctypes.c_int, [_p, _i32, _p]),
    "vpa_metadata_from_block_tables": (ctypes.c_int, [_p, _i32, _p, _i32, _p, _i32, _p, _i32,
                                                      _i64, _p]),
    "vpa_metadata_from_attention_masks": (ctypes.c_int, [_p, _i32, _p, _i32, _p, _i32, _i32,
                                                         _i64, _p]),
    "vpa_metadata_from_query_lens": (ctypes.c_int, [_p, _i32, _p, _i32, _p, _i32, _i64, _p]),
    "vpa_decode_metadata_for_batch_steps": (ctypes.c_int, [_p, _i32, _p, _i32, _p, _i32, _i32,
                                                           _i64, _i64, _i32, _i32, _p, _p, _p,
                                                           _p]),
    "vpa_contiguous_slot": (ctypes.c_int, [_i64, _i64, _i64, _i64, _i32, _i64, _p]),
    "vpa_graph_batch_bucket": (_i32, [_i32, _i32]),
    "vpa_graph_batch_buckets": (ctypes.c_int, [_i32, _p, _i32, _p]),
    "vpa_bucket_block_table_cols": (_i64, [_i64, _i32]),
    "vpa_pad_decode_batch": (ctypes.c_int, [_i32, _i32, _p, _p, _p, _p, _i32, _i32, _p, _p, _p,
                                            _p]),
}


class PagedMetadata(ctypes.Structure):
    """Mirror of vpa_paged_metadata (include/vpa_host.h)."""

    _fields_ = [
        ("slot_mapping", _p),
        ("block_tables", _p),
        ("context_lens", _p),
        ("cu_seqlens_q", _p),
        ("cu_seqlens_kv", _p),
        ("cols", _i32),
        ("num_tokens", _i64),
        ("max_context_len", _i64),
        ("max_query_len", _i64),
        ("max_kv_len", _i64),
        ("causal_only", _i32),
    ]


class VpaError(RuntimeError):
    """A libvpa entry point returned a non-zero status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[vpa status {code}] {message}")
        self.code = code
        self.message = message


_lib = None


def load() -> ctypes.CDLL:
    """Load libvpa.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"libvpa.so not found at {LIB_PATH}: build it with __graft_entry__.build() "
            "(the paged-KV ops have no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(code: int) -> None:
    if code != VPA_OK:
        msg = load().vpa_last_error().decode("utf-8", "replace")
        raise VpaError(code, msg)
