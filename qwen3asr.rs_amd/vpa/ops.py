"""Tensor-level paged-KV ops over libvpa, mirroring the Candle op API.

The three functions below keep the names, argument order, argument meaning
and error behaviour of the ``mistralrs_paged_attn`` ops that vASR calls
(re-exported at ``vasr-paged-attn/src/lib.rs:20-21``):

* ``reshape_and_cache``  — ``vasr-models/src/model/thinker_text.rs:1101-1109, 1324-1332``
* ``paged_attention``    — ``thinker_text.rs:1126-1139``
* ``gather_kv_cache``    — ``thinker_text.rs:190-198, 1344-1352``

plus ``paged_attention_varlen_prefill`` named after the reference's Metal
paged prefill (``vasr-paged-attn/src/metal/varlen_prefill.rs:284-420``).

Tensors are torch tensors on a ROCm device (torch is only the carrier of
device memory and the current stream here); every computation runs in the
HIP kernels of libvpa. Shape or dtype mismatches raise ``VpaError`` with
status ``VPA_ERR_INVALID_ARGUMENT`` / ``VPA_ERR_UNSUPPORTED`` before any
launch, as the reference returns ``Err(candle_core::Error::Msg)``.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import VpaError, check

_DTYPES = {
    torch.float32: _lib.DTYPE_F32,
    torch.float16: _lib.DTYPE_F16,
    torch.bfloat16: _lib.DTYPE_BF16,
    # fp8 caches: E4M3FN bytes, as torch's float8 type or raw uint8
    torch.float8_e4m3fn: _lib.DTYPE_FP8_E4M3,
    torch.uint8: _lib.DTYPE_FP8_E4M3,
}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise VpaError(_lib.VPA_ERR_UNSUPPORTED, f"unsupported dtype {dtype}") from None


def _err(msg: str):
    return VpaError(_lib.VPA_ERR_INVALID_ARGUMENT, msg)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require_device(*ts: torch.Tensor) -> None:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise _err(f"tensor on {t.device}: paged-KV ops run on the GPU only")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise _err(f"device mismatch: {dev} vs {t.device}")


def cache_geometry(key_cache: torch.Tensor, value_cache: torch.Tensor):
    """(num_blocks, num_kv_heads, head_dim, block_size, block_stride, head_stride)
    of a key/value cache pair in the reference layout."""
    if key_cache.dim() != 5 or value_cache.dim() != 4:
        raise _err(f"key_cache must be 5-d and value_cache 4-d, got {tuple(key_cache.shape)} "
                   f"and {tuple(value_cache.shape)}")
    nb, kvh, dx, bs, x = key_cache.shape
    nbv, kvhv, d, bsv = value_cache.shape
    if (nb, kvh, bs) != (nbv, kvhv, bsv) or dx * x != d:
        raise _err(f"paged cache shape mismatch: key={tuple(key_cache.shape)} "
                   f"value={tuple(value_cache.shape)}")
    if key_cache.dtype != value_cache.dtype:
        raise _err(f"key/value cache dtype mismatch: {key_cache.dtype} vs {value_cache.dtype}")
    if x * key_cache.element_size() != 16:
        raise _err(f"key cache pack x={x} does not match 16 / {key_cache.element_size()}")
    ks, vs = key_cache.stride(), value_cache.stride()
    tile = d * bs
    # (block, head) tiles must be contiguous; the two leading strides may be
    # those of a view into a larger pool but must agree between K and V.
    if ks[2:] != (bs * x, x, 1) or vs[2:] != (bs, 1):
        raise _err("paged cache tiles must be contiguous")
    if ks[0] != vs[0] or ks[1] != vs[1]:
        raise _err(f"key/value cache strides differ: {ks[:2]} vs {vs[:2]}")
    if ks[1] < tile:
        raise _err(f"cache head stride {ks[1]} smaller than tile {tile}")
    return nb, kvh, d, bs, ks[0], ks[1]


def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, k_scale: Optional[torch.Tensor],
                      v_scale: Optional[torch.Tensor], key_cache: torch.Tensor,
                      value_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Scatter ``key``/``value`` [T, KVH, D] into the caches at ``slot_mapping`` (i64).

    Negative slots are padding and are skipped. The caches are written in
    place. For 16/32-bit caches ``k_scale``/``v_scale`` are ignored; an fp8
    cache (``torch.float8_e4m3fn`` or ``uint8``) stores E4M3FN(x / scale)
    with the one-element f32 device tensors ``k_scale``/``v_scale``."""
    _require_device(key, value, key_cache, value_cache, slot_mapping)
    nb, kvh, d, bs, bstride, hstride = cache_geometry(key_cache, value_cache)
    if key.dim() != 3 or value.shape != key.shape:
        raise _err(f"key/value must be [T, KVH, D] of equal shape, got {tuple(key.shape)} and "
                   f"{tuple(value.shape)}")
    t, kh, kd = key.shape
    if (kh, kd) != (kvh, d):
        raise _err(f"key shape {tuple(key.shape)} does not match cache heads={kvh} dim={d}")
    if key.dtype != value.dtype:
        raise _err(f"key/value dtype mismatch: {key.dtype} vs {value.dtype}")
    if slot_mapping.dtype != torch.int64 or slot_mapping.dim() != 1 or slot_mapping.numel() != t:
        raise _err(f"slot_mapping must be i64 [{t}], got {slot_mapping.dtype} "
                   f"{tuple(slot_mapping.shape)}")
    # Packed rows are used as they are; anything else is made contiguous
    # (thinker_text.rs:43-62).
    if key.stride(2) != 1 or key.stride(1) != d:
        key = key.contiguous()
    if value.stride(2) != 1 or value.stride(1) != d:
        value = value.contiguous()
    slot_mapping = slot_mapping.contiguous()
    lib = _lib.load()
    check(lib.vpa_reshape_and_cache(
        key.data_ptr(), value.data_ptr(), key.stride(0), value.stride(0), _ptr(k_scale),
        _ptr(v_scale), key_cache.data_ptr(), value_cache.data_ptr(), slot_mapping.data_ptr(), t,
        kvh, d, bs, nb, bstride, hstride, dtype_code(key.dtype), dtype_code(key_cache.dtype),
        _stream(key_cache)))


def paged_attention_workspace(num_seqs: int, num_heads: int, head_dim: int,
                              max_context_len: int, device) -> Optional[torch.Tensor]:
    """Caller-side split-K workspace (None when not needed)."""
    n = _lib.load().vpa_paged_attention_workspace_size(num_seqs, num_heads, head_dim,
                                                        max_context_len)
    if n == 0:
        return None
    # torch's caching allocator returns 512-byte aligned blocks
    return torch.empty(n, dtype=torch.uint8, device=device)


def paged_attention(q: torch.Tensor, k_scale: Optional[torch.Tensor],
                    v_scale: Optional[torch.Tensor], key_cache: torch.Tensor,
                    value_cache: torch.Tensor, block_tables: torch.Tensor,
                    context_lens: torch.Tensor, alibi_slopes: Optional[torch.Tensor],
                    max_context_len: int, softmax_scale: float, softcapping: float,
                    sinks: Optional[torch.Tensor], *, out: Optional[torch.Tensor] = None,
                    workspace: Optional[torch.Tensor] = None,
                    planned: bool = False) -> torch.Tensor:
    """Single-token decode attention over the paged cache; returns [B, H, D].

    ``out`` and ``workspace`` are optional pre-allocated buffers (for callers
    that capture the call in a HIP graph); otherwise they are allocated from
    torch's caching allocator. ``planned=True`` uses the work list that
    ``paged_attention_plan`` wrote into ``workspace`` for this step's
    context lengths instead of building it again."""
    _require_device(q, key_cache, value_cache, block_tables, context_lens)
    nb, kvh, d, bs, bstride, hstride = cache_geometry(key_cache, value_cache)
    if q.dim() != 3 or q.shape[2] != d:
        raise _err(f"q must be [B, H, {d}], got {tuple(q.shape)}")
    b, h, _ = q.shape
    if block_tables.dtype != torch.uint32 or block_tables.dim() != 2 or block_tables.shape[0] != b:
        raise _err(f"block_tables must be u32 [{b}, cols], got {block_tables.dtype} "
                   f"{tuple(block_tables.shape)}")
    if context_lens.dtype != torch.uint32 or context_lens.shape != (b,):
        raise _err(f"context_lens must be u32 [{b}], got {context_lens.dtype} "
                   f"{tuple(context_lens.shape)}")
    q = q.contiguous()
    block_tables = block_tables.contiguous()
    context_lens = context_lens.contiguous()
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise _err("out must be a contiguous tensor shaped and typed like q")
    lib = _lib.load()
    need = lib.vpa_paged_attention_workspace_size(b, h, d, int(max_context_len))
    if workspace is None and need > 0:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    if planned and workspace is None:
        raise _err("planned=True needs the workspace paged_attention_plan filled")
    fn = lib.vpa_paged_attention_planned if planned else lib.vpa_paged_attention
    check(fn(
        out.data_ptr(), q.data_ptr(), _ptr(k_scale), _ptr(v_scale), key_cache.data_ptr(),
        value_cache.data_ptr(), block_tables.data_ptr(), block_tables.shape[1],
        context_lens.data_ptr(), _ptr(alibi_slopes), int(max_context_len), float(softmax_scale),
        float(softcapping), _ptr(sinks), b, h, kvh, d, bs, nb, bstride, hstride,
        dtype_code(q.dtype), dtype_code(key_cache.dtype), _ptr(workspace), ws_bytes,
        _stream(q)))
    return out


def reshape_and_cache_paged_attention(q: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                                      k_scale: Optional[torch.Tensor],
                                      v_scale: Optional[torch.Tensor], key_cache: torch.Tensor,
                                      value_cache: torch.Tensor, block_tables: torch.Tensor,
                                      context_lens: torch.Tensor, max_context_len: int,
                                      softmax_scale: float, *, out: Optional[torch.Tensor] = None,
                                      workspace: Optional[torch.Tensor] = None,
                                      planned: bool = False) -> torch.Tensor:
    """``reshape_and_cache`` of one new K/V row per sequence ([B, KVH, D], the
    query's dtype) at position ``context_lens[s] - 1`` of its block table,
    then ``paged_attention`` over the caches, behind one call (one launch for
    small batches over 16-bit caches); returns [B, H, D]. Equal to the two
    calls with that slot mapping as long as no two sequences' last positions
    share a block."""
    _require_device(q, key, value, key_cache, value_cache, block_tables, context_lens)
    nb, kvh, d, bs, bstride, hstride = cache_geometry(key_cache, value_cache)
    if q.dim() != 3 or q.shape[2] != d:
        raise _err(f"q must be [B, H, {d}], got {tuple(q.shape)}")
    b, h, _ = q.shape
    if key.shape != (b, kvh, d) or value.shape != key.shape:
        raise _err(f"key/value must be [{b}, {kvh}, {d}], got {tuple(key.shape)} and "
                   f"{tuple(value.shape)}")
    if key.dtype != q.dtype or value.dtype != q.dtype:
        raise _err(f"key/value dtype must be the query's {q.dtype}")
    if block_tables.dtype != torch.uint32 or block_tables.dim() != 2 or block_tables.shape[0] != b:
        raise _err(f"block_tables must be u32 [{b}, cols], got {block_tables.dtype} "
                   f"{tuple(block_tables.shape)}")
    if context_lens.dtype != torch.uint32 or context_lens.shape != (b,):
        raise _err(f"context_lens must be u32 [{b}], got {context_lens.dtype} "
                   f"{tuple(context_lens.shape)}")
    if key.stride(2) != 1 or key.stride(1) != d:
        key = key.contiguous()
    if value.stride(2) != 1 or value.stride(1) != d:
        value = value.contiguous()
    q = q.contiguous()
    block_tables = block_tables.contiguous()
    context_lens = context_lens.contiguous()
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise _err("out must be a contiguous tensor shaped and typed like q")
    lib = _lib.load()
    need = lib.vpa_paged_attention_workspace_size(b, h, d, int(max_context_len))
    if workspace is None and need > 0:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    if planned and workspace is None:
        raise _err("planned=True needs the workspace paged_attention_plan filled")
    fn = (lib.vpa_reshape_and_cache_paged_attention_planned if planned
          else lib.vpa_reshape_and_cache_paged_attention)
    check(fn(
        out.data_ptr(), q.data_ptr(), key.data_ptr(), value.data_ptr(), key.stride(0),
        value.stride(0), _ptr(k_scale), _ptr(v_scale), key_cache.data_ptr(),
        value_cache.data_ptr(), block_tables.data_ptr(), block_tables.shape[1],
        context_lens.data_ptr(), int(max_context_len), float(softmax_scale), b, h, kvh, d, bs, nb,
        bstride, hstride, dtype_code(q.dtype), dtype_code(key_cache.dtype), _ptr(workspace),
        ws_bytes, _stream(q)))
    return out


def paged_attention_plan(context_lens: torch.Tensor, max_context_len: int,
                         block_table_stride: int, num_heads: int, key_cache: torch.Tensor,
                         value_cache: torch.Tensor, dtype: torch.dtype,
                         workspace: torch.Tensor) -> None:
    """Build one step's decode work list into ``workspace`` (shared by the
    ``paged_attention(..., planned=True)`` calls of all layers of the step)."""
    _require_device(context_lens, workspace)
    nb, kvh, d, bs, _, _ = cache_geometry(key_cache, value_cache)
    if context_lens.dtype != torch.uint32 or context_lens.dim() != 1:
        raise _err(f"context_lens must be u32 1-d, got {context_lens.dtype}")
    check(_lib.load().vpa_paged_attention_plan(
        context_lens.contiguous().data_ptr(), int(max_context_len), int(block_table_stride),
        context_lens.shape[0], num_heads, kvh, d, bs, dtype_code(dtype), workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), _stream(context_lens)))


def paged_cache_read(key_cache: torch.Tensor, value_cache: torch.Tensor,
                     block_tables: torch.Tensor, max_context_len: int, num_heads: int,
                     workspace: torch.Tensor, sink: torch.Tensor, magic: int = 0x9E3779B9) -> None:
    """The decode's read pattern with no compute (``vpa_paged_cache_read``):
    every K/V byte of each sequence's context, through the work list that
    ``paged_attention_plan`` left in ``workspace``. A measurement op: its rate
    is the gather bandwidth the decode can reach. ``sink`` (u32 [1]) is
    written only where a checksum equals ``magic``."""
    _require_device(key_cache, value_cache, block_tables, workspace, sink)
    nb, kvh, d, bs, bstride, hstride = cache_geometry(key_cache, value_cache)
    if block_tables.dtype != torch.uint32 or block_tables.dim() != 2:
        raise _err("block_tables must be u32 2-d")
    if sink.dtype != torch.uint32 or sink.numel() < 1:
        raise _err("sink must be a u32 tensor")
    block_tables = block_tables.contiguous()
    check(_lib.load().vpa_paged_cache_read(
        key_cache.data_ptr(), value_cache.data_ptr(), block_tables.data_ptr(),
        block_tables.shape[1], int(max_context_len), block_tables.shape[0], num_heads, kvh, d,
        bs, nb, bstride, hstride, dtype_code(key_cache.dtype), workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), int(magic) & 0xFFFFFFFF, sink.data_ptr(),
        _stream(key_cache)))


def gather_kv_cache(key_cache: torch.Tensor, value_cache: torch.Tensor,
                    k_scale: Optional[torch.Tensor], v_scale: Optional[torch.Tensor],
                    block_tables: torch.Tensor, cu_seqlens_kv: torch.Tensor,
                    out_dtype: torch.dtype, *, total_tokens: Optional[int] = None
                    ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Gather each sequence's tokens into packed K, V [sum(kv_lens), KVH, D].

    ``total_tokens`` (= cu_seqlens_kv[-1]) may be given by a caller that
    knows the lengths on the host; otherwise it is read from the device."""
    _require_device(key_cache, value_cache, block_tables, cu_seqlens_kv)
    nb, kvh, d, bs, bstride, hstride = cache_geometry(key_cache, value_cache)
    if block_tables.dtype != torch.uint32 or block_tables.dim() != 2:
        raise _err(f"block_tables must be u32 2-d, got {block_tables.dtype} "
                   f"{tuple(block_tables.shape)}")
    num_seqs = block_tables.shape[0]
    if cu_seqlens_kv.dtype != torch.uint32 or cu_seqlens_kv.shape != (num_seqs + 1,):
        raise _err(f"cu_seqlens_kv must be u32 [{num_seqs + 1}], got {cu_seqlens_kv.dtype} "
                   f"{tuple(cu_seqlens_kv.shape)}")
    if total_tokens is None:
        total_tokens = int(cu_seqlens_kv[-1].item())
    block_tables = block_tables.contiguous()
    cu_seqlens_kv = cu_seqlens_kv.contiguous()
    out_k = torch.empty((total_tokens, kvh, d), dtype=out_dtype, device=key_cache.device)
    out_v = torch.empty_like(out_k)
    check(_lib.load().vpa_gather_kv_cache(
        out_k.data_ptr(), out_v.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
        _ptr(k_scale), _ptr(v_scale), block_tables.data_ptr(), block_tables.shape[1],
        cu_seqlens_kv.data_ptr(), num_seqs, total_tokens, kvh, d, bs, nb, bstride, hstride,
        dtype_code(key_cache.dtype), dtype_code(out_dtype), _stream(key_cache)))
    return out_k, out_v


def paged_attention_varlen_prefill(q: torch.Tensor, key_cache: torch.Tensor,
                                   value_cache: torch.Tensor, block_tables: torch.Tensor,
                                   context_lens: torch.Tensor, cu_seqlens_q: torch.Tensor,
                                   k_scale: Optional[torch.Tensor], v_scale: Optional[torch.Tensor],
                                   scale: float, softcapping: float, *, causal: bool = False,
                                   max_query_len: Optional[int] = None,
                                   max_context_len: Optional[int] = None,
                                   out: Optional[torch.Tensor] = None,
                                   denom_eps: Optional[float] = None) -> torch.Tensor:
    """Varlen prefill attention of packed queries over the paged cache.

    Argument order and meaning follow the reference's Metal op
    (``vasr-paged-attn/src/metal/varlen_prefill.rs:284-295``), which is
    non-causal; ``causal=True`` gives the bottom-right causal attention that
    the CUDA build computes with gather_kv_cache + flash varlen
    (``thinker_text.rs:1344-1365``). ``q`` is [total_q, H, D] bf16/f16/f32;
    sequence s owns rows cu_seqlens_q[s]..cu_seqlens_q[s+1]-1 and the first
    context_lens[s] cached tokens (its own new tokens included). The maxima
    size the grid; a caller that knows them on the host passes them to skip
    a device read. ``denom_eps`` is added to the softmax denominator; by
    default 1e-6 without ``causal`` (the Metal kernel,
    ``prefill_paged_attn.metal:1300``) and 0 with it (flash attention).
    Returns [total_q, H, D]."""
    _require_device(q, key_cache, value_cache, block_tables, context_lens, cu_seqlens_q)
    nb, kvh, d, bs, bstride, hstride = cache_geometry(key_cache, value_cache)
    if softcapping != 1.0:
        raise VpaError(_lib.VPA_ERR_UNSUPPORTED, f"softcapping must be 1.0, got {softcapping}")
    if q.dim() != 3 or q.shape[2] != d:
        raise _err(f"q must be [total_q, H, {d}], got {tuple(q.shape)}")
    tq, h, _ = q.shape
    if block_tables.dtype != torch.uint32 or block_tables.dim() != 2:
        raise _err(f"block_tables must be u32 2-d, got {block_tables.dtype} "
                   f"{tuple(block_tables.shape)}")
    num_seqs = block_tables.shape[0]
    if cu_seqlens_q.dtype != torch.uint32 or cu_seqlens_q.shape != (num_seqs + 1,):
        raise _err(f"cu_seqlens_q must be u32 [{num_seqs + 1}], got {cu_seqlens_q.dtype} "
                   f"{tuple(cu_seqlens_q.shape)}")
    if context_lens.dtype != torch.uint32 or context_lens.shape != (num_seqs,):
        raise _err(f"context_lens must be u32 [{num_seqs}], got {context_lens.dtype} "
                   f"{tuple(context_lens.shape)}")
    if max_query_len is None:
        max_query_len = int((cu_seqlens_q[1:].long() - cu_seqlens_q[:-1].long()).max().item()) \
            if num_seqs else 0
    if max_context_len is None:
        max_context_len = int(context_lens.long().max().item()) if num_seqs else 0
    q = q.contiguous()
    block_tables = block_tables.contiguous()
    context_lens = context_lens.contiguous()
    cu_seqlens_q = cu_seqlens_q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    elif out.shape != q.shape or out.dtype != q.dtype or not out.is_contiguous():
        raise _err("out must be a contiguous tensor shaped and typed like q")
    check(_lib.load().vpa_chunked_prefill_paged_attention(
        out.data_ptr(), q.data_ptr(), _ptr(k_scale), _ptr(v_scale), key_cache.data_ptr(),
        value_cache.data_ptr(), block_tables.data_ptr(), block_tables.shape[1],
        cu_seqlens_q.data_ptr(), context_lens.data_ptr(), num_seqs, int(max_query_len),
        int(max_context_len), tq, float(scale),
        float((0.0 if causal else 1e-6) if denom_eps is None else denom_eps), int(bool(causal)),
        h, kvh, d, bs, nb, bstride,
        hstride, dtype_code(q.dtype), dtype_code(key_cache.dtype), _stream(q)))
    return out


# ---- next-token selection and EOS state on the device -------------------------

def argmax_token_ids_from_logits(logits: torch.Tensor, *,
                                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Next-token ids [B] (u32, on the device) of logits [B, V]: the first
    maximum of each row, NaN handled as candle's argmax (generation.rs:443-460),
    without the reference's host read-back."""
    _require_device(logits)
    if logits.dim() == 1:
        logits = logits[None, :]
    if logits.dim() != 2:
        raise _err(f"logits must be [B, V], got {tuple(logits.shape)}")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    b, v = logits.shape
    if out is None:
        out = torch.empty(b, dtype=torch.uint32, device=logits.device)
    elif out.dtype != torch.uint32 or out.shape != (b,) or not out.is_contiguous():
        raise _err(f"out must be a contiguous u32 [{b}] tensor")
    check(_lib.load().vpa_argmax_rows(logits.data_ptr(), logits.stride(0), v, b,
                                      dtype_code(logits.dtype), out.data_ptr(),
                                      _stream(logits)))
    return out


class DecodeTokenState:
    """Device-resident next-token state of a batch decode loop.

    Mirrors the fields of PagedBatchState that the step-start bookkeeping
    touches (paged_batch_engine.rs:28-42): ``next_ids`` (pending ids),
    ``finished`` (u8), ``generated`` [B, capacity] with ``gen_len``, plus the
    ``input_ids`` buffer a captured decode graph reads and the 4-byte
    ``active_count``."""

    def __init__(self, batch: int, capacity: int, eos_token_ids, device):
        eos = list(eos_token_ids)
        if not eos:
            raise _err("eos_token_ids is empty")
        self.batch, self.capacity = batch, capacity
        self.eos_fill_id = int(eos[0])
        self.eos_ids = torch.tensor(eos, dtype=torch.uint32, device=device)
        self.next_ids = torch.zeros(batch, dtype=torch.uint32, device=device)
        self.finished = torch.zeros(batch, dtype=torch.uint8, device=device)
        self.generated = torch.zeros((batch, max(capacity, 1)), dtype=torch.uint32, device=device)
        self.gen_len = torch.zeros(batch, dtype=torch.uint32, device=device)
        self.input_ids = torch.zeros(batch, dtype=torch.uint32, device=device)
        self.active_count = torch.zeros(1, dtype=torch.uint32, device=device)

    def select(self, logits: torch.Tensor) -> None:
        """next_ids <- argmax of the step's logits rows (all rows of the batch)."""
        argmax_token_ids_from_logits(logits, out=self.next_ids)

    def consume(self, prev_slot_mapping: Optional[torch.Tensor] = None) -> None:
        """Step start (paged_batch_engine.rs:640-667): pending EOS ids finish
        their rows, other pending ids are appended and become input_ids;
        finished rows feed the EOS fill id. With the previous step's
        ``prev_slot_mapping`` (i64 [batch]), a row that did not run in that
        step (negative slot) feeds its input id again and appends nothing."""
        if prev_slot_mapping is not None and (prev_slot_mapping.dtype != torch.int64 or
                                              prev_slot_mapping.shape != (self.batch,)):
            raise _err(f"prev_slot_mapping must be i64 [{self.batch}]")
        check(_lib.load().vpa_decode_consume_tokens(
            self.next_ids.data_ptr(), self.finished.data_ptr(), _ptr(prev_slot_mapping),
            self.generated.data_ptr(),
            self.gen_len.data_ptr(), self.capacity, self.eos_ids.data_ptr(),
            self.eos_ids.numel(), self.eos_fill_id, self.input_ids.data_ptr(),
            self.active_count.data_ptr(), self.batch, _stream(self.next_ids)))


class DeviceBlockAllocator:
    """Device-resident KV block allocation and decode-step metadata for a
    fixed batch of rows (``vpa_allocate_rows`` / ``vpa_decode_step_metadata`` /
    ``vpa_release_blocks``): the PagedBlockManager of
    paged_cache_runtime.rs:217-380 (FIFO free list of ids 1..num_blocks-1)
    and decode_metadata_for_batch_step of paged_kv_cache.rs:924-1059, with
    every buffer on the device so a captured decode graph can run them."""

    def __init__(self, num_blocks: int, block_size: int, batch: int, cols: int, device):
        import numpy as np

        if num_blocks < 2 or block_size <= 0 or batch < 0 or cols <= 0:
            raise _err("bad allocator sizes")
        self.block_size, self.batch, self.cols = block_size, batch, cols
        self.ring_capacity = num_blocks
        ring = np.zeros(num_blocks, dtype=np.uint32)
        ring[:num_blocks - 1] = np.arange(1, num_blocks, dtype=np.uint32)
        self.free_ring = torch.from_numpy(ring).to(device)
        self.free_ring_state = torch.tensor([0, num_blocks - 1], dtype=torch.uint32, device=device)
        self.block_tables = torch.zeros((batch, cols), dtype=torch.uint32, device=device)
        self.row_blocks = torch.zeros(batch, dtype=torch.uint32, device=device)
        self.positions = torch.zeros(batch, dtype=torch.uint32, device=device)
        self.slot_mapping = torch.full((batch,), -1, dtype=torch.int64, device=device)
        self.context_lens = torch.ones(batch, dtype=torch.uint32, device=device)
        self.status = torch.zeros(3, dtype=torch.uint32, device=device)
        self.ok = torch.zeros(batch, dtype=torch.uint8, device=device)

    def _common(self):
        return (self.free_ring.data_ptr(), self.free_ring_state.data_ptr(), self.ring_capacity)

    def allocate(self, target_tokens: torch.Tensor) -> torch.Tensor:
        """Grow rows to hold target_tokens[r] tokens (u32 [batch]); returns ``ok``."""
        ring, state, cap = self._common()
        check(_lib.load().vpa_allocate_rows(
            self.block_tables.data_ptr(), self.cols, self.row_blocks.data_ptr(),
            target_tokens.contiguous().data_ptr(), self.ok.data_ptr(), ring, state, cap,
            self.block_size, self.batch, _stream(self.block_tables)))
        return self.ok

    def step(self, finished: Optional[torch.Tensor] = None):
        """One decode step: returns (slot_mapping, context_lens) device tensors."""
        ring, state, cap = self._common()
        check(_lib.load().vpa_decode_step_metadata(
            self.block_tables.data_ptr(), self.cols, self.row_blocks.data_ptr(),
            self.positions.data_ptr(), _ptr(finished), ring, state, cap, self.block_size,
            self.slot_mapping.data_ptr(), self.context_lens.data_ptr(), self.status.data_ptr(),
            self.batch, _stream(self.block_tables)))
        return self.slot_mapping, self.context_lens

    def release(self, keep_blocks: torch.Tensor) -> None:
        """Rows keep their first keep_blocks[r] blocks (u32 [batch]), the rest go back."""
        ring, state, cap = self._common()
        check(_lib.load().vpa_release_blocks(
            self.block_tables.data_ptr(), self.cols, self.row_blocks.data_ptr(),
            keep_blocks.contiguous().data_ptr(), ring, state, cap, self.batch,
            _stream(self.block_tables)))

