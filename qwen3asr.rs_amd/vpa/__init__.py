"""vpa — MI355X-native paged-KV hot path of the Qwen3-ASR decoder.

Hand-written HIP kernels for gfx950 behind the C ABI of ``include/vpa.h``
(``libvpa.so``), with the Candle-op-shaped tensor API of
``mistralrs_paged_attn`` (as re-exported by ``vasr-paged-attn``) on top.
"""

from ._lib import VpaError  # noqa: F401
from .ops import (  # noqa: F401
    DecodeTokenState,
    DeviceBlockAllocator,
    argmax_token_ids_from_logits,
    cache_geometry,
    gather_kv_cache,
    paged_attention,
    paged_attention_plan,
    paged_cache_read,
    paged_attention_varlen_prefill,
    paged_attention_workspace,
    reshape_and_cache,
    reshape_and_cache_paged_attention,
)
from .graph import DecodeGraphCache  # noqa: F401
from .step import DeviceDecodeStep  # noqa: F401

__all__ = [
    "DecodeGraphCache",
    "DecodeTokenState",
    "DeviceBlockAllocator",
    "DeviceDecodeStep",
    "VpaError",
    "argmax_token_ids_from_logits",
    "cache_geometry",
    "gather_kv_cache",
    "paged_attention",
    "paged_attention_plan",
    "paged_cache_read",
    "paged_attention_varlen_prefill",
    "paged_attention_workspace",
    "reshape_and_cache",
    "reshape_and_cache_paged_attention",
]
