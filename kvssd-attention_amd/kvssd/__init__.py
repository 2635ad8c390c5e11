"""KVSSD: packed, tiered KV-cache primitives with fused MI355X (gfx950) decode attention.

Public names match the reference package (src/kvssd/__init__.py:3-26).
"""

from .attention import packed_attention, reference_attention
from .backends import available_attention_backends, resolve_attention_backend
from .format import CacheSpec
from .pipeline import KVSSDPipeline
from .quant import dequantize_tensor, quantize_tensor
from .selectors import AllBlocks, RecentSinkBlocks
from .store import KVCacheStore
from .storage import available_storage_backends, resolve_storage_backend

__all__ = [
    "AllBlocks",
    "CacheSpec",
    "KVCacheStore",
    "KVSSDPipeline",
    "RecentSinkBlocks",
    "dequantize_tensor",
    "available_attention_backends",
    "available_storage_backends",
    "packed_attention",
    "quantize_tensor",
    "reference_attention",
    "resolve_attention_backend",
    "resolve_storage_backend",
]
