"""Attention orchestration over packed blocks (reference: src/kvssd/attention.py:13-134)."""

from __future__ import annotations

import math
from collections.abc import Sequence

import torch

from .backends import AttentionBackend, PackedBatch, resolve_attention_backend
from .backends.reference import ReferenceAttentionBackend
from .format import PackedKVBlock
from .quant import dequantize_tensor

# The fused native kernel here is the HIP one.  ``require_cuda_kernel=True`` in the
# reference means "the fused native kernel must run"; on ROCm that kernel is
# the ``hip`` backend, so the flag resolves to it.
NATIVE_BACKEND = "hip"
_NATIVE_ALIASES = (None, "auto", "cuda", "hip")


def reference_attention(
    query: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    sm_scale: float | None = None,
) -> torch.Tensor:
    """Decode attention with query [QH,D] and K/V [T,KVH,D], including GQA.

    The reference's dense path (src/kvssd/attention.py:13-31): fp32 scores
    scaled by ``sm_scale`` (default 1/sqrt(D)), softmax over the tokens, the
    result cast to the query's dtype.  The query heads are grouped by the kv
    head they read ([KVH, QH/KVH, D]), so each kv head's keys and values take
    part in one batched product instead of being gathered per query head."""
    if query.ndim != 2 or keys.ndim != 3 or keys.shape != values.shape:
        raise ValueError("expected query [QH,D] and matching keys/values [T,KVH,D]")
    q_heads, dim = query.shape
    _, kv_heads, key_dim = keys.shape
    if key_dim != dim or q_heads % kv_heads:
        raise ValueError("head_dim mismatch or query heads not divisible by KV heads")
    scale = 1.0 / math.sqrt(dim) if sm_scale is None else sm_scale
    grouped = query.float().reshape(kv_heads, q_heads // kv_heads, dim)
    k_t = keys.float().permute(1, 2, 0).contiguous()  # [KVH, D, T]
    v = values.float().permute(1, 0, 2).contiguous()  # [KVH, T, D]
    weights = torch.softmax(torch.matmul(grouped, k_t) * scale, dim=-1)
    return torch.matmul(weights, v).reshape(q_heads, dim).to(query.dtype)


def packed_attention_reference(
    query: torch.Tensor,
    blocks: Sequence[PackedKVBlock],
    sm_scale: float | None = None,
) -> torch.Tensor:
    """Packed blocks through the portable dequantize-then-attend backend
    (src/kvssd/attention.py:34-47): each block contributes its first
    ``valid_tokens`` rows, the result is cast to the query's dtype."""
    if not blocks:
        raise ValueError("at least one block is required")
    if not _uniform(blocks):
        # blocks of different shapes or codecs: each dequantised on its own,
        # their valid rows concatenated, as the reference does
        keys = torch.cat([dequantize_tensor(b.key, torch.float32)[: b.valid_tokens] for b in blocks], dim=0)
        values = torch.cat([dequantize_tensor(b.value, torch.float32)[: b.valid_tokens] for b in blocks], dim=0)
        return reference_attention(query, keys.to(query.device), values.to(query.device), sm_scale)
    scale = 1.0 / math.sqrt(query.shape[-1]) if sm_scale is None else sm_scale
    batch = PackedBatch(*stack_blocks(blocks, query.device), blocks[0].key.bits, blocks[0].key.group_size)
    out, _ = ReferenceAttentionBackend().run(query, batch, scale)
    return out.to(query.dtype)


def _fields(block: PackedKVBlock) -> tuple[torch.Tensor, ...]:
    return (block.key.packed, block.value.packed, block.key.scales, block.value.scales)


def _uniform(blocks: Sequence[PackedKVBlock]) -> bool:
    """Whether every block has the first one's array shapes and dtypes and its codec."""
    first = blocks[0]
    sig = [(t.shape, t.dtype) for t in _fields(first)]
    codec = (first.key.bits, first.key.group_size, first.value.bits, first.value.group_size)
    return all(
        [(t.shape, t.dtype) for t in _fields(b)] == sig
        and (b.key.bits, b.key.group_size, b.value.bits, b.value.group_size) == codec
        for b in blocks
    )


def stack_blocks(blocks: Sequence[PackedKVBlock], device: torch.device) -> tuple[torch.Tensor, ...]:
    """PackedBatch tensors (packed K, packed V, scales K, scales V, valid) of
    ``blocks`` on ``device`` (src/kvssd/attention.py:50-60).

    Each array is assembled once in host memory, block by block, and crosses
    to the device in one copy; the valid counts follow as one int32 tensor.
    Blocks whose arrays differ in shape or dtype from the first block's raise
    RuntimeError, as the reference's ``torch.stack`` does (nothing is
    broadcast)."""
    if not blocks:
        raise ValueError("at least one block is required")
    sig = [(t.shape, t.dtype) for t in _fields(blocks[0])]
    for i, block in enumerate(blocks):
        got = [(t.shape, t.dtype) for t in _fields(block)]
        if got != sig:
            raise RuntimeError(
                f"stack expects each tensor to be equal size and dtype, but got {got} at entry {i} "
                f"and {sig} at entry 0"
            )
    device = torch.device(device)
    fields = (
        lambda b: b.key.packed,
        lambda b: b.value.packed,
        lambda b: b.key.scales,
        lambda b: b.value.scales,
    )
    arrays = []
    for field in fields:
        first = field(blocks[0])
        host = torch.empty((len(blocks), *first.shape), dtype=first.dtype)
        for row, block in enumerate(blocks):
            host[row].copy_(field(block))
        arrays.append(host.to(device))
    counts = torch.tensor([int(b.valid_tokens) for b in blocks], dtype=torch.int32)
    return (*arrays, counts.to(device))


def native_backend_available() -> bool:
    """True when the fused HIP kernels can run on the current GPU."""
    try:
        resolve_attention_backend(NATIVE_BACKEND, torch.device("cuda"))
    except RuntimeError:
        return False
    return True


# The reference's name for the same question (src/kvssd/attention.py:63-68).
cuda_extension_available = native_backend_available


def fused_attention_tensors(
    query: torch.Tensor,
    packed_k: torch.Tensor,
    packed_v: torch.Tensor,
    scales_k: torch.Tensor,
    scales_v: torch.Tensor,
    valid_tokens: torch.Tensor,
    bits: int,
    group_size: int,
    sm_scale: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(out fp32 [QH, D], lse fp32 [QH]) of the fused HIP kernels over one
    PackedBatch: the low-level entry point of src/kvssd/attention.py:71-88,
    which fails closed when the native backend is unavailable."""
    native = resolve_attention_backend(NATIVE_BACKEND, query.device)
    batch = PackedBatch(packed_k, packed_v, scales_k, scales_v, valid_tokens, bits, group_size)
    return native.run(query, batch, sm_scale)


def merge_attention_chunks(
    left_output: torch.Tensor,
    left_lse: torch.Tensor,
    right_output: torch.Tensor,
    right_lse: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Exactly merge independently normalized attention chunks using log normalizers.

    L = logaddexp(La, Lb), O = Oa e^(La - L) + Ob e^(Lb - L).  A chunk with
    L = -inf (no tokens) contributes nothing; two empty chunks give O = 0,
    L = -inf, the attention result over their (empty) union.
    """
    merged = torch.logaddexp(left_lse, right_lse)
    finite = torch.isfinite(merged)
    safe = torch.where(finite, merged, torch.zeros_like(merged))
    w_left = torch.where(finite, torch.exp(left_lse - safe), torch.zeros_like(merged)).unsqueeze(-1)
    w_right = torch.where(finite, torch.exp(right_lse - safe), torch.zeros_like(merged)).unsqueeze(-1)
    left = torch.where(w_left != 0, left_output * w_left, torch.zeros_like(left_output))
    right = torch.where(w_right != 0, right_output * w_right, torch.zeros_like(right_output))
    return left + right, merged


def resolve_required(
    require_cuda_kernel: bool, attention_backend: str | AttentionBackend | None, device: torch.device
) -> AttentionBackend:
    """Backend resolution shared by packed_attention and the pipeline
    (src/kvssd/attention.py:116-119, src/kvssd/pipeline.py:44-48)."""
    if require_cuda_kernel and not (
        attention_backend in _NATIVE_ALIASES
        or getattr(attention_backend, "name", None) == NATIVE_BACKEND
    ):
        raise ValueError("require_cuda_kernel conflicts with a non-CUDA attention backend")
    if require_cuda_kernel and (attention_backend is None or isinstance(attention_backend, str)):
        attention_backend = NATIVE_BACKEND
    return resolve_attention_backend(attention_backend, device)


def packed_attention(
    query: torch.Tensor,
    blocks: Sequence[PackedKVBlock],
    sm_scale: float | None = None,
    require_cuda_kernel: bool = False,
    attention_backend: str | AttentionBackend | None = None,
) -> torch.Tensor:
    """Run packed attention through an explicit or automatically selected backend."""
    if not blocks:
        raise ValueError("at least one block is required")
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(query.shape[-1])
    backend = resolve_required(require_cuda_kernel, attention_backend, query.device)
    kp, vp, ks, vs, valid = stack_blocks(blocks, query.device)
    batch = PackedBatch(kp, vp, ks, vs, valid, blocks[0].key.bits, blocks[0].key.group_size)
    output, _lse = backend.run(query, batch, scale)
    return output.to(query.dtype)
