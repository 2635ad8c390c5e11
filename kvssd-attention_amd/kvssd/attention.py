"""Attention orchestration over packed blocks (reference: src/kvssd/attention.py:13-134)."""

from __future__ import annotations

import math
from collections.abc import Sequence

import torch

from .backends import AttentionBackend, PackedBatch, resolve_attention_backend
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
    """Decode attention with query [QH,D] and K/V [T,KVH,D], including GQA."""
    if query.ndim != 2 or keys.ndim != 3 or keys.shape != values.shape:
        raise ValueError("expected query [QH,D] and matching keys/values [T,KVH,D]")
    q_heads, dim = query.shape
    if keys.shape[2] != dim or q_heads % keys.shape[1]:
        raise ValueError("head_dim mismatch or query heads not divisible by KV heads")
    head_map = torch.arange(q_heads, device=query.device) // (q_heads // keys.shape[1])
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(dim)
    scores = torch.einsum("hd,thd->ht", query.float(), keys[:, head_map].float()) * scale
    weights = torch.softmax(scores, dim=-1)
    return torch.einsum("ht,thd->hd", weights, values[:, head_map].float()).to(query.dtype)


def packed_attention_reference(
    query: torch.Tensor,
    blocks: Sequence[PackedKVBlock],
    sm_scale: float | None = None,
) -> torch.Tensor:
    if not blocks:
        raise ValueError("at least one block is required")
    keys = torch.cat([dequantize_tensor(b.key)[: b.valid_tokens] for b in blocks]).to(query.device)
    values = torch.cat([dequantize_tensor(b.value)[: b.valid_tokens] for b in blocks]).to(query.device)
    return reference_attention(query, keys, values, sm_scale)


def stack_blocks(blocks: Sequence[PackedKVBlock], device: torch.device) -> tuple[torch.Tensor, ...]:
    """Coalesce blocks into PackedBatch tensors (kp, vp, ks, vs, valid) on ``device``."""
    if not blocks:
        raise ValueError("at least one block is required")
    device = torch.device(device)
    kwargs = {"device": device, "non_blocking": device.type == "cuda"}
    return (
        torch.stack([b.key.packed for b in blocks]).to(**kwargs),
        torch.stack([b.value.packed for b in blocks]).to(**kwargs),
        torch.stack([b.key.scales for b in blocks]).to(**kwargs),
        torch.stack([b.value.scales for b in blocks]).to(**kwargs),
        torch.tensor([b.valid_tokens for b in blocks], dtype=torch.int32, device=device),
    )


def native_backend_available() -> bool:
    """True when the fused HIP kernels can run on the current GPU."""
    try:
        resolve_attention_backend(NATIVE_BACKEND, torch.device("cuda"))
        return True
    except RuntimeError:
        return False


# Name kept for API compatibility with the reference (src/kvssd/attention.py:63-68).
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
    """Low-level fused entry point returning normalized output and log-sum-exp statistics."""
    backend = resolve_attention_backend(NATIVE_BACKEND, query.device)
    return backend.run(
        query,
        PackedBatch(packed_k, packed_v, scales_k, scales_v, valid_tokens, bits, group_size),
        sm_scale,
    )


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
