"""Portable PyTorch dequantize-then-attend backend.

Same contract and arithmetic as the reference's ReferenceAttentionBackend
(src/kvssd/backends/reference.py:9-50): fp32 dequantisation, concatenation of
each block's first ``valid`` rows, GQA map ``qh // (QH/KVH)``, fp32 scores,
log-sum-exp and softmax.  It is the reference API's portable backend (the only
one on CPU) and never reports itself as accelerated, so the pipeline does not
route its streamed GPU path through it.
"""

from __future__ import annotations

import torch

from ..quant import unpack_codes
from .base import BackendAvailability, PackedBatch


class ReferenceAttentionBackend:
    name = "reference"

    def probe(self, device: torch.device) -> BackendAvailability:
        return BackendAvailability(
            self.name, True, False, False, "portable PyTorch dequantize-then-attend reference", device.type
        )

    def run(self, query: torch.Tensor, batch: PackedBatch, sm_scale: float) -> tuple[torch.Tensor, torch.Tensor]:
        batch.validate(query)
        head_dim = query.shape[-1]
        mid = 1 << (batch.bits - 1)

        def dequant(packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
            codes = unpack_codes(packed, batch.bits, head_dim).float() - mid
            return codes * scales.float().repeat_interleave(batch.group_size, dim=-1)

        keys = dequant(batch.packed_k, batch.scales_k)
        values = dequant(batch.packed_v, batch.scales_v)
        # block i contributes the rows [i, :valid[i]] (Python slice rules: a
        # negative count drops that many rows from the end of the block)
        counts = [int(v) for v in batch.valid_tokens.tolist()]
        keys = torch.cat([keys[i, :n] for i, n in enumerate(counts)], dim=0)
        values = torch.cat([values[i, :n] for i, n in enumerate(counts)], dim=0)
        q_heads, kv_heads = query.shape[0], keys.shape[1]
        head_map = torch.arange(q_heads, device=query.device) // (q_heads // kv_heads)
        scores = torch.einsum("hd,thd->ht", query.float(), keys[:, head_map]) * sm_scale
        lse = torch.logsumexp(scores, dim=-1)
        out = torch.einsum("ht,thd->hd", torch.softmax(scores, dim=-1), values[:, head_map])
        return out, lse
