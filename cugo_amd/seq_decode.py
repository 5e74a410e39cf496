"""Incremental decoding of the event-sequence policy over a per-row KV cache.

`cached_step(model, cache, x, slots=None, rows=None)` computes what the reference's
`SeqNet.cached_step` computes (python/cugo_seq50.py:291-322) for any module laid out
like it: `model.encoder.layers` of pre-norm `nn.TransformerEncoderLayer`s
(norm1 -> packed in-projection -> attention -> out_proj; norm2 -> linear1 -> activation
-> linear2) and a cache with `k`, `v` ([layers, rows, heads, slots, dh]), `length`,
`heads`, `slots`, `row_ids`.  The per-layer `index_put_` of the new key/value and the
decode attention run as one HIP launch (`decode_attention_append`).

`KVCache` mirrors the reference cache (python/cugo_seq50.py:325-339) with the slot count
as a parameter (the reference fixes it at MAX_EVENTS + 2 = 50).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .cugo_seq_attention50 import decode_attention_append


class KVCache:
    """Per-row keys/values of every layer (bf16, head-major) plus per-row lengths."""

    def __init__(self, layers: int, rows: int, heads: int, d_model: int, slots: int,
                 device: torch.device, dtype: torch.dtype = torch.bfloat16) -> None:
        self.heads = heads
        self.slots = slots
        self.k = torch.zeros((layers, rows, heads, slots, d_model // heads), dtype=dtype,
                             device=device)
        self.v = torch.zeros_like(self.k)
        self.length = torch.zeros(rows, dtype=torch.int64, device=device)
        self.row_ids = torch.arange(rows, device=device)


def cached_step(model: nn.Module, cache, x: torch.Tensor, slots: int | None = None,
                rows: torch.Tensor | None = None) -> torch.Tensor:
    """One token per cache row (x [n, d]); its key/value go to slot cache.length[row].

    Each token attends every cached slot plus itself; `slots` bounds the slot index;
    `rows` names each token's cache row (default: every row in order).  Returns the
    final hidden state [n, d].  Same steps as python/cugo_seq50.py:291-322."""
    n, d = x.shape
    heads = cache.heads
    dh = d // heads
    t = cache.slots if slots is None else min(slots, cache.slots)
    row_ids = cache.row_ids if rows is None else rows
    length = cache.length if rows is None else cache.length.index_select(0, row_ids)
    pos = length.clamp_max(t - 1)
    for i, layer in enumerate(model.encoder.layers):
        attn = layer.self_attn
        q, k, v = F.linear(layer.norm1(x), attn.in_proj_weight, attn.in_proj_bias).chunk(3, -1)
        a = decode_attention_append(q.reshape(n, heads, dh), k.reshape(n, heads, dh),
                                    v.reshape(n, heads, dh), cache.k[i], cache.v[i], pos,
                                    row_ids)
        x = x + attn.out_proj(a.reshape(n, d))
        x = x + layer.linear2(layer.activation(layer.linear1(layer.norm2(x))))
    return x
