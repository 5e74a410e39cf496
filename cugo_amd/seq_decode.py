"""Incremental decoding of the event-sequence policy over a per-row KV cache.

`cached_step(model, cache, x, slots=None, rows=None)` computes what the reference's
`SeqNet.cached_step` computes (python/cugo_seq50.py:291-322) for any module laid out
like it: `model.encoder.layers` of pre-norm `nn.TransformerEncoderLayer`s
(norm1 -> packed in-projection -> attention -> out_proj; norm2 -> linear1 -> activation
-> linear2) and a cache with `k`, `v` ([layers, rows, heads, slots, dh]), `length`,
`heads`, `slots`, `row_ids`.  The per-layer `index_put_` of the new key/value and the
decode attention run as one HIP launch (`decode_attention_append`, reading q, k and v in
place from the packed in-projection), and each residual add with the pre-norm that
follows it as another (`add_layernorm`).

`KVCache` mirrors the reference cache (python/cugo_seq50.py:325-339) with the slot count
as a parameter (the reference fixes it at MAX_EVENTS + 2 = 50).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .cugo_seq_attention50 import decode_attention_append
from .cugo_torch50_ext import load_extension


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


_FUSED_WIDTHS = (64, 128, 256, 512, 1024)
_EXT = None


def _ext():
    global _EXT
    if _EXT is None:
        _EXT = load_extension()
    return _EXT


def _add_norm(x: torch.Tensor, y: torch.Tensor | None, norm: nn.Module):
    """(x + y, norm(x + y)), or (x, norm(x)) for y None: one HIP launch
    (`add_layernorm`) for an affine LayerNorm over the last dim of a bf16/fp32 row of a
    supported width, torch's two ops otherwise."""
    if (isinstance(norm, nn.LayerNorm) and norm.weight is not None and norm.bias is not None
            and x.dim() == 2 and x.dtype in (torch.bfloat16, torch.float32)
            and norm.weight.dtype == x.dtype and tuple(norm.normalized_shape) == (x.shape[1],)
            and x.shape[1] in _FUSED_WIDTHS and (y is None or y.dtype == x.dtype)):
        out = _ext().add_layernorm(x.contiguous(), y, norm.weight.detach(), norm.bias.detach(),
                                   norm.eps)
        return out[0], out[1]
    x = x if y is None else x + y
    return x, norm(x)


def cached_step(model: nn.Module, cache, x: torch.Tensor, slots: int | None = None,
                rows: torch.Tensor | None = None) -> torch.Tensor:
    """One token per cache row (x [n, d]); its key/value go to slot cache.length[row].

    Each token attends every cached slot plus itself; `slots` bounds the slot index;
    `rows` names each token's cache row (default: every row in order).  Returns the
    final hidden state [n, d].  Same steps as python/cugo_seq50.py:291-322; each residual
    add and the pre-norm after it run as one launch, and q, k and v are read in place from
    the packed in-projection."""
    n, d = x.shape
    heads = cache.heads
    dh = d // heads
    t = cache.slots if slots is None else min(slots, cache.slots)
    row_ids = cache.row_ids if rows is None else rows
    length = cache.length if rows is None else cache.length.index_select(0, row_ids)
    pos = length.clamp_max(t - 1)
    layers = model.encoder.layers
    x, h = _add_norm(x, None, layers[0].norm1)
    for i, layer in enumerate(layers):
        attn = layer.self_attn
        q, k, v = F.linear(h, attn.in_proj_weight, attn.in_proj_bias).chunk(3, -1)
        a = decode_attention_append(q.reshape(n, heads, dh), k.reshape(n, heads, dh),
                                    v.reshape(n, heads, dh), cache.k[i], cache.v[i], pos,
                                    row_ids)
        x, h = _add_norm(x, attn.out_proj(a.reshape(n, d)), layer.norm2)
        m = layer.linear2(layer.activation(layer.linear1(h)))
        if i + 1 < len(layers):
            x, h = _add_norm(x, m, layers[i + 1].norm1)
        else:
            x = x + m
    return x
