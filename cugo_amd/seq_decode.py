"""Incremental decoding of the event-sequence policy over a per-row KV cache.

`cached_step(model, cache, x, slots=None, rows=None)` computes what the reference's
`SeqNet.cached_step` computes (python/cugo_seq50.py:291-322) for any module laid out
like it: `model.encoder.layers` of pre-norm `nn.TransformerEncoderLayer`s
(norm1 -> packed in-projection -> attention -> out_proj; norm2 -> linear1 -> activation
-> linear2) and a cache with `k`, `v` ([layers, rows, heads, slots, dh]), `length`,
`heads`, `slots`, `row_ids`.  The per-layer `index_put_` of the new key/value and the
decode attention run as one HIP launch (`decode_attention_append`, reading q, k and v in
place from the packed in-projection), each bf16 linear layer as one (`linear`), out_proj
with the residual add and the pre-norm that follows it as one (`linear_add_layernorm`), and
the feed-forward half (linear1, GELU, linear2, the residual add and the next norm) as one
(`ffn`, the hidden layer kept on chip).

`KVCache` mirrors the reference cache (python/cugo_seq50.py:325-339) with the slot count
as a parameter (the reference fixes it at MAX_EVENTS + 2 = 50).
"""

from __future__ import annotations

import weakref

import torch
import torch.nn.functional as F
from torch import nn

from .cugo_seq_attention50 import decode_attention_append, decode_order
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


def add_norm(x: torch.Tensor, y: torch.Tensor | None, norm: nn.Module):
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


def is_exact_gelu(act) -> bool:
    """The exact (erf) GELU, as a function or a module."""
    return act is F.gelu or (isinstance(act, nn.GELU) and act.approximate == "none")


def _fits_linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> bool:
    """The shapes and alignments `linear` takes (include/cugo_hip.h, cugo_linear)."""
    return (x.dim() == 2 and x.is_cuda and x.dtype == torch.bfloat16 and x.stride(1) == 1
            and weight.dtype == torch.bfloat16 and weight.dim() == 2
            and weight.shape[1] <= x.shape[1] and x.shape[1] in (64, 128, 256, 512, 1024)
            and (x.shape[0] <= 1 or x.stride(0) % 8 == 0)
            and x.data_ptr() % 16 == 0
            and (bias is None or (bias.dtype == torch.bfloat16 and bias.is_contiguous()
                                  and bias.data_ptr() % 8 == 0)))


_PACKED: dict[int, tuple] = {}


def packed_weight(weight: torch.Tensor, k_pad: int | None = None) -> torch.Tensor:
    """`weight` [n, k] in the fragment order `linear` reads (mlp_pack_weight with n padded
    to 16 and k to k_pad, zeros past k), built on first use and rebuilt into the same
    buffer when the weight changes in place (its version), so a captured HIP graph reads
    the new values."""
    n, k = weight.shape
    kp = k if k_pad is None else k_pad
    key = (weight.data_ptr(), weight._version)
    slot = (id(weight), kp)
    hit = _PACKED.get(slot)
    rows = (n + 15) // 16 * 16
    if (hit is None or hit[0]() is not weight or hit[2].device != weight.device
            or hit[2].numel() != rows * kp):
        hit = (weakref.ref(weight), key,
               _ext().mlp_pack_weight(weight.detach().contiguous(), rows, kp))
    elif hit[1] != key:
        hit[2].copy_(_ext().mlp_pack_weight(weight.detach().contiguous(), rows, kp))
        hit = (hit[0], key, hit[2])
    _PACKED[slot] = hit
    return hit[2]


def prepare_linears(model: nn.Module) -> None:
    """Packs every encoder layer's linear weights now (before a HIP-graph capture)."""
    for layer in model.encoder.layers:
        for w in (layer.self_attn.in_proj_weight, layer.self_attn.out_proj.weight,
                  layer.linear1.weight, layer.linear2.weight):
            if w.dtype == torch.bfloat16 and w.is_cuda:
                packed_weight(w)


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
           gelu: bool = False, residual: torch.Tensor | None = None,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """F.linear(x, weight, bias), then F.gelu when `gelu`, then residual + that when a
    residual is given ([rows, N], or an [N] row for every row): one HIP launch (`linear`)
    for bf16 rows with K in {64, ..., 1,024} (with a residual, N a multiple of 4), torch's
    ops otherwise; into `out` when given.  x may be wider than the weight's K when its
    extra columns are zeros (a padded input: the packed weight is zero there too)."""
    if x.shape[-1] != weight.shape[1] and not _fits_linear(x, weight, bias):
        x = x[..., :weight.shape[1]]
    n = weight.shape[0]
    if _fits_linear(x, weight, bias) and (
            residual is None or (residual.dtype == torch.bfloat16 and residual.is_contiguous()
                                 and residual.shape in ((x.shape[0], n), (n,))
                                 and n % 4 == 0)):
        return _ext().linear(x, packed_weight(weight, x.shape[1]), n,
                             None if bias is None else bias.detach(), gelu,
                             residual=None if residual is None else residual.detach(), out=out)
    y = F.linear(x, weight, bias)
    y = F.gelu(y) if gelu else y
    y = y if residual is None else residual + y
    return y if out is None else out.copy_(y)


def linear_add_norm(u: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                    x: torch.Tensor, norm: nn.Module):
    """add_norm(x, F.linear(u, weight, bias), norm): one HIP launch
    (`linear_add_layernorm`) for bf16 rows 256 wide, `linear` and `add_norm` otherwise."""
    if (_fits_linear(u, weight, bias) and weight.shape[0] == 256 and x.dim() == 2
            and x.dtype == torch.bfloat16 and x.shape == (u.shape[0], 256)
            and isinstance(norm, nn.LayerNorm) and norm.weight is not None
            and norm.bias is not None and norm.weight.dtype == torch.bfloat16
            and tuple(norm.normalized_shape) == (256,)):
        out = _ext().linear_add_layernorm(u, packed_weight(weight),
                                          None if bias is None else bias.detach(),
                                          x.contiguous(), norm.weight.detach(),
                                          norm.bias.detach(), norm.eps)
        return out[0], out[1]
    return add_norm(x, linear(u, weight, bias), norm)


def _fits_ffn(layer, h: torch.Tensor, x: torch.Tensor, norm: nn.Module | None) -> bool:
    """The shapes `ffn` takes: bf16 rows 256 wide, a 1,024-wide hidden layer with the exact
    GELU, and (when given) an affine bf16 LayerNorm over 256 columns."""
    l1, l2 = layer.linear1, layer.linear2
    return (h.dim() == 2 and h.is_cuda and h.dtype == torch.bfloat16 and h.shape[1] == 256
            and h.stride(1) == 1 and (h.shape[0] <= 1 or h.stride(0) % 8 == 0)
            and h.data_ptr() % 16 == 0 and x.dtype == torch.bfloat16 and x.is_contiguous()
            and x.shape == h.shape and is_exact_gelu(layer.activation)
            and tuple(l1.weight.shape) == (1024, 256) and tuple(l2.weight.shape) == (256, 1024)
            and l1.weight.dtype == torch.bfloat16 and l2.weight.dtype == torch.bfloat16
            and l1.bias is not None and l2.bias is not None
            and l1.bias.dtype == torch.bfloat16 and l2.bias.dtype == torch.bfloat16
            and (norm is None or (isinstance(norm, nn.LayerNorm) and norm.weight is not None
                                  and norm.bias is not None
                                  and norm.weight.dtype == torch.bfloat16
                                  and tuple(norm.normalized_shape) == (256,))))


def feed_forward(layer, h: torch.Tensor, x: torch.Tensor, norm: nn.Module | None = None):
    """x + linear2(activation(linear1(h))) of a pre-norm encoder layer
    (python/cugo_seq50.py:319-322), h = norm2(x), and with `norm` also norm of that:
    returns x_out, or (x_out, norm(x_out)).  One HIP launch (`ffn`, the hidden layer kept
    on chip) for the d = 256, 1,024-wide bf16 layer; linear (GELU) and linear_add_norm /
    linear with the residual otherwise, which give the same bits."""
    if _fits_ffn(layer, h, x, norm):
        l1, l2 = layer.linear1, layer.linear2
        out = _ext().ffn(h, x, packed_weight(l1.weight), l1.bias.detach(),
                         packed_weight(l2.weight), l2.bias.detach(),
                         None if norm is None else norm.weight.detach(),
                         None if norm is None else norm.bias.detach(),
                         1e-5 if norm is None else norm.eps)
        return out[0] if norm is None else (out[0], out[1])
    if is_exact_gelu(layer.activation):
        u = linear(h, layer.linear1.weight, layer.linear1.bias, gelu=True)
    else:
        u = layer.activation(linear(h, layer.linear1.weight, layer.linear1.bias))
    if norm is None:
        return linear(u, layer.linear2.weight, layer.linear2.bias, residual=x)
    return linear_add_norm(u, layer.linear2.weight, layer.linear2.bias, x, norm)


def attention_tail(layer, att: torch.Tensor, x: torch.Tensor, norm: nn.Module | None = None):
    """The rest of a pre-norm encoder layer after its attention (python/cugo_seq50.py:
    317-322): x1 = x + out_proj(att), then feed_forward(layer, norm2(x1), x1, norm).  One
    HIP launch (`out_proj_ffn`: neither x1 nor norm2(x1) leaves the chip) for the d = 256
    bf16 layer `feed_forward` fuses with a biased out_proj and an affine bf16 norm2;
    linear_add_norm and feed_forward otherwise, which give the same bits."""
    op, n2 = layer.self_attn.out_proj, layer.norm2
    if (_fits_ffn(layer, att, x, norm) and _fits_linear(att, op.weight, op.bias)
            and tuple(op.weight.shape) == (256, 256) and op.bias is not None
            and isinstance(n2, nn.LayerNorm) and n2.weight is not None and n2.bias is not None
            and n2.weight.dtype == torch.bfloat16 and n2.bias.dtype == torch.bfloat16
            and tuple(n2.normalized_shape) == (256,)):
        l1, l2 = layer.linear1, layer.linear2
        out = _ext().out_proj_ffn(att, x, packed_weight(op.weight), op.bias.detach(),
                                  n2.weight.detach(), n2.bias.detach(), n2.eps,
                                  packed_weight(l1.weight), l1.bias.detach(),
                                  packed_weight(l2.weight), l2.bias.detach(),
                                  None if norm is None else norm.weight.detach(),
                                  None if norm is None else norm.bias.detach(),
                                  1e-5 if norm is None else norm.eps)
        return out[0] if norm is None else (out[0], out[1])
    x, h = linear_add_norm(att, op.weight, op.bias, x, n2)
    return feed_forward(layer, h, x, norm)


def order_pays(n: int, slots: int) -> bool:
    """Whether a longest-first query order (decode_order) is worth its launch: on caches
    longer than 64 slots the decode splits each query's slots over two wavefronts of a
    4-wavefront workgroup, and past 2,048 queries (8 heads a wavefront, ~120 VGPRs: four
    wavefronts a SIMD, 4,096 on the chip) the launch runs in more than one round, where
    the order decides which rows start last.  Measured at 4,096 queries of a 320-slot
    cache, us a launch natural / longest first: rows to a uniform target in [1, 320]
    149.7 / 136.0, rows filled to ~308 slots 231.2 / 233.5, one game a row 18.2 / 18.4."""
    return slots > 64 and n > 2048


def cached_step(model: nn.Module, cache, x: torch.Tensor, slots: int | None = None,
                rows: torch.Tensor | None = None, pos: torch.Tensor | None = None) -> torch.Tensor:
    """One token per cache row (x [n, d]); its key/value go to slot cache.length[row].

    Each token attends every cached slot plus itself; `slots` bounds the slot index;
    `rows` names each token's cache row (default: every row in order); `pos`, if given,
    the slot of each token in place of its row's length.  Returns the
    final hidden state [n, d].  Same steps as python/cugo_seq50.py:291-322; each residual
    add and the pre-norm after it run in the launch of the linear layer before them, q, k
    and v are read in place from the packed in-projection, and linear1 + GELU is one
    launch."""
    n, d = x.shape
    heads = cache.heads
    dh = d // heads
    t = cache.slots if slots is None else min(slots, cache.slots)
    row_ids = cache.row_ids if rows is None else rows
    if pos is None:
        pos = cache.length if rows is None else cache.length.index_select(0, row_ids)
    # The decode kernel takes positions past the last slot as the last slot itself.
    pos = pos if t == cache.slots else pos.clamp_max(t - 1)
    # Longest rows first, for every layer's decode, where rows may be long and ragged and
    # the launch takes more than one round of workgroups (results do not depend on it).
    order = decode_order(pos, t) if order_pays(n, cache.slots) else None
    layers = model.encoder.layers
    x, h = add_norm(x, None, layers[0].norm1)
    for i, layer in enumerate(layers):
        attn = layer.self_attn
        q, k, v = linear(h, attn.in_proj_weight, attn.in_proj_bias).chunk(3, -1)
        a = decode_attention_append(q.reshape(n, heads, dh), k.reshape(n, heads, dh),
                                    v.reshape(n, heads, dh), cache.k[i], cache.v[i], pos,
                                    row_ids, order=order)
        if i + 1 < len(layers):
            x, h = attention_tail(layer, a.reshape(n, d), x, layers[i + 1].norm1)
        else:
            x = attention_tail(layer, a.reshape(n, d), x)
    return x


def cached_step_pair(model: nn.Module, cache, x: torch.Tensor, split: int, pos_a: torch.Tensor,
                     pos_b: torch.Tensor, rows_b: torch.Tensor,
                     final_norm: nn.Module | None = None, prune: bool = True,
                     h: torch.Tensor | None = None):
    """cached_step for two groups of tokens at once: rows [0, split) of x (group a, one
    token for each of the cache rows 0 .. split - 1, written at slot pos_a[r]) and rows
    [split, n) (group b, one token for cache row rows_b[j], at slot pos_b[j]).  At every
    layer group a's keys and values are appended before group b attends, so b sees what
    it would see had a been through every layer first (cached_step(a), then
    cached_step(b)); a reads no slot of b (a token reads the slots below its own, and b
    writes at or above a's).  The linear layers run once over both groups.  Positions past
    the last slot are taken as the last slot.  Returns group b's final hidden states
    [n - split, d], and with `final_norm` also final_norm of them (in the last layer's
    launch).  Group a's outputs are not returned: the callers' a tokens are event tokens,
    whose outputs the reference discards (cugo_seq_selfplay50.py:156), so at the last layer
    (`prune`) they only append their key and value (`kv_append`) and skip the attention,
    out_proj and feed-forward; b's outputs and every cache slot are the bits of the full
    pass (`prune=False`).  `h`, if given, is the first layer's norm1 of x, already written
    by the launches that made x."""
    n, d = x.shape
    heads = cache.heads
    dh = d // heads
    layers = model.encoder.layers
    if h is None:
        x, h = add_norm(x, None, layers[0].norm1)
    att = torch.empty((n, heads, dh), dtype=x.dtype, device=x.device)
    for i, layer in enumerate(layers):
        sa = layer.self_attn
        last = i + 1 == len(layers)
        q, k, v = (t.reshape(n, heads, dh)
                   for t in linear(h, sa.in_proj_weight, sa.in_proj_bias).chunk(3, -1))
        if last and prune:  # a's key and value only: nothing reads its outputs past here
            _ext().kv_append(k[:split], v[:split], cache.k[i], cache.v[i], pos_a)
        else:
            decode_attention_append(q[:split], k[:split], v[:split], cache.k[i], cache.v[i],
                                    pos_a, None, out=att[:split])
        decode_attention_append(q[split:], k[split:], v[split:], cache.k[i], cache.v[i], pos_b,
                                rows_b, out=att[split:])
        if last:  # b's rows only
            return attention_tail(layer, att[split:].view(n - split, d), x[split:], final_norm)
        x, h = attention_tail(layer, att.view(n, d), x, layers[i + 1].norm1)
    return x
