"""Drop-in for the reference module `cugo_seq_attention50`
(python/cugo_seq_attention50.py:43-62): single-query attention over a KV cache.

`decode_attention(q, keys, values, pos, use_triton=True, rows=None)` keeps the
reference signature and result: q [n, heads, dh]; keys/values [rows, heads, slots, dh]
(contiguous); pos [n] and rows [n] int64 (rows defaults to 0..n-1) -> [n, heads, dh]
in q's dtype, each query attending slots 0..pos of its row.  It always runs the gfx950
HIP kernel (`cugo_decode_attention` of libcugo_hip.so); `use_triton` is accepted for
call compatibility and selects nothing, because there is one implementation.  There is
no CPU path: tensors that are not on the GPU raise.

`decode_attention_append` is the reference caller's KV append plus decode
(python/cugo_seq50.py:313-320: `index_put_` of the new key/value at slot pos, then
`decode_attention`) in one launch.

Both take an optional `order` (int32 [n], a permutation of the queries): the order in
which the launch serves them.  It changes no result.  `decode_order(pos, slots)` gives the
longest-first order, with which ragged rows end a launch with short work instead of long
rows started late.
"""

from __future__ import annotations

import torch

from cugo_amd.cugo_torch50_ext import load_extension

_EXT = None


def _ext():
    global _EXT
    if _EXT is None:
        _EXT = load_extension()
    return _EXT


def _check_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError("decode_attention runs on the GPU only; got a CPU tensor")


def decode_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, pos: torch.Tensor,
                     use_triton: bool = True, rows: torch.Tensor | None = None,
                     order: torch.Tensor | None = None) -> torch.Tensor:
    """q [n, heads, dh]; keys/values [rows, heads, slots, dh] (contiguous); pos [n] and
    rows [n] int64 (rows defaults to 0..n-1) -> [n, heads, dh]."""
    del use_triton  # one implementation: the HIP kernel
    _check_device(q, keys, values, pos)
    return _ext().decode_attention(q, keys, values, pos, rows, order)


def decode_attention_append(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                            keys: torch.Tensor, values: torch.Tensor, pos: torch.Tensor,
                            rows: torch.Tensor | None = None,
                            out: torch.Tensor | None = None,
                            order: torch.Tensor | None = None) -> torch.Tensor:
    """Writes k_new/v_new [n, heads, dh] to slot pos[i] of row rows[i] of keys/values (in
    place, cast to the cache dtype), then returns decode_attention over slots 0..pos
    (written into `out`, contiguous [n, heads, dh], when given)."""
    _check_device(q, k_new, v_new, keys, values, pos)
    return _ext().decode_attention_append(q, k_new, v_new, keys, values, pos, rows, out, order)


def decode_order(pos: torch.Tensor, slots: int) -> torch.Tensor:
    """int32 [n]: the queries longest first by min(pos, slots - 1) (negative pos last),
    binned by length; for `order`.  One small launch."""
    _check_device(pos)
    return _ext().decode_order(pos, slots)
