"""Decode-attention oracle (TEST INFRASTRUCTURE ONLY).

Only tests/ and bench.py import this module, as the checker; the product path never
does.  Two restatements of the reference's single-query attention
(python/cugo_seq_attention50.py:43-62):

* `matmul_path` - the reference's own two-matmul formulation
  (python/cugo_seq_attention50.py:58-62): gather the rows, scores = q @ K^T in q's dtype,
  cast to fp32 and scale, mask slots > pos with -inf, fp32 softmax, cast the
  probabilities back to q's dtype, then @ V.  Torch on whatever device the inputs are.
* `brute_force` - float64 numpy loops over (query, head, slot), written from the
  definition out[i,h] = sum_t softmax_t(q . K[r,h,t] / sqrt(dh)) V[r,h,t] over
  t = 0..min(pos, slots-1); small shapes only.  It pins `matmul_path` (tests/) and
  is pinned itself by closed forms: pos = 0 gives V[r,h,0]; equal keys give the mean
  of V[r,h,0..pos]; one key far above the rest gives that slot's V.
"""

from __future__ import annotations

import numpy as np


def matmul_path(q, keys, values, pos, rows=None):
    """cugo_seq_attention50.py:58-62 restated (torch tensors in, torch tensor out)."""
    import torch

    n, heads, dh = q.shape
    slots = keys.shape[2]
    scale = dh ** -0.5
    if rows is None:
        rows = torch.arange(n, device=q.device)
    keys, values = keys.index_select(0, rows), values.index_select(0, rows)
    mask = torch.arange(slots, device=q.device).view(1, 1, 1, slots) <= pos.view(n, 1, 1, 1)
    # [n, heads, 1, dh] @ [n, heads, dh, slots]; the transposed operand is made contiguous
    # before the batched product.
    kt = keys.transpose(-1, -2).to(q.dtype).contiguous()
    scores = torch.matmul(q.unsqueeze(2), kt).float() * scale
    probs = torch.softmax(scores.masked_fill(~mask, float("-inf")), -1).to(q.dtype)
    return torch.matmul(probs, values.to(q.dtype).contiguous()).squeeze(2)


def brute_force(q: np.ndarray, keys: np.ndarray, values: np.ndarray, pos: np.ndarray,
                rows: np.ndarray | None = None) -> np.ndarray:
    """float64 reference from the definition; arrays are numpy (any float dtype)."""
    q = np.asarray(q, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    values = np.asarray(values, dtype=np.float64)
    n, heads, dh = q.shape
    slots = keys.shape[2]
    rows = np.arange(n) if rows is None else np.asarray(rows)
    out = np.empty((n, heads, dh), dtype=np.float64)
    scale = 1.0 / np.sqrt(dh)
    for i in range(n):
        r = int(rows[i])
        p = int(pos[i])
        for h in range(heads):
            if p < 0 or r < 0 or r >= keys.shape[0]:
                out[i, h] = np.nan
                continue
            last = min(p, slots - 1)
            s = np.array([float(np.dot(q[i, h], keys[r, h, t])) * scale for t in range(last + 1)])
            w = np.exp(s - s.max())
            w /= w.sum()
            acc = np.zeros(dh)
            for t in range(last + 1):
                acc += w[t] * values[r, h, t]
            out[i, h] = acc
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r[nan] = 0x7FC0
    return r
