"""Event-sequence policy oracle (TEST INFRASTRUCTURE ONLY).

Only tests/ and bench.py import this module, as the checker; the product path never
does.  Restatements of the reference's sequence-policy pieces that the self-play step
uses:

* `encode_events_np` / `encode_start_np` - the observer-relative token vectors of
  python/cugo_seq50.py:91-110 and :113-128, as float64 numpy arrays built bit by bit
  (414 and 274 columns).  Pinned in tests/test_cpu_seq_oracle.py by hand-built events
  and openings whose tokens follow from the reference's slot list (played, own drawn,
  flipped, my gain, opponent gain, my loss, opponent loss, shown; "my" = player 0's
  words for observer seat 0 and player 1's for seat 1) and from the start-word layout
  (hand0, hand1, floor, captured0, captured1, mission, neutral,
  type | mult << 8 | first << 16 | m0 << 24 | m1 << 32, torch50.h:684-698).
* `token_reference` - SeqNet.event_token / start_token (cugo_seq50.py:271-282) on top of
  those vectors with the reference's bf16 roundings: the Linear in float64, rounded to
  the weight dtype, then + position, rounded, then + token_type, rounded.
* `reference_cached_step` - SeqNet.cached_step (cugo_seq50.py:291-322): index_put_ of the
  new key/value, then the matmul decode path (oracle.decode_ref.matmul_path).  Pinned by
  the fact that incremental decoding must equal the full causal forward of the same
  prefix (tests/test_cpu_seq_step_pins.py, float64, ragged rows, the slot clamp).
* `gumbel_reference` - the sampling lines of WaveCollector._step
  (cugo_seq_selfplay50.py:125-130) on supplied uniforms, in torch.  Pinned by closed
  forms and sampled frequencies (same test file).
"""

from __future__ import annotations

import numpy as np

from oracle.decode_ref import matmul_path

EVENT_IN = 8 * 50 + 12 + 2
START_IN = 5 * 50 + 12 + 8 + 4
KINDS = 12
MAX_EVENTS = 48
_CARDS = (1 << 50) - 1


def _bits(x: int, width: int = 50) -> np.ndarray:
    x = int(x) & ((1 << 64) - 1)
    return np.array([(x >> j) & 1 for j in range(width)], dtype=np.float64)


def encode_events_np(words: np.ndarray, seat: np.ndarray) -> np.ndarray:
    """[n, 9] int64 event words, [n] seats -> [n, 414] float64 tokens
    (cugo_seq50.py:91-110 for one event per row)."""
    words = np.asarray(words, dtype=np.int64).reshape(-1, 9)
    seat = np.asarray(seat, dtype=np.int64).reshape(-1)
    out = np.zeros((words.shape[0], EVENT_IN), dtype=np.float64)
    for i, (ev, s) in enumerate(zip(words.view(np.uint64), seat)):
        header = int(ev[8])
        me = (header & 0xFF) == int(s)
        kind = (header >> 8) & 0xFF
        first = int(s) == 0
        slots = (ev[0], ev[1] if me else 0, ev[2],
                 ev[3] if first else ev[4], ev[4] if first else ev[3],
                 ev[5] if first else ev[6], ev[6] if first else ev[5], ev[7])
        for k, m in enumerate(slots):
            out[i, 50 * k:50 * (k + 1)] = _bits(int(m))
        out[i, 400 + min(kind, KINDS - 1)] = 1.0
        out[i, 412] = 1.0 if me else 0.0
        out[i, 413] = 0.0 if me else float(_bits(int(ev[1])).sum())
    return out


def encode_start_np(start: np.ndarray, seat: np.ndarray) -> np.ndarray:
    """[n, 8] int64 start words, [n] seats -> [n, 274] float64 tokens
    (cugo_seq50.py:113-128)."""
    start = np.asarray(start, dtype=np.int64).reshape(-1, 8)
    seat = np.asarray(seat, dtype=np.int64).reshape(-1)
    out = np.zeros((start.shape[0], START_IN), dtype=np.float64)
    for i, (st, s) in enumerate(zip(start.view(np.uint64), seat)):
        first = int(s) == 0
        st = [int(w) for w in st]
        planes = (st[0] if first else st[1], st[2], st[3] if first else st[4],
                  st[4] if first else st[3], st[5])
        for k, m in enumerate(planes):
            out[i, 50 * k:50 * (k + 1)] = _bits(m)
        out[i, 250:262] = _bits(st[6], 12)
        header = st[7]
        out[i, 262 + min(header & 0xFF, 7)] = 1.0
        m0, m1 = ((header >> 24) & 0xFF) / 8.0, ((header >> 32) & 0xFF) / 8.0
        out[i, 270] = ((header >> 8) & 0xFF) / 4.0
        out[i, 271] = 1.0 if ((header >> 16) & 1) == int(s) else 0.0
        out[i, 272] = m0 if first else m1
        out[i, 273] = m1 if first else m0
    return out


def token_reference(tokens: np.ndarray, weight, bias, position_row, token_type_row):
    """Linear (float64 sum over the token, weight [d, in] as in nn.Linear) then the
    position and token-type adds, each result rounded to the weight dtype; torch tensors
    in (any device), a tensor of the weight dtype out."""
    import torch

    dt = weight.dtype
    t = torch.as_tensor(tokens, dtype=torch.float64, device=weight.device)
    # the reference casts the token to the weight dtype first (`.to(dtype)`)
    t = t.to(dt).to(torch.float64)
    r1 = (t @ weight.to(torch.float64).T + bias.to(torch.float64)).to(dt)
    r2 = (r1.to(torch.float64) + position_row.to(torch.float64)).to(dt)
    return (r2.to(torch.float64) + token_type_row.to(torch.float64)).to(dt)


def reference_cached_step(model, cache, x, rows=None, slots=None):
    """cugo_seq50.py:291-322 restated with the matmul decode path: token i goes to cache
    row rows[i] (default: row i) at slot min(length[row], t - 1), t = min(slots,
    cache.slots), and attends slots 0..that slot; returns the last layer's residual
    stream [n, d].  Pinned in tests/test_cpu_seq_step_pins.py against the full causal
    forward of nn.TransformerEncoder."""
    import torch
    import torch.nn.functional as F

    n, d = x.shape
    heads, dh = cache.heads, d // cache.heads
    t = cache.slots if slots is None else min(slots, cache.slots)
    if rows is None:
        rows = torch.arange(n, device=x.device)
    pos = cache.length.index_select(0, rows).clamp_max(t - 1)
    head_ids = torch.arange(heads, device=x.device).view(1, heads)
    flat_rows = (rows.view(n, 1) * heads + head_ids).flatten()
    flat_pos = pos.repeat_interleave(heads)
    for i, layer in enumerate(model.encoder.layers):
        attn = layer.self_attn
        q, k, v = F.linear(layer.norm1(x), attn.in_proj_weight, attn.in_proj_bias).chunk(3, -1)
        kc, vc = cache.k[i], cache.v[i]
        kc.view(-1, cache.slots, dh).index_put_((flat_rows, flat_pos),
                                                k.reshape(n * heads, dh).to(kc.dtype))
        vc.view(-1, cache.slots, dh).index_put_((flat_rows, flat_pos),
                                                v.reshape(n * heads, dh).to(vc.dtype))
        a = matmul_path(q.reshape(n, heads, dh), kc, vc, pos, rows)
        x = x + attn.out_proj(a.reshape(n, d))
        x = x + layer.linear2(layer.activation(layer.linear1(layer.norm2(x))))
    return x


def gumbel_reference(logits, legal, uniforms):
    """cugo_seq_selfplay50.py:125-130 with `torch.rand_like(masked)` replaced by the
    supplied uniforms: (actions, logp).  Pinned in tests/test_cpu_seq_step_pins.py by
    closed forms (one legal action, k equal logits, a dominant draw) and by the action
    frequencies of many draws against the legal softmax."""
    import torch

    masked = logits.masked_fill(~legal, -1.0e30)
    gumbel = -torch.log(-torch.log(uniforms.clamp(1e-20, 1.0)))
    actions = (masked + gumbel).argmax(1)
    logp = torch.log_softmax(masked, 1).gather(1, actions.unsqueeze(1)).squeeze(1)
    return actions, logp
