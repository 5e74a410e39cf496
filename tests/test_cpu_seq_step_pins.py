"""Pins of oracle/seq_ref.py's decoder step and sampler by facts the mathematics fixes.

* `reference_cached_step` (python/cugo_seq50.py:291-322 restated) decodes one token per
  cache row against the keys and values of the tokens cached before it.  A causal
  pre-norm encoder computes each position from the positions at or before it only, so
  the step's output must equal the full causal forward of nn.TransformerEncoder over the
  row's cached prefix followed by the new token, at the last position.  That holds for
  every row of a ragged batch in any row order, for a query token whose slot the next
  event overwrites (the cache length is not advanced), and at the slot clamp (a row
  whose length reached the slots bound t writes slot t - 1 and attends slots 0..t - 1:
  the forward over the first t - 1 cached tokens and the new one).
* `gumbel_reference` (python/cugo_seq_selfplay50.py:125-130 restated) is Gumbel-max
  sampling from the softmax of the legal logits: one legal action is always chosen with
  log-probability 0, k equal legal logits give -log k, the largest perturbed logit wins,
  illegal actions never win for uniforms in [0, 1), and the action frequencies of many
  draws follow the legal softmax.

Each check is shown to fail for a planted mistake in the oracle (a swapped pre-norm, an
off-by-one slot, the log-probability over every action, the noise added unmasked), so a
shared misreading of the reference by the oracle and the GPU path cannot stay green.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch
from torch import nn

import oracle.seq_ref as seq_ref
from oracle.seq_ref import gumbel_reference, reference_cached_step

D, HEADS, LAYERS = 32, 4, 2
# matmul_path casts the scores to float32 as the reference does (cugo_seq_attention50.py:60),
# so an otherwise float64 step agrees with the float64 forward to float32 rounding.
TOL = 1e-5


class _Cache:
    """The fields reference_cached_step reads, in float64."""

    def __init__(self, rows: int, slots: int) -> None:
        self.heads, self.slots = HEADS, slots
        self.k = torch.zeros((LAYERS, rows, HEADS, slots, D // HEADS), dtype=torch.float64)
        self.v = torch.zeros_like(self.k)
        self.length = torch.zeros(rows, dtype=torch.int64)


def _model(seed: int = 0) -> nn.Module:
    torch.manual_seed(seed)
    layer = nn.TransformerEncoderLayer(D, HEADS, 4 * D, dropout=0.0, activation="gelu",
                                       batch_first=True, norm_first=True)
    model = nn.Module()
    model.encoder = nn.TransformerEncoder(layer, LAYERS, enable_nested_tensor=False)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0.0, 0.3)  # large enough that attention is far from uniform
    return model.double().eval()


def _causal_last(model: nn.Module, tokens: torch.Tensor) -> torch.Tensor:
    """Full causal forward of nn.TransformerEncoder over [T, d]; the last position."""
    t = tokens.shape[0]
    mask = nn.Transformer.generate_square_subsequent_mask(t, dtype=torch.float64)
    out = model.encoder(tokens.unsqueeze(0), mask=mask, is_causal=True)
    return out[0, -1]


def _replay(model: nn.Module, oracle_model: nn.Module | None = None, length_shift: int = 0,
            seed: int = 1) -> float:
    """Ragged decoding through reference_cached_step against the full forward; returns the
    largest relative error over every token.  `oracle_model` / `length_shift` plant a
    mistake on the oracle's side only (a different module, an off-by-one slot)."""
    oracle_model = model if oracle_model is None else oracle_model
    rows_n, cache_slots, bound = 7, 12, 9
    g = torch.Generator().manual_seed(seed)
    cache = _Cache(rows_n, cache_slots)
    history: list[list[torch.Tensor]] = [[] for _ in range(rows_n)]
    worst = 0.0
    clamp_hits = query_hits = 0
    with torch.no_grad():
        for step in range(16):
            rows = torch.randperm(rows_n, generator=g)[:5]
            x = torch.randn(5, D, generator=g, dtype=torch.float64)
            advance = torch.rand(5, generator=g) < 0.75  # events advance, queries do not
            saved = cache.length.clone()
            cache.length += length_shift
            got = reference_cached_step(oracle_model, cache, x, rows, slots=bound)
            cache.length.copy_(saved)
            for i, r in enumerate(rows.tolist()):
                pos = min(len(history[r]), bound - 1)
                clamp_hits += len(history[r]) >= bound - 1
                query_hits += not bool(advance[i])
                want = _causal_last(model, torch.stack(history[r][:pos] + [x[i]]))
                err = float((got[i] - want).norm() / want.norm())
                worst = max(worst, err)
                if advance[i]:
                    history[r].append(x[i])
                    cache.length[r] += 1
    assert clamp_hits > 0 and query_hits > 0  # both regimes were exercised
    return worst


def test_cached_step_equals_full_causal_forward():
    assert _replay(_model()) <= TOL


def test_cached_step_pin_catches_a_swapped_prenorm():
    model = _model()
    swapped = copy.deepcopy(model)
    for layer in swapped.encoder.layers:  # norm2 before attention, norm1 before the MLP
        layer.norm1, layer.norm2 = layer.norm2, layer.norm1
    with torch.no_grad():
        for layer in model.encoder.layers:  # make the two norms differ
            layer.norm2.weight.mul_(1.7)
    assert _replay(model, oracle_model=swapped) > 100 * TOL


def test_cached_step_pin_catches_an_off_by_one_slot():
    assert _replay(_model(), length_shift=1) > 100 * TOL


def test_cached_step_default_rows_and_slots():
    """rows=None is row i for token i; slots=None bounds by the cache's own slot count."""
    model = _model(3)
    g = torch.Generator().manual_seed(4)
    a, b = _Cache(4, 6), _Cache(4, 6)
    with torch.no_grad():
        for _ in range(8):  # runs past the cache's 6 slots: the clamp at cache.slots - 1
            x = torch.randn(4, D, generator=g, dtype=torch.float64)
            ya = reference_cached_step(model, a, x)
            yb = reference_cached_step(model, b, x, torch.arange(4), slots=6)
            assert torch.equal(ya, yb)
            a.length += 1
            b.length += 1


# -- Gumbel-max sampling --------------------------------------------------------------


def _logp_over_all_actions(logits, legal, uniforms):
    """A planted mistake: the log-probability normalised over every action."""
    actions, _ = gumbel_reference(logits, legal, uniforms)
    return actions, torch.log_softmax(logits, 1).gather(1, actions.unsqueeze(1)).squeeze(1)


def _noise_unmasked(logits, legal, uniforms):
    """A planted mistake: the argmax over the unmasked logits."""
    gumbel = -torch.log(-torch.log(uniforms.clamp(1e-20, 1.0)))
    actions = (logits + gumbel).argmax(1)
    masked = logits.masked_fill(~legal, -1.0e30)
    return actions, torch.log_softmax(masked, 1).gather(1, actions.unsqueeze(1)).squeeze(1)


def _closed_forms(sampler) -> None:
    g = torch.Generator().manual_seed(5)
    n, a = 64, 179
    logits = torch.randn(n, a, generator=g) * 3.0
    u = torch.rand(n, a, generator=g)
    # one legal action: always it, log-probability exactly 0
    only = torch.randint(0, a, (n,), generator=g)
    legal = torch.zeros(n, a, dtype=torch.bool)
    legal[torch.arange(n), only] = True
    act, lp = sampler(logits, legal, u)
    assert torch.equal(act, only)
    assert torch.equal(lp, torch.zeros(n))
    # k equal legal logits among large illegal ones: -log k, and never an illegal action
    for k in (2, 3, 7, 50, 179):
        legal = torch.zeros(n, a, dtype=torch.bool)
        for i in range(n):
            legal[i, torch.randperm(a, generator=g)[:k]] = True
        flat = torch.where(legal, torch.full((n, a), 0.25), logits.abs() + 50.0)
        act, lp = sampler(flat, legal, u)
        assert bool(legal[torch.arange(n), act].all())
        assert torch.allclose(lp, torch.full((n,), -float(np.log(k))), atol=1e-5)
    # extreme uniforms: 0 (clamped to 1e-20) and the largest float32 below 1
    legal = torch.rand(n, a, generator=g) < 0.3
    legal[:, 0] = True
    for value in (0.0, float(np.nextafter(np.float32(1.0), np.float32(0.0)))):
        act, _ = sampler(logits, legal, torch.full((n, a), value))
        assert bool(legal[torch.arange(n), act].all())
    # a legal action whose draw is 1 (gumbel +inf) wins
    hot = torch.randint(0, a, (n,), generator=g)
    legal[torch.arange(n), hot] = True
    u1 = u.clone()
    u1[torch.arange(n), hot] = 1.0
    act, _ = sampler(logits, legal, u1)
    assert torch.equal(act, hot)


def _frequencies(sampler) -> None:
    """20,000 draws of one row: the count of each action within 4 sigma of the legal
    softmax (binomial sigma), and no illegal action."""
    g = torch.Generator().manual_seed(6)
    a, draws = 179, 20000
    logits = torch.randn(1, a, generator=g) * 1.5
    legal = torch.rand(1, a, generator=g) < 0.1
    legal[0, :3] = True
    rows_l = logits.expand(draws, a).contiguous()
    rows_m = legal.expand(draws, a).contiguous()
    act, lp = sampler(rows_l, rows_m, torch.rand(draws, a, generator=g))
    p = torch.softmax(logits.double().masked_fill(~legal, -float("inf")), 1)[0]
    counts = torch.bincount(act, minlength=a).double()
    sigma = torch.sqrt(draws * p * (1 - p)).clamp_min(1.0)
    assert bool((counts[~legal[0]] == 0).all())
    assert bool(((counts - draws * p).abs() <= 4 * sigma).all())
    assert torch.allclose(lp.double(), p.log()[act], atol=1e-5)


def test_gumbel_closed_forms():
    _closed_forms(gumbel_reference)


def test_gumbel_frequencies_follow_the_legal_softmax():
    _frequencies(gumbel_reference)


@pytest.mark.parametrize("planted", [_logp_over_all_actions, _noise_unmasked])
def test_gumbel_pins_catch_planted_mistakes(planted):
    with pytest.raises(AssertionError):
        _closed_forms(planted)
        _frequencies(planted)


def test_matmul_path_is_the_oracles_attention():
    """The step reads attention through oracle.decode_ref.matmul_path (itself pinned to the
    float64 brute force in tests/test_cpu_decode_oracle.py)."""
    assert seq_ref.matmul_path.__module__ == "oracle.decode_ref"
