"""Paired evaluation (python/cugo_eval50.py:137-361) on the HIP engine.

Pinned end to end against the oracle engine: two policies whose greedy choice is known
in closed form (the first legal action, the last legal action: a zero-weight Linear with
a descending or ascending bias) play the duplicated deals on the CPU oracle, and every
summary field must equal what those games give.  Self-play of one policy on both seats
of a pair plays the same game twice, so every pair scores 0.  The greedy kernel is
checked against torch's masked argmax.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.conftest import announce

pytestmark = pytest.mark.gpu

DEV = "cuda"


def fixed_choice(last: bool) -> torch.nn.Module:
    """Logits that do not depend on the state: argmax over the legal mask picks the first
    (or the last) legal action."""
    lin = torch.nn.Linear(720, 179)
    with torch.no_grad():
        lin.weight.zero_()
        order = torch.arange(179, dtype=torch.float32)
        lin.bias.copy_(order if last else -order)
    return lin.to(DEV)


def test_masked_argmax_matches_torch(ext):
    announce("masked_argmax")
    g = torch.Generator(device=DEV).manual_seed(9)
    logits = torch.randn(5000, 179, generator=g, device=DEV)
    legal = torch.rand(5000, 179, generator=g, device=DEV) < 0.2
    legal[:3] = False
    logits[3:6] = 1.0  # ties: the first legal index
    want = logits.masked_fill(~legal, -1.0e30).argmax(1)
    assert torch.equal(ext.masked_argmax(logits, legal), want)
    lb = logits.to(torch.bfloat16)
    want_b = lb.float().masked_fill(~legal, -1.0e30).argmax(1)
    assert torch.equal(ext.masked_argmax(lb, legal), want_b)


def oracle_games(ref, seeds, first, a_seat, choose):
    """Plays every game to the end on the oracle with A = choose[0], B = choose[1]
    (functions legal row -> action); returns final reward0, nagari, excluded, steps."""
    n = seeds.size
    states = ref.create(seeds, first)
    reward = np.zeros(n, dtype=np.float32)
    nagari = np.zeros(n, dtype=bool)
    excluded = np.zeros(n, dtype=bool)
    ids = np.arange(n)
    steps = 0
    for step in range(200):
        if ids.size == 0:
            break
        _, legal, player, done, status = ref.observe(states, ids)
        assert (status == 0).all()
        if step == 0:
            excluded[ids[done]] = True
            keep = ~done
            ids, legal, player = ids[keep], legal[keep], player[keep]
            if ids.size == 0:
                break
        steps += 1
        acts = np.array([choose[0 if p == s else 1](row)
                         for row, p, s in zip(legal, player, a_seat[ids])])
        r, d, nag, st, _ = ref.step(states, acts, ids)
        assert (st == 0).all()
        ended = d
        reward[ids] = np.where(ended, r, 0.0)
        nagari[ids] = ended & nag
        ids = ids[~d]
    return reward, nagari, excluded, steps


def test_paired_eval_against_oracle_games(ext, ref):
    announce("paired eval vs oracle games")
    from cugo_amd.paired_eval import evaluate_paired
    from cugo_amd.seq_selfplay import make_seeds

    pairs = 200
    got = evaluate_paired(ext, fixed_choice(False), fixed_choice(True), pairs, seed_offset=900,
                          max_steps=128, use_amp=False)
    seeds, first = make_seeds(pairs, 900, "cpu")
    seeds = np.tile(seeds.numpy(), 2)
    first = np.tile(first.numpy(), 2)
    a_seat = (np.arange(2 * pairs) >= pairs).astype(np.int64)
    first_legal = lambda row: int(np.flatnonzero(row)[0])   # noqa: E731
    last_legal = lambda row: int(np.flatnonzero(row)[-1])   # noqa: E731
    reward, nagari, excluded, steps = oracle_games(ref, seeds, first, a_seat,
                                                   (first_legal, last_legal))
    score = np.where(a_seat == 0, reward, -reward)
    s0, s1 = score[:pairs], score[pairs:]
    v0, v1 = ~excluded[:pairs], ~excluded[pairs:]
    pair = (s0 + s1) * 0.5
    both = v0 & v1
    wdl = lambda x: (int((x > 0).sum()), int((x < 0).sum()), int((x == 0).sum()))  # noqa: E731
    assert got.decision_steps == steps
    assert (got.evaluated_pairs, got.evaluated_games, got.predecision_excluded) == (
        int(both.sum()), int((~excluded).sum()), int(excluded.sum()))
    assert (got.a_wins, got.b_wins, got.draws) == wdl(score[~excluded])
    assert (got.a_p0_wins, got.a_p0_losses, got.a_p0_draws) == wdl(s0[v0])
    assert (got.a_p1_wins, got.a_p1_losses, got.a_p1_draws) == wdl(s1[v1])
    assert (got.pair_wins, got.pair_losses, got.pair_draws) == wdl(pair[both])
    assert (got.terminal, got.nagari) == (int((~nagari).sum()), int(nagari.sum()))
    assert got.mean_pair_score_a == pytest.approx(float(pair[both].mean()), rel=1e-6, abs=1e-6)
    assert got.mean_score_a == pytest.approx(float(score[~excluded].mean()), rel=1e-6, abs=1e-6)
    assert got.pair_score_std == pytest.approx(float(pair[both].std(ddof=1)), rel=1e-5)


def test_paired_self_play_scores_zero(ext):
    announce("paired self-play")
    from cugo_amd.paired_eval import evaluate_paired

    torch.manual_seed(4)
    model = torch.nn.Sequential(torch.nn.Linear(720, 128), torch.nn.ReLU(),
                                torch.nn.Linear(128, 179)).to(DEV)
    got = evaluate_paired(ext, model, model, 500, seed_offset=17, max_steps=128, use_amp=False)
    assert got.mean_pair_score_a == 0.0 and got.pair_draws == got.evaluated_pairs
    assert (got.a_p0_wins, got.a_p0_losses) == (got.a_p1_losses, got.a_p1_wins)
    assert got.games == 1000 and got.seconds > 0
    # sampling from the softmax plays, too (its outcome depends on torch's RNG)
    s = evaluate_paired(ext, model, model, 100, seed_offset=3, max_steps=128, use_amp=True,
                        sample_a=True, sample_b=True)
    assert s.a_wins + s.b_wins + s.draws == s.evaluated_games


def test_paired_eval_graph_equals_eager(ext):
    """The captured step and the eager one play the same games: identical summaries (all
    fields but the time) for two different MLP policies under fp16 autocast; the Linear
    weights cast to fp16 once give autocast's own outputs bit for bit."""
    announce("paired eval: graph replay vs eager steps")
    from dataclasses import asdict

    from cugo_amd.paired_eval import evaluate_paired

    def mlp(seed):
        torch.manual_seed(seed)
        return torch.nn.Sequential(torch.nn.Linear(720, 256), torch.nn.ReLU(),
                                   torch.nn.Linear(256, 179)).to(DEV)

    a, b = mlp(5), mlp(6)
    # the fp16 copy of the Linear weights computes what autocast computes, bit for bit
    from cugo_amd.paired_eval import _half_linears

    x = torch.randn(1000, 720, device=DEV)
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.float16):
        assert torch.equal(_half_linears(a)(x), a(x))
    runs = [asdict(evaluate_paired(ext, a, b, 300, seed_offset=41, max_steps=128, use_amp=True,
                                   graph=g)) for g in (True, False, True)]
    for r in runs:
        r.pop("seconds")
    assert runs[0] == runs[1] == runs[2]
    assert runs[0]["evaluated_games"] > 0 and runs[0]["decision_steps"] > 10
