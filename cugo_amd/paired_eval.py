"""Paired evaluation on the HIP engine (python/cugo_eval50.py:137-361, `evaluate_paired`).

Every deal is played twice, model A on seat 0 in game i and on seat 1 in game pairs + i,
so deal luck cancels in the pair score.  A decision step observes the games still
running, evaluates each model on the rows where its seat moves, takes the greedy action
(the `masked_argmax` kernel: argmax of the fp32 logits with illegal actions at -1e30) or
samples from the softmax, steps the engine, and drops finished games.  Summary fields and
their meaning are the reference's `EvalSummary` (cugo_eval50.py:27-61).

Policies are modules mapping the [n, 720] features to logits (or a tuple whose first
item is the logits), like the reference's PpoActor; sequence policies with event
histories are not handled here.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass

import torch
from torch import nn

from .seq_selfplay import make_seeds


@dataclass
class EvalSummary:
    pairs: int
    games: int
    evaluated_pairs: int
    evaluated_games: int
    predecision_excluded: int
    a_wins: int
    b_wins: int
    draws: int
    a_p0_wins: int
    a_p0_losses: int
    a_p0_draws: int
    a_p1_wins: int
    a_p1_losses: int
    a_p1_draws: int
    pair_wins: int
    pair_losses: int
    pair_draws: int
    mean_score_a: float
    mean_score_a_p0: float
    mean_score_a_p1: float
    mean_pair_score_a: float
    pair_score_std: float
    pair_score_se: float
    pair_score_ci95_low: float
    pair_score_ci95_high: float
    terminal: int
    nagari: int
    decision_steps: int
    seconds: float

    @property
    def games_per_s(self) -> float:
        return self.games / self.seconds


def _actions(ext, model: nn.Module, features, legal, use_amp: bool, sample: bool):
    """cugo_eval50.py:112-127 for a features-only policy."""
    with torch.autocast(device_type="cuda", dtype=torch.float16, enabled=use_amp):
        out = model(features)
    logits = (out[0] if isinstance(out, tuple) else out).float().contiguous()
    if sample:
        masked = logits.masked_fill(~legal, -1.0e30)
        return torch.multinomial(torch.softmax(masked, dim=1), 1).squeeze(1)
    return ext.masked_argmax(logits, legal)


def _wdl(x: torch.Tensor) -> tuple[int, int, int]:
    return int((x > 0).sum()), int((x < 0).sum()), int((x == 0).sum())


def _mean(x: torch.Tensor) -> float:
    return float(x.mean()) if x.numel() else 0.0


def evaluate_paired(ext, model_a: nn.Module, model_b: nn.Module, pairs: int, seed_offset: int,
                    max_steps: int, use_amp: bool, sample_a: bool = False,
                    sample_b: bool = False) -> EvalSummary:
    if pairs <= 0:
        raise ValueError("pairs must be positive")
    if max_steps <= 0:
        raise ValueError("max_steps must be positive")
    dev = torch.device("cuda")
    seeds, first = make_seeds(pairs, seed_offset, dev)
    games = 2 * pairs
    states = ext.create(seeds.repeat(2), first.repeat(2))
    a_seat = (torch.arange(games, device=dev) >= pairs).long()  # A moves first seat in game i
    final_reward0 = torch.zeros(games, device=dev)
    final_nagari = torch.zeros(games, dtype=torch.bool, device=dev)
    excluded = torch.zeros(games, dtype=torch.bool, device=dev)  # over before any decision
    bad = torch.zeros(3, dtype=torch.int64, device=dev)  # observe, legal, step
    ok = int(ext.STATUS_OK)
    model_a.eval()
    model_b.eval()
    ids = torch.arange(games, device=dev)
    decision_steps = 0
    finished_all = False
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.inference_mode():
        for step in range(max_steps):
            if ids.numel() == 0:
                finished_all = True
                break
            features, legal, players, done, status = ext.observe_indexed(states, ids)
            fine = status == ok
            any_legal = legal.any(1)
            if step == 0:
                # games already over, or unplayable, at the deal leave the evaluation
                excluded.index_fill_(0, ids[done], True)
                live = ~done
                bad[0] += (live & ~fine).sum()
                bad[1] += (live & fine & ~any_legal).sum()
                keep = live & fine & any_legal
                ids, features, legal, players = ids[keep], features[keep], legal[keep], players[keep]
                if ids.numel() == 0:
                    finished_all = True
                    break
            else:
                bad[0] += (~fine).sum()
                bad[1] += (fine & (done | ~any_legal)).sum()
            decision_steps += 1
            a_moves = players.long() == a_seat.index_select(0, ids)
            actions = torch.empty(ids.numel(), dtype=torch.int64, device=dev)
            for model, rows, sample in ((model_a, a_moves, sample_a), (model_b, ~a_moves, sample_b)):
                at = torch.nonzero(rows).squeeze(1)
                if at.numel():
                    actions[at] = _actions(ext, model, features[at], legal[at], use_amp, sample)
            reward0, new_done, nagari, step_status, _ = ext.step_indexed(states, ids, actions)
            step_ok = step_status == ok
            bad[2] += (~step_ok).sum()
            ended = step_ok & new_done
            final_reward0[ids] = torch.where(ended, reward0, torch.zeros_like(reward0))
            final_nagari[ids] = ended & nagari
            ids = ids[step_ok & ~new_done]
        else:
            finished_all = ids.numel() == 0
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0

    observe_bad, legal_bad, step_bad = (int(x) for x in bad.tolist())
    if observe_bad:
        raise RuntimeError(f"observe failed on {observe_bad} active visits")
    if legal_bad:
        raise RuntimeError(f"active state had invalid/no legal actions on {legal_bad} visits")
    if step_bad:
        raise RuntimeError(f"step failed on {step_bad} active visits")
    if not finished_all:
        raise RuntimeError(f"not all games finished within {max_steps} decision steps")

    score = torch.where(a_seat == 0, final_reward0, -final_reward0)  # A's points
    s0, s1 = score[:pairs], score[pairs:]
    pair_score = (s0 + s1) * 0.5
    v0, v1 = ~excluded[:pairs], ~excluded[pairs:]
    both = v0 & v1
    valid = score[~excluded]
    vp = pair_score[both]
    n_pairs = int(both.sum())
    mean_pair = _mean(vp)
    std = float(vp.std(unbiased=True)) if n_pairs > 1 else 0.0
    se = std / math.sqrt(n_pairs) if n_pairs > 1 else 0.0
    half = 1.959963984540054 * se
    a_w, b_w, d = _wdl(valid)
    p0 = _wdl(s0[v0])
    p1 = _wdl(s1[v1])
    pw = _wdl(vp)
    return EvalSummary(
        pairs=pairs, games=games, evaluated_pairs=n_pairs,
        evaluated_games=int((~excluded).sum()), predecision_excluded=int(excluded.sum()),
        a_wins=a_w, b_wins=b_w, draws=d,
        a_p0_wins=p0[0], a_p0_losses=p0[1], a_p0_draws=p0[2],
        a_p1_wins=p1[0], a_p1_losses=p1[1], a_p1_draws=p1[2],
        pair_wins=pw[0], pair_losses=pw[1], pair_draws=pw[2],
        mean_score_a=_mean(valid), mean_score_a_p0=_mean(s0[v0]), mean_score_a_p1=_mean(s1[v1]),
        mean_pair_score_a=mean_pair, pair_score_std=std, pair_score_se=se,
        pair_score_ci95_low=mean_pair - half, pair_score_ci95_high=mean_pair + half,
        terminal=int((~final_nagari).sum()), nagari=int(final_nagari.sum()),
        decision_steps=decision_steps, seconds=seconds)
