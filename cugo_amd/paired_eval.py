"""Paired evaluation on the HIP engine (python/cugo_eval50.py:137-361, `evaluate_paired`).

Every deal is played twice, model A on seat 0 in game i and on seat 1 in game pairs + i,
so deal luck cancels in the pair score.  A decision step observes the games, evaluates
each model, takes for every game the greedy action of the model whose seat moves (the
`masked_argmax` kernel: argmax of the fp32 logits with illegal actions at -1e30) or a
sample from its softmax, and steps the engine; finished games stay resident, masked.  Summary fields and
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


def _half_linears(model: nn.Module) -> nn.Module:
    """A copy of `model` whose nn.Linear weights and biases are already float16: under fp16
    autocast a Linear casts them at every call (a cast launch per parameter and step), to
    exactly these values, so the copy computes what the model computes without them."""
    import copy

    twin = copy.deepcopy(model)
    for m in twin.modules():
        if isinstance(m, nn.Linear):
            m.weight.data = m.weight.data.half()
            if m.bias is not None:
                m.bias.data = m.bias.data.half()
    return twin


def _wdl(x: torch.Tensor) -> tuple[int, int, int]:
    return int((x > 0).sum()), int((x < 0).sum()), int((x == 0).sum())


def _mean(x: torch.Tensor) -> float:
    return float(x.mean()) if x.numel() else 0.0


def evaluate_paired(ext, model_a: nn.Module, model_b: nn.Module, pairs: int, seed_offset: int,
                    max_steps: int, use_amp: bool, sample_a: bool = False,
                    sample_b: bool = False, graph: bool = True) -> EvalSummary:
    """cugo_eval50.py:137-361 on resident games: every step observes all 2 pairs games,
    evaluates both models on every row, keeps model A's action where A's seat moves and
    B's elsewhere, and steps every game; rows of games that are over are masked out of
    the outcome and the checks (the reference drops them instead, which needs the count of
    survivors on the host every step).  The per-row decisions are the reference's; the
    step is one HIP-graph replay (greedy policies; `graph=False` or sampling: eager), and
    the host reads whether games are left one step behind, so the GPU never waits."""
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
    active = torch.zeros(games, dtype=torch.bool, device=dev)   # games still being played
    bad = torch.zeros(3, dtype=torch.int64, device=dev)  # observe, legal, step
    steps_dev = torch.zeros((), dtype=torch.int64, device=dev)  # decision steps
    ok = int(ext.STATUS_OK)
    model_a.eval()
    model_b.eval()
    if use_amp:
        same = model_b is model_a
        model_a = _half_linears(model_a)
        model_b = model_a if same else _half_linears(model_b)

    any_active = torch.zeros(1, dtype=torch.int32, device=dev)  # set in a step, counted after

    def step() -> None:
        # the checks, the count and the per-game choice of model are one launch before the
        # step and one after it (paired_select / paired_update, selfplay.hip)
        features, legal, players, done, status = ext.observe(states)
        act_a = _actions(ext, model_a, features, legal, use_amp, sample_a)
        act_b = _actions(ext, model_b, features, legal, use_amp, sample_b)
        actions = ext.paired_select(active, status, done, legal.any(1), players, a_seat, act_a,
                                    act_b, bad, any_active)
        reward0, new_done, nagari, step_status, _ = ext.step(states, actions)
        ext.paired_update(active, step_status, new_done, reward0, nagari, final_reward0,
                          final_nagari, bad, any_active, steps_dev.view(1))

    replay = step
    flags = torch.zeros(2, dtype=torch.bool, pin_memory=True)
    with torch.inference_mode():
        if graph and not (sample_a or sample_b):
            # warm-up steps on a side stream (library handles, allocator blocks), then the
            # capture; the state they touched is put back
            kept = [states, final_reward0, final_nagari, active, bad, steps_dev, any_active]
            saved = [t.clone() for t in kept]
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                step()
                step()
            torch.cuda.current_stream().wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step()
            for t, v in zip(kept, saved):
                t.copy_(v)
            replay = g.replay
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        # the deal: games over already, or unplayable, leave the evaluation before step 0
        _, legal, _, done, status = ext.observe(states)
        fine = status == ok
        any_legal = legal.any(1)
        excluded.copy_(done)
        bad[0] += (~done & ~fine).sum()
        bad[1] += (~done & fine & ~any_legal).sum()
        active.copy_(~done & fine & any_legal)
        stream = torch.cuda.current_stream()
        finished_all = False
        behind = None  # (event, flag slot) of the step before the latest
        for k in range(max_steps):
            replay()
            flags[k & 1].copy_(active.any(), non_blocking=True)
            queued = (torch.cuda.Event(), k & 1)
            queued[0].record(stream)
            if behind is not None:
                behind[0].synchronize()
                if not bool(flags[behind[1]]):
                    finished_all = True
                    break
            behind = queued
        else:
            finished_all = not bool(active.any())
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0
    decision_steps = int(steps_dev)

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
