"""Paired evaluation on the HIP engine (python/cugo_eval50.py:137-361, `evaluate_paired`).

Every deal is played twice, model A on seat 0 in game i and on seat 1 in game pairs + i,
so deal luck cancels in the pair score.  A decision step observes the games, evaluates
each model, takes for every game the greedy action of the model whose seat moves (the
`masked_argmax` kernel: argmax of the fp32 logits with illegal actions at -1e30) or a
sample from its softmax, and steps the engine; finished games stay resident, masked.
Summary fields and their meaning are the reference's `EvalSummary`
(cugo_eval50.py:27-61).

Two kinds of policy, as in the reference (`policy_logits`, cugo_seq50.py:347-365):

* features-only modules mapping the [n, 720] features to logits (or a tuple whose first
  item is the logits), like the reference's PpoActor, under fp16 autocast with use_amp;
* sequence policies (`uses_history`, cugo_amd.seq_selfplay.SeqPolicy, into which a
  reference SeqNet state_dict loads), run in bf16 with use_amp as the reference does
  (cugo_eval50.py:120-121).  The reference builds a History of every game's opening and
  committed events (cugo_eval50.py:169, :258-263) and runs the dense forward over
  [opening, events, query] for each mover (`SeqNet.forward`, cugo_seq50.py:208-224).  Here
  each sequence policy keeps one KV-cache row per game, for the seat it plays there: the
  opening token at slot 0, one event token per committed event of either seat (its own
  view of it), and each step a query token in the slot after them.  A step's event
  tokens go through the layers with the next step's queries, in one pass
  (`cached_step_pair`), as the sequence self-play does; incremental decoding computes
  what the dense forward computes at the query.  A policy's pass keeps the queries of its
  movers only (`paired_movers`): the others' rows are skipped by the decode, as the
  reference feeds each model its movers (cugo_eval50.py:130-135).
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass

import torch
from torch import nn

from .seq_selfplay import MAX_EVENTS, make_seeds


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


def _choose(ext, logits: torch.Tensor, legal: torch.Tensor, sample: bool) -> torch.Tensor:
    """The greedy action (argmax of the legal logits as float32) or a softmax sample
    (cugo_eval50.py:124-127)."""
    if sample:
        masked = logits.float().masked_fill(~legal, -1.0e30)
        return torch.multinomial(torch.softmax(masked, dim=1), 1).squeeze(1)
    return ext.masked_argmax(logits.contiguous(), legal)


class _SequenceSeat:
    """A sequence policy's part of the resident games: one KV-cache row per game for the
    seat the policy plays in it (`seat`), the rows of the step's pass (the last step's
    event tokens in [0, games), this step's queries in [games, 2 games)), the slots the
    waiting event tokens go to, and the query input rows (features ++ legal in the policy
    dtype, zero-padded to a width `linear` takes)."""

    def __init__(self, model: nn.Module, seat: torch.Tensor, games: int, dev,
                 q_inputs: dict) -> None:
        from .seq_selfplay import ACTIONS, FEATURES, policy_cache

        for name in ("query_from_input", "event_token", "start_token", "readout", "prepare"):
            if not hasattr(model, name):
                raise TypeError("a sequence policy must be a cugo_amd.seq_selfplay.SeqPolicy "
                                "(a reference SeqNet state_dict loads into one)")
        self.model, self.seat, self.games = model, seat, games
        dtype = model.event_in.weight.dtype
        d = model.position.shape[1]
        self.cache = policy_cache(model, games, dev)
        self.pair = torch.zeros((2 * games, d), dtype=dtype, device=dev)
        self.pair_h = torch.zeros_like(self.pair)  # norm1 of the rows, from their launches
        # slots of the waiting event tokens and of the next queries; -1 skips a row (an
        # event not kept, the query of a game that is over)
        self.event_pos = torch.full((games,), -1, dtype=torch.int64, device=dev)
        self.query_pos = torch.full((games,), -1, dtype=torch.int64, device=dev)
        cols = model.kept_columns()
        width = FEATURES if cols is None else len(cols)
        need = width + ACTIONS
        stride = next((k for k in (64, 128, 256, 512, 1024) if k >= need), need)
        # the query input rows, shared by the policies that read the same columns in the
        # same dtype (filled once a step)
        key = (None if cols is None else tuple(cols), dtype, stride)
        if key not in q_inputs:
            q_inputs[key] = (None if cols is None else
                             torch.tensor(cols, dtype=torch.int32, device=dev),
                             torch.zeros((games, stride), dtype=dtype, device=dev))
        self.columns, self.q_in = q_inputs[key]
        self.ids = torch.arange(games, device=dev)
        model.prepare()

    def open(self, start: torch.Tensor, active: torch.Tensor) -> None:
        """Every game's opening token (cugo_seq50.py:271-274, seen from `seat`) into slot 0;
        no event waits, and the first queries go to slot 1 of the games being played."""
        m, cache = self.model, self.cache
        cache.length.zero_()
        m.cached_step(cache, m.start_token(start, self.seat), 1)
        cache.length.fill_(1)
        self.event_pos.fill_(-1)
        torch.where(active, cache.length, torch.full_like(cache.length, -1), out=self.query_pos)

    def logits(self) -> torch.Tensor:
        """The last step's kept event tokens and the query of every game still being played
        whose mover sits in this policy's seat (its input rows in `q_in`, filled this step)
        through the layers together (the queries attend the events' keys at every layer),
        then the readout of the queries: [games, 179] logits in the policy dtype (NaN in the
        rows of the other games, whose rows the decode skips: no cache read or write;
        nothing reads those logits)."""
        from .seq_decode import cached_step_pair

        m, g = self.model, self.games
        m.query_from_input(self.q_in, out=self.pair[g:], norm_out=self.pair_h[g:])
        hidden, normed = cached_step_pair(m, self.cache, self.pair, g, self.event_pos,
                                          self.query_pos, self.ids, final_norm=m.norm,
                                          h=self.pair_h)
        return m.readout(hidden, normed)  # the queries' (the events' are not kept)

    def events(self, events: torch.Tensor, count: torch.Tensor) -> None:
        """This step's event tokens, each game's from `seat`'s view at position 1 + count
        (cugo_seq50.py:276-282), waiting for the next step's pass."""
        self.model.event_token(events, self.seat, count, out=self.pair[:self.games],
                               norm_out=self.pair_h[:self.games])


def _bf16_twin(model: nn.Module) -> nn.Module:
    """The policy in bf16: fp16 autocast is not used for sequence models, which run in
    bf16 (cugo_eval50.py:120-121); parameters that are bf16 already are kept as they are."""
    import copy

    if next(model.parameters()).dtype == torch.bfloat16:
        return model
    return copy.deepcopy(model).to(torch.bfloat16).eval()


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
                    sample_b: bool = False, graph: bool = True,
                    trace: list | None = None) -> EvalSummary:
    """cugo_eval50.py:137-361 on resident games: every step observes all 2 pairs games,
    evaluates both models on every row, keeps model A's action where A's seat moves and
    B's elsewhere, and steps every game; rows of games that are over are masked out of
    the outcome and the checks (the reference drops them instead, which needs the count of
    survivors on the host every step).  The per-row decisions are the reference's; the
    step is one HIP-graph replay (greedy policies; `graph=False` or sampling: eager), and
    the host reads whether games are left one step behind, so the GPU never waits.
    Either model may be a sequence policy (`uses_history`, a SeqPolicy).  `trace`, when
    given, receives one dict a decision step: copies of every game's chosen action and
    of both models' logits ("actions", "logits_a", "logits_b")."""
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
    same = model_b is model_a
    seq = [bool(getattr(m, "uses_history", False)) for m in (model_a, model_b)]
    if use_amp:
        # features-only policies: the Linear weights cast to fp16 once; sequence
        # policies: bf16 (cugo_eval50.py:120-121)
        model_a = _bf16_twin(model_a) if seq[0] else _half_linears(model_a)
        model_b = model_a if same else (_bf16_twin(model_b) if seq[1] else
                                        _half_linears(model_b))
    # Sequence policies keep their event histories as KV caches, one row per game for the
    # seat they play (A: a_seat, B: the other); both models may be one module.
    ids = torch.arange(games, device=dev)
    q_inputs: dict = {}  # (columns, dtype, stride) -> (int32 columns, query input rows)
    seq_seats = [(_SequenceSeat(m, a_seat if k == 0 else 1 - a_seat, games, dev, q_inputs)
                  if seq[k] else None) for k, m in enumerate((model_a, model_b))]
    histories = [s for s in seq_seats if s is not None]
    count = torch.zeros(games, dtype=torch.int64, device=dev)  # committed events per game
    start = ext.start(states) if histories else None  # the openings (History, cugo_seq50.py:56)

    any_active = torch.zeros(1, dtype=torch.int32, device=dev)  # set in a step, counted after
    playing = torch.zeros(1, dtype=torch.int32, device=dev)  # 1 after a step with games left

    last: dict[str, torch.Tensor] = {}  # the latest step's outputs, for `trace`

    def logits_actions(k: int, model, features, legal, sample: bool):
        if seq_seats[k] is not None:
            logits = seq_seats[k].logits()
        else:
            with torch.autocast(device_type="cuda", dtype=torch.float16, enabled=use_amp):
                out = model(features)
            logits = (out[0] if isinstance(out, tuple) else out).float()
        last[("logits_a", "logits_b")[k]] = logits
        return _choose(ext, logits, legal, sample)

    def step() -> None:
        # the checks, the count and the per-game choice of model are one launch before the
        # step and one after it (paired_select / paired_update, selfplay.hip)
        features, legal, players, done, status = ext.observe(states)
        for columns, q_in in q_inputs.values():  # the sequence policies' query input rows
            ext.query_input(features, legal, columns, q_in)
        for h in histories:  # a sequence policy answers for its movers only (the others'
            ext.paired_movers(players, h.seat, h.query_pos)  # queries are skipped)
        act_a = logits_actions(0, model_a, features, legal, sample_a)
        act_b = logits_actions(1, model_b, features, legal, sample_b)
        actions = ext.paired_select(active, status, done, legal.any(1), players, a_seat, act_a,
                                    act_b, bad, any_active, playing)
        last["actions"] = actions
        if histories:
            reward0, new_done, nagari, step_status, committed, events = (
                ext.step_events_indexed(states, ids, actions))
            for h in histories:
                h.events(events, count)
            slots = [x for h in histories for x in (h.cache.length, h.event_pos, h.query_pos)]
            ext.paired_events(active, step_status, committed, new_done, count, *slots)
        else:
            reward0, new_done, nagari, step_status, _ = ext.step(states, actions)
        ext.paired_update(active, step_status, new_done, reward0, nagari, final_reward0,
                          final_nagari, bad, any_active, steps_dev.view(1), playing)

    replay = step
    flags = torch.zeros(2, dtype=torch.int32, pin_memory=True)
    with torch.inference_mode():
        if graph and not (sample_a or sample_b):
            # warm-up steps on a side stream (library handles, allocator blocks), then the
            # capture; the state they touched is put back
            kept = [states, final_reward0, final_nagari, active, bad, steps_dev, any_active,
                    count]
            for h in histories:
                kept += [h.cache.length, h.event_pos, h.query_pos, h.pair]
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
        for h in histories:
            h.open(start, active)
        stream = torch.cuda.current_stream()
        finished_all = False
        behind = None  # (event, flag slot) of the step before the latest
        for k in range(max_steps):
            replay()
            if trace is not None:
                trace.append({name: t.clone() for name, t in last.items()})
            flags[k & 1].copy_(playing[0], non_blocking=True)
            queued = (torch.cuda.Event(), k & 1)
            queued[0].record(stream)
            if behind is not None:
                behind[0].synchronize()
                if not int(flags[behind[1]]):
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
    if histories and int(count.max()) > MAX_EVENTS:
        raise RuntimeError(f"a game committed more than {MAX_EVENTS} events")

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
