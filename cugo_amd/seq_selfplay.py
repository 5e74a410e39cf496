"""GPU-resident self-play of the event-sequence policy on the HIP engine.

`SeqPolicy` is the inference half of the reference's `SeqNet` (python/cugo_seq50.py:131-323)
in either query form: "hybrid" (query token = the 720 features + the 179-bit legal mask)
or "events" (the 171 context columns `CONTEXT_INDEX` + the mask).  It keeps
the same submodules and parameter names (`event_in`, `start_in`, `query_in`, `position`,
`token_type`, `encoder`, `norm`, `head`), so a reference state_dict loads into it.  Its
opening and event tokens are HIP kernels (`start_tokens`, `event_tokens`): each row sums
the Linear weight columns of its token's set bits instead of materialising the 0/1 token
and running a GEMM, with the reference's bf16 roundings.  `cached_step` appends the new
key/value and attends in one HIP launch per layer (`seq_decode.cached_step`).

`SelfPlayWave` is the reference's `WaveCollector` (python/cugo_seq_selfplay50.py:36-238),
frozen-opponent pool included: a wave of games advances one decision per step -
observe, one query token per game on the mover's cache row, readout, masked Gumbel-max
sampling (a HIP kernel on the uniforms torch draws), the engine step with its event
record, one event token per seat appended to the caches - and the whole step is captured
once as a HIP graph and replayed.  The policy runs in its weights' dtype (bf16 or fp32)
with no autocast.
"""

from __future__ import annotations

import torch
from torch import nn

from .cugo_torch50_ext import load_extension
from .seq_decode import KVCache, cached_step

FEATURES = 720
ACTIONS = 179
EVENT_WORDS = 9
START_WORDS = 8
MAX_EVENTS = 48                       # cugo_seq50.py:37
EVENT_IN = 8 * 50 + 12 + 2            # cugo_seq50.py:40
START_IN = 5 * 50 + 12 + 8 + 4        # cugo_seq50.py:41
STOP_POINTS_COLUMN = 471              # cugo_contract50.py:31
# Events-mode query columns (cugo_contract50.py:34-36): the v3 decision context, own
# hand, table counts and the round multiplier.
CONTEXT_V3 = [*range(200, 250), *range(396, 453), *range(471, 476), 552]
CONTEXT_INDEX = [*CONTEXT_V3, *range(0, 50), *range(491, 496), 557, 710, 711]
SIGNED_GOLDEN = -7046029254386353131  # cugo_ppo_nets50.py:11
SEED_BASE = 0x243F6A8885A308D3        # cugo_ppo_nets50.py:12


def make_seeds(batch: int, offset: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """Deal seeds and first players of games offset .. offset + batch - 1
    (cugo_ppo_nets50.py:15-17)."""
    index = torch.arange(batch, dtype=torch.int64, device=device)
    return index.mul(SIGNED_GOLDEN).add(SEED_BASE + offset), index.bitwise_and(1)


def stop_points(features: torch.Tensor) -> torch.Tensor:
    """Settled points of stopping now, from the fp32 features (cugo_contract50.py:40-42)."""
    return torch.round(torch.exp2(12.0 * features[:, STOP_POINTS_COLUMN].float()) - 1.0).long()


class SeqPolicy(nn.Module):
    """SeqNet for incremental inference: start/event/query tokens, the cached decoder step
    and the readout head.  mode "hybrid": the query carries all 720 features; "events":
    only the CONTEXT_INDEX columns (cugo_seq50.py:143-150)."""

    def __init__(self, mode: str = "hybrid", outputs: int = ACTIONS, d_model: int = 256,
                 layers: int = 4, heads: int = 8) -> None:
        super().__init__()
        if mode not in ("hybrid", "events"):
            raise ValueError("mode must be hybrid or events")
        self.mode = mode
        d = d_model
        width = FEATURES if mode == "hybrid" else len(CONTEXT_INDEX)
        self.register_buffer("context_index", torch.tensor(CONTEXT_INDEX), persistent=False)
        self.event_in = nn.Linear(EVENT_IN, d)
        self.start_in = nn.Linear(START_IN, d)
        self.query_in = nn.Sequential(nn.Linear(width + ACTIONS, 2 * d), nn.GELU(),
                                      nn.Linear(2 * d, d))
        self.position = nn.Parameter(torch.zeros(MAX_EVENTS + 1, d))
        self.token_type = nn.Parameter(torch.zeros(3, d))
        nn.init.normal_(self.position, std=0.02)
        nn.init.normal_(self.token_type, std=0.02)
        layer = nn.TransformerEncoderLayer(d, heads, 4 * d, dropout=0.0, activation="gelu",
                                           batch_first=True, norm_first=True)
        self.encoder = nn.TransformerEncoder(layer, layers, enable_nested_tensor=False)
        self.norm = nn.LayerNorm(d)
        self.head = nn.Sequential(nn.Linear(d, d), nn.GELU(), nn.Linear(d, outputs))
        self._ext = None
        self._transposed: dict[str, tuple[tuple, torch.Tensor]] = {}

    # -- token kernels ---------------------------------------------------------------

    def ext(self):
        if self._ext is None:
            self._ext = load_extension()
        return self._ext

    def _weight_t(self, name: str) -> torch.Tensor:
        """The Linear weight transposed to [in, d] (the kernels' column layout), refreshed
        when the weight changes (in-place updates bump its version) into the same buffer,
        so a captured HIP graph reads the new weights."""
        w = getattr(self, name).weight
        key = (w.data_ptr(), w._version)
        hit = self._transposed.get(name)
        if (hit is None or hit[1].dtype != w.dtype or hit[1].device != w.device
                or hit[1].shape != (w.shape[1], w.shape[0])):
            hit = (key, w.detach().t().contiguous())
        elif hit[0] != key:
            hit[1].copy_(w.detach().t())
            hit = (key, hit[1])
        self._transposed[name] = hit
        return hit[1]

    def prepare(self) -> None:
        """Build the transposed token weights now (before a HIP-graph capture)."""
        self._weight_t("event_in")
        self._weight_t("start_in")

    def start_token(self, start: torch.Tensor, seat: torch.Tensor) -> torch.Tensor:
        """cugo_seq50.py:271-274: start_in(encode_start) + position[0] + token_type[0]."""
        return self.ext().start_tokens(start.contiguous(), seat.contiguous(),
                                       self._weight_t("start_in"), self.start_in.bias.detach(),
                                       self.position.detach(), self.token_type.detach())

    def event_token(self, words: torch.Tensor, seat: torch.Tensor,
                    index: torch.Tensor) -> torch.Tensor:
        """cugo_seq50.py:276-282: event_in(encode_events) + position[1 + min(index, 47)]
        + token_type[1].  Row r reads words[r % len(words)] and index[r % len(words)], so one
        copy of the events serves every seat that observes them."""
        return self.ext().event_tokens(words.contiguous(), seat.contiguous(), index.contiguous(),
                                       self._weight_t("event_in"), self.event_in.bias.detach(),
                                       self.position.detach(), self.token_type.detach())

    def query_token(self, features: torch.Tensor, legal: torch.Tensor) -> torch.Tensor:
        """cugo_seq50.py:166-180: query_in(features ++ legal) + token_type[2]; events mode
        keeps the CONTEXT_INDEX columns of 720-wide features."""
        if self.mode == "events" and features.shape[-1] == FEATURES:
            features = features.index_select(-1, self.context_index)
        dt = self.event_in.weight.dtype
        return self.query_from_input(torch.cat((features.to(dt), legal.to(dt)), -1))

    def kept_columns(self) -> list[int] | None:
        """Feature columns a rollout keeps for this mode (cugo_seq50.py:342-344)."""
        return None if self.mode == "hybrid" else CONTEXT_INDEX

    def query_from_input(self, q_in: torch.Tensor) -> torch.Tensor:
        """query_token on the already concatenated input [n, 720 + 179]."""
        return self.query_in(q_in) + self.token_type[2]

    def readout(self, h: torch.Tensor) -> torch.Tensor:
        """cugo_seq50.py:187-189 and :288-289."""
        out = self.head(self.norm(h))
        return out.squeeze(-1) if out.shape[-1] == 1 else out

    def cached_step(self, cache: KVCache, x: torch.Tensor, slots: int | None = None,
                    rows: torch.Tensor | None = None) -> torch.Tensor:
        """cugo_seq50.py:291-322, the append and decode of each layer in one HIP launch."""
        return cached_step(self, cache, x, slots, rows)


def policy_cache(policy: SeqPolicy, rows: int, device, slots: int = MAX_EVENTS + 2) -> KVCache:
    """The reference's KVCache(model, rows) (cugo_seq50.py:325-339): opening + events + one
    scratch slot for the query, bf16, head-major."""
    layers = len(policy.encoder.layers)
    heads = policy.encoder.layers[0].self_attn.num_heads
    d = policy.position.shape[1]
    return KVCache(layers, rows, heads, d, slots, torch.device(device))


class SelfPlayWave:
    """Self-play of `wave` games at a time, one HIP graph per decision step
    (WaveCollector, cugo_seq_selfplay50.py:36-238).  With an opponent and pool_games > 0,
    games 0 .. pool_games - 1 of a wave played with `pool=True` put the frozen opponent on
    the seat the learner does not hold."""

    def __init__(self, ext, actor: SeqPolicy, wave: int, max_steps: int = 64,
                 opponent: SeqPolicy | None = None, pool_games: int = 0) -> None:
        device = next(actor.parameters()).device
        if not 0 <= pool_games <= wave:
            raise ValueError(f"pool_games ({pool_games}) must lie in [0, {wave}]")
        if opponent is not None and opponent.kept_columns() != actor.kept_columns():
            # both read the one query input the step builds from the kept columns
            raise ValueError("the opponent's query mode must be the actor's")
        self.ext, self.actor, self.w, self.max_steps = ext, actor, wave, max_steps
        self.opponent, self.p = opponent, (pool_games if opponent is not None else 0)
        w = wave
        self.ids = torch.arange(w, device=device)
        self.seats2 = torch.cat((torch.zeros(w, dtype=torch.int64, device=device),
                                 torch.ones(w, dtype=torch.int64, device=device)))
        seeds, first = make_seeds(w, 0, device)
        self.states = ext.create(seeds, first)
        self.events = torch.zeros((w, MAX_EVENTS, EVENT_WORDS), dtype=torch.int64, device=device)
        self.count = torch.zeros(w, dtype=torch.int64, device=device)
        self.start = torch.zeros((w, START_WORDS), dtype=torch.int64, device=device)
        self.learner_seat = torch.zeros(w, dtype=torch.int64, device=device)
        self.cache = policy_cache(actor, 2 * w, device)  # row = seat * w + game
        # row = pool game (the opponent's seat)
        self.opp_cache = (policy_cache(opponent, max(1, self.p), device)
                          if opponent is not None else None)
        cols = actor.kept_columns()
        self.columns = (None if cols is None
                        else torch.tensor(cols, dtype=torch.int32, device=device))
        width = FEATURES if cols is None else len(cols)
        s = max_steps
        self.rec_features = torch.zeros((s, w, width), dtype=torch.bfloat16, device=device)
        self.rec_legal = torch.zeros((s, w, ACTIONS), dtype=torch.bool, device=device)
        self.rec_logp = torch.zeros((s, w), dtype=torch.float32, device=device)
        self.rec_long = {name: torch.zeros((s, w), dtype=torch.int64, device=device)
                         for name in ("actions", "opp_hand", "stock", "stop_points", "seat",
                                      "count")}
        self.rec_valid = torch.zeros((s, w), dtype=torch.bool, device=device)
        self.step_index = torch.zeros(1, dtype=torch.int64, device=device)
        self.final_reward0 = torch.zeros(w, device=device)
        self.final_nagari = torch.zeros(w, dtype=torch.bool, device=device)
        self.finished = torch.zeros(w, dtype=torch.bool, device=device)
        self.started = torch.zeros(w, dtype=torch.bool, device=device)
        self.bad = torch.zeros((), dtype=torch.int64, device=device)
        self.ok = int(ext.STATUS_OK)
        def native(pool_games: int):
            return ext.SelfPlayState(
                w, s, self.step_index, self.count, self.events, self.cache.length,
                self.final_reward0, self.final_nagari, self.finished, self.bad,
                self.rec_features, self.rec_legal, self.rec_logp, self.rec_long["actions"],
                self.rec_long["opp_hand"], self.rec_long["stock"], self.rec_long["stop_points"],
                self.rec_long["seat"], self.rec_long["count"], self.rec_valid, self.columns,
                pool_games, self.learner_seat,
                None if self.opp_cache is None else self.opp_cache.length)
        self.native = {False: native(0)}
        if self.p > 0:
            self.native[True] = native(self.p)
        # Sampling noise: None draws torch.rand_like inside the step (the reference's
        # choice); a tensor [wave, ACTIONS] is read instead (set by a caller that draws
        # its own uniforms before each step).
        self.noise: torch.Tensor | None = None
        self.graph: torch.cuda.CUDAGraph | None = None
        self.graph_pool: bool | None = None
        self.logits: torch.Tensor | None = None

    @torch.no_grad()
    def reset(self, seeds: torch.Tensor, first: torch.Tensor, learner_seat: torch.Tensor,
              pool: bool = False) -> None:
        """cugo_seq_selfplay50.py:78-106."""
        self.states.copy_(self.ext.create(seeds, first))
        self.start.copy_(self.ext.start(self.states))
        self.events.zero_()
        self.count.zero_()
        self.learner_seat.copy_(learner_seat)
        done = self.ext.observe_indexed(self.states, self.ids)[3]
        self.started.copy_(~done)
        self.finished.copy_(done)
        self.final_reward0.zero_()
        self.final_nagari.zero_()
        self.bad.zero_()
        self.step_index.zero_()
        self.rec_valid.zero_()
        self.cache.length.zero_()
        actor = self.actor
        actor.cached_step(self.cache, actor.start_token(self.start.repeat(2, 1), self.seats2), 1)
        self.cache.length.fill_(1)
        if pool and self.p > 0:
            p, opp = self.p, self.opponent
            self.opp_cache.length.zero_()
            opp.cached_step(self.opp_cache, opp.start_token(self.start[:p], 1 - self.learner_seat[:p]), 1)
            self.opp_cache.length.fill_(1)

    @torch.no_grad()
    def step(self, pool: bool = False) -> None:
        """One decision of every game (cugo_seq_selfplay50.py:108-163).  The torch
        bookkeeping around the policy runs as two kernels (`SelfPlayState.prepare` before
        the query, `.advance` after the event tokens)."""
        ids, actor, ext = self.ids, self.actor, self.ext
        pool = pool and self.p > 0
        native = self.native[pool]
        features, legal, players, done, status = ext.observe_indexed(self.states, ids)
        stock = ext.stock_indexed(self.states, ids)
        q_in, query_rows = native.prepare(self.states, features, legal, players, done, status,
                                          stock, actor.event_in.weight.dtype)
        hidden = actor.cached_step(self.cache, actor.query_from_input(q_in), rows=query_rows)
        logits = actor.readout(hidden)  # the kernel reads bf16 logits as the fp32 .float()
        if pool:
            # the opponent answers every pool game; its logits count where it moves
            p, opp = self.p, self.opponent
            opp_logits = opp.readout(opp.cached_step(self.opp_cache, opp.query_from_input(q_in[:p])))
            opp_move = players[:p].long() != self.learner_seat[:p]
            logits = torch.cat((torch.where(opp_move.unsqueeze(1), opp_logits.to(logits.dtype),
                                            logits[:p]), logits[p:]))
        self.logits = logits  # the last step's logits (kept for inspection)
        uniforms = (torch.rand(logits.shape, dtype=torch.float32, device=logits.device)
                    if self.noise is None else self.noise)
        actions, logp = ext.gumbel_sample(logits.contiguous(), legal, uniforms)
        reward0, new_done, nagari, step_status, committed, events = ext.step_events_indexed(
            self.states, ids, actions)
        actor.cached_step(self.cache, actor.event_token(events, self.seats2, self.count))
        if pool:
            opp = self.opponent
            opp.cached_step(self.opp_cache, opp.event_token(events[:p], 1 - self.learner_seat[:p],
                                                            self.count[:p]))
        native.advance(done, reward0, new_done, nagari, step_status, committed, events, actions,
                       logp)
        self.step_index += 1

    @torch.no_grad()
    def capture(self, pool: bool = False) -> None:
        """Record step(pool) once as a HIP graph (cugo_seq_selfplay50.py:165-180)."""
        pool = pool and self.p > 0
        if self.graph is not None and self.graph_pool == pool:
            return
        self.graph = None
        self.actor.prepare()
        if self.opponent is not None:
            self.opponent.prepare()
        seeds, first = make_seeds(self.w, 0, self.states.device)
        self.reset(seeds, first, torch.zeros_like(self.learner_seat), pool)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):  # warm-up (GEMM handles, allocator) outside the capture
                self.step(pool)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self.step(pool)
        self.graph, self.graph_pool = graph, pool

    @torch.no_grad()
    def play(self, seeds: torch.Tensor, first: torch.Tensor, learner_seat: torch.Tensor,
             pool: bool = False) -> int:
        """Plays one wave to the end by replaying the captured step; returns the number of
        steps replayed (cugo_seq_selfplay50.py:203-219)."""
        self.capture(pool)
        self.reset(seeds, first, learner_seat, pool)
        for k in range(self.max_steps):
            self.graph.replay()
            if (k + 1) % 4 == 0 and k + 1 >= 16 and bool(self.finished.all()):
                steps = k + 1
                break
        else:
            if not bool(self.finished.all()):
                raise RuntimeError(f"games did not finish within {self.max_steps} steps")
            steps = self.max_steps
        if int(self.bad):
            raise RuntimeError(f"{int(self.bad)} bad observe/step results in a wave")
        if int(self.count.max()) > MAX_EVENTS:
            raise RuntimeError("event log overflow")
        return steps

    @torch.no_grad()
    def collect(self, games: int, seed_offset: int, opponent_state: dict | None = None) -> dict:
        """Plays `games` games, a multiple of the wave (cugo_seq_selfplay50.py:182-238).
        With opponent_state (loaded into the opponent in place, so the captured step keeps
        its pointers) the first pool_games of every wave face it.  Returns the outcomes
        the reference returns, plus what it hands its rollout storage and event log: the
        learner's decisions step-major within each wave (`decisions`) and every game's
        event log, count and opening (`log`)."""
        if games % self.w:
            raise ValueError(f"games ({games}) must be a multiple of the wave size ({self.w})")
        device = self.states.device
        pool = opponent_state is not None and self.p > 0
        if pool:
            self.opponent.load_state_dict(opponent_state)
            self.opponent.prepare()
        seeds, first = make_seeds(games, seed_offset, device)
        learner_seat = torch.randint(2, (games,), device=device)
        vs_pool = torch.zeros(games, dtype=torch.bool, device=device)
        final_reward0 = torch.zeros(games, device=device)
        final_nagari = torch.zeros(games, dtype=torch.bool, device=device)
        started = torch.zeros(games, dtype=torch.bool, device=device)
        log = {"events": torch.zeros((games, MAX_EVENTS, EVENT_WORDS), dtype=torch.int64,
                                     device=device),
               "count": torch.zeros(games, dtype=torch.int64, device=device),
               "start": torch.zeros((games, START_WORDS), dtype=torch.int64, device=device)}
        parts: dict[str, list[torch.Tensor]] = {k: [] for k in (
            "features", "legal", "actions", "logp", "opp_hand", "stock", "stop_points",
            "env_ids", "seat", "count")}
        steps = 0
        for offset in range(0, games, self.w):
            part = slice(offset, offset + self.w)
            steps = max(steps, self.play(seeds[part], first[part], learner_seat[part], pool))
            at = torch.nonzero(self.rec_valid)  # step-major: decisions stay in game order
            s_idx, g_idx = at[:, 0], at[:, 1]
            parts["features"].append(self.rec_features[s_idx, g_idx])
            parts["legal"].append(self.rec_legal[s_idx, g_idx])
            parts["logp"].append(self.rec_logp[s_idx, g_idx])
            parts["env_ids"].append(offset + g_idx)
            for name in ("actions", "opp_hand", "stock", "stop_points", "seat", "count"):
                parts[name].append(self.rec_long[name][s_idx, g_idx])
            log["events"][part] = self.events
            log["count"][part] = self.count
            log["start"][part] = self.start
            final_reward0[part] = self.final_reward0
            final_nagari[part] = self.final_nagari
            started[part] = self.started
            if pool:
                vs_pool[offset:offset + self.p] = True
        return {"final_reward0": final_reward0, "final_nagari": final_nagari,
                "started": started, "learner_seat": learner_seat, "vs_pool": vs_pool,
                "steps": steps, "decisions": {k: torch.cat(v) for k, v in parts.items()},
                "log": log}
