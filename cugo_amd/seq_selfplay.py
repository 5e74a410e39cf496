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
from .seq_decode import (KVCache, _fits_linear, add_norm, cached_step, cached_step_pair,
                         is_exact_gelu, linear, packed_weight, prepare_linears)

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

    uses_history = True  # cugo_seq50.py:134: callers feed it event histories

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
        """Build the transposed token weights and the packed encoder weights now (before a
        HIP-graph capture)."""
        self._weight_t("event_in")
        self._weight_t("start_in")
        prepare_linears(self)
        for lin in (self.head[0], self.head[2]):
            if lin.weight.dtype == torch.bfloat16 and lin.weight.is_cuda:
                packed_weight(lin.weight)

    def start_token(self, start: torch.Tensor, seat: torch.Tensor) -> torch.Tensor:
        """cugo_seq50.py:271-274: start_in(encode_start) + position[0] + token_type[0]."""
        return self.ext().start_tokens(start.contiguous(), seat.contiguous(),
                                       self._weight_t("start_in"), self.start_in.bias.detach(),
                                       self.position.detach(), self.token_type.detach())

    def _norm1(self) -> nn.Module:
        """The first encoder layer's norm1 (the pre-norm every token meets first)."""
        return self.encoder.layers[0].norm1

    def _fused_norm1(self) -> bool:
        """Whether the token launches can write norm1 of their tokens themselves: an
        affine LayerNorm over d in the tokens' dtype."""
        n1 = self._norm1()
        dt = self.event_in.weight.dtype
        return (isinstance(n1, nn.LayerNorm) and n1.weight is not None and n1.bias is not None
                and n1.weight.dtype == dt and n1.bias.dtype == dt
                and tuple(n1.normalized_shape) == (self.position.shape[1],))

    def event_token(self, words: torch.Tensor, seat: torch.Tensor, index: torch.Tensor,
                    out: torch.Tensor | None = None,
                    norm_out: torch.Tensor | None = None) -> torch.Tensor:
        """cugo_seq50.py:276-282: event_in(encode_events) + position[1 + min(index, 47)]
        + token_type[1].  Row r reads words[r % len(words)] and index[r % len(words)], so one
        copy of the events serves every seat that observes them.  Written into `out` when
        given; with `norm_out`, the first layer's norm1 of the tokens is written there too
        (in the same launch where the norm allows)."""
        fused = norm_out is not None and self._fused_norm1()
        n1 = self._norm1()
        x = self.ext().event_tokens(words.contiguous(), seat.contiguous(), index.contiguous(),
                                    self._weight_t("event_in"), self.event_in.bias.detach(),
                                    self.position.detach(), self.token_type.detach(), out,
                                    n1.weight.detach() if fused else None,
                                    n1.bias.detach() if fused else None,
                                    n1.eps if fused else 1e-5, norm_out if fused else None)
        if norm_out is not None and not fused:
            norm_out.copy_(add_norm(x, None, n1)[1])
        return x

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

    def query_from_input(self, q_in: torch.Tensor, out: torch.Tensor | None = None,
                         norm_out: torch.Tensor | None = None) -> torch.Tensor:
        """query_token on the already concatenated input [n, 720 + 179] (into `out` when
        given); q_in may carry zero columns past the input width (SelfPlayState.prepare's
        padded rows), so that the first layer and its GELU run as one `linear` launch.
        With `norm_out`, the first layer's norm1 of the tokens is written there too (in the
        second layer's launch where the shapes allow)."""
        first, act, second = self.query_in
        if is_exact_gelu(act):
            h = linear(q_in, first.weight, first.bias, gelu=True)
        else:
            h = act(linear(q_in, first.weight, first.bias))
        # + token_type[2] rounded after the layer's own rounding, as torch adds the two
        tt = self.token_type[2]
        if (norm_out is not None and self._fused_norm1() and tt.dtype == torch.bfloat16
                and second.weight.shape[0] == 256 and second.bias is not None
                and _fits_linear(h, second.weight, second.bias)):
            n1 = self._norm1()
            x, _ = self.ext().linear_add_layernorm(
                h, packed_weight(second.weight, h.shape[1]), second.bias.detach(), tt.detach(),
                n1.weight.detach(), n1.bias.detach(), n1.eps, out=out, ln_out=norm_out)
            return x
        x = linear(h, second.weight, second.bias, residual=tt, out=out)
        if norm_out is not None:
            norm_out.copy_(add_norm(x, None, self._norm1())[1])
        return x

    def readout(self, h: torch.Tensor, normed: torch.Tensor | None = None) -> torch.Tensor:
        """cugo_seq50.py:187-189 and :288-289: head(norm(h)), the norm as one HIP launch
        (or `normed`, norm(h) already computed), the head's first Linear with its GELU as
        another and its output Linear as a third where they fit."""
        if h.dim() == 2 and is_exact_gelu(self.head[1]):
            z = add_norm(h, None, self.norm)[1] if normed is None else normed
            u = linear(z, self.head[0].weight, self.head[0].bias, gelu=True)
            out = linear(u, self.head[2].weight, self.head[2].bias)
        else:
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


DONE_BYTE = 239  # TorchEnv50::done (torch50.h:108-121)
RECORD_LONG = ("actions", "opp_hand", "stock", "stop_points", "seat", "count")


class _WaveTensors:
    """Every device tensor of one wave of `w` games, made from one table of names, shapes
    and dtypes; `per_wave` lists those a new wave starts from zero."""

    def __init__(self, w: int, steps: int, width: int, device) -> None:
        i64, b, f32 = torch.int64, torch.bool, torch.float32
        table = {
            "events": ((w, MAX_EVENTS, EVENT_WORDS), i64), "count": ((w,), i64),
            "start": ((w, START_WORDS), i64), "learner_seat": ((w,), i64),
            "rec_features": ((steps, w, width), torch.bfloat16),
            "rec_legal": ((steps, w, ACTIONS), b), "rec_logp": ((steps, w), f32),
            "rec_valid": ((steps, w), b), "step_index": ((2,), i64),
            "final_reward0": ((w,), f32), "final_nagari": ((w,), b), "finished": ((w,), b),
            "started": ((w,), b), "bad": ((), i64),
        }
        for name, (shape, dtype) in table.items():
            setattr(self, name, torch.zeros(shape, dtype=dtype, device=device))
        self.rec_long = {k: torch.zeros((steps, w), dtype=i64, device=device) for k in RECORD_LONG}
        self.per_wave = [self.events, self.count, self.rec_valid, self.step_index,
                         self.final_reward0, self.final_nagari, self.bad]


class SelfPlayWave:
    """Self-play of `wave` games at a time on the HIP engine, one HIP graph replay per
    decision step.  Plays what the reference's WaveCollector plays
    (cugo_seq_selfplay50.py:36-238) and leaves the same tensors behind (events, count,
    start, rec_*, final_reward0, final_nagari, finished, started, bad).  With an opponent
    and pool_games > 0, a wave started with pool=True seats the frozen opponent opposite
    the learner in its first pool_games games.

    KV cache rows: the learner's policy keeps one row per seat and game, row
    seat * wave + game (the query goes to the mover's row, event tokens to both); the
    opponent keeps one row per pool game, for its own seat."""

    def __init__(self, ext, actor: SeqPolicy, wave: int, max_steps: int = 64,
                 opponent: SeqPolicy | None = None, pool_games: int = 0) -> None:
        if not 0 <= pool_games <= wave:
            raise ValueError(f"pool_games must be between 0 and the wave size {wave}, "
                             f"got {pool_games}")
        if opponent is not None and opponent.kept_columns() != actor.kept_columns():
            raise ValueError("actor and opponent read different query columns")
        dev = next(actor.parameters()).device
        cols = actor.kept_columns()
        self.ext, self.actor, self.opponent = ext, actor, opponent
        self.w, self.max_steps = wave, max_steps
        self.p = pool_games if opponent is not None else 0
        self.t = _WaveTensors(wave, max_steps, FEATURES if cols is None else len(cols), dev)
        self.ids = torch.arange(wave, device=dev)
        self.seats2 = torch.arange(2 * wave, device=dev) // wave  # seat of each cache row
        self.states = ext.create(*make_seeds(wave, 0, dev))
        self.cache = policy_cache(actor, 2 * wave, dev)
        self.opp_cache = None if opponent is None else policy_cache(opponent, max(1, self.p), dev)
        self.columns = None if cols is None else torch.tensor(cols, dtype=torch.int32, device=dev)
        self.native = {pool: self._native(pool) for pool in ((False, True) if self.p else (False,))}
        # Gumbel noise: None draws Philox4x32-10 uniforms in the sampling kernel (seeded
        # once from torch's generator; the epoch advances with every step, in the advance
        # kernel); a [wave, 179] float32 tensor is read instead (its caller refills it
        # between replays).
        self.noise: torch.Tensor | None = None
        self.seed = int(torch.randint(0, 2**62, (1,)).item())
        self.noise_epoch = torch.zeros(1, dtype=torch.int64, device=dev)
        for native in self.native.values():
            native.set_noise_epoch(self.noise_epoch)
        self.logits: torch.Tensor | None = None  # the last step's logits
        self.graph: torch.cuda.CUDAGraph | None = None  # one step, for `pool` below
        self.graph_pool: bool | None = None
        # 1 while a game is still being played after a step (prepare clears it, advance
        # sets it); copied behind each replay into pinned host memory
        self.playing = torch.zeros(1, dtype=torch.int32, device=dev)
        for native in self.native.values():
            native.set_playing(self.playing)
        self._done_flags = torch.zeros(2, dtype=torch.int32, pin_memory=True)
        # The learner's event tokens of a step wait in rows [0, 2 w) of `pair` and go
        # through the layers with the next step's queries (rows [2 w, 3 w)), in one pass
        # (cached_step_pair); event_pos holds the slots they go to (-1 for an event that
        # is not kept: no committed action, or a game already over, whose row the decode
        # skips, as it skips the query of a finished game).  flush() runs them alone.
        d = actor.position.shape[1]
        self.pair = torch.zeros((3 * wave, d), dtype=actor.event_in.weight.dtype, device=dev)
        # the first layer's norm1 of those rows, written by the launches that make them
        self.pair_h = torch.zeros_like(self.pair)
        # The query input's rows padded with zeros to a depth `linear` takes (1,024 for the
        # 899 columns of the hybrid mode), or unpadded where none fits.
        q_width = (FEATURES if cols is None else len(cols)) + ACTIONS
        self.q_stride = next((k for k in (64, 128, 256, 512, 1024) if k >= q_width), 0)
        self.event_pos = torch.zeros(2 * wave, dtype=torch.int64, device=dev)
        for native in self.native.values():  # advance writes the slots of a step's events
            native.set_event_pos(self.event_pos)

    # the reference's tensor names, for callers of the wave's outcome
    def __getattr__(self, name: str):
        t = self.__dict__.get("t")
        if t is not None and hasattr(t, name):
            return getattr(t, name)
        raise AttributeError(name)

    def _native(self, pool: bool):
        """The prepare/advance kernels' view of this wave's tensors."""
        t, rl = self.t, self.t.rec_long
        return self.ext.SelfPlayState(
            self.w, self.max_steps, t.step_index, t.count, t.events, self.cache.length,
            t.final_reward0, t.final_nagari, t.finished, t.bad, t.rec_features, t.rec_legal,
            t.rec_logp, rl["actions"], rl["opp_hand"], rl["stock"], rl["stop_points"],
            rl["seat"], rl["count"], t.rec_valid, self.columns, self.p if pool else 0,
            t.learner_seat, None if self.opp_cache is None else self.opp_cache.length)

    @staticmethod
    def _open(policy: SeqPolicy, cache: KVCache, start: torch.Tensor, seat: torch.Tensor) -> None:
        """Every row's opening token into slot 0 of `cache`."""
        cache.length.zero_()
        policy.cached_step(cache, policy.start_token(start, seat), 1)
        cache.length.fill_(1)

    @torch.no_grad()
    def reset(self, seeds: torch.Tensor, first: torch.Tensor, learner_seat: torch.Tensor,
              pool: bool = False) -> None:
        """Deals a new wave (the reference's _reset, cugo_seq_selfplay50.py:78-106)."""
        t = self.t
        self.states.copy_(self.ext.create(seeds, first))
        t.start.copy_(self.ext.start(self.states))
        t.learner_seat.copy_(learner_seat)
        for x in t.per_wave:
            x.zero_()
        over = self.states[:, DONE_BYTE] != 0  # a game dealt finished (initial Chongtong)
        t.finished.copy_(over)
        t.started.copy_(~over)
        self._open(self.actor, self.cache, t.start.repeat(2, 1), self.seats2)
        if pool and self.p:
            self._open(self.opponent, self.opp_cache, t.start[:self.p],
                       1 - t.learner_seat[:self.p])
        # no events wait: the first step's event rows are skipped
        self.pair[:2 * self.w].zero_()
        self.event_pos.fill_(-1)

    @torch.no_grad()
    def step(self, pool: bool = False) -> None:
        """One decision of every game (the reference's _step,
        cugo_seq_selfplay50.py:108-163); the bookkeeping around the policy is two HIP
        launches (SelfPlayState.prepare before the query, .advance after the event
        tokens).  The learner's event tokens of this step enter its cache at the next
        step (with that step's queries) or at flush(); until then the cache holds the
        step's query in their slots, which no later token reads.  Rows of finished games
        and of events not kept are skipped by the decode (no cache read or write; their
        hidden states and logits are NaN, and nothing reads them)."""
        ext, actor, t, w = self.ext, self.actor, self.t, self.w
        pool = pool and self.p > 0
        native = self.native[pool]
        features, legal, players, done, status = ext.observe_indexed(self.states, self.ids)
        # stock None: prepare records stock_indexed's words from the state rows itself
        q_in, query_rows, query_pos = native.prepare(self.states, features, legal, players, done,
                                                     status, None, actor.event_in.weight.dtype,
                                                     self.q_stride)
        # the last step's event tokens (both seats' rows) and this step's queries through
        # the layers together; the queries attend the events' new keys at every layer
        actor.query_from_input(q_in, out=self.pair[2 * w:], norm_out=self.pair_h[2 * w:])
        hidden, normed = cached_step_pair(actor, self.cache, self.pair, 2 * w, self.event_pos,
                                          query_pos, query_rows, final_norm=actor.norm,
                                          h=self.pair_h)
        logits = actor.readout(hidden, normed)  # the queries' (the events' are not kept)
        if pool:
            p, opp = self.p, self.opponent
            theirs = opp.readout(opp.cached_step(self.opp_cache, opp.query_from_input(q_in[:p])))
            their_turn = (players[:p].long() != t.learner_seat[:p]).unsqueeze(1)
            logits = torch.cat((torch.where(their_turn, theirs.to(logits.dtype), logits[:p]),
                                logits[p:]))
        self.logits = logits
        if self.noise is not None:
            actions, logp = ext.gumbel_sample(logits.contiguous(), legal, self.noise)
        else:
            actions, logp = ext.gumbel_sample_philox(logits.contiguous(), legal, self.seed,
                                                     self.noise_epoch, 0)
        reward0, new_done, nagari, step_status, committed, events = ext.step_events_indexed(
            self.states, self.ids, actions)
        actor.event_token(events, self.seats2, t.count, out=self.pair[:2 * w],
                          norm_out=self.pair_h[:2 * w])
        if pool:
            opp.cached_step(self.opp_cache,
                            opp.event_token(events[:p], 1 - t.learner_seat[:p], t.count[:p]))
        native.advance(done, reward0, new_done, nagari, step_status, committed, events, actions,
                       logp)  # and the step counter (step_index[1])

    @torch.no_grad()
    def flush(self) -> None:
        """Runs the last step's waiting event tokens through the learner's layers, so its
        cache holds every event as the reference's does after the same steps."""
        cached_step(self.actor, self.cache, self.pair[:2 * self.w], pos=self.event_pos)

    def _capture_step(self, pool: bool) -> torch.cuda.CUDAGraph:
        """step(pool) as a HIP graph.  Library handles, the caching allocator's blocks and
        the token weights are set up by two eager steps on a side stream first, so the
        capture records kernel launches only."""
        self.actor.prepare()
        if self.opponent is not None:
            self.opponent.prepare()
        self.reset(*make_seeds(self.w, 0, self.states.device),
                   torch.zeros_like(self.t.learner_seat), pool)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.step(pool)
            self.step(pool)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self.step(pool)
        return graph

    @torch.no_grad()
    def capture(self, pool: bool = False) -> None:
        """Captures one step (for `pool`) into self.graph unless it already holds it."""
        pool = pool and self.p > 0
        if self.graph is None or self.graph_pool != pool:
            self.graph, self.graph_pool = None, None
            self.graph, self.graph_pool = self._capture_step(pool), pool

    @torch.no_grad()
    def play(self, seeds: torch.Tensor, first: torch.Tensor, learner_seat: torch.Tensor,
             pool: bool = False) -> int:
        """Deals a wave and replays the step until every game has finished; returns the
        number of steps run.  After each replay the step's playing flag (set by its
        advance launch while a game is left) is copied to pinned host memory behind it,
        and the host reads the flag of the replay before the one it has just queued, so
        the GPU never waits for the host: the wave runs at most one step past its end."""
        self.capture(pool)
        self.reset(seeds, first, learner_seat, pool)
        flags, t = self._done_flags, self.t
        stream = torch.cuda.current_stream()
        queued = None  # (event, steps, flag slot) of the latest replay
        steps = 0
        while True:
            behind = queued
            if steps < self.max_steps:
                self.graph.replay()
                steps += 1
                flags[steps & 1].copy_(self.playing[0], non_blocking=True)
                queued = (torch.cuda.Event(), steps, steps & 1)
                queued[0].record(stream)
            if behind is not None:
                behind[0].synchronize()
                if not int(flags[behind[2]]):  # no game left after that step
                    break
                if behind[1] == self.max_steps:
                    raise RuntimeError(f"a wave ran {self.max_steps} steps with games left")
        self.flush()
        problems = int(t.bad)
        if problems:
            raise RuntimeError(f"{problems} observe or step results of active games were "
                               "not ok in this wave")
        if int(t.count.max()) > MAX_EVENTS:
            raise RuntimeError(f"a game committed more than {MAX_EVENTS} events")
        return steps

    def _decisions(self, offset: int) -> dict[str, torch.Tensor]:
        """The learner's recorded decisions of the last wave in step-major order (each
        step's games in order), as the reference appends them to its storage."""
        t = self.t
        flat = torch.nonzero(t.rec_valid.flatten()).squeeze(1)
        step_of, game_of = flat // self.w, flat % self.w
        out = {"features": t.rec_features[step_of, game_of],
               "legal": t.rec_legal[step_of, game_of], "logp": t.rec_logp[step_of, game_of],
               "env_ids": offset + game_of}
        out.update({k: v.flatten()[flat] for k, v in t.rec_long.items()})
        return out

    @torch.no_grad()
    def collect(self, games: int, seed_offset: int, opponent_state: dict | None = None) -> dict:
        """Plays games seed_offset .. seed_offset + games - 1, wave by wave (the
        reference's collect, cugo_seq_selfplay50.py:182-238; games must be a multiple of
        the wave).  opponent_state, loaded into the opponent in place so the captured
        graph keeps reading the same weights, puts it in the first pool_games of every
        wave.  Returns the reference's outcome tensors, the learner's decisions
        ("decisions", what the reference hands its rollout storage) and every game's
        event log, count and opening ("log")."""
        if games % self.w:
            raise ValueError(f"{games} games do not split into waves of {self.w}")
        dev = self.states.device
        pool = opponent_state is not None and self.p > 0
        if pool:
            self.opponent.load_state_dict(opponent_state)
            self.opponent.prepare()
        seeds, first = make_seeds(games, seed_offset, dev)
        learner_seat = torch.randint(2, (games,), device=dev)
        waves: list[dict[str, torch.Tensor]] = []
        decisions: list[dict[str, torch.Tensor]] = []
        steps = 0
        t = self.t
        for offset in range(0, games, self.w):
            part = slice(offset, offset + self.w)
            steps = max(steps, self.play(seeds[part], first[part], learner_seat[part], pool))
            decisions.append(self._decisions(offset))
            vs_pool = torch.zeros(self.w, dtype=torch.bool, device=dev)
            vs_pool[:self.p if pool else 0] = True
            waves.append({"final_reward0": t.final_reward0.clone(),
                          "final_nagari": t.final_nagari.clone(), "started": t.started.clone(),
                          "vs_pool": vs_pool, "events": t.events.clone(),
                          "count": t.count.clone(), "start": t.start.clone()})
        joined = {k: torch.cat([wv[k] for wv in waves]) for k in waves[0]}
        return {"final_reward0": joined["final_reward0"], "final_nagari": joined["final_nagari"],
                "started": joined["started"], "learner_seat": learner_seat,
                "vs_pool": joined["vs_pool"], "steps": steps,
                "decisions": {k: torch.cat([d[k] for d in decisions]) for k in decisions[0]},
                "log": {k: joined[k] for k in ("events", "count", "start")}}
