"""GPU-resident self-play of the event-sequence policy on the HIP engine.

`SeqPolicy` is the inference half of the reference's `SeqNet` in its "hybrid" form
(python/cugo_seq50.py:131-323: query token = the 720 features + the 179-bit legal mask):
the same submodules and parameter names (`event_in`, `start_in`, `query_in`, `position`,
`token_type`, `encoder`, `norm`, `head`), so a reference state_dict loads into it.  Its
opening and event tokens are HIP kernels (`start_tokens`, `event_tokens`): each row sums
the Linear weight columns of its token's set bits instead of materialising the 0/1 token
and running a GEMM, with the reference's bf16 roundings.  `cached_step` appends the new
key/value and attends in one HIP launch per layer (`seq_decode.cached_step`).

`SelfPlayWave` is the reference's `WaveCollector` (python/cugo_seq_selfplay50.py:36-238)
without the frozen-opponent pool: a wave of games advances one decision per step -
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
    """SeqNet (hybrid query) for incremental inference: start/event/query tokens, the
    cached decoder step and the readout head."""

    def __init__(self, outputs: int = ACTIONS, d_model: int = 256, layers: int = 4,
                 heads: int = 8) -> None:
        super().__init__()
        d = d_model
        self.event_in = nn.Linear(EVENT_IN, d)
        self.start_in = nn.Linear(START_IN, d)
        self.query_in = nn.Sequential(nn.Linear(FEATURES + ACTIONS, 2 * d), nn.GELU(),
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
        """The Linear weight transposed to [in, d] (the kernels' column layout), kept
        until the weight changes (in-place updates bump its version)."""
        w = getattr(self, name).weight
        key = (w.data_ptr(), w._version, w.dtype, w.device)
        hit = self._transposed.get(name)
        if hit is None or hit[0] != key:
            hit = (key, w.detach().t().contiguous())
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
        """cugo_seq50.py:166-180 (hybrid): query_in(features ++ legal) + token_type[2]."""
        dt = self.event_in.weight.dtype
        return self.query_from_input(torch.cat((features.to(dt), legal.to(dt)), -1))

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
    (WaveCollector without the opponent pool, cugo_seq_selfplay50.py:36-238)."""

    def __init__(self, ext, actor: SeqPolicy, wave: int, max_steps: int = 64) -> None:
        device = next(actor.parameters()).device
        self.ext, self.actor, self.w, self.max_steps = ext, actor, wave, max_steps
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
        s = max_steps
        self.rec_features = torch.zeros((s, w, FEATURES), dtype=torch.bfloat16, device=device)
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
        self.native = ext.SelfPlayState(
            w, s, self.step_index, self.count, self.events, self.cache.length,
            self.final_reward0, self.final_nagari, self.finished, self.bad, self.rec_features,
            self.rec_legal, self.rec_logp, self.rec_long["actions"], self.rec_long["opp_hand"],
            self.rec_long["stock"], self.rec_long["stop_points"], self.rec_long["seat"],
            self.rec_long["count"], self.rec_valid)
        # Sampling noise: None draws torch.rand_like inside the step (the reference's
        # choice); a tensor [wave, ACTIONS] is read instead (set by a caller that draws
        # its own uniforms before each step).
        self.noise: torch.Tensor | None = None
        self.graph: torch.cuda.CUDAGraph | None = None
        self.logits: torch.Tensor | None = None

    @torch.no_grad()
    def reset(self, seeds: torch.Tensor, first: torch.Tensor, learner_seat: torch.Tensor) -> None:
        """cugo_seq_selfplay50.py:78-106 (no pool)."""
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

    @torch.no_grad()
    def step(self) -> None:
        """One decision of every game (cugo_seq_selfplay50.py:108-163, no pool).  The torch
        bookkeeping around the policy runs as two kernels (`SelfPlayState.prepare` before
        the query, `.advance` after the event tokens)."""
        ids, actor, ext = self.ids, self.actor, self.ext
        features, legal, players, done, status = ext.observe_indexed(self.states, ids)
        stock = ext.stock_indexed(self.states, ids)
        q_in, query_rows = self.native.prepare(self.states, features, legal, players, done,
                                               status, stock, actor.event_in.weight.dtype)
        hidden = actor.cached_step(self.cache, actor.query_from_input(q_in), rows=query_rows)
        logits = actor.readout(hidden)  # the kernel reads bf16 logits as the fp32 .float()
        self.logits = logits  # the last step's logits (kept for inspection)
        uniforms = (torch.rand(logits.shape, dtype=torch.float32, device=logits.device)
                    if self.noise is None else self.noise)
        actions, logp = ext.gumbel_sample(logits.contiguous(), legal, uniforms)
        reward0, new_done, nagari, step_status, committed, events = ext.step_events_indexed(
            self.states, ids, actions)
        actor.cached_step(self.cache, actor.event_token(events, self.seats2, self.count))
        self.native.advance(done, reward0, new_done, nagari, step_status, committed, events,
                            actions, logp)
        self.step_index += 1

    @torch.no_grad()
    def capture(self) -> None:
        """Record step() once as a HIP graph (cugo_seq_selfplay50.py:165-180)."""
        if self.graph is not None:
            return
        self.actor.prepare()
        seeds, first = make_seeds(self.w, 0, self.states.device)
        self.reset(seeds, first, torch.zeros_like(self.learner_seat))
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):  # warm-up (GEMM handles, allocator) outside the capture
                self.step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self.step()
        self.graph = graph

    @torch.no_grad()
    def play(self, seeds: torch.Tensor, first: torch.Tensor, learner_seat: torch.Tensor) -> int:
        """Plays one wave to the end by replaying the captured step; returns the number of
        steps replayed (cugo_seq_selfplay50.py:203-219)."""
        self.capture()
        self.reset(seeds, first, learner_seat)
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
