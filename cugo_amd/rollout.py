"""MLP PPO self-play rollouts on the HIP engine.

The reference's collector (python/cugo_ppo50.py:321-450, `collect`) plays each step as
observe -> actor forward -> masked sampling -> step, records (features, legal, action,
logp) per decision and the settled reward at the end.  This module plays the same loop
over a resident batch of games with auto-reset, for a residual MLP actor:

  * engine: `step_observe_spares` in one launch per step: the step of every game with the
    sampled actions, each finished row given its next game (seed base + i + B *
    generation, first player i & 1) from a pre-dealt spare (`refill_spares` every REFILL
    steps; a stale spare is dealt into its slot first), then the next step's observation
    of the new states (720 features written as bf16 straight into the rollout buffer, +
    the 179-way mask).  The horizon's first observation is `observe_bf16`; an actor the
    one-launch forward does not serve gets `observe` (float32 features) and
    `step_reset_spares` as two launches;
  * actor: one HIP launch for the whole forward pass (`mlp_forward`: MFMA GEMMs with a
    128-row tile's activations kept on chip from the input layer to the heads, reading
    the buffer's bf16 features), for the 512-wide actor; any
    other width runs `fused_forward`: bf16 GEMMs through PyTorch-ROCm (hipBLASLt), the bias
    and ReLU of each block's first Linear fused into its GEMM, each residual add fused with
    the next LayerNorm (`add_layernorm`, one HIP launch);
  * sampling: the Gumbel-max draw over the legal actions and its log-probability in one
    HIP launch (`gumbel_sample_philox`), its uniforms drawn in the kernel from
    Philox4x32-10 keyed by a seed taken once from the caller's generator, the rollout's
    epoch (a device counter raised once per horizon, so a captured graph draws fresh
    noise on every replay) and the step; with fixed `noise` [B, 179], `gumbel_sample` on
    those uniforms.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn
from torch.nn import functional as F

REFILL = 32  # steps between pre-deals of the next games
SPARE_SLOTS = 2  # pre-dealt games per row


class ResidualBlock(nn.Module):
    """h + fc2(relu(fc1(norm(h))))."""

    def __init__(self, d: int) -> None:
        super().__init__()
        self.norm = nn.LayerNorm(d)
        self.fc1 = nn.Linear(d, d)
        self.fc2 = nn.Linear(d, d)

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        return h + self.fc2(torch.relu(self.fc1(self.norm(h))))


class ResidualMlpActor(nn.Module):
    """720 features -> Linear(720, d) -> `blocks` residual blocks -> LayerNorm -> 179
    logits and a scalar value.  `forward` is the plain PyTorch form; `fused_forward` the
    rollout's."""

    def __init__(self, d: int = 512, blocks: int = 3, features: int = 720,
                 actions: int = 179) -> None:
        super().__init__()
        self.inp = nn.Linear(features, d)
        self.blocks = nn.ModuleList(ResidualBlock(d) for _ in range(blocks))
        self.norm = nn.LayerNorm(d)
        self.logits = nn.Linear(d, actions)
        self.value = nn.Linear(d, 1)

    def forward(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        h = self.inp(x)
        for block in self.blocks:
            h = block(h)
        h = self.norm(h)
        return self.logits(h), self.value(h).squeeze(-1)

    def flops_per_row(self) -> int:
        """Multiply-adds x 2 of one forward pass (the Linear layers)."""
        return 2 * sum(m.in_features * m.out_features for m in self.modules()
                       if isinstance(m, nn.Linear))


def fused_forward(ext, actor: ResidualMlpActor, x: torch.Tensor):
    """actor(x) for a bf16 actor on a contiguous bf16 [n, 720] input: the same layers,
    with fc1's bias and ReLU in its GEMM's epilogue and every residual add fused with the
    LayerNorm that follows it.  Returns (logits [n, 179], value [n]) in bf16."""
    h = F.linear(x, actor.inp.weight, actor.inp.bias)
    norms = [b.norm for b in actor.blocks] + [actor.norm]
    _, z = ext.add_layernorm(h, None, norms[0].weight, norms[0].bias, norms[0].eps)
    for k, block in enumerate(actor.blocks):
        u = torch._addmm_activation(block.fc1.bias, z, block.fc1.weight.t())
        y = torch.addmm(block.fc2.bias, u, block.fc2.weight.t())
        nxt = norms[k + 1]
        h, z = ext.add_layernorm(h, y, nxt.weight, nxt.bias, nxt.eps)
    logits = F.linear(z, actor.logits.weight, actor.logits.bias)
    value = F.linear(z, actor.value.weight, actor.value.bias).squeeze(-1)
    return logits, value


def mlp_kernel_fits(actor: ResidualMlpActor) -> bool:
    """Whether `mlp_forward` serves this actor (hidden width 512, at most 4 blocks, the
    input width a multiple of 8 up to 768, at most 255 actions)."""
    return (actor.inp.out_features == 512 and len(actor.blocks) <= 4
            and actor.inp.in_features % 8 == 0 and actor.inp.in_features <= 768
            and actor.logits.out_features <= 255)


@dataclass
class PackedActor:
    """A bf16 ResidualMlpActor's parameters as `mlp_forward` reads them: the matrices in
    the kernel's MFMA operand order (`mlp_pack_weight`), the head as one matrix (the logits
    weight with the value weight as its last row) and one bias."""

    w_in: torch.Tensor
    b_in: torch.Tensor
    ln_w: list
    ln_b: list
    w1: list
    b1: list
    w2: list
    b2: list
    w_head: torch.Tensor
    b_head: torch.Tensor
    actions: int
    eps: float


MAX_FEATURES = 768  # the kernel's padded input width
HEAD_ROWS = 256     # the kernel's padded head width


@torch.no_grad()
def pack_actor(ext, actor: ResidualMlpActor) -> PackedActor:
    """The actor's parameters packed for `mlp_forward`; pack again after they change."""
    d = actor.inp.out_features

    def pack(w: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
        return ext.mlp_pack_weight(w.contiguous(), rows, cols)

    blocks = actor.blocks
    head = torch.cat([actor.logits.weight, actor.value.weight]).contiguous()
    return PackedActor(
        w_in=pack(actor.inp.weight, d, MAX_FEATURES), b_in=actor.inp.bias.contiguous(),
        ln_w=[b.norm.weight.contiguous() for b in blocks] + [actor.norm.weight.contiguous()],
        ln_b=[b.norm.bias.contiguous() for b in blocks] + [actor.norm.bias.contiguous()],
        w1=[pack(b.fc1.weight, d, d) for b in blocks],
        b1=[b.fc1.bias.contiguous() for b in blocks],
        w2=[pack(b.fc2.weight, d, d) for b in blocks],
        b2=[b.fc2.bias.contiguous() for b in blocks],
        w_head=pack(head, HEAD_ROWS, d),
        b_head=torch.cat([actor.logits.bias, actor.value.bias]).contiguous(),
        actions=actor.logits.out_features, eps=actor.norm.eps)


def mlp_forward(ext, packed: PackedActor, x: torch.Tensor,
                x_copy: torch.Tensor | None = None, value: torch.Tensor | None = None):
    """The actor's forward pass in one HIP launch (`pack_actor` of a bf16 actor): x [n, F]
    float32 or bf16 (contiguous); x_copy, if given, receives x rounded to bf16; `value`, if
    given, receives the values (f32 [n]).  Returns (logits bf16 [n, A], value f32 [n]).
    bf16 operands with fp32 accumulation; the residual stream stays fp32 between
    blocks."""
    p = packed
    return ext.mlp_actor_forward(x, x_copy, p.w_in, p.b_in, p.ln_w, p.ln_b, p.w1, p.b1, p.w2,
                                 p.b2, p.w_head, p.b_head, p.actions, p.eps, value)


@dataclass
class RolloutBuffer:
    """`horizon` steps of B games: the actor's bf16 input, the legal mask, the sampled
    action and its log-probability, the value estimate, and the step's reward for seat 0
    (non-zero only when the game settles) and done flag."""

    features: torch.Tensor  # bf16 [H, B, 720]
    legal: torch.Tensor     # bool [H, B, 179]
    action: torch.Tensor    # int64 [H, B]
    logp: torch.Tensor      # f32 [H, B]
    value: torch.Tensor     # f32 [H, B]
    reward: torch.Tensor    # f32 [H, B]
    done: torch.Tensor      # bool [H, B]

    @classmethod
    def empty(cls, horizon: int, batch: int, device) -> "RolloutBuffer":
        def e(*shape, dtype):
            return torch.empty((horizon, batch, *shape), dtype=dtype, device=device)
        return cls(e(720, dtype=torch.bfloat16), e(179, dtype=torch.bool), e(dtype=torch.int64),
                   e(dtype=torch.float32), e(dtype=torch.float32), e(dtype=torch.float32),
                   e(dtype=torch.bool))


class MlpRollout:
    """B resident games played by `actor` with auto-reset.  Game j of row i is dealt
    from seed base_seed + i + B * j with first player i & 1 (j = generation[i]).

    `collect()` plays `horizon` steps eagerly; `capture()` records those steps once as a
    HIP graph and `replay()` plays the next `horizon` steps from it (no per-op launch cost
    on the host).  The sampler's uniforms come from Philox4x32-10 (seeded from
    `generator`, or torch's default generator), or from `noise` [B, 179] when set, which
    every step then reads."""

    def __init__(self, ext, actor: ResidualMlpActor, batch: int, horizon: int,
                 base_seed: int, generator: torch.Generator | None = None) -> None:
        self.ext, self.actor = ext, actor
        self.batch, self.horizon, self.base = batch, horizon, base_seed
        dev = next(actor.parameters()).device
        idx = torch.arange(batch, dtype=torch.int64, device=dev)
        self.states = ext.create(idx + base_seed, idx & 1)
        self.generation = torch.zeros(batch, dtype=torch.int32, device=dev)
        # step_reset_spares re-seeds a finished row's sampler word; the actor does not
        # use it.
        self.sampler = ext.seed_samplers(batch, base_seed, self.generation)
        self.spares = torch.empty((SPARE_SLOTS * batch, 248), dtype=torch.uint8, device=dev)
        self.spare_gen = torch.zeros(SPARE_SLOTS * batch, dtype=torch.int32, device=dev)
        self.buffer = RolloutBuffer.empty(horizon, batch, dev)
        self.generator = generator
        self.noise: torch.Tensor | None = None
        # the Philox key and the horizon counter (device memory, raised by _steps)
        self.seed = int(torch.randint(0, 2**62, (1,), generator=generator, device=dev).item())
        self.epoch = torch.zeros(1, dtype=torch.int64, device=dev)
        self.graph: torch.cuda.CUDAGraph | None = None
        # the one-launch forward where it fits the actor, else the layer-by-layer one
        self.fused_kernel = mlp_kernel_fits(actor)
        self.packed = pack_actor(ext, actor) if self.fused_kernel else None
        self.observation = None  # the last step's observe outputs
        self.step_out = None     # the last step's step outputs

    def observe(self, t: int):
        """Step t's observation (the next games are pre-dealt every REFILL steps).  With the
        one-launch actor, the features are written as bf16 straight into the buffer's row
        t (`observe_bf16`: the float32 features rounded as torch rounds them), which the
        actor reads."""
        if t % REFILL == 0:
            self.ext.refill_spares(self.spares, self.spare_gen, self.generation, self.base)
        if self.fused_kernel:  # features and mask straight into the buffer's row t
            self.observation = self.ext.observe_bf16(self.states, self.buffer.features[t],
                                                     legal=self.buffer.legal[t])
        else:
            self.observation = self.ext.observe(self.states)
        return self.observation

    def act(self, t: int):
        """The actor's action for every game of the last observation, recorded in row t
        of the buffer."""
        features, legal = self.observation[0], self.observation[1]
        buf = self.buffer
        if self.fused_kernel:
            # features and legal are the buffer's rows t; the value, action and
            # log-probability are written into theirs
            logits, _ = mlp_forward(self.ext, self.packed, features, value=buf.value[t])
        else:
            x = buf.features[t]
            x.copy_(features)
            logits, value = fused_forward(self.ext, self.actor, x)
            buf.legal[t].copy_(legal)
            buf.value[t].copy_(value)
        if self.noise is not None:
            self.ext.gumbel_sample(logits, legal, self.noise, actions=buf.action[t],
                                   logp=buf.logp[t])
        else:
            self.ext.gumbel_sample_philox(logits, legal, self.seed, self.epoch, t,
                                          actions=buf.action[t], logp=buf.logp[t])
        return buf.action[t]

    def repack(self) -> None:
        """Re-reads the actor's parameters after they changed (the one-launch forward reads
        a packed copy; a captured graph reads the same tensors, updated in place)."""
        if self.fused_kernel:
            fresh = pack_actor(self.ext, self.actor)
            if self.packed is None:
                self.packed = fresh
                return
            for name in ("w_in", "b_in", "w_head", "b_head"):
                getattr(self.packed, name).copy_(getattr(fresh, name))
            for name in ("ln_w", "ln_b", "w1", "b1", "w2", "b2"):
                for old, new in zip(getattr(self.packed, name), getattr(fresh, name)):
                    old.copy_(new)

    def step(self, t: int, action: torch.Tensor):
        """Steps every game with `action` (re-dealing finished ones); the reward and done
        flag go straight into the buffer's row t."""
        self.step_out = self.ext.step_reset_spares(
            self.states, action, self.base, self.generation, self.sampler, self.spares,
            self.spare_gen, reward=self.buffer.reward[t], done=self.buffer.done[t])
        return self.step_out

    def step_observe(self, t: int, action: torch.Tensor):
        """step(t, action), then step t + 1's observation of the new states, in one launch
        (`step_observe_spares`): the reward and done flag go into the buffer's row t, the
        bf16 features and mask into row t + 1."""
        if (t + 1) % REFILL == 0:
            self.ext.refill_spares(self.spares, self.spare_gen, self.generation, self.base)
        buf = self.buffer
        out = self.ext.step_observe_spares(
            self.states, action, self.base, self.generation, self.sampler, self.spares,
            self.spare_gen, buf.features[t + 1], reward=buf.reward[t], done=buf.done[t],
            legal=buf.legal[t + 1])
        self.step_out, self.observation = out[:5], out[5:]
        return self.step_out

    def _steps(self) -> None:
        self.epoch.add_(1)  # fresh sampler noise for this horizon (a kernel: graph-safe)
        self.observe(0)
        for t in range(self.horizon):
            action = self.act(t)
            if self.fused_kernel and t + 1 < self.horizon:
                self.step_observe(t, action)
            else:
                self.step(t, action)
                if t + 1 < self.horizon:
                    self.observe(t + 1)

    @torch.no_grad()
    def collect(self) -> RolloutBuffer:
        """`horizon` steps into the buffer, issued eagerly (the games carry on across
        calls)."""
        self._steps()
        return self.buffer

    @torch.no_grad()
    def capture(self) -> None:
        """Records `horizon` steps as one HIP graph.  Two eager steps on a side stream set
        up the GEMM handles and the allocator's blocks first; they advance the games."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for t in range(2):
                self.observe(t)
                self.step(t, self.act(t))
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self._steps()
        self.graph = graph

    def replay(self) -> RolloutBuffer:
        """The next `horizon` steps from the captured graph."""
        if self.graph is None:
            raise RuntimeError("capture() the rollout before replaying it")
        self.graph.replay()
        return self.buffer

    def games_completed(self) -> int:
        return int(self.generation.sum(dtype=torch.int64).item())
