"""The MLP PPO rollout (cugo_amd/rollout.py) on the GPU.

The engine side is checked against the oracle: the actor's sampled actions are replayed
on the oracle, and every step's observation, step outputs and the rows after the
auto-reset must be identical.  The actor's fused forward pass is checked against the
plain float32 PyTorch forward of the same module, within a bf16 tolerance.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.ref import splitmix_first
from tests.conftest import announce
from tests.test_gpu_engine import assert_observe_equal, assert_step_equal, to_np

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _actor(seed: int, std: float):
    from cugo_amd.rollout import ResidualMlpActor

    torch.manual_seed(seed)
    actor = ResidualMlpActor()
    with torch.no_grad():
        for p in actor.parameters():
            p.normal_(0.0, std)
    return actor.to(DEV)


def test_rollout_engine_matches_oracle(ext, ref):
    """C4's loop at its full batch, 32,768 games, for 40 steps, the step alone and the
    fused step + next observation on alternate steps: observation (bf16 features equal
    to the oracle's float32 ones rounded as torch rounds them), actions drawn from the
    legal set, step outputs and the rows after every step's auto-reset, against the
    oracle stepping the same actions and re-dealing finished rows from seed base + i +
    32,768 * generation."""
    from cugo_amd.rollout import MlpRollout

    announce("MLP rollout engine vs oracle (32,768 x 40)")
    n, steps, base = 32768, 40, 0x243F6A8885A308D3 + 0xC4
    actor = _actor(0, 0.02).to(torch.bfloat16).eval()
    gen = torch.Generator(device=DEV).manual_seed(1)
    ro = MlpRollout(ext, actor, n, steps, base, generator=gen)
    seeds = (np.uint64(base) + np.arange(n, dtype=np.uint64)).view(np.int64)
    host = ref.create(seeds, np.arange(n, dtype=np.int64) & 1)
    assert np.array_equal(to_np(ro.states), host)
    hgen = np.zeros(n, dtype=np.int64)
    with torch.no_grad():
        obs = ro.observe(0)
        for t in range(steps):
            robs = ref.observe(host)
            # the rollout keeps bf16 features: the oracle's float32 features, rounded
            want = torch.from_numpy(robs[0]).to(torch.bfloat16).view(torch.int16)
            assert obs[0].dtype == torch.bfloat16
            assert torch.equal(obs[0].view(torch.int16).cpu(), want), f"features, step {t}"
            assert_observe_equal((obs[0].float(),) + tuple(obs[1:]),
                                 (obs[0].float().cpu().numpy(),) + tuple(robs[1:]),
                                 f"observation, step {t}")
            action = ro.act(t)
            a = to_np(action)
            legal = robs[1]
            live = ~robs[3]
            assert legal[np.arange(n)[live], a[live]].all(), f"illegal action, step {t}"
            # odd steps: the fused step + next observation the rollout loop uses; even
            # steps: the step alone, then observe
            fused = t % 2 == 1 and t + 1 < steps
            out = ro.step_observe(t, action) if fused else ro.step(t, action)
            rout = ref.step(host, a)
            assert_step_equal(out, rout, f"step {t}")
            ended = np.nonzero(rout[1])[0]
            hgen[ended] += 1
            new_seeds = (np.uint64(base) + ended.astype(np.uint64)
                         + np.uint64(n) * hgen[ended].astype(np.uint64)).view(np.int64)
            host[ended] = ref.create(new_seeds, ended & 1)
            assert np.array_equal(to_np(ro.states), host), f"rows after step {t}"
            buf = ro.buffer
            assert np.array_equal(to_np(buf.reward[t]).view(np.uint32),
                                  rout[0].view(np.uint32)), t
            assert np.array_equal(to_np(buf.done[t]), rout[1]), t
            assert np.array_equal(to_np(buf.legal[t]), legal), t
            assert buf.features[t].data_ptr() == obs[0].data_ptr(), t
            lp = to_np(buf.logp[t])
            assert (lp[live] <= 1e-6).all() and np.isfinite(lp[live]).all(), t
            if t + 1 < steps:
                obs = ro.observation if fused else ro.observe(t + 1)
    assert np.array_equal(to_np(ro.generation), hgen)
    # the re-seeded sampler words of finished rows (unused by the actor) are the
    # driver's: SplitMix64 of the row's current seed
    rows = np.nonzero(hgen)[0][:64]
    want = [splitmix_first(int(base + i + n * hgen[i]) & (2**64 - 1)) for i in rows]
    assert np.array_equal(to_np(ro.sampler).view(np.uint64)[rows], np.array(want, np.uint64))
    assert hgen.sum() > n  # most games finished at least once in 40 steps


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gumbel_sample_philox(ext, dtype):
    """gumbel_sample_philox draws exactly the oracle's Philox4x32-10 uniforms (bit for bit,
    every row and action, at a partial last block of rows), and its actions and
    log-probabilities equal gumbel_sample's on those uniforms; the epoch is read from
    device memory at run time (a new epoch, new noise), and a repeat call draws the same."""
    from oracle.philox_ref import gumbel_uniforms

    announce(f"Gumbel-max with Philox uniforms ({dtype})")
    n, a = 3001, 179
    g = torch.Generator(device=DEV).manual_seed(3)
    logits = (torch.randn(n, a, generator=g, device=DEV) * 3).to(dtype)
    legal = torch.rand(n, a, generator=g, device=DEV) < 0.3
    legal[5] = False  # a row with no legal action
    legal[6] = False
    legal[6, 178] = True
    seed = 0x5EED1234ABCD9876
    epoch = torch.tensor([41], dtype=torch.int64, device=DEV)
    u = torch.full((n, a), float("nan"), device=DEV)
    act, lp = ext.gumbel_sample_philox(logits, legal, seed, epoch, 9, uniforms_out=u)
    want_u = gumbel_uniforms(seed, 41, 9, np.arange(n), a)
    assert np.array_equal(u.cpu().numpy().view(np.uint32), want_u.view(np.uint32))
    ref_act, ref_lp = ext.gumbel_sample(logits, legal, u)
    assert torch.equal(act, ref_act)
    assert torch.equal(lp.view(torch.int32), ref_lp.view(torch.int32))
    assert int(act[6]) == 178
    again = ext.gumbel_sample_philox(logits, legal, seed, epoch, 9)
    assert torch.equal(again[0], act) and torch.equal(again[1].view(torch.int32), lp.view(torch.int32))
    epoch.fill_(42)
    u2 = torch.empty_like(u)
    ext.gumbel_sample_philox(logits, legal, seed, epoch, 9, uniforms_out=u2)
    assert np.array_equal(u2.cpu().numpy(), gumbel_uniforms(seed, 42, 9, np.arange(n), a))
    assert float((u2 == u).float().mean()) < 1e-3


def test_fused_forward_matches_float32(ext):
    """fused_forward (bf16 GEMMs with the bias + ReLU epilogue, fused add + LayerNorm)
    against the module's own forward in float32 on the same bf16 inputs: relative
    Frobenius error of the logits and values at most 2e-2 (bf16 rounding through eight
    layers), and the greedy actions agree on at least 97 % of the rows."""
    from cugo_amd.rollout import fused_forward

    announce("MLP actor fused forward vs float32")
    actor32 = _actor(3, 0.05).float().eval()
    actor16 = _actor(3, 0.05).to(torch.bfloat16).eval()
    g = torch.Generator(device=DEV).manual_seed(5)
    x = (torch.rand(4096, 720, generator=g, device=DEV) < 0.2).float()
    x[:, 453:479] = torch.rand(4096, 26, generator=g, device=DEV)
    xb = x.to(torch.bfloat16)
    with torch.no_grad():
        want_l, want_v = actor32(xb.float())
        got_l, got_v = fused_forward(ext, actor16, xb.contiguous())
        plain_l, _ = actor16(xb)
    for got, want in ((got_l, want_l), (got_v, want_v)):
        rel = float((got.float() - want).norm() / want.norm())
        assert rel <= 2e-2, rel
    assert float((got_l.float() - plain_l.float()).norm() / plain_l.float().norm()) <= 2e-2
    agree = float((got_l.float().argmax(1) == want_l.argmax(1)).float().mean())
    assert agree >= 0.97, agree


def _features(n: int, seed: int) -> torch.Tensor:
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = (torch.rand(n, 720, generator=g, device=DEV) < 0.2).float()
    x[:, 453:479] = torch.rand(n, 26, generator=g, device=DEV)
    return x


@pytest.mark.parametrize("n,dtype,blocks", [(4096 + 37, torch.float32, 3),
                                            (1000, torch.bfloat16, 3),
                                            (130, torch.float32, 1)])
def test_mlp_kernel_matches_float32(ext, n, dtype, blocks):
    """mlp_forward (the whole actor in one launch: MFMA GEMMs, LayerNorms and the heads on a
    128-row tile) against the module's own forward in float32 on the same bf16 inputs:
    relative Frobenius error of the logits and values at most 2e-2, the greedy actions
    agree on at least 97 % of the rows, and the bf16 copy of the input equals torch's
    rounding.  Row counts that leave a partial last tile; float32 and bf16 inputs; one and
    three blocks."""
    from cugo_amd.rollout import ResidualMlpActor, fused_forward, mlp_forward, pack_actor

    announce(f"MLP actor kernel vs float32 (n={n}, {dtype}, {blocks} blocks)")
    torch.manual_seed(11)
    base = ResidualMlpActor(blocks=blocks)
    with torch.no_grad():
        for p in base.parameters():
            p.normal_(0.0, 0.05)
    actor16 = base.to(DEV).to(torch.bfloat16).eval()
    actor32 = ResidualMlpActor(blocks=blocks).to(DEV)
    actor32.load_state_dict({k: v.float() for k, v in actor16.state_dict().items()})
    x = _features(n, 5)
    xb = x.to(torch.bfloat16)
    copy = torch.full_like(xb, float("nan"))
    packed = pack_actor(ext, actor16)
    with torch.no_grad():
        want_l, want_v = actor32.eval()(xb.float())
        got_l, got_v = mlp_forward(ext, packed, (x if dtype == torch.float32 else xb).contiguous(),
                                   copy)
        layered_l, layered_v = fused_forward(ext, actor16, xb.contiguous())
    assert got_l.dtype == torch.bfloat16 and got_v.dtype == torch.float32
    assert tuple(got_l.shape) == (n, 179) and tuple(got_v.shape) == (n,)
    assert torch.equal(copy, xb)
    for got, want in ((got_l, want_l), (got_v, want_v)):
        rel = float((got.float() - want).norm() / want.norm())
        assert rel <= 2e-2, rel
    assert float((layered_l.float() - want_l).norm() / want_l.norm()) <= 2e-2
    agree = float((got_l.float().argmax(1) == want_l.argmax(1)).float().mean())
    assert agree >= 0.97, agree
    # repeatable, and an empty batch is a no-op
    with torch.no_grad():
        again_l, again_v = mlp_forward(ext, packed, (x if dtype == torch.float32 else xb).contiguous())
        empty_l, empty_v = mlp_forward(ext, packed, x[:0].contiguous())
    assert torch.equal(again_l, got_l) and torch.equal(again_v, got_v)
    assert tuple(empty_l.shape) == (0, 179) and tuple(empty_v.shape) == (0,)


def test_mlp_kernel_rejects_other_shapes(ext):
    """Widths the kernel does not serve raise instead of running: hidden 256, or an input
    width that is not a multiple of 8."""
    from cugo_amd.rollout import ResidualMlpActor, mlp_forward, mlp_kernel_fits, pack_actor

    narrow = ResidualMlpActor(d=256).to(DEV).to(torch.bfloat16)
    odd = ResidualMlpActor(features=722).to(DEV).to(torch.bfloat16)
    assert not mlp_kernel_fits(narrow) and not mlp_kernel_fits(odd)
    with pytest.raises(RuntimeError):
        mlp_forward(ext, pack_actor(ext, narrow), _features(64, 1))
    with pytest.raises(RuntimeError):
        mlp_forward(ext, pack_actor(ext, odd), torch.zeros(64, 722, device=DEV))


def test_rollout_graph_replay_equals_eager(ext):
    """capture() + replay() plays what collect() plays: two rollouts from the same deals
    with the same fixed noise, one eager and one from the captured graph, for two horizons
    of 40 steps (refills at steps 0 and 32 of each): identical rows, generations, samplers
    and buffers after each horizon."""
    from cugo_amd.rollout import MlpRollout

    announce("MLP rollout graph replay vs eager")
    n, horizon, base = 8192, 40, 0x1234567
    actor = _actor(1, 0.05).to(torch.bfloat16).eval()
    a = MlpRollout(ext, actor, n, horizon, base)
    b = MlpRollout(ext, actor, n, horizon, base)
    noise = torch.rand((n, 179), generator=torch.Generator(device=DEV).manual_seed(9),
                       device=DEV)
    a.noise, b.noise = noise, noise
    with torch.no_grad():
        b.capture()  # runs two eager warm-up steps (t = 0, 1) before recording
        for t in range(2):
            a.observe(t)
            a.step(t, a.act(t))
        for _ in range(2):
            a.collect()
            b.replay()
            torch.cuda.synchronize()
            for x, y in ((a.states, b.states), (a.generation, b.generation),
                         (a.sampler, b.sampler)):
                assert torch.equal(x, y)
            for name in ("features", "legal", "action", "logp", "value", "reward", "done"):
                assert torch.equal(getattr(a.buffer, name), getattr(b.buffer, name)), name
    assert a.games_completed() > n


def test_rollout_captured_horizons_match_oracle(ext, ref):
    """C4 in the form bench.py times it (bench.make_rollout: B = 32,768, the 3 x 512 bf16
    actor, a 128-step horizon captured once as a HIP graph and replayed, Philox uniforms
    drawn in the sampler).  The capture's two eager warm-up steps and two replayed
    horizons (refills at steps 0, 32, 64 and 96 of each; the epoch raised by each replay)
    against the oracle stepping the recorded actions: every one of the 256 steps' bf16
    features, mask, reward and done flag, the rows, generations and re-seeded sampler
    words after each horizon, every action legal.  The sampler's draw is checked on a
    1,024-row sample at steps 0, 31, 32, 95 and 127 of each horizon: the Philox uniforms
    of (seed, epoch, step) from the oracle's Philox, the actor's logits on the recorded
    features, and the oracle's Gumbel-max give the recorded action, value and
    log-probability."""
    from bench import ROLLOUT_BASE, make_rollout
    from cugo_amd.rollout import mlp_forward
    from oracle.philox_ref import gumbel_uniforms
    from oracle.seq_ref import gumbel_reference

    announce("MLP rollout: two captured 128-step horizons at 32,768 games vs oracle")
    n, horizon, base = 32768, 128, ROLLOUT_BASE
    ro = make_rollout(ext, torch, n, horizon)
    assert ro.fused_kernel and ro.noise is None
    idx = np.arange(n, dtype=np.uint64)
    host = ref.create((np.uint64(base) + idx).view(np.int64), np.arange(n, dtype=np.int64) & 1)
    assert np.array_equal(to_np(ro.states), host)
    hgen = np.zeros(n, dtype=np.int64)

    def oracle_step(actions: np.ndarray, label: str):
        rout = ref.step(host, actions)
        ended = np.nonzero(rout[1])[0]
        hgen[ended] += 1
        seeds = (np.uint64(base) + ended.astype(np.uint64)
                 + np.uint64(n) * hgen[ended].astype(np.uint64)).view(np.int64)
        host[ended] = ref.create(seeds, ended & 1)
        return rout

    def rows_match(label: str):
        assert np.array_equal(to_np(ro.states), host), f"rows after {label}"
        assert np.array_equal(to_np(ro.generation), hgen), f"generations after {label}"
        done_rows = np.nonzero(hgen)[0][:256]
        want = [splitmix_first(int(base + i + n * hgen[i]) & (2**64 - 1)) for i in done_rows]
        assert np.array_equal(to_np(ro.sampler).view(np.uint64)[done_rows],
                              np.array(want, np.uint64)), f"samplers after {label}"

    buf = ro.buffer
    with torch.no_grad():
        ro.capture()  # records the horizon; its two eager warm-up steps run first
        torch.cuda.synchronize()
        for t in range(2):
            oracle_step(to_np(buf.action[t]), f"warm-up step {t}")
        rows_match("the warm-up steps")
        sample_rows = np.sort(np.random.default_rng(41).choice(n, 1024, replace=False))
        rows_dev = torch.from_numpy(sample_rows).to(DEV)
        for epoch in (1, 2):
            ro.replay()
            torch.cuda.synchronize()
            assert int(ro.epoch) == epoch
            for t in range(horizon):
                label = f"horizon {epoch}, step {t}"
                if t % 32 == 0:
                    print(f"  {label}", flush=True)
                robs = ref.observe(host)
                want = torch.from_numpy(robs[0]).to(torch.bfloat16).view(torch.int16)
                assert torch.equal(buf.features[t].view(torch.int16).cpu(), want), \
                    f"features, {label}"
                legal = robs[1]
                assert np.array_equal(to_np(buf.legal[t]), legal), f"legal, {label}"
                a = to_np(buf.action[t])
                live = ~robs[3]
                assert legal[np.arange(n)[live], a[live]].all(), f"illegal action, {label}"
                lp = to_np(buf.logp[t])
                assert (lp[live] <= 1e-6).all() and np.isfinite(lp[live]).all(), label
                if t in (0, 31, 32, 95, 127):
                    x = buf.features[t].index_select(0, rows_dev).contiguous()
                    logits, value = mlp_forward(ext, ro.packed, x)
                    u = torch.from_numpy(gumbel_uniforms(ro.seed, epoch, t, sample_rows, 179))
                    legal_s = buf.legal[t].index_select(0, rows_dev)
                    act, logp = gumbel_reference(logits.float(), legal_s, u.to(DEV))
                    assert torch.equal(act, buf.action[t].index_select(0, rows_dev)), \
                        f"sampled actions, {label}"
                    assert torch.allclose(logp, buf.logp[t].index_select(0, rows_dev),
                                          atol=1e-5), f"log-probabilities, {label}"
                    assert torch.equal(value, buf.value[t].index_select(0, rows_dev)), \
                        f"values, {label}"
                rout = oracle_step(a, label)
                assert np.array_equal(to_np(buf.reward[t]).view(np.uint32),
                                      rout[0].view(np.uint32)), f"reward, {label}"
                assert np.array_equal(to_np(buf.done[t]), rout[1]), f"done, {label}"
            rows_match(f"horizon {epoch}")
    assert hgen.sum() > 4 * n  # about 13 games a row in 258 steps
