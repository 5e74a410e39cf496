"""GPU parity: every operation of the HIP extension against the oracle.

The checker is the oracle (oracle/matgo/, the plain-C restatement of the reference
engine, driven through oracle/ref.py) on the same inputs; the oracle itself is pinned by
the golden fixtures and the reference's own build (tests/test_cpu_oracle*.py).  Integer,
byte and mask outputs must be identical and float features/rewards bit-identical
(compared as raw 32-bit patterns).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.ref import (PADDING, SEED_BASE, fnv_update, FNV_OFFSET, sample_actions,
                        splitmix_first, step_record)
from tests.conftest import GOLDEN, announce

pytestmark = pytest.mark.gpu

DEV = "cuda"


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def f32_bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def c1_seeds(n: int, base: int = SEED_BASE):
    idx = np.arange(n, dtype=np.uint64)
    seeds = (np.uint64(base) + idx).view(np.int64)
    return seeds, (np.arange(n, dtype=np.int64) & 1)


def assert_observe_equal(gpu_out, ref_out, label: str) -> None:
    f, legal, player, done, status = (to_np(t) for t in gpu_out)
    rf, rlegal, rplayer, rdone, rstatus = ref_out
    bad = np.nonzero((f32_bits(f) != f32_bits(rf)).any(axis=1))[0]
    assert bad.size == 0, f"{label}: features differ in rows {bad[:8]}"
    assert np.array_equal(legal, rlegal), f"{label}: legal masks differ"
    assert np.array_equal(player, rplayer), f"{label}: players differ"
    assert np.array_equal(done, rdone), f"{label}: done differs"
    assert np.array_equal(status, rstatus), f"{label}: status differs"


def assert_step_equal(gpu_out, ref_out, label: str) -> None:
    names = ("reward", "done", "nagari", "status", "committed", "events")
    for name, g, r in zip(names, gpu_out, ref_out):
        g = to_np(g)
        if name == "reward":
            assert np.array_equal(f32_bits(g), f32_bits(r)), f"{label}: reward differs"
        else:
            assert np.array_equal(g, r), f"{label}: {name} differs"


def test_create_and_start(ext, ref):
    announce("create_and_start")
    seeds, first = c1_seeds(4096)
    rng = np.random.default_rng(7)
    seeds = np.concatenate([seeds, rng.integers(-2**63, 2**63 - 1, 4033, dtype=np.int64)])
    first = np.concatenate([first, rng.integers(0, 5, 4033, dtype=np.int64)])
    states = ext.create(torch.from_numpy(seeds).to(DEV), torch.from_numpy(first).to(DEV))
    rows = to_np(states)
    expect = ref.create(seeds, first)
    assert np.array_equal(rows, expect)
    assert np.array_equal(to_np(ext.start(states)), ref.start(expect))
    golden = np.load(GOLDEN / "rows.npz")
    g = ext.create(torch.from_numpy(golden["seeds"]).to(DEV),
                   torch.from_numpy(golden["first"]).to(DEV))
    assert np.array_equal(to_np(g), golden["created"])
    assert np.array_equal(to_np(ext.start(g)), golden["start"])


def test_random_policy_games_match_reference(ext, ref):
    """The C1 protocol: 4,096 games to the end in lockstep with the reference; every
    observation, step output, event record and row byte compared, and the per-game
    digests checked against the golden fixture."""
    announce("random_policy_lockstep_c1")
    n = 4096
    seeds, first = c1_seeds(n)
    states = ext.create(torch.from_numpy(seeds).to(DEV), torch.from_numpy(first).to(DEV))
    host = ref.create(seeds, first)
    sampler = np.array([splitmix_first(int(s) & (2**64 - 1)) for s in seeds], dtype=np.uint64)
    digest = np.full(n, FNV_OFFSET, dtype=np.uint64)
    steps = np.zeros(n, dtype=np.int32)
    ids = torch.arange(n, device=DEV)
    for step in range(128):
        obs = ext.observe(states)
        robs = ref.observe(host)
        assert_observe_equal(obs, robs, f"observe step {step}")
        active = ~robs[3]
        if not active.any():
            break
        assert robs[1][active].any(axis=1).all(), "active game without a legal action"
        actions = sample_actions(robs[1], sampler, active)
        out = ext.step_events_indexed(states, ids, torch.from_numpy(actions).to(DEV))
        rout = ref.step(host, actions, events=True)
        assert_step_equal(out, rout, f"step {step}")
        assert np.array_equal(to_np(states), host), f"rows differ after step {step}"
        rec = step_record(robs[0], robs[1], robs[2], robs[3], robs[4], actions, *rout)
        digest[active] = fnv_update(digest[active], rec[active])
        steps[active] += 1
    golden = np.load(GOLDEN / "c1_random_policy.npz")
    assert np.array_equal(steps, golden["steps"])
    assert np.array_equal(digest, golden["digest"])
    rewards = np.array([ref.reward0(r) for r in host], dtype=np.int64)
    assert np.array_equal(rewards, golden["final_reward"])


def test_wild_actions_and_indexed_rows(ext, ref):
    """Out-of-range and illegal actions, invalid/duplicate ids, odd batch sizes."""
    announce("wild_actions_indexed")
    rng = np.random.default_rng(11)
    n = 1000  # not a multiple of 64
    seeds = rng.integers(-2**63, 2**63 - 1, n, dtype=np.int64)
    first = rng.integers(0, 2, n, dtype=np.int64)
    states = ext.create(torch.from_numpy(seeds).to(DEV), torch.from_numpy(first).to(DEV))
    host = ref.create(seeds, first)
    sampler = np.array([splitmix_first(int(s) & (2**64 - 1)) for s in seeds], dtype=np.uint64)
    for step in range(60):
        ids = rng.permutation(n)[: rng.integers(1, n)].astype(np.int64)
        obs_ids = np.concatenate([ids, [-1, n, n + 5, ids[0], ids[0]]]).astype(np.int64)
        obs = ext.observe_indexed(states, torch.from_numpy(obs_ids).to(DEV))
        assert_observe_equal(obs, ref.observe(host, obs_ids), f"observe_indexed {step}")
        _, legal, _, done, _ = ref.observe(host, ids)
        actions = sample_actions(legal, sampler[ids], ~done)
        wild = rng.random(ids.size) < 0.15
        actions[wild] = rng.integers(-3, 185, int(wild.sum()))
        step_ids = np.concatenate([ids, [-7, n]]).astype(np.int64)
        step_actions = np.concatenate([actions, [0, 1]]).astype(np.int64)
        if step % 2:
            out = ext.step_indexed(states, torch.from_numpy(step_ids).to(DEV),
                                   torch.from_numpy(step_actions).to(DEV))
            rout = ref.step(host, step_actions, ids=step_ids)
        else:
            out = ext.step_events_indexed(states, torch.from_numpy(step_ids).to(DEV),
                                          torch.from_numpy(step_actions).to(DEV))
            rout = ref.step(host, step_actions, ids=step_ids, events=True)
        assert_step_equal(out, rout, f"step_indexed {step}")
        assert np.array_equal(to_np(states), host), f"rows differ after indexed step {step}"


def test_full_batch_step_matches(ext, ref):
    announce("full_batch_step")
    golden = np.load(GOLDEN / "rows.npz")
    mid = golden["mid"]
    for name, actions in (("first", golden["first_legal"]), ("wild", golden["wild"])):
        states = torch.from_numpy(mid.copy()).to(DEV)
        out = ext.step(states, torch.from_numpy(actions).to(DEV))
        host = mid.copy()
        rout = ref.step(host, actions)
        assert_step_equal(out, rout, f"step {name}")
        assert np.array_equal(to_np(states), host)
        assert np.array_equal(host, golden[f"after_{name}"])


def test_golden_rows_observe_hands_stock(ext):
    announce("golden_rows")
    golden = np.load(GOLDEN / "rows.npz")
    states = torch.from_numpy(golden["mid"]).to(DEV)
    f, legal, player, done, status = (to_np(t) for t in ext.observe(states))
    assert np.array_equal(f32_bits(f), f32_bits(golden["features"]))
    assert np.array_equal(legal, golden["legal"])
    assert np.array_equal(player, golden["player"])
    assert np.array_equal(done, golden["done"])
    assert np.array_equal(status, golden["status"])
    ids = torch.arange(states.shape[0], device=DEV)
    assert np.array_equal(to_np(ext.hands_indexed(states, ids)), golden["hands"])
    assert np.array_equal(to_np(ext.stock_indexed(states, ids)), golden["stock"])


def test_branch_and_clone(ext, ref):
    announce("branch_clone")
    golden = np.load(GOLDEN / "rows.npz")
    parents_np = golden["mid"]
    parents = torch.from_numpy(parents_np).to(DEV)
    snapshot = parents.clone()
    m = parents_np.shape[0]
    rng = np.random.default_rng(3)
    ids = np.concatenate([rng.integers(0, m, 5000), [-1, m, m + 3]]).astype(np.int64)
    actions = rng.integers(-2, 181, ids.size).astype(np.int64)
    legal = golden["legal"]
    pick = rng.random(ids.size) < 0.7
    for k in np.nonzero(pick & (ids >= 0) & (ids < m))[0]:
        choices = np.nonzero(legal[ids[k]])[0]
        if choices.size:
            actions[k] = choices[k % choices.size]
    tid, tact = torch.from_numpy(ids).to(DEV), torch.from_numpy(actions).to(DEV)
    out = ext.branch_indexed(parents, tid, tact)
    rout = ref.branch(parents_np, ids, actions)
    assert np.array_equal(to_np(out[0]), rout[0]), "children differ"
    assert_step_equal(out[1:], rout[1:], "branch outputs")
    assert torch.equal(parents, snapshot), "parents changed"
    clones = ext.clone_indexed(parents, tid)
    assert np.array_equal(to_np(clones), ref.clone(parents_np, ids))
    # branch == clone + step on valid parents (branch50_smoke.py:113-115)
    valid = torch.from_numpy((ids >= 0) & (ids < m)).to(DEV)
    split = ext.step(clones, tact)
    assert torch.equal(out[0][valid], clones[valid])
    for a, b in zip(out[1:], split):
        assert torch.equal(a[valid], b[valid])


def test_branch_one_parent_waves(ext, ref):
    """branch_indexed where every child of a 64-child wave has the same parent (the
    scalar-head path) and where one lane differs or the shared id is invalid (the per-lane
    path), against the oracle: every golden mid-game parent kind (pending floor choices,
    finished games, ordinary decisions), every action id in turn plus out-of-range ones,
    and a partial last wave."""
    announce("branch one-parent waves")
    golden = np.load(GOLDEN / "rows.npz")
    parents_np = golden["mid"]
    m = parents_np.shape[0]
    legal = golden["legal"]
    pending = np.nonzero(parents_np[:, 27 * 8 + 3] != 0)[0]   # pactive byte of word 27
    finished = np.nonzero(parents_np[:, 29 * 8 + 7] != 0)[0]  # done byte of word 29
    ordinary = np.setdiff1d(np.arange(m), np.concatenate([pending, finished]))
    assert pending.size > 0 and finished.size > 0
    rng = np.random.default_rng(29)
    chosen = np.concatenate([pending[:24], finished[:8], rng.choice(ordinary, 96, replace=False)])
    ids, acts = [], []
    for w, p in enumerate(chosen):
        wave = np.full(64, p, dtype=np.int64)
        a = (np.arange(64) + 64 * (w % 3)) % 181 - 1  # -1 .. 179 over three waves
        good = np.nonzero(legal[p])[0]
        if good.size:  # most lanes legal
            a[::2] = good[np.arange(32) % good.size]
        if w % 17 == 5:
            wave[63] = (p + 1) % m  # one lane with another parent
        ids.append(wave)
        acts.append(a)
    ids.append(np.full(64, m, dtype=np.int64))  # a wave of one invalid parent id
    acts.append(np.zeros(64, dtype=np.int64))
    ids.append(np.full(37, chosen[0], dtype=np.int64))  # a partial last wave
    acts.append(np.arange(37, dtype=np.int64))
    ids, acts = np.concatenate(ids), np.concatenate(acts)
    parents = torch.from_numpy(parents_np).to(DEV)
    snapshot = parents.clone()
    out = ext.branch_indexed(parents, torch.from_numpy(ids).to(DEV), torch.from_numpy(acts).to(DEV))
    rout = ref.branch(parents_np, ids, acts)
    assert np.array_equal(to_np(out[0]), rout[0]), "children differ"
    assert_step_equal(out[1:], rout[1:], "one-parent branch outputs")
    assert torch.equal(parents, snapshot)
    status = to_np(out[4])
    assert (status == 0).sum() > 1000 and (status == -1).sum() == 64


def test_empty_batches(ext):
    announce("empty_batches")
    states = ext.create(torch.zeros(4, dtype=torch.long, device=DEV),
                        torch.zeros(4, dtype=torch.long, device=DEV))
    empty = torch.empty(0, dtype=torch.long, device=DEV)
    assert tuple(ext.clone_indexed(states, empty).shape) == (0, 248)
    br = ext.branch_indexed(states, empty, empty)
    assert tuple(br[0].shape) == (0, 248) and all(t.numel() == 0 for t in br[1:])
    assert ext.observe_indexed(states, empty)[0].shape == (0, 720)
    assert ext.create(empty, empty).shape == (0, 248)
    ev = ext.step_events_indexed(states, empty, empty)
    assert tuple(ev[5].shape) == (0, 9)


def test_shape_errors_raise(ext):
    announce("shape_errors")
    states = ext.create(torch.zeros(4, dtype=torch.long, device=DEV),
                        torch.zeros(4, dtype=torch.long, device=DEV))
    with pytest.raises(RuntimeError, match="states second dimension"):
        ext.observe(torch.zeros(4, 100, dtype=torch.uint8, device=DEV))
    with pytest.raises(RuntimeError, match="same batch size"):
        ext.step(states, torch.zeros(3, dtype=torch.long, device=DEV))
    with pytest.raises(RuntimeError, match="wrong dtype"):
        ext.step(states, torch.zeros(4, dtype=torch.int32, device=DEV))
    with pytest.raises(RuntimeError, match="CUDA tensor"):
        ext.observe(states.cpu())


def test_driver_sample_and_reset(ext, ref):
    """The random-policy driver kernels: GPU sampler == numpy sampler; reset_done
    re-creates exactly the finished rows from their next seed."""
    announce("driver_sample_reset")
    n = 3000
    base = 0x1234567
    gen = torch.zeros(n, dtype=torch.int32, device=DEV)
    sampler = ext.seed_samplers(n, base, gen)
    host_sampler = np.array([splitmix_first(base + i) for i in range(n)], dtype=np.uint64)
    assert np.array_equal(to_np(sampler).view(np.uint64), host_sampler)
    seeds = (np.uint64(base) + np.arange(n, dtype=np.uint64)).view(np.int64)
    states = ext.create(torch.from_numpy(seeds).to(DEV),
                        torch.from_numpy(np.arange(n) & 1).to(DEV))
    completed = torch.zeros(1, dtype=torch.long, device=DEV)
    for _ in range(30):
        _, legal, _, done, _ = ext.observe(states)
        actions = ext.sample_uniform(legal, sampler)
        expect = sample_actions(to_np(legal), host_sampler, np.ones(n, dtype=bool))
        assert np.array_equal(to_np(actions), expect)
        _, sdone, _, _, _ = ext.step(states, actions)
        before = to_np(gen).copy()
        ext.reset_done(states, sdone, base, gen, sampler, completed)
        reset = to_np(sdone)
        after = to_np(gen)
        assert np.array_equal(after, before + reset)
        rows = to_np(states)
        for k, i in enumerate(np.nonzero(reset)[0]):
            seed = (base + int(i) + n * int(after[i])) & (2**64 - 1)
            host_sampler[i] = splitmix_first(seed)
            if k < 8:
                expect_row = ref.create(np.array([seed], dtype=np.uint64).view(np.int64),
                                        np.array([i & 1]))
                assert np.array_equal(rows[i], expect_row[0])
    assert int(completed.item()) == int(to_np(gen).sum())


def test_driver_spare_reset_matches_reset(ext):
    """reset_done_spares (next games pre-dealt by refill_spares every few steps, dealt
    inline when a spare is stale) leaves states, generations, samplers and the completed
    count identical to reset_done."""
    announce("driver_spare_reset")
    n = 2500
    base = 0x7654321
    seeds = (np.uint64(base) + np.arange(n, dtype=np.uint64)).view(np.int64)
    first = torch.from_numpy(np.arange(n) & 1).to(DEV)
    a = ext.create(torch.from_numpy(seeds).to(DEV), first)
    b = a.clone()
    gen_a = torch.zeros(n, dtype=torch.int32, device=DEV)
    gen_b = gen_a.clone()
    smp_a = ext.seed_samplers(n, base, gen_a)
    smp_b = smp_a.clone()
    done_a = torch.zeros(1, dtype=torch.long, device=DEV)
    done_b = done_a.clone()
    spares = torch.zeros((n, 248), dtype=torch.uint8, device=DEV)
    spare_gen = torch.zeros(n, dtype=torch.int32, device=DEV)
    # c: the same batch as two slices on their own streams, seeds strided by the batch
    # (no counter: completed=None; generation counts the finished games)
    c = a.clone()
    gen_c, smp_c = gen_a.clone(), smp_a.clone()
    spares_c = torch.zeros_like(spares)
    spare_gen_c = torch.zeros_like(spare_gen)
    half = n // 2  # even
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for step in range(60):
        if step % 3 == 0:
            ext.refill_spares(spares, spare_gen, gen_b, base)
        _, legal, _, _, _ = ext.observe(a)
        actions = ext.sample_uniform(legal, smp_a)
        smp_b.copy_(smp_a)
        smp_c.copy_(smp_a)
        _, sdone, _, _, _ = ext.step(a, actions)
        ext.step(b, actions)
        ext.reset_done(a, sdone, base, gen_a, smp_a, done_a)
        ext.reset_done_spares(b, sdone, base, gen_b, smp_b, done_b, spares, spare_gen)
        cur = torch.cuda.current_stream()
        for k, st in enumerate(streams):
            st.wait_stream(cur)
            with torch.cuda.stream(st):
                r = slice(k * half, (k + 1) * half)
                if step % 5 == 0:
                    ext.refill_spares(spares_c[r], spare_gen_c[r], gen_c[r], base + k * half, n)
                _, cdone, _, _, _ = ext.step(c[r], actions[r])
                ext.reset_done_spares(c[r], cdone, base + k * half, gen_c[r], smp_c[r], None,
                                      spares_c[r], spare_gen_c[r], n)
        for st in streams:
            cur.wait_stream(st)
        assert torch.equal(a, b) and torch.equal(a, c), step
        assert torch.equal(gen_a, gen_b) and torch.equal(smp_a, smp_b), step
        assert torch.equal(gen_a, gen_c) and torch.equal(smp_a, smp_c), step
    assert int(done_a.item()) == int(done_b.item()) == int(gen_c.sum().item()) > n


def test_step_reset_spares_matches_step_then_reset(ext):
    """step_reset_spares == step followed by reset_done_spares (no counter): the same step
    outputs, states, generations and samplers, with spares refilled every few steps so
    that both the spare copy and the inline deal occur; also as two strided slices."""
    announce("step_reset_spares")
    n = 2500  # a partial last tile
    base = 0x3141592
    seeds = (np.uint64(base) + np.arange(n, dtype=np.uint64)).view(np.int64)
    a = ext.create(torch.from_numpy(seeds).to(DEV), torch.from_numpy(np.arange(n) & 1).to(DEV))
    gen_a = torch.zeros(n, dtype=torch.int32, device=DEV)
    smp_a = ext.seed_samplers(n, base, gen_a)
    spares_a = torch.zeros((n, 248), dtype=torch.uint8, device=DEV)
    sg_a = torch.zeros(n, dtype=torch.int32, device=DEV)
    b, gen_b, smp_b, spares_b, sg_b = (t.clone() for t in (a, gen_a, smp_a, spares_a, sg_a))
    c, gen_c, smp_c, spares_c, sg_c = (t.clone() for t in (a, gen_a, smp_a, spares_a, sg_a))
    half = n // 2  # even
    for step in range(60):
        if step % 4 == 0:
            ext.refill_spares(spares_a, sg_a, gen_a, base)
            ext.refill_spares(spares_b, sg_b, gen_b, base)
        if step % 6 == 0:  # slice 1 never gets spares: its rows are all dealt inline
            ext.refill_spares(spares_c[:half], sg_c[:half], gen_c[:half], base, n)
        _, _, _, _, _, actions = ext.observe_sample(a, smp_a)
        smp_b.copy_(smp_a)
        smp_c.copy_(smp_a)
        out_a = ext.step(a, actions)
        ext.reset_done_spares(a, out_a[1], base, gen_a, smp_a, None, spares_a, sg_a)
        out_b = ext.step_reset_spares(b, actions, base, gen_b, smp_b, spares_b, sg_b)
        parts = []
        for k in range(2):
            r = slice(k * half, (k + 1) * half)
            parts.append(ext.step_reset_spares(c[r], actions[r], base + k * half, gen_c[r],
                                               smp_c[r], spares_c[r], sg_c[r], n))
        for j in range(5):
            assert torch.equal(out_a[j], out_b[j]), (step, j)
            assert torch.equal(out_a[j], torch.cat([parts[0][j], parts[1][j]])), (step, j)
        assert torch.equal(a, b) and torch.equal(a, c), step
        assert torch.equal(gen_a, gen_b) and torch.equal(smp_a, smp_b), step
        assert torch.equal(gen_a, gen_c) and torch.equal(smp_a, smp_c), step
    assert int(gen_a.sum().item()) > n


@pytest.mark.parametrize("bf16", [True, False])
def test_step_observe_spares_matches_step_then_observe(ext, bf16):
    """step_observe_spares == step_reset_spares followed by observe (float32 features) or
    observe_bf16 of the new states: the five step outputs, the five observation outputs,
    the rows, generations and samplers, bit for bit, over 60 steps with spares refilled
    every few steps (spare copies and stale spares both occur), at a partial last tile."""
    announce(f"step_observe_spares (bf16={bf16})")
    n = 2500
    base = 0x5772156
    seeds = (np.uint64(base) + np.arange(n, dtype=np.uint64)).view(np.int64)
    a = ext.create(torch.from_numpy(seeds).to(DEV), torch.from_numpy(np.arange(n) & 1).to(DEV))
    gen_a = torch.zeros(n, dtype=torch.int32, device=DEV)
    smp_a = ext.seed_samplers(n, base, gen_a)
    sp_a = torch.zeros((2 * n, 248), dtype=torch.uint8, device=DEV)
    sg_a = torch.zeros(2 * n, dtype=torch.int32, device=DEV)
    b, gen_b, smp_b, sp_b, sg_b = (t.clone() for t in (a, gen_a, smp_a, sp_a, sg_a))
    feats = torch.full((n, 720), float("nan"), device=DEV,
                       dtype=torch.bfloat16 if bf16 else torch.float32)
    for step in range(60):
        if step % 7 == 0:
            ext.refill_spares(sp_a, sg_a, gen_a, base)
            ext.refill_spares(sp_b, sg_b, gen_b, base)
        _, _, _, _, _, actions = ext.observe_sample(a, smp_a)
        smp_b.copy_(smp_a)
        st = ext.step_reset_spares(a, actions, base, gen_a, smp_a, sp_a, sg_a)
        if bf16:
            ob = ext.observe_bf16(a, torch.empty_like(feats))
        else:
            ob = ext.observe(a)
        fused = ext.step_observe_spares(b, actions, base, gen_b, smp_b, sp_b, sg_b, feats)
        assert fused[5].data_ptr() == feats.data_ptr()
        for k, want in enumerate(list(st) + list(ob)):
            got = fused[k]
            if got.is_floating_point():  # bit patterns (NaN-safe)
                got, want = got.view(torch.int16 if bf16 and k == 5 else torch.int32), \
                    want.view(torch.int16 if bf16 and k == 5 else torch.int32)
            assert torch.equal(got, want), (step, k)
        assert torch.equal(a, b) and torch.equal(gen_a, gen_b) and torch.equal(smp_a, smp_b), step
    assert int(gen_a.sum().item()) > n


def test_branch_observe_matches_branch_then_observe(ext):
    """branch_observe_indexed == branch_indexed followed by observe_indexed of the children:
    every output bit-identical, with invalid and duplicate parent ids, wild actions and a
    partial last tile; the parents are not modified."""
    announce("branch_observe_indexed")
    rows = torch.from_numpy(np.load(GOLDEN / "rows.npz")["mid"]).to(DEV)
    m = rows.shape[0]
    g = np.random.default_rng(41)
    n = 5000
    ids = g.integers(0, m, n)
    ids[:7] = [-1, m, m + 100, 0, 0, 5, -7]
    actions = g.integers(-3, 185, n)
    ids_t = torch.from_numpy(ids).to(DEV)
    act_t = torch.from_numpy(actions).to(DEV)
    before = rows.clone()
    fused = ext.branch_observe_indexed(rows, ids_t, act_t)
    assert torch.equal(rows, before)
    br = ext.branch_indexed(rows, ids_t, act_t)
    ob = ext.observe_indexed(br[0], torch.arange(n, device=DEV))
    for k, want in enumerate(list(br) + list(ob)):
        assert torch.equal(fused[k], want), k
    assert ext.branch_observe_indexed(rows, ids_t[:0], act_t[:0])[0].shape == (0, 248)


def test_play_random_matches_observe_sample_then_step(ext):
    """play_random == observe_sample followed by step_reset_spares: all eleven outputs,
    the rows, generations and samplers, over 60 steps with spares refilled every few
    steps (spare and inline re-deals both occur), at a partial last tile."""
    announce("play_random")
    n = 3001 * 2  # a partial last tile, even
    base = 0x2718281
    seeds = (np.uint64(base) + np.arange(n, dtype=np.uint64)).view(np.int64)
    a = ext.create(torch.from_numpy(seeds).to(DEV), torch.from_numpy(np.arange(n) & 1).to(DEV))
    gen_a = torch.zeros(n, dtype=torch.int32, device=DEV)
    smp_a = ext.seed_samplers(n, base, gen_a)
    sp_a = torch.zeros((n, 248), dtype=torch.uint8, device=DEV)
    sg_a = torch.zeros(n, dtype=torch.int32, device=DEV)
    b, gen_b, smp_b, sp_b, sg_b = (t.clone() for t in (a, gen_a, smp_a, sp_a, sg_a))
    for step in range(60):
        if step % 5 == 0:
            ext.refill_spares(sp_a, sg_a, gen_a, base)
            ext.refill_spares(sp_b, sg_b, gen_b, base)
        obs = ext.observe_sample(a, smp_a)
        st = ext.step_reset_spares(a, obs[5], base, gen_a, smp_a, sp_a, sg_a)
        fused = ext.play_random(b, smp_b, base, gen_b, sp_b, sg_b)
        for k, want in enumerate(list(obs) + list(st)):
            assert torch.equal(fused[k], want), (step, k)
        assert torch.equal(a, b) and torch.equal(gen_a, gen_b) and torch.equal(smp_a, smp_b), step
    assert int(gen_a.sum().item()) > n


def test_observe_sample_matches_observe_then_sample(ext):
    """observe_sample == observe followed by sample_uniform: the same five observation
    outputs, actions and sampler words, over a random-policy run with resets (so rows
    at every stage of a game, finished rows with an empty mask included)."""
    announce("observe_sample")
    n = 4100  # a partial last tile
    base = 0x5A5A5A5
    seeds = (np.uint64(base) + np.arange(n, dtype=np.uint64)).view(np.int64)
    states = ext.create(torch.from_numpy(seeds).to(DEV),
                        torch.from_numpy(np.arange(n) & 1).to(DEV))
    gen = torch.zeros(n, dtype=torch.int32, device=DEV)
    smp_a = ext.seed_samplers(n, base, gen)
    smp_b = smp_a.clone()
    empty = 0
    for step in range(40):
        obs = ext.observe(states)
        actions = ext.sample_uniform(obs[1], smp_a)
        fused = ext.observe_sample(states, smp_b)
        for k in range(5):
            assert torch.equal(obs[k], fused[k]), (step, k)
        assert torch.equal(actions, fused[5]) and torch.equal(smp_a, smp_b), step
        empty += int((actions < 0).sum().item())
        _, done, _, _, _ = ext.step(states, actions)
        if step % 7 == 6:  # leave finished rows in place for a few steps first
            ext.reset_done(states, done, base, gen, smp_a)
            smp_b.copy_(smp_a)
    assert empty > 0 and int(gen.sum().item()) > 0
    assert ext.observe_sample(states[:0], smp_a[:0])[5].numel() == 0


def test_repeatable(ext):
    announce("repeatable")
    golden = np.load(GOLDEN / "rows.npz")
    a = torch.from_numpy(golden["mid"]).to(DEV)
    b = a.clone()
    acts = torch.from_numpy(golden["first_legal"]).to(DEV)
    oa, ob = ext.step(a, acts), ext.step(b, acts)
    assert torch.equal(a, b)
    for x, y in zip(oa, ob):
        assert torch.equal(x, y)
    f1 = ext.observe(a)[0]
    f2 = ext.observe(a)[0]
    assert torch.equal(f1, f2)


def test_padding_bytes_zero(ext):
    announce("padding_zero")
    seeds, first = c1_seeds(512)
    states = ext.create(torch.from_numpy(seeds).to(DEV), torch.from_numpy(first).to(DEV))
    rows = to_np(states)
    for lo, hi in PADDING:
        assert not rows[:, lo:hi].any()


def test_play_random_full_batch_matches_oracle(ext, ref):
    """The random-policy loop at its full size: 65,536 resident games, 24 play_random
    launches with the spares refilled every 8 (the loop the throughput figure times).
    Each step's observation, actions and step outputs, and the rows after it, against the
    oracle playing the same protocol: observe, the uniform legal draw, step, and a
    finished game's row re-dealt from seed base + i + 65,536 * generation with a fresh
    sampler.  Most games finish within 24 steps, so spare and inline re-deals both run."""
    announce("play_random full batch vs oracle")
    n = 65536
    seeds, first = c1_seeds(n)
    states = ext.create(torch.from_numpy(seeds).to(DEV), torch.from_numpy(first).to(DEV))
    host = ref.create(seeds, first)
    gen = torch.zeros(n, dtype=torch.int32, device=DEV)
    smp = ext.seed_samplers(n, SEED_BASE, gen)
    sampler = np.array([splitmix_first(int(s) & (2**64 - 1)) for s in seeds], dtype=np.uint64)
    assert np.array_equal(to_np(smp).view(np.uint64), sampler)
    spares = torch.zeros((n, 248), dtype=torch.uint8, device=DEV)
    spare_gen = torch.zeros(n, dtype=torch.int32, device=DEV)
    hgen = np.zeros(n, dtype=np.int64)
    for step in range(24):
        if step % 8 == 0:
            ext.refill_spares(spares, spare_gen, gen, SEED_BASE, n)
        out = ext.play_random(states, smp, SEED_BASE, gen, spares, spare_gen, n)
        robs = ref.observe(host)
        assert_observe_equal(out[:5], robs, f"observation, step {step}")
        actions = sample_actions(robs[1], sampler, ~robs[3])
        assert np.array_equal(to_np(out[5]), actions), f"actions, step {step}"
        rout = ref.step(host, actions)
        assert_step_equal(out[6:], rout, f"step {step}")
        ended = np.nonzero(rout[1])[0]
        hgen[ended] += 1
        new_seeds = ((np.uint64(SEED_BASE) + ended.astype(np.uint64)
                      + np.uint64(n) * hgen[ended].astype(np.uint64))).view(np.int64)
        host[ended] = ref.create(new_seeds, ended & 1)
        sampler[ended] = [splitmix_first(int(s) & (2**64 - 1)) for s in new_seeds]
        assert np.array_equal(to_np(states), host), f"rows, step {step}"
    assert np.array_equal(to_np(gen), hgen)
    assert np.array_equal(to_np(smp).view(np.uint64), sampler)
    assert hgen.sum() > n // 2


def test_play_random_bench_block_every_step_matches_oracle(ext, ref):
    """The throughput loop exactly as bench.py runs it: 65,536 resident games, two spare
    slots (spares [2 x 65,536, 248]), blocks of refill_spares then one play_random launch
    of 32 steps, three blocks.  The launch keeps every step's outputs (record=True: the
    same kernel, writing step s to its own block of rows), and each of the 96 steps'
    observation (features as bit patterns, mask, player, done, status), action and step
    outputs is compared with the oracle playing the same protocol, then the rows,
    generations and samplers after each block."""
    announce("play_random bench block (65,536 x 32 steps x 3, 2 slots) vs oracle")
    n, k, slots = 65536, 32, 2
    seeds, first = c1_seeds(n)
    states = ext.create(torch.from_numpy(seeds).to(DEV), torch.from_numpy(first).to(DEV))
    host = ref.create(seeds, first)
    gen = torch.zeros(n, dtype=torch.int32, device=DEV)
    smp = ext.seed_samplers(n, SEED_BASE, gen)
    sampler = np.array([splitmix_first(int(s) & (2**64 - 1)) for s in seeds], dtype=np.uint64)
    spares = torch.zeros((slots * n, 248), dtype=torch.uint8, device=DEV)
    spare_gen = torch.zeros(slots * n, dtype=torch.int32, device=DEV)
    hgen = np.zeros(n, dtype=np.int64)
    for block in range(3):
        ext.refill_spares(spares, spare_gen, gen, SEED_BASE, n)
        out = ext.play_random(states, smp, SEED_BASE, gen, spares, spare_gen, n, k, record=True)
        assert tuple(out[0].shape) == (k, n, 720) and tuple(out[10].shape) == (k, n)
        for step in range(k):
            label = f"block {block}, step {step}"
            robs = ref.observe(host)
            assert_observe_equal([t[step] for t in out[:5]], robs, f"observation, {label}")
            actions = sample_actions(robs[1], sampler, ~robs[3])
            assert np.array_equal(to_np(out[5][step]), actions), f"actions, {label}"
            rout = ref.step(host, actions)
            assert_step_equal([t[step] for t in out[6:]], rout, label)
            ended = np.nonzero(rout[1])[0]
            hgen[ended] += 1
            new_seeds = ((np.uint64(SEED_BASE) + ended.astype(np.uint64)
                          + np.uint64(n) * hgen[ended].astype(np.uint64))).view(np.int64)
            host[ended] = ref.create(new_seeds, ended & 1)
            sampler[ended] = [splitmix_first(int(s) & (2**64 - 1)) for s in new_seeds]
        del out
        assert np.array_equal(to_np(states), host), f"rows after block {block}"
        assert np.array_equal(to_np(gen), hgen), f"generations after block {block}"
        assert np.array_equal(to_np(smp).view(np.uint64), sampler), f"samplers, block {block}"
    # most rows finished at least twice, so both slots' spares and inline deals ran
    assert (hgen >= 2).mean() > 0.5, np.bincount(hgen)


@pytest.mark.parametrize("n", [3001 * 2 + 2, 65536])
def test_play_random_record_matches_single_steps(ext, n):
    """record=True changes where the outputs go, never what they are: a recorded launch
    of K steps gives, in block s, the outputs of the s-th of K one-step launches, and the
    same rows, generations and samplers, at a partial last tile (n not a multiple of 4
    or 64: the blocks are padded to a multiple of 4 rows) and at the full batch."""
    announce(f"play_random record (n={n})")
    base = 0x5A5A5A5A
    seeds = (np.uint64(base) + np.arange(n, dtype=np.uint64)).view(np.int64)
    a = ext.create(torch.from_numpy(seeds).to(DEV), torch.from_numpy(np.arange(n) & 1).to(DEV))
    gen_a = torch.zeros(n, dtype=torch.int32, device=DEV)
    smp_a = ext.seed_samplers(n, base, gen_a)
    sp_a = torch.zeros((2 * n, 248), dtype=torch.uint8, device=DEV)
    sg_a = torch.zeros(2 * n, dtype=torch.int32, device=DEV)
    b, gen_b, smp_b, sp_b, sg_b = (t.clone() for t in (a, gen_a, smp_a, sp_a, sg_a))
    for block, k in enumerate([5, 32, 1]):
        ext.refill_spares(sp_a, sg_a, gen_a, base)
        ext.refill_spares(sp_b, sg_b, gen_b, base)
        rec = ext.play_random(b, smp_b, base, gen_b, sp_b, sg_b, steps=k, record=True)
        for step in range(k):
            single = ext.play_random(a, smp_a, base, gen_a, sp_a, sg_a)
            for j, (x, y) in enumerate(zip(single, rec)):
                assert torch.equal(x, y[step]), (block, step, j)
        assert torch.equal(a, b) and torch.equal(gen_a, gen_b) and torch.equal(smp_a, smp_b), block
    empty = ext.play_random(b[:0], smp_b[:0], base, gen_b[:0], sp_b[:0], sg_b[:0], steps=3,
                            record=True)
    assert tuple(empty[0].shape) == (3, 0, 720)


def test_branch_observe_full_batch(ext, ref):
    """The branch stress at its full size: 4,096 mid-game roots x 256 children (child k of
    a root takes legal[k] while k < count, else legal[xorshift % count]) through
    branch_observe_indexed.  32,768 sampled children against the oracle (branch, then
    observe of the child), and the whole batch equal to branch_indexed followed by
    observe_indexed; the roots are not modified."""
    announce("branch_observe full batch")
    roots_n, per = 4096, 256
    idx = torch.arange(roots_n, dtype=torch.int64, device=DEV)
    roots = ext.create(idx * 7919 + SEED_BASE, idx & 1)
    gen = torch.zeros(roots_n, dtype=torch.int32, device=DEV)
    smp = ext.seed_samplers(roots_n, SEED_BASE, gen)
    depth = torch.from_numpy(np.random.default_rng(17).integers(3, 16, roots_n)).to(DEV)
    for t in range(15):
        _, legal, _, _, _ = ext.observe(roots)
        acts = ext.sample_uniform(legal, smp)
        acts = torch.where(depth > t, acts, torch.full_like(acts, -1))
        keep = roots.clone()
        ext.step(roots, acts)
        roots = torch.where((depth > t).unsqueeze(1), roots, keep)
    roots_np = to_np(roots)
    _, legal, _, _, _ = ref.observe(roots_np)
    g = np.random.default_rng(23)
    ids = np.repeat(np.arange(roots_n, dtype=np.int64), per)
    k = np.tile(np.arange(per, dtype=np.int64), roots_n)
    counts = legal.sum(axis=1)[ids]
    draw = g.integers(0, 2**62, ids.size)
    pick = np.where(k < counts, k, draw % np.maximum(counts, 1))
    order = np.argsort(~legal, axis=1, kind="stable")  # legal actions first, ascending
    actions = np.where(counts > 0, order[ids, pick], -1).astype(np.int64)
    ids_t, act_t = torch.from_numpy(ids).to(DEV), torch.from_numpy(actions).to(DEV)
    before = roots.clone()
    fused = ext.branch_observe_indexed(roots, ids_t, act_t)
    assert torch.equal(roots, before)
    sample = np.sort(g.choice(ids.size, 32768, replace=False))
    rch = ref.branch(roots_np, ids[sample], actions[sample])
    assert np.array_equal(to_np(fused[0][torch.from_numpy(sample).to(DEV)]), rch[0])
    sel = torch.from_numpy(sample).to(DEV)
    assert_step_equal([t[sel] for t in fused[1:6]], rch[1:], "sampled children")
    robs = ref.observe(rch[0])
    assert_observe_equal([t[sel] for t in fused[6:11]], robs, "sampled children's observation")
    br = ext.branch_indexed(roots, ids_t, act_t)
    for j, want in enumerate(br):
        assert torch.equal(fused[j], want), j
    del br
    ob = ext.observe_indexed(fused[0], torch.arange(ids.size, device=DEV))
    for j, want in enumerate(ob):
        assert torch.equal(fused[6 + j], want), j


@pytest.mark.parametrize("n", [3001 * 2, 65536])
def test_play_random_steps_match_single_steps(ext, n):
    """play_random(steps=K) == K calls of one step: rows, generations, samplers and the
    eleven outputs of the last step, for K = 1, 3, 8, 16 and 32 (the bench's block) over several
    blocks, with the spares refilled only every other block (so spare and inline re-deals
    both occur), at a partial last tile and at the full batch."""
    announce(f"play_random steps (n={n})")
    base = 0x31415926
    seeds = (np.uint64(base) + np.arange(n, dtype=np.uint64)).view(np.int64)
    a = ext.create(torch.from_numpy(seeds).to(DEV), torch.from_numpy(np.arange(n) & 1).to(DEV))
    gen_a = torch.zeros(n, dtype=torch.int32, device=DEV)
    smp_a = ext.seed_samplers(n, base, gen_a)
    sp_a = torch.zeros((n, 248), dtype=torch.uint8, device=DEV)
    sg_a = torch.zeros(n, dtype=torch.int32, device=DEV)
    b, gen_b, smp_b, sp_b, sg_b = (t.clone() for t in (a, gen_a, smp_a, sp_a, sg_a))
    for block, k in enumerate([8, 3, 16, 1, 32, 16]):
        if block % 2 == 0:
            ext.refill_spares(sp_a, sg_a, gen_a, base)
            ext.refill_spares(sp_b, sg_b, gen_b, base)
        for _ in range(k):
            single = ext.play_random(a, smp_a, base, gen_a, sp_a, sg_a)
        multi = ext.play_random(b, smp_b, base, gen_b, sp_b, sg_b, steps=k)
        for j, (x, y) in enumerate(zip(single, multi)):
            assert torch.equal(x, y), (block, k, j)
        assert torch.equal(a, b) and torch.equal(gen_a, gen_b) and torch.equal(smp_a, smp_b), block
    assert int(gen_a.sum().item()) > n // 2
    with pytest.raises(RuntimeError):
        ext.play_random(b, smp_b, base, gen_b, sp_b, sg_b, steps=0)


@pytest.mark.parametrize("slots", [2, 4])
def test_spare_slots_do_not_change_results(ext, slots):
    """Several pre-dealt games per row (spares [slots * n, 248], slot-major) change where
    a finished row's next game comes from, never which game it is: play_random blocks of
    16 steps, and step_reset_spares / reset_done_spares step by step, give the same rows,
    generations, samplers and outputs as one slot, at a partial last tile."""
    announce(f"spare slots ({slots})")
    n, base = 3001 * 2, 0x27182818
    seeds = (np.uint64(base) + np.arange(n, dtype=np.uint64)).view(np.int64)
    a = ext.create(torch.from_numpy(seeds).to(DEV), torch.from_numpy(np.arange(n) & 1).to(DEV))
    gen_a = torch.zeros(n, dtype=torch.int32, device=DEV)
    smp_a = ext.seed_samplers(n, base, gen_a)
    b, gen_b, smp_b = a.clone(), gen_a.clone(), smp_a.clone()
    sp_a = torch.zeros((n, 248), dtype=torch.uint8, device=DEV)
    sg_a = torch.zeros(n, dtype=torch.int32, device=DEV)
    sp_b = torch.zeros((slots * n, 248), dtype=torch.uint8, device=DEV)
    sg_b = torch.zeros(slots * n, dtype=torch.int32, device=DEV)
    for block in range(4):
        ext.refill_spares(sp_a, sg_a, gen_a, base)
        ext.refill_spares(sp_b, sg_b, gen_b, base)
        x = ext.play_random(a, smp_a, base, gen_a, sp_a, sg_a, steps=16)
        y = ext.play_random(b, smp_b, base, gen_b, sp_b, sg_b, steps=16)
        for j, (u, v) in enumerate(zip(x, y)):
            assert torch.equal(u, v), (block, j)
        assert torch.equal(a, b) and torch.equal(gen_a, gen_b) and torch.equal(smp_a, smp_b), block
    # the two-launch path: every slot's refill, then single steps with auto-reset
    ext.refill_spares(sp_a, sg_a, gen_a, base)
    ext.refill_spares(sp_b, sg_b, gen_b, base)
    for t in range(12):
        _, _, _, _, _, act = ext.observe_sample(a, smp_a)
        _, _, _, _, _, act_b = ext.observe_sample(b, smp_b)
        assert torch.equal(act, act_b), t
        if t % 2:
            x = ext.step_reset_spares(a, act, base, gen_a, smp_a, sp_a, sg_a)
            y = ext.step_reset_spares(b, act, base, gen_b, smp_b, sp_b, sg_b)
        else:
            x = ext.step(a, act)
            y = ext.step(b, act)
            ext.reset_done_spares(a, x[1].bool(), base, gen_a, smp_a, None, sp_a, sg_a)
            ext.reset_done_spares(b, y[1].bool(), base, gen_b, smp_b, None, sp_b, sg_b)
        for j, (u, v) in enumerate(zip(x, y)):
            assert torch.equal(u, v), (t, j)
        assert torch.equal(a, b) and torch.equal(gen_a, gen_b) and torch.equal(smp_a, smp_b), t
    assert int(gen_a.sum().item()) > n
    with pytest.raises(RuntimeError):
        ext.refill_spares(torch.zeros((3 * n, 248), dtype=torch.uint8, device=DEV),
                          torch.zeros(3 * n, dtype=torch.int32, device=DEV), gen_b, base)
