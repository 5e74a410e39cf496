"""Writes the golden fixtures under tests/golden/ from the reference engine build.

    python tests/golden/make_golden.py

Runs the reference's own header-only engine (oracle/_ref/libcugo_ref.so, built by
`make -C oracle ref` from the reference checkout) and stores inputs and expected
outputs as .npz data:

  c1_random_policy.npz  4,096 random-policy games (seed = 0x243F6A8885A308D3 + i,
                        first = i & 1, sampler xorshift64 seeded by SplitMix64(seed)):
                        per-game FNV-1a digest of every decision record, decision count
                        and exact final reward of player 0; plus the full records of
                        games 0..15 (first 64 decisions).
  rows.npz              created rows and start records of games 0..255; mid-game rows
                        (incl. pending floor choices) with their observations, hands,
                        stock peeks and the step results of a fixed action list.
  canonical.npz         digests of the canonical whole-game driver (see canonical()).
  scenarios.npz         the hand-built rule scenarios of scenarios.py, played (see
                        scenario_fixture()).

    python tests/golden/make_golden.py canonical     (one fixture only)
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle.ref import SEED_BASE, RefEngine, sample_actions, splitmix_first  # noqa: E402


def c1(ref: RefEngine) -> None:
    digest, steps, reward, records, total = ref.play_random(SEED_BASE, 4096, threads=8,
                                                            record_games=16, record_cap=64)
    np.savez_compressed(HERE / "c1_random_policy.npz", digest=digest, steps=steps,
                        final_reward=reward, records=records, total=np.int64(total))
    print(f"c1: games=4096 decisions={total} mean={total / 4096:.2f}")


def rows(ref: RefEngine) -> None:
    n = 256
    idx = np.arange(n, dtype=np.int64)
    seeds = (np.uint64(SEED_BASE) + idx.astype(np.uint64)).view(np.int64)
    first = idx & 1
    created = ref.create(seeds, first)
    start = ref.start(created)
    # Play every game forward by a seed-dependent number of random decisions and keep
    # the intermediate rows: a mix of primary, Go/Stop, Gukjin, pending floor-choice and
    # finished states.
    states = created.copy()
    sampler = np.array([splitmix_first(int(s) & (2**64 - 1)) for s in seeds], dtype=np.uint64)
    keep = []
    for step in range(40):
        _, legal, _, done, _ = ref.observe(states)
        actions = sample_actions(legal, sampler, ~done)
        ref.step(states, actions)
        if step % 4 == 3:
            keep.append(states.copy())
    mid = np.concatenate(keep, axis=0)
    obs = ref.observe(mid)
    ids = np.arange(mid.shape[0], dtype=np.int64)
    hands = ref.hands(mid, ids)
    stock = ref.stock(mid, ids)
    # A fixed action list over every row: first legal action, and out-of-range ones.
    legal = obs[1]
    first_legal = np.where(legal.any(axis=1), legal.argmax(axis=1), -1).astype(np.int64)
    wild = (ids * 37) % 183 - 2
    stepped = mid.copy()
    out_first = ref.step(stepped, first_legal, events=True)
    stepped_wild = mid.copy()
    out_wild = ref.step(stepped_wild, wild, events=True)
    np.savez_compressed(
        HERE / "rows.npz", seeds=seeds, first=first, created=created, start=start, mid=mid,
        features=obs[0], legal=obs[1], player=obs[2], done=obs[3], status=obs[4], hands=hands,
        stock=stock, first_legal=first_legal, after_first=stepped,
        first_out=np.stack([o.astype(np.float64) for o in out_first[:5]]),
        first_events=out_first[5], wild=wild, after_wild=stepped_wild,
        wild_out=np.stack([o.astype(np.float64) for o in out_wild[:5]]), wild_events=out_wild[5])
    pending = int((mid[:, 219] != 0).sum())
    print(f"rows: created={n} mid={mid.shape[0]} pending={pending} done={int(obs[3].sum())}")


GOLDEN_GAMMA = 0x9E3779B97F4A7C15


def canonical(ref: RefEngine) -> None:
    """Canonical-driver digests (rollout_canonical_torch50, five words a game): the
    8,192 seeds of the reference's rollout-equivalence test (torch50_test.cpp:160-191),
    4,096 seeds of its GPU bench (cuda_rollout50_bench.cu:22-33, warm-up base), and 512
    of those games cut at 5 primary actions (the max-actions ending)."""
    def seeds_of(base: int, n: int) -> np.ndarray:
        i = np.arange(n, dtype=np.uint64)
        return (np.uint64(base) + i * np.uint64(GOLDEN_GAMMA)).view(np.int64)

    test_seeds = seeds_of(0x1F83D9ABFB41BD6B, 8192)
    bench_seeds = seeds_of(0x6A09E667F3BCC909, 4096)
    test_first = np.arange(8192, dtype=np.int64) & 1
    bench_first = np.arange(4096, dtype=np.int64) & 1
    np.savez_compressed(
        HERE / "canonical.npz", test_seeds=test_seeds, test_first=test_first,
        test_digest=ref.rollout_canonical(test_seeds, test_first),
        bench_seeds=bench_seeds, bench_first=bench_first,
        bench_digest=ref.rollout_canonical(bench_seeds, bench_first),
        bench_explicit=ref.rollout_canonical(bench_seeds, bench_first, explicit=True),
        cut_digest=ref.rollout_canonical(bench_seeds[:512], bench_first[:512], max_actions=5))
    print("canonical: 8,192 + 4,096 + 512 digests")


def scenario_fixture(ref: RefEngine) -> None:
    """The hand-built rule scenarios of tests/golden/scenarios.py played on the reference
    build: for each step of each scenario the row before it, its observation, the action,
    the step outputs with the event record, and the row after; for each scenario's first
    row its start words, hands and stock peek, and one child for every legal action plus
    an illegal and an out-of-range one (branch_indexed)."""
    from tests.golden.scenarios import scenarios

    rec = {k: [] for k in ("step_scenario", "step_row", "step_action", "features", "legal",
                           "player", "done", "status", "reward", "step_done", "nagari",
                           "step_status", "committed", "events", "after")}
    br = {k: [] for k in ("branch_scenario", "branch_action", "children", "b_reward", "b_done",
                          "b_nagari", "b_status", "b_committed")}
    names, firsts = [], []
    for k, (name, first, actions, _) in enumerate(scenarios()):
        names.append(name)
        firsts.append(first)
        rows = first[None].copy()
        for a in actions:
            f, legal, player, done, status = ref.observe(rows)
            before = rows.copy()
            out = ref.step(rows, np.array([a], dtype=np.int64), events=True)
            for key, v in zip(("step_scenario", "step_row", "step_action", "features", "legal",
                               "player", "done", "status", "reward", "step_done", "nagari",
                               "step_status", "committed", "events", "after"),
                              (np.array([k]), before, np.array([a], dtype=np.int64), f, legal,
                               player, done, status, *out, rows.copy())):
                rec[key].append(v)
            print(f"  {name:26s} action {a:3d} -> status {int(out[3][0])} done {int(out[1][0])} "
                  f"reward {float(out[0][0]):g}")
        _, legal, _, _, _ = ref.observe(first[None])
        acts = np.concatenate([np.nonzero(legal[0])[0], [0 if not legal[0, 0] else 1, 400]])
        acts = np.unique(acts).astype(np.int64)
        out = ref.branch(first[None], np.zeros(acts.size, dtype=np.int64), acts)
        for key, v in zip(br, (np.full(acts.size, k), acts, *out)):
            br[key].append(v)
    firsts = np.stack(firsts)
    ids = np.arange(len(firsts), dtype=np.int64)
    np.savez_compressed(
        HERE / "scenarios.npz", names=np.array(names), first=firsts, start=ref.start(firsts),
        hands=ref.hands(firsts, ids), stock=ref.stock(firsts, ids),
        **{k: np.concatenate(v) for k, v in rec.items()},
        **{k: np.concatenate(v) for k, v in br.items()})
    print(f"scenarios: {len(names)} scenarios, {sum(map(len, rec['step_action']))} steps, "
          f"{sum(map(len, br['branch_action']))} children")


def main() -> None:
    ref = RefEngine(reference=True)
    what = sys.argv[1:] or ["c1", "rows", "canonical", "scenarios"]
    for name in what:
        {"c1": c1, "rows": rows, "canonical": canonical,
         "scenarios": scenario_fixture}[name](ref)


if __name__ == "__main__":
    main()
