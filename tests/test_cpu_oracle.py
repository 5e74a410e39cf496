"""CPU: the oracle (reference engine build) against the golden fixtures and against
facts the rules fix independently of any implementation."""

from __future__ import annotations

import numpy as np

from oracle.ref import (FNV_OFFSET, PADDING, SEED_BASE, fnv_update, sample_actions,
                        splitmix_first, step_record)
from tests.conftest import GOLDEN


def test_c1_digests_match_golden(ref):
    golden = np.load(GOLDEN / "c1_random_policy.npz")
    digest, steps, reward, records, total = ref.play_random(SEED_BASE, 4096, threads=4,
                                                            record_games=16, record_cap=64)
    assert np.array_equal(digest, golden["digest"])
    assert np.array_equal(steps, golden["steps"])
    assert np.array_equal(reward, golden["final_reward"])
    assert np.array_equal(records, golden["records"])
    assert total == int(golden["total"])


def test_batch_protocol_reproduces_digests(ref):
    """The numpy batch driver (sampler, record layout, FNV) used by the GPU tests gives
    the golden digests when run over the oracle's batch operations."""
    golden = np.load(GOLDEN / "c1_random_policy.npz")
    n = 256
    idx = np.arange(n, dtype=np.uint64)
    seeds = (np.uint64(SEED_BASE) + idx).view(np.int64)
    host = ref.create(seeds, np.arange(n) & 1)
    sampler = np.array([splitmix_first(int(s) & (2**64 - 1)) for s in seeds], dtype=np.uint64)
    digest = np.full(n, FNV_OFFSET, dtype=np.uint64)
    for _ in range(128):
        obs = ref.observe(host)
        active = ~obs[3]
        if not active.any():
            break
        actions = sample_actions(obs[1], sampler, active)
        out = ref.step(host, actions, events=True)
        rec = step_record(*obs, actions, *out)
        digest[active] = fnv_update(digest[active], rec[active])
    assert np.array_equal(digest, golden["digest"][:n])


def test_golden_rows_reproduce(ref):
    g = np.load(GOLDEN / "rows.npz")
    assert np.array_equal(ref.create(g["seeds"], g["first"]), g["created"])
    assert np.array_equal(ref.start(g["created"]), g["start"])
    f, legal, player, done, status = ref.observe(g["mid"])
    assert np.array_equal(f.view(np.uint32), g["features"].view(np.uint32))
    assert np.array_equal(legal, g["legal"]) and np.array_equal(status, g["status"])
    ids = np.arange(g["mid"].shape[0])
    assert np.array_equal(ref.hands(g["mid"], ids), g["hands"])
    assert np.array_equal(ref.stock(g["mid"], ids), g["stock"])
    host = g["mid"].copy()
    ref.step(host, g["first_legal"])
    assert np.array_equal(host, g["after_first"])


def test_deal_partitions_the_deck(ref):
    """create(): 10/10/8 deal plus 22 stock partition the 50 cards (deal.h:82-92);
    floor bonus cards move to the first player's pile (turn50.h:150-167)."""
    rng = np.random.default_rng(1)
    seeds = rng.integers(-2**63, 2**63 - 1, 2000, dtype=np.int64)
    first = rng.integers(0, 2, 2000, dtype=np.int64)
    rows = ref.create(seeds, first)
    w = rows.view(np.uint64)
    hand0, hand1, floor, stock, cap0, cap1 = (w[:, k] for k in range(6))
    deck = (1 << 50) - 1
    assert np.all((hand0 | hand1 | floor | stock | cap0 | cap1) == deck)
    pop = np.vectorize(lambda x: bin(int(x)).count("1"))
    assert np.all(pop(hand0) == 10) and np.all(pop(hand1) == 10)
    total = pop(hand0) + pop(hand1) + pop(floor) + pop(stock) + pop(cap0) + pop(cap1)
    assert np.all(total == 50)
    bonus = 3 << 48
    assert not np.any(floor & bonus)
    assert not np.any(np.where(first == 0, cap1, cap0))
    for lo, hi in PADDING:
        assert not rows[:, lo:hi].any()


def test_stock_peek_is_the_future(ref):
    """stock_indexed's 8 predicted cards are exactly what later draws take
    (torch50_ext.cu:336-363): replaying draws with the row's own SplitMix64 stream."""
    g = np.load(GOLDEN / "rows.npz")
    mid = g["mid"]
    peek = ref.stock(mid, np.arange(mid.shape[0])).view(np.uint64)
    w = mid.view(np.uint64)
    mask64 = (1 << 64) - 1
    for r in range(0, mid.shape[0], 37):
        stock, state = int(w[r, 3]), int(w[r, 6])
        for k in range(8):
            count = bin(stock).count("1")
            if count == 0:
                expect = 0xFF
            else:
                while True:  # Lemire bounded draw with rejection (rng.h:34-54)
                    state = (state + 0x9E3779B97F4A7C15) & mask64
                    z = state
                    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask64
                    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask64
                    x = (z ^ (z >> 31)) >> 32
                    prod = x * count
                    low = prod & 0xFFFFFFFF
                    if low < count and low < ((-count) % (1 << 32)) % count:
                        continue
                    rank = prod >> 32
                    break
                bits = [b for b in range(64) if stock >> b & 1]
                card = bits[rank]
                stock &= ~(1 << card)
                expect = card if card < 48 else 0xFF
            got = (int(peek[r]) >> (8 * k)) & 0xFF
            assert got == expect, (r, k)
            if expect == 0xFF:
                assert all(((int(peek[r]) >> (8 * j)) & 0xFF) == 0xFF for j in range(k, 8))
                break


def test_final_rewards_are_zero_sum_settlements(ref):
    """Every random-policy game ends done; reward0 is an integer whose float cast is
    what step reports at the end (torch50_ext.cu:101)."""
    g = np.load(GOLDEN / "c1_random_policy.npz")
    rec = g["records"]
    for game in range(rec.shape[0]):
        steps = int(g["steps"][game])
        if steps == 0:  # finished at the deal (initial Chongtong, terminal50.h:226-252)
            continue
        last = rec[game, min(steps, rec.shape[1]) - 1]
        reward = last[3071:3075].view(np.float32)[0]
        done = last[3075]
        if steps <= rec.shape[1]:
            assert done == 1
            assert reward == np.float32(g["final_reward"][game])
