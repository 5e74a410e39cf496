"""Pins of the redeal oracle (oracle/redeal_ref.py, restating python/cugo_ppo50.py:122-148).

A hand-built row fixes every word the redeal writes; on the 2,560 golden mid-game rows
(tests/golden/rows.npz, written from the reference engine) with random keys, what the
rules fix for any row is checked: the unknown cards are conserved, the opponent keeps as
many free cards, shown cards stay in hand, the new free cards are the smallest-key
unknown cards, held follows the new hand, and no other word changes.
"""

from __future__ import annotations

import numpy as np

from oracle.redeal_ref import (HAND0, HAND1, HELD0, HELD1, REV0, REV1, RNG, STOCK,
                               redeal_np)
from tests.conftest import GOLDEN


def mask(*cards):
    m = 0
    for c in cards:
        m |= 1 << c
    return m


def bits(m):
    return {j for j in range(64) if (int(m) >> j) & 1}


def test_hand_built_row():
    w = np.zeros((1, 31), dtype=np.uint64)
    w[0, HAND0] = mask(1, 2, 3)
    w[0, HAND1] = mask(10, 11, 12, 13)
    w[0, REV1] = mask(13)                   # shown by a shake: stays in the hand
    w[0, STOCK] = mask(20, 21, 22, 23, 24)
    w[0, HELD1] = mask(10, 11, 12, 13, 30)  # 30 was held earlier and played
    w[0, 4] = mask(40)                      # a capture: untouched
    keys = np.full((1, 50), 0.9, dtype=np.float32)
    keys[0, 21], keys[0, 10], keys[0, 24] = 0.1, 0.2, 0.3   # the three smallest unknown keys
    keys[0, 1] = 0.0                        # the observer's own card: not unknown
    out = redeal_np(w, np.array([0]), keys, np.array([12345]))
    assert bits(out[0, HAND1]) == {10, 13, 21, 24}
    assert bits(out[0, STOCK]) == {11, 12, 20, 22, 23}
    assert bits(out[0, HELD1]) == {10, 13, 21, 24, 30}
    assert int(out[0, RNG]) == 12345
    untouched = [k for k in range(31) if k not in (HAND1, STOCK, HELD1, RNG)]
    assert np.array_equal(out[0, untouched], w[0, untouched])
    # the other seat redeals player 0's hand instead
    out1 = redeal_np(w, np.array([1]), keys, np.array([7]))
    assert len(bits(out1[0, HAND0])) == 3 and bits(out1[0, HAND1]) == {10, 11, 12, 13}


def test_golden_rows_invariants():
    rows = np.load(GOLDEN / "rows.npz")["mid"]
    words = rows.view(np.uint64).reshape(-1, 31)
    n = words.shape[0]
    rng = np.random.default_rng(5)
    seat = rng.integers(0, 2, n)
    keys = rng.random((n, 50), dtype=np.float32)
    out = redeal_np(words, seat, keys, rng.integers(-2**62, 2**62, n))
    moved = 0
    for i in range(n):
        s0 = seat[i] == 0
        opp, opp_held, opp_rev = (HAND1, HELD1, REV1) if s0 else (HAND0, HELD0, REV0)
        hand, new_hand = int(words[i, opp]), int(out[i, opp])
        fixed = hand & int(words[i, opp_rev])
        free = hand & ~fixed
        unknown = free | int(words[i, STOCK])
        assert new_hand | int(out[i, STOCK]) == unknown | fixed
        assert new_hand & int(out[i, STOCK]) == 0
        assert new_hand & fixed == fixed
        new_free = new_hand & ~fixed
        assert bin(new_free).count("1") == bin(free).count("1")
        # exactly the smallest keys among the unknown cards
        unk = sorted(bits(unknown), key=lambda j: (keys[i, j], j))
        assert bits(new_free) == set(unk[:bin(free).count("1")])
        held = int(words[i, opp_held])
        assert int(out[i, opp_held]) == ((held & ~hand) | new_hand)
        keep = [k for k in range(31) if k not in (opp, STOCK, opp_held, RNG)]
        assert np.array_equal(out[i, keep], words[i, keep])
        moved += new_hand != hand
    assert moved > n // 2
