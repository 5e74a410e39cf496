"""Redeal oracle (TEST INFRASTRUCTURE ONLY).

Only tests/ import this module, as the checker.  `redeal_np` restates `_redeal`
(python/cugo_ppo50.py:122-148) on [n, 31] uint64 state words with the random draws
supplied (keys [n, 50], rng [n]); equal keys rank by card id (a stable argsort; the
reference's argsort leaves the order of equal keys open).  Pinned in
tests/test_cpu_redeal_oracle.py by a hand-built row and by what the rules fix for any
row: the unknown cards (opponent's unshown hand plus stock) are conserved, the opponent
keeps the same number of free cards, shown cards stay, the selected cards are exactly
the smallest-key unknown cards, held follows the new hand, every other word is untouched.
"""

from __future__ import annotations

import numpy as np

HAND0, HAND1, STOCK, RNG, HELD0, HELD1, REV0, REV1 = 0, 1, 3, 6, 20, 21, 22, 23
MASK64 = (1 << 64) - 1


def redeal_np(words: np.ndarray, seat: np.ndarray, keys: np.ndarray, rng: np.ndarray) -> np.ndarray:
    """New [n, 31] uint64 words (the input is not modified)."""
    out = np.array(words, dtype=np.uint64, copy=True)
    for i in range(out.shape[0]):
        w = [int(x) for x in out[i]]
        s0 = int(seat[i]) == 0
        hand = w[HAND1] if s0 else w[HAND0]
        fixed = hand & (w[REV1] if s0 else w[REV0])
        held = w[HELD1] if s0 else w[HELD0]
        free = hand & ~fixed & MASK64
        unknown = free | w[STOCK]
        count = bin(free).count("1")
        k = np.where([(unknown >> j) & 1 for j in range(50)], keys[i], 2.0)
        order = np.argsort(k, kind="stable")
        new_free = 0
        for j in order[:count]:
            new_free |= 1 << int(j)
        new_hand = fixed | new_free
        new_held = (held & ~hand & MASK64) | new_hand
        out[i, STOCK] = unknown & ~new_free & MASK64
        out[i, HAND1 if s0 else HAND0] = new_hand
        out[i, HELD1 if s0 else HELD0] = new_held
        out[i, RNG] = int(rng[i]) & MASK64
    return out
