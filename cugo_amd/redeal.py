"""Redealt worlds: the observer's view fixed, the hidden cards dealt again.

`redeal(ext, states, seat)` is the reference's `_redeal` (python/cugo_ppo50.py:122-148) on
[N, 248] rows in place: the observer's opponent gets a uniform new unrevealed hand from
the cards the observer cannot see, the rest is the stock, the stock order is reseeded and
held follows the new hand.  The reference's random draws are made the same way, in the
same order (`torch.rand(n, 50)` keys, then `torch.randint(-2**62, 2**62, (n,))` RNG words),
so with the same torch generator state the worlds are the reference's; the card
selection runs as the HIP kernel `redeal` (ties between equal keys go to the lower card id,
an order the reference's argsort leaves open).

`redeal_worlds(ext, states, env_rows, seat, worlds, tries)` is the reference function
(cugo_ppo50.py:151-172): world-major copies of the rows, each redealt until the observer's
features and legal mask are unchanged, a row keeping its real deal after `tries` misses.
"""

from __future__ import annotations

import torch

STATE_BYTES = 248


def redeal(ext, states: torch.Tensor, seat: torch.Tensor) -> None:
    """In place on [N, 248] rows; seat [N] int64 is each row's observer."""
    n = states.shape[0]
    keys = torch.rand(n, 50, device=states.device)
    rng = torch.randint(-2**62, 2**62, (n,), device=states.device)
    ext.redeal(states, seat.contiguous(), keys, rng)


def redeal_worlds(ext, states: torch.Tensor, env_rows: torch.Tensor, seat: torch.Tensor,
                  worlds: int, tries: int = 8) -> torch.Tensor:
    """[worlds * R, 248] copies of the rows, world-major, each redealt so the observer's
    features and legal actions are unchanged (cugo_ppo50.py:151-172).  Each try redeals
    and observes only the rows still without a world, from the real deal again; the test
    against the real observation and the copy of the accepted worlds are one launch
    (`accept_worlds`), and the count of rows left is the try's one host read (the next
    try's draws are sized by it, as the reference's are)."""
    if states.shape[1] != STATE_BYTES:
        raise RuntimeError("the state rows must be 248 bytes")
    base = states.index_select(0, env_rows)
    dev = base.device
    rows = base.shape[0]
    f_real, l_real, _, _, _ = ext.observe_indexed(base, torch.arange(rows, device=dev))
    real = base.repeat(worlds, 1)
    seats = seat.repeat(worlds)
    out = real.clone()
    missing = torch.arange(real.shape[0], device=dev)  # rows without a world yet
    for _ in range(tries):
        if missing.numel() == 0:
            break
        cand = real.index_select(0, missing)
        redeal(ext, cand, seats.index_select(0, missing))
        f, l, _, _, _ = ext.observe_indexed(cand, torch.arange(missing.numel(), device=dev))
        # world-major: copy k of row r is row k * rows + r, compared with real row r
        same = ext.accept_worlds(f, l, f_real, l_real, missing, cand, out)
        missing = missing[~same]
    return out
