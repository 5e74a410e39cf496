"""GPU parity of the redeal kernel and redealt worlds (python/cugo_ppo50.py:122-172).

The kernel against the oracle (oracle/redeal_ref.py, pinned in
tests/test_cpu_redeal_oracle.py) on the golden mid-game rows with the same draws: rows
bit-identical.  `redeal` draws its keys and RNG words as the reference does (torch.rand,
then torch.randint), checked by replaying the generator.  `redeal_worlds`: every world
shows the observer the same features and mask as the real deal, only the opponent's hand,
the stock, held and the RNG word move, and most rows get a new deal.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.redeal_ref import HAND0, HAND1, HELD0, HELD1, RNG, STOCK, redeal_np
from tests.conftest import GOLDEN, announce

pytestmark = pytest.mark.gpu

DEV = "cuda"


def test_redeal_kernel_matches_oracle(ext):
    announce("redeal kernel vs oracle")
    rows = np.load(GOLDEN / "rows.npz")["mid"]
    n = rows.shape[0]
    g = np.random.default_rng(31)
    seat = g.integers(0, 2, n)
    keys = g.random((n, 50), dtype=np.float32)
    keys[:8, :] = 0.5                     # all keys equal: ties go to the lower card id
    rng = g.integers(-2**62, 2**62, n)
    states = torch.from_numpy(rows.copy()).to(DEV)
    ext.redeal(states, torch.from_numpy(seat).to(DEV), torch.from_numpy(keys).to(DEV),
               torch.from_numpy(rng).to(DEV))
    want = redeal_np(rows.view(np.uint64).reshape(n, 31), seat, keys, rng)
    got = states.cpu().numpy().view(np.uint64).reshape(n, 31)
    bad = np.nonzero((got != want).any(1))[0]
    assert bad.size == 0, bad[:8]
    assert ext.redeal(states[:0], torch.zeros(0, dtype=torch.int64, device=DEV),
                      torch.zeros((0, 50), device=DEV),
                      torch.zeros(0, dtype=torch.int64, device=DEV)) is None


def test_redeal_draws_like_the_reference(ext):
    """redeal() consumes torch's generator as the reference's _redeal does: rand(n, 50)
    keys, then randint(-2**62, 2**62, (n,)) RNG words."""
    announce("redeal draws")
    from cugo_amd.redeal import redeal

    rows = np.load(GOLDEN / "rows.npz")["mid"][:700]
    n = rows.shape[0]
    seat = torch.from_numpy(np.arange(n) % 2).to(DEV)
    states = torch.from_numpy(rows.copy()).to(DEV)
    torch.manual_seed(77)
    redeal(ext, states, seat)
    torch.manual_seed(77)
    keys = torch.rand(n, 50, device=DEV)
    rng = torch.randint(-2**62, 2**62, (n,), device=DEV)
    want = redeal_np(rows.view(np.uint64).reshape(n, 31), seat.cpu().numpy(),
                     keys.cpu().numpy(), rng.cpu().numpy())
    assert np.array_equal(states.cpu().numpy().view(np.uint64).reshape(n, 31), want)


def _mid_game_rows(ext, n, seed):
    idx = torch.arange(n, dtype=torch.int64, device=DEV)
    states = ext.create(idx * 31337 + seed, idx & 1)
    gen = torch.zeros(n, dtype=torch.int32, device=DEV)
    sampler = ext.seed_samplers(n, seed, gen)
    steps = torch.from_numpy(np.random.default_rng(seed).integers(2, 14, n)).to(DEV)
    for t in range(14):
        _, legal, _, done, _ = ext.observe(states)
        actions = ext.sample_uniform(legal, sampler)
        actions = torch.where(steps > t, actions, torch.full_like(actions, -1))
        keep = states.clone()
        ext.step(states, actions)
        states = torch.where((steps > t).unsqueeze(1), states, keep)
    _, _, player, done, _ = ext.observe(states)
    live = torch.nonzero(~done).squeeze(1)
    return states.index_select(0, live), player.long().index_select(0, live)


def test_redeal_worlds_keep_the_observers_view(ext):
    announce("redeal_worlds")
    from cugo_amd.redeal import redeal_worlds

    states, player = _mid_game_rows(ext, 3000, 0x77)
    r = states.shape[0]
    env_rows = torch.arange(r, device=DEV)
    worlds = 4
    torch.manual_seed(1)
    out = redeal_worlds(ext, states, env_rows, player, worlds)
    assert out.shape == (worlds * r, 248)
    ids = torch.arange(worlds * r, device=DEV)
    f, l, _, _, _ = ext.observe_indexed(out, ids)
    f0, l0, _, _, _ = ext.observe_indexed(states, env_rows)
    assert torch.equal(f, f0.repeat(worlds, 1)) and torch.equal(l, l0.repeat(worlds, 1))
    w_out = out.cpu().numpy().view(np.uint64).reshape(-1, 31)
    w_in = np.tile(states.cpu().numpy().view(np.uint64).reshape(-1, 31), (worlds, 1))
    seat = player.repeat(worlds).cpu().numpy()
    mine = np.where(seat[:, None] == 0, w_in[:, [HAND0, HELD0]], w_in[:, [HAND1, HELD1]])
    mine_out = np.where(seat[:, None] == 0, w_out[:, [HAND0, HELD0]], w_out[:, [HAND1, HELD1]])
    assert np.array_equal(mine, mine_out)          # the observer's own hand and held
    free_words = [k for k in range(31) if k not in (HAND0, HAND1, STOCK, HELD0, HELD1, RNG)]
    assert np.array_equal(w_out[:, free_words], w_in[:, free_words])
    changed = (w_out[:, STOCK] != w_in[:, STOCK]).mean()
    assert changed > 0.5, changed
    torch.manual_seed(1)
    again = redeal_worlds(ext, states, env_rows, player, worlds)
    assert torch.equal(out, again)
    # the same torch draws through the reference's loop in torch ops (cugo_ppo50.py:151-172:
    # compare, gather and copy per try) give the same worlds
    torch.manual_seed(1)
    assert torch.equal(out, _worlds_in_torch_ops(ext, states, env_rows, player, worlds))


def _worlds_in_torch_ops(ext, states, env_rows, seat, worlds, tries=8):
    from cugo_amd.redeal import redeal

    base = states.index_select(0, env_rows)
    rows = base.shape[0]
    f_real, l_real, _, _, _ = ext.observe_indexed(base, torch.arange(rows, device=DEV))
    real = base.repeat(worlds, 1)
    seats = seat.repeat(worlds)
    out = real.clone()
    missing = torch.arange(real.shape[0], device=DEV)
    for _ in range(tries):
        if missing.numel() == 0:
            break
        cand = real.index_select(0, missing)
        redeal(ext, cand, seats.index_select(0, missing))
        f, l, _, _, _ = ext.observe_indexed(cand, torch.arange(missing.numel(), device=DEV))
        of = missing % rows
        same = (f == f_real.index_select(0, of)).all(1) & (l == l_real.index_select(0, of)).all(1)
        out.index_copy_(0, missing[same], cand[same])
        missing = missing[~same]
    return out


def test_accept_worlds_edges(ext):
    """accept_worlds: an empty try; a row index outside `out` is neither written nor kept;
    a candidate differing in one feature or one legal bit is not kept."""
    announce("accept_worlds edges")
    states, player = _mid_game_rows(ext, 64, 0x78)
    r = states.shape[0]
    f, l, _, _, _ = ext.observe_indexed(states, torch.arange(r, device=DEV))
    out = torch.zeros_like(states)
    empty = ext.accept_worlds(f[:0], l[:0], f, l, torch.zeros(0, dtype=torch.int64, device=DEV),
                              states[:0], out)
    assert empty.shape == (0,) and not bool(out.any())
    missing = torch.arange(r, device=DEV)
    missing[0] = r + 5   # outside out
    f2, l2 = f.clone(), l.clone()
    f2[1, 7] += 1.0
    l2[2, 3] = ~l2[2, 3]
    same = ext.accept_worlds(f2, l2, f, l, missing, states, out)
    want = torch.ones(r, dtype=torch.bool, device=DEV)
    want[:3] = False
    assert torch.equal(same, want)
    assert not bool(out[:3].any()) and torch.equal(out[3:], states[3:])
