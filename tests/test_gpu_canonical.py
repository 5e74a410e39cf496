"""GPU parity of the canonical whole-game driver (ext.rollout_canonical, the reference's
rollout_canonical_torch50, torch50.h:598-619): five digest words a game, identical to the
golden digests the reference build wrote and to the oracle on large seed families."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.ref import SEED_BASE, canonical_field
from tests.conftest import GOLDEN, announce

pytestmark = pytest.mark.gpu

DEV = "cuda"
GAMMA = np.uint64(0x9E3779B97F4A7C15)


def run(ext, seeds: np.ndarray, first: np.ndarray, cap: int = 128) -> np.ndarray:
    out = ext.rollout_canonical(torch.from_numpy(seeds).to(DEV), torch.from_numpy(first).to(DEV),
                                cap)
    return out.cpu().numpy()


def test_canonical_matches_golden(ext):
    announce("canonical driver vs golden digests")
    g = np.load(GOLDEN / "canonical.npz")
    assert np.array_equal(run(ext, g["test_seeds"], g["test_first"]), g["test_digest"])
    assert np.array_equal(run(ext, g["bench_seeds"], g["bench_first"]), g["bench_digest"])
    assert np.array_equal(run(ext, g["bench_seeds"][:512], g["bench_first"][:512], 5),
                          g["cut_digest"])


@pytest.mark.parametrize("family", ["c2", "spaced"])
def test_canonical_matches_oracle(ext, ref, family):
    """262,144 games: the C2 seeds (base + i, first = i & 1) or golden-ratio-spaced seeds
    with first = 0, at max_actions 128 and 9, and a partial last tile."""
    n = 262144 + 37
    announce(f"canonical driver vs oracle ({family}, {n} games)")
    i = np.arange(n, dtype=np.uint64)
    if family == "c2":
        seeds, first = (np.uint64(SEED_BASE) + i).view(np.int64), (i & np.uint64(1)).astype(np.int64)
    else:
        seeds, first = (np.uint64(0x3C6EF372FE94F82B) + i * GAMMA).view(np.int64), np.zeros(n, np.int64)
    for cap in (128, 9):
        got = run(ext, seeds, first, cap)
        want = ref.rollout_canonical(seeds, first, max_actions=cap)
        bad = np.nonzero((got != want).any(axis=1))[0]
        assert bad.size == 0, (cap, bad[:8], got[bad[:2]], want[bad[:2]])
    ends = np.bincount(canonical_field(got, "end"), minlength=5)
    assert ends[4] > 0 and ends[0] > 0  # cap 9: both max-actions and terminal endings


def test_canonical_edges(ext, ref):
    announce("canonical driver edges")
    seeds = (np.uint64(SEED_BASE) + np.arange(100, dtype=np.uint64)).view(np.int64)
    first = np.arange(100, dtype=np.int64) & 1
    zero = run(ext, seeds, first, 0)  # no action taken: max-actions, or a dealt Chongtong
    assert np.array_equal(zero, ref.rollout_canonical(seeds, first, max_actions=0))
    assert (canonical_field(zero, "actions") == 0).all()
    empty = ext.rollout_canonical(torch.zeros(0, dtype=torch.int64, device=DEV),
                                  torch.zeros(0, dtype=torch.int64, device=DEV))
    assert tuple(empty.shape) == (0, 5)
    with pytest.raises(RuntimeError):
        ext.rollout_canonical(torch.zeros(4, dtype=torch.int64, device=DEV),
                              torch.zeros(4, dtype=torch.int64, device=DEV), 70000)
    with pytest.raises(RuntimeError):
        ext.rollout_canonical(torch.zeros(4, dtype=torch.int64, device=DEV),
                              torch.zeros(3, dtype=torch.int64, device=DEV))
