"""CPU: the canonical whole-game driver (rollout_canonical_torch50, torch50.h:598-619).

The oracle's restatement (oracle/matgo/canonical.h) is pinned by the golden digests the
reference build wrote (tests/golden/canonical.npz) and, where the reference build is
present (oracle/_ref), by a differential sweep against it; the reference's own
equivalence of its torch and explicit drivers (torch50_test.cpp:160-191) is checked on
the same build.  The HIP driver takes the canonical action without re-running the
reference's canonicalize_* probes on a copy of the state; that every probe returns kOk in
the states play reaches is checked here on the oracle, which keeps the probes.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle.ref import ORACLE_LIB, REF_LIB, SEED_BASE, RefEngine, canonical_field
from tests.conftest import GOLDEN

GAMMA = np.uint64(0x9E3779B97F4A7C15)
needs_ref = pytest.mark.skipif(not REF_LIB.exists(), reason="reference build (oracle/_ref) absent")


def spaced_seeds(base: int, n: int) -> np.ndarray:
    return (np.uint64(base) + np.arange(n, dtype=np.uint64) * GAMMA).view(np.int64)


def test_oracle_matches_golden_digests(ref):
    g = np.load(GOLDEN / "canonical.npz")
    assert np.array_equal(ref.rollout_canonical(g["test_seeds"], g["test_first"]), g["test_digest"])
    assert np.array_equal(ref.rollout_canonical(g["bench_seeds"], g["bench_first"]),
                          g["bench_digest"])
    cut = ref.rollout_canonical(g["bench_seeds"][:512], g["bench_first"][:512], max_actions=5)
    assert np.array_equal(cut, g["cut_digest"])
    # what the fixtures cover: terminal and nagari endings, every terminal reason,
    # post-chance choices, and the max-actions ending of the cut games
    d = g["test_digest"]
    assert set(np.unique(canonical_field(d, "end"))) == {0, 1}
    assert set(np.unique(canonical_field(d, "terminal_reason"))) == {0, 1, 2, 3, 4, 5}
    assert canonical_field(d, "choice_actions").max() >= 3
    assert (canonical_field(g["cut_digest"], "end") == 4).sum() > 400
    # the torch driver's words 0-3 are the explicit driver's (the reference's own check)
    assert np.array_equal(g["bench_digest"][:, :4], g["bench_explicit"][:, :4])


@needs_ref
@pytest.mark.parametrize("base,first_mode", [(SEED_BASE, "alternate"),
                                             (0x6A09E667F3BCC909, "alternate"),
                                             (0xBB67AE8584CAA73B, "zero")])
def test_oracle_matches_reference_build(ref, base, first_mode):
    """65,536 games a seed family (unit-stride C2 seeds, and the reference GPU bench's
    golden-ratio-spaced bases), max_actions 128, then 20 and 3."""
    n = 65536
    seeds = ((np.uint64(base) + np.arange(n, dtype=np.uint64)).view(np.int64)
             if base == SEED_BASE else spaced_seeds(base, n))
    first = (np.arange(n, dtype=np.int64) & 1) if first_mode == "alternate" else np.zeros(n, np.int64)
    reference = RefEngine(reference=True)
    for cap in (128, 20, 3):
        want = reference.rollout_canonical(seeds, first, max_actions=cap)
        got = ref.rollout_canonical(seeds, first, max_actions=cap)
        bad = np.nonzero((want != got).any(axis=1))[0]
        assert bad.size == 0, (cap, bad[:8], want[bad[:2]], got[bad[:2]])
        if cap == 128:
            explicit = reference.rollout_canonical(seeds, first, max_actions=cap, explicit=True)
            assert np.array_equal(want[:, :4], explicit[:, :4])


@pytest.mark.parametrize("random_policy", [0, 1])
def test_canonical_probes_pass_in_reachable_states(random_policy):
    """Every canonicalize_* probe (rollout50.h:400-489) returns kOk in each decision state
    of 40,000 games, played with the canonical action or with uniform random legal
    actions; a planted failure (a probe run on a state with no stock) is counted."""
    lib = ctypes.CDLL(str(ORACLE_LIB))
    fn = lib.cugo_oracle_canonical_probe_failures
    fn.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    fn.restype = None
    out = np.zeros(2, dtype=np.int64)
    fn(ctypes.c_uint64(0x5851F42D4C957F2D + random_policy), 40000, random_policy, 8,
       out.ctypes.data)
    states, failures = int(out[0]), int(out[1])
    assert states > 40000 * (15 if random_policy else 10), states
    assert failures == 0, failures
    fn(ctypes.c_uint64(0x5851F42D4C957F2D), 2000, 2, 8, out.ctypes.data)
    assert out[1] > out[0] // 2, out  # the planted stock-less probes fail and are counted
