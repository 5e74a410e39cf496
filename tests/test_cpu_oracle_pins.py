"""CPU: the oracle (oracle/matgo/, plain C) pinned by the reference's own known answers
and, where the reference checkout is built (oracle/_ref), by a differential sweep
against the reference engine itself.

Known answers restated from the reference's tests: tests/score_test.cpp:40-111,
tests/game50_test.cpp:80-93 and tests/settlement50_test.cpp:46-125.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.ref import (ORACLE_LIB, REF_LIB, SEED_BASE, OracleRules, RefEngine, sample_actions,
                        splitmix_first)


def card(month: int, slot: int) -> int:
    return month * 4 + slot


def bit(c: int) -> int:
    return 1 << c


BRIGHT = bit(card(0, 0)) | bit(card(2, 0)) | bit(card(7, 0)) | bit(card(10, 0)) | bit(card(11, 0))
RAIN = card(11, 0)
ANIMAL = sum(bit(card(m, s)) for m, s in ((1, 0), (3, 0), (4, 0), (5, 0), (6, 0), (7, 1), (8, 0),
                                          (9, 0), (11, 1)))
RIBBON = sum(bit(card(m, s)) for m, s in ((0, 1), (1, 1), (2, 1), (3, 1), (4, 1), (5, 1), (6, 1),
                                          (8, 1), (9, 1), (11, 2)))
PLAIN_PI = sum(bit(card(m, s)) for m in range(11) for s in (2, 3))
DOUBLE_PI = bit(card(10, 1)) | bit(card(11, 3))
GODORI = bit(card(1, 0)) | bit(card(3, 0)) | bit(card(7, 1))
HONGDAN = bit(card(0, 1)) | bit(card(1, 1)) | bit(card(2, 1))
GUKJIN = card(8, 0)
STD_DECK = (1 << 48) - 1
FLAG_GODORI, FLAG_HONGDAN, FLAG_CHODAN, FLAG_CHEONGDAN, FLAG_MEONGTTA = 1, 2, 4, 8, 16


@pytest.fixture(scope="module")
def rules():
    return OracleRules()


def first_n(mask: int, n: int) -> int:
    out = 0
    for b in range(64):
        if n == 0:
            break
        if mask >> b & 1:
            out |= 1 << b
            n -= 1
    return out


def test_bright_scoring(rules):  # score_test.cpp:40-53
    assert rules.score(bit(card(0, 0)) | bit(card(2, 0)) | bit(card(7, 0)))["bright_points"] == 3
    assert rules.score(bit(card(0, 0)) | bit(card(2, 0)) | bit(RAIN))["bright_points"] == 2
    assert rules.score(BRIGHT & ~bit(RAIN))["bright_points"] == 4
    assert rules.score(BRIGHT)["bright_points"] == 15


def test_animal_ribbon_pi_scoring(rules):  # score_test.cpp:55-88
    g = rules.score(GODORI)
    assert g["animal_count"] == 3 and g["animal_points"] == 5 and g["flags"] & FLAG_GODORI
    a = rules.score(ANIMAL)
    assert a["animal_count"] == 9 and a["animal_points"] == 10 and a["flags"] & FLAG_MEONGTTA
    r = rules.score(RIBBON)
    assert r["ribbon_count"] == 10 and r["ribbon_points"] == 15
    assert r["flags"] & FLAG_HONGDAN and r["flags"] & FLAG_CHODAN and r["flags"] & FLAG_CHEONGDAN
    ten = sum(bit(card(m, s)) for m in range(5) for s in (2, 3))
    assert rules.score(ten)["pi_units"] == 10 and rules.score(ten)["pi_points"] == 1
    assert rules.score(DOUBLE_PI)["pi_units"] == 4


def test_gukjin_dual_use(rules):  # score_test.cpp:90-111
    a = rules.score(bit(GUKJIN))
    assert a["animal_count"] == 1 and a["pi_units"] == 0
    c = rules.score(bit(GUKJIN), gukjin_as_pi=True)
    assert c["animal_count"] == 0 and c["pi_units"] == 2
    full, conv = rules.score(STD_DECK), rules.score(STD_DECK, gukjin_as_pi=True)
    assert full["pi_units"] == 26 and full["total_points"] == 57
    assert conv["pi_units"] == 28 and conv["total_points"] == 58


def test_go_adjusted_points(rules):  # game50_test.cpp:80-88
    assert [rules.go_points(7, g) for g in range(6)] == [7, 8, 9, 20, 44, 96]
    assert rules.go_points(11, 3) == (11 + 3) * 2 and rules.go_points(11, 4) == (11 + 4) * 4


def stop_row(winner: int, cap0: int, cap1: int) -> np.ndarray:
    """A zero TerminalGameState50 row finished by Stop (settlement50_test.cpp:25-30)."""
    row = np.zeros(248, dtype=np.uint8)
    w = row.view(np.uint64)
    w[4], w[5] = cap0, cap1  # captured0 / captured1 (turn50.h:92-115)
    row[128] = winner        # terminal_winner (terminal50.h:74-102)
    row[129] = 1             # TerminalReason50::kStop
    return row


def test_plain_stop_settlement(rules):  # settlement50_test.cpp:52-67
    row = stop_row(0, GODORI | HONGDAN, first_n(PLAIN_PI, 8))
    s = rules.settle(row)
    assert s["status"] == 0 and s["final_points"] == rules.score(GODORI | HONGDAN)["total_points"]


def test_all_stop_multipliers(rules):  # settlement50_test.cpp:69-104
    winner = first_n(ANIMAL, 7) | first_n(BRIGHT, 3) | first_n(PLAIN_PI, 10)
    loser = first_n(PLAIN_PI & ~winner, 7)
    row = stop_row(0, winner, loser)
    row[96], row[97] = 3, 1  # go_count0 = 3, go_count1 = 1 (game50.h:38-48)
    row[108] = 1             # bombs0 (special50.h:25-32)
    row[104] = 1             # shaken0 = month 0
    s = rules.settle(row)
    base = rules.score(winner)["total_points"]
    assert s["status"] == 0
    assert s["final_points"] == rules.go_points(base, 3) * 4 * 16  # bomb+shake x4, four baks x16


def test_fixed_special_settlement(rules):  # settlement50_test.cpp:106-125
    row = stop_row(1, 0, first_n(ANIMAL, 7) | first_n(BRIGHT, 3) | first_n(PLAIN_PI, 10))
    row[129] = 5  # kThreePpuk
    row[136:144] = np.array([49], dtype=np.uint64).view(np.uint8)
    row[97], row[96], row[109], row[106] = 5, 1, 2, 3
    s = rules.settle(row)
    assert s["status"] == 0 and s["final_points"] == 49


def test_unfinished_does_not_settle(rules):  # settlement50_test.cpp:40-50
    row = np.zeros(248, dtype=np.uint8)
    row[128] = 0xFF
    assert rules.settle(row)["status"] == 1


needs_ref = pytest.mark.skipif(not REF_LIB.exists(), reason="reference build (oracle/_ref) absent")


@needs_ref
def test_oracle_matches_reference_build_on_random_games():
    """200,000 x 19.6 decision records hashed per game, four seed bases."""
    o, r = RefEngine(ORACLE_LIB), RefEngine(reference=True)
    for base in (1, 0xDEADBEEF, SEED_BASE + 10**9, 2**63 + 12345):
        a = o.play_random(base, 50000, threads=8)
        b = r.play_random(base, 50000, threads=8)
        for x, y in zip(a[:3], b[:3]):
            assert np.array_equal(x, y), hex(base)
        assert a[4] == b[4]


def same(a, b) -> bool:
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a, b)


@needs_ref
def test_oracle_matches_reference_build_on_wild_actions():
    """Mid-game rows from random seeds; 20% of actions illegal or out of range; every
    operation's outputs and the row bytes after each step compared exactly."""
    o, r = RefEngine(ORACLE_LIB), RefEngine(reference=True)
    rng = np.random.default_rng(0)
    n = 8192
    seeds = rng.integers(-2**63, 2**63 - 1, n, dtype=np.int64)
    first = rng.integers(0, 2, n).astype(np.int64)
    so, sr = o.create(seeds, first), r.create(seeds, first)
    assert np.array_equal(so, sr)
    sampler = np.array([splitmix_first(int(s) & (2**64 - 1)) for s in seeds], dtype=np.uint64)
    ids = np.arange(n, dtype=np.int64)
    for step in range(64):
        oo, ro = o.observe(so), r.observe(sr)
        assert all(same(x, y) for x, y in zip(oo, ro)), step
        assert same(o.hands(so, ids), r.hands(sr, ids)) and same(o.stock(so, ids), r.stock(sr, ids))
        assert same(o.start(so), r.start(sr))
        acts = sample_actions(ro[1], sampler, ~ro[3])
        acts = np.where(rng.random(n) < 0.2, rng.integers(-3, 182, n), acts)
        bo, br = o.branch(so, ids[::5], acts[::5]), r.branch(sr, ids[::5], acts[::5])
        assert all(same(x, y) for x, y in zip(bo, br)), step
        to, tr = o.step(so, acts, events=True), r.step(sr, acts, events=True)
        assert all(same(x, y) for x, y in zip(to, tr)), step
        assert np.array_equal(so, sr), step
        if ro[3].all():
            break
