"""CPU: the hand-built rule scenarios (tests/golden/scenarios.py, written from the
reference's tests/hangame_rules50_test.cpp and tests/terminal50_test.cpp).

The fixture holds what the reference build did on each scenario.  These tests check
that each scenario exercises its rule with the outcome the reference's own test
requires, and that the oracle reproduces every recorded output bit for bit."""

from __future__ import annotations

import numpy as np
import pytest

from tests.conftest import GOLDEN
from tests.golden.scenarios import (BRIGHTS3, GODORI, REASON_BONUS_CT, REASON_STOP,
                                    REASON_THREE_PPUK, card, cards, field, month_cards,
                                    pi_cards)

FIX = np.load(GOLDEN / "scenarios.npz")
NAMES = [str(n) for n in FIX["names"]]


def steps_of(name: str) -> np.ndarray:
    return np.nonzero(FIX["step_scenario"] == NAMES.index(name))[0]


def after(name: str, k: int = -1) -> np.ndarray:
    return FIX["after"][steps_of(name)[k]]


def legal_at(name: str, k: int) -> set[int]:
    return set(np.nonzero(FIX["legal"][steps_of(name)[k]])[0].tolist())


def value(name: str, key: str, k: int = -1):
    return FIX[key][steps_of(name)[k]]


def popcount(x) -> int:
    return bin(int(x)).count("1")


def test_every_step_ok_or_finished():
    ok = FIX["step_status"] == 0
    finished = FIX["step_status"] == 9  # stepping a finished game
    assert (ok | finished).all(), [NAMES[s] for s in FIX["step_scenario"][~(ok | finished)]]
    assert len(NAMES) == 25


def test_neutral_ppuk_and_last_turn_rules():  # hangame_rules50_test.cpp:87-180
    r = after("neutral_ppuk_capture")
    assert int(field(r, "captured0")[0]) & month_cards(3) == month_cards(3)
    assert popcount(field(r, "captured1")[0]) == 1 and field(r, "neutral_ppuk")[0] == 0
    victim = pi_cards(6, 2)
    r = after("last_turn_jjok")
    assert field(r, "captured1")[0] == victim
    assert int(field(r, "captured0")[0]) & cards((0, 0), (0, 1)) == cards((0, 0), (0, 1))
    r = after("last_turn_no_ppuk")
    assert field(r, "ppuk_months")[0] == 0 and int(field(r, "captured0")[0]) >> card(1, 0) & 1
    r = after("ppuk_before_last_turn")
    assert field(r, "ppuk_months")[0] == 1 << 1
    assert int(field(r, "floor")[0]) & cards((1, 0), (1, 1), (1, 2)) == cards((1, 0), (1, 1), (1, 2))
    assert field(after("last_turn_bonus"), "captured1")[0] == cards((1, 2))
    r = after("auto_stop_after_turn_19")
    assert field(r, "terminal_reason")[0] == REASON_STOP and field(r, "terminal_winner")[0] == 0
    assert value("auto_stop_after_turn_19", "step_done") and value("auto_stop_after_turn_19", "reward") > 0
    assert legal_at("go_stop_mid_game", 1) == {123, 124}
    assert field(after("go_stop_mid_game"), "go0")[0] == 1


def test_settlement_rules():  # hangame_rules50_test.cpp:183-226: 9-point winner
    rewards = {n: float(value(n, "reward")) for n in
               ("settle_void", "settle_gwang_bak", "settle_pi_bak", "settle_eight_pi",
                "settle_carry_mission", "nagari_side_payment")}
    assert rewards == {"settle_void": 0.0, "settle_gwang_bak": 18.0, "settle_pi_bak": 36.0,
                       "settle_eight_pi": 18.0, "settle_carry_mission": 9.0 * 4 * 2 * 3,
                       "nagari_side_payment": -14.0}
    assert value("nagari_side_payment", "nagari")


def test_gukjin_prompt_before_go_stop():  # hangame_rules50_test.cpp:245-262
    assert legal_at("gukjin_prompt", 1) == {177, 178}
    assert legal_at("gukjin_prompt", 2) == {123, 124}
    assert int(field(after("gukjin_prompt", 1), "owner1")[0]) != 0


def test_forced_specials_and_four_shake():  # hangame_rules50_test.cpp:297-323
    bomb = legal_at("forced_bomb", 0)
    assert {card(4, 0), card(4, 1), card(4, 2)}.isdisjoint(bomb) and {card(6, 0), 102} <= bomb
    grenade = legal_at("forced_grenade", 0)
    assert {card(4, 0), card(4, 1)}.isdisjoint(grenade) and 114 in grenade
    assert 50 + card(4, 0) in legal_at("four_card_shake", 0)
    r = after("four_card_shake")
    assert field(r, "shaken4_0")[0] == 1 << 4 and field(r, "shaken0")[0] == 0


def test_mission_sweep_ttadak():  # hangame_rules50_test.cpp:327-431
    r = after("mission_completed")
    assert field(r, "mission_multi0")[0] == 3 and field(r, "mission_multi1")[0] == 0
    r = after("sweep")
    assert int(field(r, "floor")[0]) & ((1 << 48) - 1) == 0
    assert popcount(field(r, "captured1")[0]) == 1
    assert field(after("ttadak_turn_0"), "side0")[0] == 7
    assert field(after("ttadak_turn_2"), "side0")[0] == 0


def test_public_observation():  # hangame_rules50_test.cpp:438-479
    f = value("neutral_ppuk_observed", "features", 0)
    assert f[479 + 3] == 1.0  # the neutral ppuk month plane (features 479-490)
    r = after("shake_reveals")
    assert field(r, "revealed0")[0] == cards((4, 0), (4, 1), (4, 2))
    assert field(r, "actor")[0] == 1


def test_three_ppuk_and_bonus_chongtong():  # terminal50_test.cpp:118-176
    r = after("third_ppuk_ends_game")
    assert field(r, "terminal_reason")[0] == REASON_THREE_PPUK and field(r, "side0")[0] == 42
    assert value("third_ppuk_ends_game", "reward") == 49.0
    assert legal_at("bonus_chongtong", 1) == {125, 126}
    r = after("bonus_chongtong")
    assert field(r, "terminal_reason")[0] == REASON_BONUS_CT and field(r, "terminal_winner")[0] == 0


def test_oracle_reproduces_fixture(ref):
    f, legal, player, done, status = ref.observe(FIX["step_row"])
    assert np.array_equal(f.view(np.uint32), FIX["features"].view(np.uint32))
    for got, key in ((legal, "legal"), (player, "player"), (done, "done"), (status, "status")):
        assert np.array_equal(got, FIX[key]), key
    rows = FIX["step_row"].copy()
    out = ref.step(rows, FIX["step_action"], events=True)
    for got, key in zip(out, ("reward", "step_done", "nagari", "step_status", "committed",
                              "events")):
        assert np.array_equal(got, FIX[key]), key
    assert np.array_equal(rows, FIX["after"])
    children = ref.branch(FIX["first"], FIX["branch_scenario"], FIX["branch_action"])
    for got, key in zip(children, ("children", "b_reward", "b_done", "b_nagari", "b_status",
                                   "b_committed")):
        assert np.array_equal(got, FIX[key]), key
    ids = np.arange(len(NAMES), dtype=np.int64)
    assert np.array_equal(ref.start(FIX["first"]), FIX["start"])
    assert np.array_equal(ref.hands(FIX["first"], ids), FIX["hands"])
    assert np.array_equal(ref.stock(FIX["first"], ids), FIX["stock"])
