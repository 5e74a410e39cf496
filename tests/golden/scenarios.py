"""Hand-built rule scenarios as 248-byte rows (test data; no engine code).

The reference checks its Hangame rule differences and its terminal rules on states built
by hand (tests/hangame_rules50_test.cpp:61-562, tests/terminal50_test.cpp:153-206), at the
turn, game or terminal level.  Here each such situation is written as a whole torch row
(TorchEnv50, include/cugo/game/torch50.h:108-121, field offsets as measured with offsetof
on the reference build) at a decision point, with the actions that play it out: a small
stock makes every draw the one the scenario names.  make_golden.py runs them through the
reference build; tests check the HIP engine and the oracle against that, and check the
rule each scenario is about against the reference test's own expectations.
"""

from __future__ import annotations

import numpy as np

# field -> (byte offset, numpy dtype) of the 248-byte row
FIELDS = {
    "hand0": (0, "<u8"), "hand1": (8, "<u8"), "floor": (16, "<u8"), "stock": (24, "<u8"),
    "captured0": (32, "<u8"), "captured1": (40, "<u8"), "rng": (48, "<u8"),
    "pending_bonus": (56, "<u8"), "ppuk_months": (64, "<u2"), "owner1": (66, "<u2"),
    "bonus2_ppuk": (68, "<u2"), "bonus3_ppuk": (70, "<u2"), "turn_index": (72, "<u2"),
    "actor": (74, "u1"), "phase": (75, "u1"), "pending_played": (76, "u1"),
    "pending_drawn": (77, "u1"), "mission_cards": (80, "<u8"), "neutral_ppuk": (88, "<u2"),
    "go0": (96, "u1"), "go1": (97, "u1"), "last_go0": (98, "u1"), "last_go1": (99, "u1"),
    "decision_actor": (100, "u1"), "game_winner": (101, "u1"), "gukjin_decision": (102, "u1"),
    "shaken0": (104, "<u2"), "shaken1": (106, "<u2"), "bombs0": (108, "u1"), "bombs1": (109, "u1"),
    "credits0": (110, "u1"), "credits1": (111, "u1"), "shaken4_0": (112, "<u2"),
    "shaken4_1": (114, "<u2"), "ppuk_count0": (120, "u1"), "ppuk_count1": (121, "u1"),
    "ppuk_streak0": (122, "u1"), "ppuk_streak1": (123, "u1"), "chongtong_actor": (124, "u1"),
    "chongtong_months": (126, "<u2"), "terminal_winner": (128, "u1"),
    "terminal_reason": (129, "u1"), "terminal_points": (136, "<u8"), "side0": (144, "<i4"),
    "round_multiplier": (148, "u1"), "mission_type": (149, "u1"), "mission_multiplier": (150, "u1"),
    "mission_multi0": (151, "u1"), "mission_multi1": (152, "u1"), "held0": (160, "<u8"),
    "held1": (168, "<u8"), "revealed0": (176, "<u8"), "revealed1": (184, "<u8"),
    "pending_active": (219, "u1"), "status": (238, "u1"), "done": (239, "u1"),
    "nagari": (240, "u1"),
}
NO_CARD, NO_PLAYER = 0xFF, 0xFF
DECK = (1 << 50) - 1
BONUS2, BONUS3 = 48, 49
PLAY, RESOLVE = 0, 2
REASON_STOP, REASON_BONUS_CT, REASON_THREE_PPUK = 1, 4, 5
# action indices (policy50.h:15-35, torch50.h:16-22)
A_BONUS, A_SHAKE, A_BOMB, A_GRENADE = 48, 50, 98, 110
A_GO, A_STOP, A_CT_WIN, A_CHOICE, A_GUKJIN_PI = 123, 124, 125, 127, 177


def card(month: int, slot: int) -> int:
    return month * 4 + slot


def cards(*pairs) -> int:
    m = 0
    for month, slot in pairs:
        m |= 1 << card(month, slot)
    return m


def month_cards(month: int) -> int:
    return 0xF << (4 * month)


def pi_cards(first_month: int, count: int) -> int:
    """`count` plain pi (slots 2, 3) from first_month on (hangame_rules50_test.cpp:24-32)."""
    m, month = 0, first_month
    while count > 0:
        for slot in (2, 3):
            if count > 0:
                m |= 1 << card(month, slot)
                count -= 1
        month += 1
    return m


BRIGHTS3 = cards((0, 0), (2, 0), (7, 0))
GODORI = cards((1, 0), (3, 0), (7, 1))  # hwatu.h:69-72
GUKJIN = card(8, 0)


def row(**fields) -> np.ndarray:
    """A row at a play-phase decision of actor 0 with no decision, chongtong or terminal
    pending, round multiplier 1, and the given fields on top."""
    base = {"actor": 0, "phase": PLAY, "pending_played": NO_CARD, "pending_drawn": NO_CARD,
            "decision_actor": NO_PLAYER, "game_winner": NO_PLAYER, "chongtong_actor": NO_PLAYER,
            "terminal_winner": NO_PLAYER, "round_multiplier": 1, "rng": 7}
    base.update(fields)
    out = np.zeros(248, dtype=np.uint8)
    for name, value in base.items():
        at, dt = FIELDS[name]
        out[at:at + np.dtype(dt).itemsize] = np.array([value], dtype=dt).view(np.uint8)
    return out


def field(rows: np.ndarray, name: str) -> np.ndarray:
    """Field `name` of one row [248] or of rows [n, 248]."""
    at, dt = FIELDS[name]
    r = np.atleast_2d(rows)
    size = np.dtype(dt).itemsize
    return np.ascontiguousarray(r[:, at:at + size]).view(dt).reshape(-1)


def scenarios() -> list[tuple[str, np.ndarray, list[int], str]]:
    """(name, first row, actions played from it in order, reference location)."""
    victim = pi_cards(6, 2)
    late_win = BRIGHTS3 | GODORI  # 3 brights (3) + godori (5) = 8 points
    out = []

    def add(name, r, actions, where):
        out.append((name, r, list(actions), where))

    # hangame 2: the played card takes a dealt (neutral) triple and steals one pi
    add("neutral_ppuk_capture",
        row(hand0=cards((3, 3), (6, 0)), hand1=cards((7, 0)),
            floor=cards((3, 0), (3, 1), (3, 2), (9, 0)), neutral_ppuk=1 << 3,
            captured1=victim, stock=cards((5, 0)), turn_index=4),
        [card(3, 3)], "hangame_rules50_test.cpp:87-104")
    # hangame 3: last turn - jjok without a steal, no ppuk, a bonus without a steal
    add("last_turn_jjok",
        row(hand0=cards((0, 0)), hand1=cards((8, 1)), floor=cards((1, 0)), stock=cards((0, 1)),
            captured1=victim, turn_index=18),
        [card(0, 0)], "hangame_rules50_test.cpp:121-131")
    add("last_turn_no_ppuk",
        row(hand0=cards((1, 1)), hand1=cards((8, 1)), floor=cards((1, 0)), stock=cards((1, 2)),
            captured1=victim, turn_index=18),
        [card(1, 1)], "hangame_rules50_test.cpp:133-143")
    add("ppuk_before_last_turn",
        row(hand0=cards((1, 1), (6, 0)), hand1=cards((8, 1), (9, 1)), floor=cards((1, 0)),
            stock=cards((1, 2)), captured1=victim, turn_index=17),
        [card(1, 1)], "hangame_rules50_test.cpp:145-150")
    add("last_turn_bonus",
        row(hand0=1 << BONUS2, hand1=cards((8, 1)), stock=cards((0, 0)),
            captured1=cards((1, 2)), turn_index=18),
        [A_BONUS], "hangame_rules50_test.cpp:152-163")
    add("auto_stop_after_turn_19",
        row(hand0=cards((5, 0)), floor=cards((6, 0)), stock=cards((9, 0)), captured0=late_win,
            captured1=cards((9, 1)), turn_index=19),
        [card(5, 0)], "hangame_rules50_test.cpp:165-180")
    add("go_stop_mid_game",
        row(hand0=cards((5, 0), (5, 1)), hand1=cards((8, 1), (9, 1)), floor=cards((6, 0)),
            stock=cards((9, 0), (10, 0)), captured0=late_win, turn_index=10),
        [card(5, 0), A_GO], "hangame_rules50_test.cpp:174-177")
    # hangame 4: pi-bak, void game, gwang-bak, carry and mission multipliers; nagari keeps
    # side payments
    winner = BRIGHTS3 | GODORI | pi_cards(0, 10)
    ribbon = cards((9, 1))
    for name, loser, rnd, mission in (("settle_void", 0, 1, 0),
                                      ("settle_gwang_bak", ribbon, 1, 0),
                                      ("settle_pi_bak", ribbon | pi_cards(5, 5), 1, 0),
                                      ("settle_eight_pi", ribbon | pi_cards(5, 8), 1, 0),
                                      ("settle_carry_mission", ribbon | pi_cards(5, 5), 2, 3)):
        add(name, row(captured0=winner, captured1=loser, round_multiplier=rnd,
                      mission_multi0=mission, terminal_winner=0, terminal_reason=REASON_STOP,
                      done=1),
            [0], "hangame_rules50_test.cpp:183-226")
    add("nagari_side_payment",
        row(round_multiplier=2, side0=-14, done=1, nagari=1), [0],
        "hangame_rules50_test.cpp:221-226")
    # hangame 5: the Gukjin prompt comes before Go/Stop and is answered once
    add("gukjin_prompt",
        row(hand0=cards((5, 0), (5, 1)), hand1=cards((10, 1), (9, 1)), floor=cards((6, 0)),
            stock=cards((9, 0), (10, 0)),
            captured0=(1 << GUKJIN) | BRIGHTS3 | pi_cards(0, 8) | GODORI, turn_index=6),
        [card(5, 0), A_GUKJIN_PI, A_GO], "hangame_rules50_test.cpp:245-262")
    # hangame 6: forced bomb and grenade months, four-card shake
    add("forced_bomb",
        row(hand0=cards((4, 0), (4, 1), (4, 2), (6, 0)), hand1=cards((7, 0)),
            floor=cards((4, 3), (9, 0)), stock=cards((10, 0), (11, 0))),
        [A_BOMB + 4], "hangame_rules50_test.cpp:297-305")
    add("forced_grenade",
        row(hand0=cards((4, 0), (4, 1), (6, 0)), hand1=cards((7, 0)),
            floor=cards((4, 2), (4, 3)), stock=cards((10, 0), (11, 0))),
        [A_GRENADE + 4], "hangame_rules50_test.cpp:307-313")
    add("four_card_shake",
        row(hand0=month_cards(4) | cards((6, 0)), hand1=cards((7, 0)), floor=cards((9, 0)),
            stock=cards((10, 0), (11, 0))),
        [A_SHAKE + card(4, 0)], "hangame_rules50_test.cpp:315-323")
    # hangame 7: a mission completed by a capture pays its multiplier
    add("mission_completed",
        row(hand0=cards((0, 2), (6, 0)), hand1=cards((7, 0)), floor=cards((0, 1)),
            stock=cards((9, 0), (10, 0)), captured0=1 << 0, mission_type=1,
            mission_multiplier=3, mission_cards=(1 << 0) | (1 << 1)),
        [card(0, 2)], "hangame_rules50_test.cpp:327-337")
    # hangame 8: sweep steals one; a first-turn ttadak pays 7, a later one nothing
    add("sweep",
        row(hand0=cards((2, 1), (6, 0)), hand1=cards((7, 0)), floor=cards((2, 0), (5, 0)),
            stock=cards((5, 1)), captured1=victim, turn_index=4),
        [card(2, 1)], "hangame_rules50_test.cpp:407-412")
    for turn in (0, 2):
        add(f"ttadak_turn_{turn}",
            row(hand0=cards((2, 2), (6, 0)), hand1=cards((7, 0)),
                floor=cards((2, 0), (2, 1), (9, 0)), stock=cards((2, 3)), captured1=victim,
                turn_index=turn),
            [card(2, 2)], "hangame_rules50_test.cpp:414-431")
    # hangame 9: public information in the observation
    add("neutral_ppuk_observed",
        row(hand0=cards((6, 0)), hand1=cards((7, 0)), floor=cards((3, 0), (3, 1), (3, 2)),
            stock=DECK & ~(cards((6, 0), (7, 0), (3, 0), (3, 1), (3, 2))), neutral_ppuk=1 << 3),
        [card(6, 0)], "hangame_rules50_test.cpp:438-452")
    shake_hand0 = cards((4, 0), (4, 1), (4, 2), (6, 0))
    shake_hand1 = cards((7, 0), (8, 0))
    shake_floor = cards((9, 0), (10, 0))
    add("shake_reveals",
        row(hand0=shake_hand0, hand1=shake_hand1, floor=shake_floor,
            stock=DECK & ~(shake_hand0 | shake_hand1 | shake_floor)),
        [A_SHAKE + card(4, 0)], "hangame_rules50_test.cpp:454-479")
    # terminal50: a third consecutive ppuk of the first player (its turn ends as turn 5)
    # ends the game at 7 points and pays 21 more (42 paid in all)
    add("third_ppuk_ends_game",
        row(hand0=cards((1, 1), (6, 0)), hand1=cards((8, 1), (9, 1)),
            floor=cards((1, 0), (2, 0), (2, 1), (2, 2), (4, 0), (4, 1), (4, 2)),
            stock=cards((1, 2)), ppuk_count0=2, ppuk_streak0=2, side0=21, turn_index=4,
            ppuk_months=(1 << 2) | (1 << 4)),
        [card(1, 1)], "terminal50_test.cpp:153-176")
    # terminal50: a bonus play whose replacement completes a month opens the Chongtong
    # choice; winning it ends the game
    add("bonus_chongtong",
        row(hand0=(1 << BONUS2) | cards((5, 0), (5, 1), (5, 2), (6, 0)), hand1=cards((7, 0)),
            floor=cards((9, 0)), stock=cards((5, 3)), turn_index=2),
        [A_BONUS, A_CT_WIN], "terminal50_test.cpp (bonus replacement Chongtong choice)")
    return out
