"""Pins of the sequence-policy oracle (oracle/seq_ref.py) by hand-built known answers.

encode_events / encode_start (python/cugo_seq50.py:91-128) are restated in numpy; these
cases fix every slot and column from the reference's slot list and the start-word layout,
so a swapped seat, slot or column fails one of them.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.seq_ref import (EVENT_IN, START_IN, encode_events_np, encode_start_np,
                            token_reference)


def mask(*cards: int) -> int:
    m = 0
    for c in cards:
        m |= 1 << c
    return m


def signed(words):
    return np.array([w - (1 << 64) if w >= (1 << 63) else w for w in words], dtype=np.int64)


def event(played=0, drawn=0, flipped=0, gain0=0, gain1=0, lost0=0, lost1=0, shown=0,
          actor=0, kind=0):
    return signed([played, drawn, flipped, gain0, gain1, lost0, lost1, shown,
                   actor | (kind << 8)])


def cols(token: np.ndarray) -> dict[int, float]:
    return {int(j): float(token[j]) for j in np.nonzero(token)[0]}


def test_event_token_from_the_actors_seat():
    ev = event(played=mask(5), drawn=mask(10), flipped=mask(20), gain0=mask(5, 20),
               lost1=mask(33), shown=mask(41), actor=0, kind=2)
    t = encode_events_np(ev[None], np.array([0]))[0]
    assert t.shape == (EVENT_IN,)
    # played 5, own drawn 10, flipped 20, my gain {5, 20}, opponent loss 33, shown 41,
    # kind 2, me
    assert cols(t) == {5: 1.0, 60: 1.0, 120: 1.0, 155: 1.0, 170: 1.0, 333: 1.0, 391: 1.0,
                       402: 1.0, 412: 1.0}


def test_event_token_from_the_other_seat():
    ev = event(played=mask(5), drawn=mask(10, 11), flipped=mask(20), gain0=mask(5, 20),
               lost1=mask(33), actor=0, kind=2)
    t = encode_events_np(ev[None], np.array([1]))[0]
    # the draw is hidden (two cards -> count 2), gains of player 0 are the opponent's,
    # losses of player 1 are mine
    assert cols(t) == {5: 1.0, 120: 1.0, 205: 1.0, 220: 1.0, 283: 1.0, 402: 1.0, 413: 2.0}


def test_event_token_seat_one_actor_and_clamps():
    ev = event(played=mask(49) | (1 << 50) | (1 << 63), drawn=mask(0), gain1=mask(7),
               lost0=mask(8), actor=1, kind=200)
    t = encode_events_np(ev[None], np.array([1]))[0]
    # bits >= 50 are outside the plane; kind clamps to 11; seat 1 reads player 1 as "my"
    assert cols(t) == {49: 1.0, 50: 1.0, 157: 1.0, 308: 1.0, 411: 1.0, 412: 1.0}
    t0 = encode_events_np(ev[None], np.array([0]))[0]
    assert cols(t0) == {49: 1.0, 207: 1.0, 258: 1.0, 411: 1.0, 413: 1.0}


def start_words(hand0, hand1, floor, cap0, cap1, mission, neutral, mtype, mult, first, m0, m1):
    return signed([hand0, hand1, floor, cap0, cap1, mission, neutral,
                   mtype | (mult << 8) | (first << 16) | (m0 << 24) | (m1 << 32)])


def test_start_token_both_seats():
    st = start_words(mask(1, 2), mask(3), mask(4), mask(5), mask(6), mask(7), 0b101, 3, 2, 1, 4, 6)
    t0 = encode_start_np(st[None], np.array([0]))[0]
    assert t0.shape == (START_IN,)
    assert cols(t0) == {1: 1.0, 2: 1.0, 54: 1.0, 105: 1.0, 156: 1.0, 207: 1.0, 250: 1.0,
                        252: 1.0, 265: 1.0, 270: 0.5, 272: 0.5, 273: 0.75}
    t1 = encode_start_np(st[None], np.array([1]))[0]
    assert cols(t1) == {3: 1.0, 54: 1.0, 106: 1.0, 155: 1.0, 207: 1.0, 250: 1.0, 252: 1.0,
                        265: 1.0, 270: 0.5, 271: 1.0, 272: 0.75, 273: 0.5}


def test_start_token_type_clamp_and_neutral_width():
    st = start_words(0, 0, 0, 0, 0, 0, (1 << 12) | 0b1, 9, 0, 0, 0, 0)
    t = encode_start_np(st[None], np.array([0]))[0]
    # neutral keeps 12 bits; mission type clamps to 7; seat 0 moves first
    assert cols(t) == {250: 1.0, 269: 1.0, 271: 1.0}


def test_token_reference_is_the_linear_plus_rows():
    torch = pytest.importorskip("torch")
    g = torch.Generator().manual_seed(0)
    d = 16
    w = torch.randn(d, EVENT_IN, generator=g)
    b = torch.randn(d, generator=g)
    pos = torch.randn(d, generator=g)
    tt = torch.randn(d, generator=g)
    tok = np.zeros((2, EVENT_IN))
    tok[0, 7] = 1.0
    tok[1, 413] = 3.0
    out = token_reference(tok, w, b, pos, tt).double()
    want0 = w[:, 7].double() + b.double() + pos.double() + tt.double()
    want1 = 3.0 * w[:, 413].double() + b.double() + pos.double() + tt.double()
    assert torch.allclose(out[0], want0, atol=1e-5)
    assert torch.allclose(out[1], want1, atol=1e-5)
