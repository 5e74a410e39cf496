"""The oracle's Philox4x32-10 (oracle/philox_ref.py) against the known-answer vectors its
authors publish with their library (Random123, kat_vectors: philox4x32 with 10 rounds),
and the sampler's uniforms against the counter layout they are defined by."""

from __future__ import annotations

import numpy as np

from oracle.philox_ref import gumbel_uniforms, philox4x32_10

KAT = [  # counter, key, output
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


def test_philox_known_answers():
    for ctr, key, want in KAT:
        got = philox4x32_10(np.array([ctr], dtype=np.uint32), key)[0]
        assert [int(x) for x in got] == list(want)


def test_philox_planted_mistake_fails():
    # a wrong round count or swapped multiplier moves every word of the first vector
    ctr, key, want = KAT[2]
    c = np.array([ctr], dtype=np.uint32)
    assert [int(x) for x in philox4x32_10(c, (key[1], key[0]))[0]] != list(want)


def test_gumbel_uniforms_layout():
    """u(r, a) is word (a // 16) % 4 of the block at counter (r, a % 16 + 64 (a // 64),
    offset, epoch) under key (seed lo, seed hi), as (word >> 8) / 2^24."""
    seed, epoch, offset = 0x0123456789ABCDEF, 7, 11
    rows = np.array([0, 1, 5, 1000], dtype=np.int64)
    u = gumbel_uniforms(seed, epoch, offset, rows, 179)
    assert u.shape == (4, 179) and u.dtype == np.float32
    assert (u >= 0).all() and (u < 1).all()
    for r_i, r in enumerate(rows):
        for a in (0, 15, 16, 63, 64, 100, 178):
            ctr = np.array([[r, a % 16 + 64 * (a // 64), offset, epoch]], dtype=np.uint32)
            w = philox4x32_10(ctr, (seed & 0xFFFFFFFF, seed >> 32))[0][(a // 16) % 4]
            assert u[r_i, a] == np.float32((int(w) >> 8) * 2.0 ** -24)
    # every (row, action) a distinct draw, roughly uniform
    big = gumbel_uniforms(seed, epoch, offset, np.arange(512), 179)
    assert len(np.unique(big)) > 0.99 * big.size
    assert abs(float(big.mean()) - 0.5) < 0.01
    hist = np.histogram(big, bins=16, range=(0, 1))[0]
    assert hist.min() > 0.9 * big.size / 16
