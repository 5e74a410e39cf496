"""Test infrastructure (the oracle): the Philox4x32-10 counter-based generator and the
Gumbel-max sampler's uniforms drawn from it, in numpy.

Only tests may import this module.  It restates the published algorithm (Salmon, Moraes,
Dror and Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC 2011): each of ten rounds
maps the 128-bit counter (c0, c1, c2, c3) under the 64-bit key (k0, k1) to
(hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1, lo(M0 c0)), and the key is bumped
by the Weyl constants (W0, W1) between rounds.  It is pinned by the known-answer vectors
the authors publish with their library (tests/test_cpu_philox.py).

The sampler's uniform for row r and action a (cugo_gumbel_sample_philox): word (a / 16) % 4
of Philox4x32-10 at counter (r mod 2^32, (a % 16) + 64 (a / 64) + 256 (r / 2^32), offset,
epoch mod 2^32) under the key (seed mod 2^32, seed / 2^32), as (word >> 8) * 2^-24.
"""

from __future__ import annotations

import numpy as np

M0, M1 = 0xD2511F53, 0xCD9E8D57
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK = 0xFFFFFFFF


def philox4x32_10(ctr: np.ndarray, key: tuple[int, int]) -> np.ndarray:
    """ctr uint32 [..., 4] -> uint32 [..., 4]."""
    c = [ctr[..., i].astype(np.uint64) for i in range(4)]
    k0, k1 = np.uint64(key[0] & MASK), np.uint64(key[1] & MASK)
    m0, m1, mask = np.uint64(M0), np.uint64(M1), np.uint64(MASK)
    for _ in range(10):
        p0 = m0 * c[0]
        p1 = m1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & mask
        hi1, lo1 = p1 >> np.uint64(32), p1 & mask
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
        k0 = (k0 + np.uint64(W0)) & mask
        k1 = (k1 + np.uint64(W1)) & mask
    return np.stack([x.astype(np.uint32) for x in c], axis=-1)


def gumbel_uniforms(seed: int, epoch: int, offset: int, rows: np.ndarray,
                    actions: int) -> np.ndarray:
    """float32 [len(rows), actions]: the uniforms cugo_gumbel_sample_philox draws for the
    given row indices."""
    rows = np.asarray(rows, dtype=np.uint64)
    a = np.arange(actions, dtype=np.uint64)
    r2, a2 = np.meshgrid(rows, a, indexing="ij")
    ctr = np.stack([r2 & np.uint64(MASK),
                    (a2 % np.uint64(16)) + np.uint64(64) * (a2 // np.uint64(64))
                    + np.uint64(256) * (r2 >> np.uint64(32)),
                    np.full_like(r2, offset & MASK),
                    np.full_like(r2, epoch & MASK)], axis=-1).astype(np.uint32)
    words = philox4x32_10(ctr, (seed & MASK, (seed >> 32) & MASK))
    pick = ((a2 // np.uint64(16)) % np.uint64(4)).astype(np.int64)
    w = np.take_along_axis(words, pick[..., None], axis=-1)[..., 0]
    return ((w >> np.uint32(8)).astype(np.float32) * np.float32(2.0 ** -24))
