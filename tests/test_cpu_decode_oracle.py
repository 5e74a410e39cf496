"""CPU: the decode-attention oracle pinned by closed forms, and the matmul restatement
(python/cugo_seq_attention50.py:58-62) pinned against the float64 brute force."""

from __future__ import annotations

import numpy as np
import torch

from oracle.decode_ref import bf16_to_f32, brute_force, f32_to_bf16, matmul_path


def rand(shape, seed, scale=1.0):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * scale


def test_brute_force_pos_zero_returns_first_value():
    q, k, v = rand((3, 2, 8), 1), rand((3, 2, 5, 8), 2), rand((3, 2, 5, 8), 3)
    out = brute_force(q, k, v, np.zeros(3, dtype=np.int64))
    np.testing.assert_allclose(out, v[:, :, 0], rtol=0, atol=1e-12)


def test_brute_force_equal_keys_give_the_mean():
    q, v = rand((2, 3, 4), 4), rand((2, 3, 6, 4), 5)
    k = np.broadcast_to(rand((2, 3, 1, 4), 6), (2, 3, 6, 4)).copy()
    pos = np.array([3, 5])
    out = brute_force(q, k, v, pos)
    for i, p in enumerate(pos):
        np.testing.assert_allclose(out[i], v[i, :, :p + 1].astype(np.float64).mean(axis=1), atol=1e-12)


def test_brute_force_dominant_key_selects_its_value():
    q = np.ones((1, 1, 4), dtype=np.float32)
    k = np.zeros((1, 1, 7, 4), dtype=np.float32)
    k[0, 0, 4] = 100.0  # score 200 / sqrt(4) = 100 above every other slot
    v = rand((1, 1, 7, 4), 7)
    out = brute_force(q, k, v, np.array([6]))
    np.testing.assert_allclose(out[0, 0], v[0, 0, 4], atol=1e-12)


def test_brute_force_rows_gather_and_pos_clamp():
    q, k, v = rand((4, 2, 8), 8), rand((6, 2, 5, 8), 9), rand((6, 2, 5, 8), 10)
    rows = np.array([5, 0, 5, 2])
    pos = np.array([2, 9, 4, 0])  # 9 >= slots: every slot
    out = brute_force(q, k, v, pos, rows)
    direct = brute_force(q, k[rows], v[rows], np.minimum(pos, 4))
    np.testing.assert_allclose(out, direct, atol=1e-12)
    assert np.isnan(brute_force(q[:1], k, v, np.array([-1]))).all()
    assert np.isnan(brute_force(q[:1], k, v, np.array([0]), np.array([6]))).all()


def test_matmul_path_matches_brute_force_fp32():
    q, k, v = rand((5, 4, 16), 11), rand((7, 4, 9, 16), 12), rand((7, 4, 9, 16), 13)
    rows = np.array([6, 1, 1, 3, 0])
    pos = np.array([0, 8, 3, 20, 5])
    got = matmul_path(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                      torch.from_numpy(pos), torch.from_numpy(rows)).numpy()
    np.testing.assert_allclose(got, brute_force(q, k, v, pos, rows), rtol=1e-5, atol=1e-6)


def test_matmul_path_bf16_within_bf16_rounding():
    qb = f32_to_bf16(rand((6, 8, 32), 14, 0.5))
    kb = f32_to_bf16(rand((6, 8, 50, 32), 15, 0.5))
    vb = f32_to_bf16(rand((6, 8, 50, 32), 16))
    pos = np.array([0, 1, 17, 48, 49, 30])
    as_t = lambda a: torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)  # noqa: E731
    got = matmul_path(as_t(qb), as_t(kb), as_t(vb), torch.from_numpy(pos)).float().numpy()
    want = brute_force(bf16_to_f32(qb), bf16_to_f32(kb), bf16_to_f32(vb), pos)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 1e-2, rel


def test_bf16_conversions_round_to_nearest_even():
    x = np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, -2.5, np.inf, np.nan], dtype=np.float32)
    bits = f32_to_bf16(x)
    assert bits[0] == 0x3F80 and bits[1] == 0x3F80 and bits[2] == 0x3F82
    assert bits[4] == 0x7F80 and bits[5] == 0x7FC0
    assert bf16_to_f32(bits[3:4])[0] == -2.5
