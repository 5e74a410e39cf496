"""Host build of the engine's bit-arithmetic helpers against plainer formulations.

tests/engine_host_check.cpp includes cugo_amd/csrc/engine.h in host code and checks the
feature record decode against feature_at, the steal selection against the reference's
card-by-card loop, the special-play months against legal_special_months, and the six
turn-taking kinds as one transition (apply_turn_action) and their post-chance probe
(probe_postchance) against the per-kind compositions, and create_env's deal against the
draw-by-draw deal (the GPU parity tests check the same functions end to end against the
oracle).  tests/engine_host_rows.cpp builds create_env on the host so that whole dealt
rows are compared with the oracle's, rejection-zone deals included.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def test_engine_helpers_match_plain_formulations(tmp_path):
    if not (Path(HIPCC).exists() or shutil.which("hipcc")):
        pytest.skip("hipcc is not installed")
    exe = tmp_path / "engine_host_check"
    subprocess.run([HIPCC, "-O1", "-std=c++17", f"-I{REPO / 'cugo_amd' / 'csrc'}",
                    f"-I{REPO / 'include'}", str(REPO / "tests" / "engine_host_check.cpp"),
                    "-o", str(exe)], check=True, capture_output=True, timeout=300)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.count("equal") == 6, out.stdout


def test_host_deal_rows_equal_oracle(tmp_path, ref):
    """create_env + pack_row built for the host: every byte of the dealt row equals the
    oracle's create for 200,000 random seeds with random first players, and for 6 seeds
    whose deal draws a Lemire product in the rejection zone (about 2.6e-7 of deals take
    that path, so random seeds never reach it)."""
    import ctypes

    import numpy as np

    if not (Path(HIPCC).exists() or shutil.which("hipcc")):
        pytest.skip("hipcc is not installed")
    lib_path = tmp_path / "libengine_rows.so"
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-shared", "-fPIC",
                    f"-I{REPO / 'cugo_amd' / 'csrc'}", f"-I{REPO / 'include'}",
                    str(REPO / "tests" / "engine_host_rows.cpp"), "-o", str(lib_path)],
                   check=True, capture_output=True, timeout=300)
    lib = ctypes.CDLL(str(lib_path))
    lib.host_create_rows.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int64, ctypes.c_void_p]
    lib.host_rejection_seeds.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int64,
                                         ctypes.c_void_p]
    lib.host_rejection_seeds.restype = ctypes.c_int64
    rare = np.zeros(6, dtype=np.int64)
    assert lib.host_rejection_seeds(ctypes.c_uint64(0x9E3779B97F4A7C15),
                                    ctypes.c_uint64(0x2545F4914F6CDD1D), 6,
                                    rare.ctypes.data) == 6
    g = np.random.default_rng(20261202)
    seeds = np.concatenate([g.integers(-2**63, 2**63 - 1, 200000, dtype=np.int64), rare])
    first = g.integers(0, 2, seeds.size, dtype=np.int64)
    rows = np.zeros((seeds.size, 31), dtype=np.uint64)
    lib.host_create_rows(seeds.ctypes.data, first.ctypes.data, seeds.size, rows.ctypes.data)
    want = ref.create(seeds, first)
    bad = np.nonzero((rows.view(np.uint8).reshape(-1, 248) != want).any(axis=1))[0]
    assert bad.size == 0, (bad[:8], seeds[bad[:8]])
    from oracle.ref import REF_LIB, RefEngine
    if REF_LIB.exists():  # the rare deals through the reference's own build as well
        assert np.array_equal(RefEngine(reference=True).create(rare, first[-6:]), want[-6:])
