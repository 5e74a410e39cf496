"""Host build of the engine's bit-arithmetic helpers against plainer formulations.

tests/engine_host_check.cpp includes cugo_amd/csrc/engine.h in host code and checks the
feature record decode against feature_at, the steal selection against the reference's
card-by-card loop, the special-play months against legal_special_months, and the six
turn-taking kinds as one transition (apply_turn_action) and their post-chance probe
(probe_postchance) against the per-kind compositions, and create_env's deal against the
draw-by-draw deal (the GPU parity tests check the same functions end to end against the
oracle).
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
