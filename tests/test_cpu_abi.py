"""CPU: the product libraries load and export their declared interface (no GPU calls)."""

from __future__ import annotations

import ctypes
import re

import numpy as np

from tests.conftest import REPO


def declared_symbols() -> list[str]:
    text = (REPO / "include" / "cugo_hip.h").read_text()
    return sorted(set(re.findall(r"\bint\s+(cugo_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(REPO / "cugo_amd" / "libcugo_hip.so"))
    names = declared_symbols()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lib, name), name
    lib.cugo_version.restype = ctypes.c_int
    assert lib.cugo_version() >> 16 == 1


def test_abi_rejects_bad_arguments_without_launching():
    lib = ctypes.CDLL(str(REPO / "cugo_amd" / "libcugo_hip.so"))
    lib.cugo_create.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                ctypes.c_void_p, ctypes.c_void_p]
    assert lib.cugo_create(None, None, -1, None, None) < 0
    assert lib.cugo_create(None, None, 5, None, None) < 0
    assert lib.cugo_create(None, None, 0, None, None) == 0
    # spare slots: 1, 2 or 4 pre-dealt games per row; any other count is refused
    P, I = ctypes.c_void_p, ctypes.c_int64
    lib.cugo_refill_spares.argtypes = [P, P, P, I, ctypes.c_uint64, I, I, P]
    buf = ctypes.create_string_buffer(64)
    for slots, want_ok in ((1, True), (2, True), (4, True), (0, False), (3, False), (8, False)):
        rc = lib.cugo_refill_spares(buf, buf, buf, 0, 0, 0, slots, None)
        assert (rc == 0) == want_ok, (slots, rc)


def test_extension_module_constants():
    import torch  # noqa: F401  (loads libc10 / libtorch, which the module links)

    from cugo_amd import _cugo_torch50_hip as m

    assert (m.FEATURE_COUNT, m.ACTION_COUNT, m.PRIMARY_ACTION_COUNT, m.CHOICE_ACTION_BEGIN,
            m.EVENT_WORDS, m.START_WORDS, m.STATE_BYTES, m.STATUS_OK) == (
                720, 179, 127, 127, 9, 8, 248, 0)
    for op in ("create", "observe", "observe_indexed", "step", "step_indexed", "clone_indexed",
               "branch_indexed", "hands_indexed", "stock_indexed", "step_events_indexed",
               "start", "decode_attention", "decode_attention_append", "sample_uniform",
               "observe_sample", "reset_done", "reset_done_spares", "refill_spares",
               "seed_samplers", "step_reset_spares", "play_random",
               "branch_observe_indexed"):
        assert callable(getattr(m, op))


def test_stop_points_table_is_the_host_log2f():
    """The baked table equals this host's libm log2f(1 + p) / 12 (torch50.h:405-408)."""
    text = (REPO / "cugo_amd" / "csrc" / "stop_bits.inc").read_text()
    values = [float.fromhex(t.strip().rstrip("f")) for t in text.replace("\n", " ").split(",")
              if t.strip()]
    assert len(values) == 4095
    libm = ctypes.CDLL("libm.so.6")
    libm.log2f.restype = ctypes.c_float
    libm.log2f.argtypes = [ctypes.c_float]
    for p in range(0, 4095, 7):
        bits = np.float32(libm.log2f(np.float32(1.0) + np.float32(p))) / np.float32(12.0)
        expect = min(np.float32(bits), np.float32(1.0))
        assert np.float32(values[p]) == expect, p
    assert values[0] == 0.0 and values[4094] < 1.0


def test_load_extension_fails_loudly_without_gpu(monkeypatch):
    import torch

    import cugo_amd

    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    try:
        cugo_amd.load_extension()
    except RuntimeError as exc:
        assert "not available" in str(exc)
    else:
        raise AssertionError("load_extension must raise without a GPU")


def test_drop_in_modules_import_under_reference_names():
    """With cugo_amd/ first on sys.path, the reference's import lines resolve to this
    package's modules (python/cugo_torch50_ext.py, python/cugo_seq_attention50.py)."""
    import subprocess
    import sys

    code = ("import sys; sys.path[:0] = [sys.argv[1], sys.argv[2]];"
            "from cugo_torch50_ext import load_extension;"
            "from cugo_seq_attention50 import decode_attention;"
            "import torch;"
            "q = torch.zeros(1, 1, 32)\n"
            "try:\n decode_attention(q, q.view(1, 1, 1, 32), q.view(1, 1, 1, 32), torch.zeros(1, dtype=torch.long))\n"
            "except RuntimeError as e:\n print('raised', e)\n")
    out = subprocess.run([sys.executable, "-c", code, str(REPO / "cugo_amd"), str(REPO)],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    assert "raised" in out.stdout and "GPU" in out.stdout


def test_policy_state_dict_names():
    """SeqPolicy carries the parameter names of a reference SeqNet(hybrid) checkpoint
    (python/cugo_seq50.py:150-167)."""
    from cugo_amd.seq_selfplay import SeqPolicy

    names = set(SeqPolicy().state_dict())
    for key in ("event_in.weight", "start_in.bias", "query_in.0.weight", "query_in.2.bias",
                "position", "token_type", "encoder.layers.3.self_attn.in_proj_weight",
                "encoder.layers.0.linear2.bias", "norm.weight", "head.2.weight"):
        assert key in names, key
    assert SeqPolicy().query_in[0].in_features == 720 + 179
