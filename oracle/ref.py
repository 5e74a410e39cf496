"""ctypes binding of the oracle libraries (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module.  It binds
  oracle/libcugo_oracle.so  the oracle: this repository's plain-C restatement of the
                            reference engine (oracle/matgo/), and
  oracle/_ref/libcugo_ref.so  this repository's harness (oracle/ref_harness.cpp) compiled
                            against the reference's own header-only engine, built only
                            where the reference checkout is present; it pins the oracle.
Both expose the reference extension's batch operations
(python/csrc/torch50_ext.cu:53-363) as CPU loops over 248-byte rows.

Arrays are numpy; rows are uint8 [n, 248].
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
REF_LIB = ORACLE_DIR / "_ref" / "libcugo_ref.so"
ORACLE_LIB = ORACLE_DIR / "libcugo_oracle.so"

STATE_BYTES = 248
FEATURES = 720
ACTIONS = 179
EVENT_WORDS = 9
START_WORDS = 8
SEED_BASE = 0x243F6A8885A308D3

_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


class _Lib:
    """Binds one library's batch API (`<prefix>_create`, ...) under short names."""

    SIG = {
        "state_bytes": ([], ctypes.c_int),
        "create": ([_P, _P, _I64, _P], None),
        "observe_indexed": ([_P, _P, _I64, _I64, _P, _P, _P, _P, _P], None),
        "step_indexed": ([_P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P], None),
        "start": ([_P, _I64, _P], None),
        "clone_indexed": ([_P, _P, _I64, _I64, _P], None),
        "branch_indexed": ([_P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P], None),
        "hands_indexed": ([_P, _P, _I64, _I64, _P], None),
        "stock_indexed": ([_P, _P, _I64, _I64, _P], None),
        "reward0": ([_P], ctypes.c_int64),
        "record_bytes": ([], ctypes.c_int),
        "play_random": ([ctypes.c_uint64, _I64, ctypes.c_int, _P, _P, _P, _P, _I64,
                         ctypes.c_int32], ctypes.c_int64),
        "branch_work": ([_P, _P, _P, _I64, ctypes.c_int, ctypes.c_int], ctypes.c_uint64),
        "rollout_canonical": ([_P, _P, _I64, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P],
                              None),
    }

    def __init__(self, lib: ctypes.CDLL, prefix: str) -> None:
        for name, (args, res) in self.SIG.items():
            fn = getattr(lib, f"{prefix}_{name}")
            fn.argtypes = args
            fn.restype = res
            setattr(self, name, fn)


class RefEngine:
    """A CPU engine with the batch API of the reference extension.  By default the
    oracle (this repository's plain-C restatement, oracle/matgo/); `reference=True`
    loads the reference's own build (oracle/_ref), which pins the restatement."""

    def __init__(self, path: Path | str | None = None, reference: bool = False,
                 threads: int | None = None) -> None:
        path = Path(path) if path is not None else (REF_LIB if reference else ORACLE_LIB)
        if not path.exists():
            hint = ("`make -C oracle ref` where the reference checkout is present" if reference
                    else "`make -C oracle oracle`")
            raise FileNotFoundError(f"{path} is missing: build it with {hint}")
        self.path = path
        self.kind = "reference" if reference else "oracle"
        cdll = ctypes.CDLL(str(path))
        self.lib = _Lib(cdll, "cugo_ref" if reference else "cugo_oracle")
        assert self.lib.state_bytes() == STATE_BYTES
        self.record_bytes = self.lib.record_bytes()
        # The oracle's contiguous batch loops (create, observe, step without ids) run on a
        # thread pool; rows are independent, so the outputs are the sequential loop's.
        setter = getattr(cdll, "cugo_oracle_set_threads", None)
        if setter is not None:
            setter.argtypes = [ctypes.c_int]
            setter.restype = None
            setter(threads if threads is not None else min(os.cpu_count() or 1, 16))

    # -- extension operations -------------------------------------------------------
    def create(self, seeds: np.ndarray, first: np.ndarray) -> np.ndarray:
        seeds = np.ascontiguousarray(seeds, dtype=np.int64)
        first = np.ascontiguousarray(first, dtype=np.int64)
        out = np.zeros((seeds.size, STATE_BYTES), dtype=np.uint8)
        self.lib.create(_ptr(seeds), _ptr(first), seeds.size, _ptr(out))
        return out

    def observe(self, states: np.ndarray, ids: np.ndarray | None = None):
        states = np.ascontiguousarray(states, dtype=np.uint8)
        n = states.shape[0] if ids is None else ids.size
        if ids is not None:
            ids = np.ascontiguousarray(ids, dtype=np.int64)
        f = np.zeros((n, FEATURES), dtype=np.float32)
        legal = np.zeros((n, ACTIONS), dtype=np.uint8)
        player = np.zeros(n, dtype=np.uint8)
        done = np.zeros(n, dtype=np.uint8)
        status = np.zeros(n, dtype=np.int16)
        self.lib.observe_indexed(_ptr(states), _ptr(ids), n, states.shape[0], _ptr(f),
                                          _ptr(legal), _ptr(player), _ptr(done), _ptr(status))
        return f, legal.astype(bool), player, done.astype(bool), status

    def step(self, states: np.ndarray, actions: np.ndarray, ids: np.ndarray | None = None,
             events: bool = False):
        """In place on `states` (a C-contiguous uint8 [N, 248] array)."""
        assert states.dtype == np.uint8 and states.flags.c_contiguous
        actions = np.ascontiguousarray(actions, dtype=np.int64)
        if ids is not None:
            ids = np.ascontiguousarray(ids, dtype=np.int64)
        n = actions.size
        reward = np.zeros(n, dtype=np.float32)
        done = np.zeros(n, dtype=np.uint8)
        nagari = np.zeros(n, dtype=np.uint8)
        status = np.zeros(n, dtype=np.int16)
        committed = np.zeros(n, dtype=np.uint8)
        ev = np.zeros((n, EVENT_WORDS), dtype=np.int64) if events else None
        self.lib.step_indexed(_ptr(states), _ptr(ids), _ptr(actions), n,
                                       states.shape[0], _ptr(reward), _ptr(done), _ptr(nagari),
                                       _ptr(status), _ptr(committed), _ptr(ev))
        out = (reward, done.astype(bool), nagari.astype(bool), status, committed.astype(bool))
        return out + (ev,) if events else out

    def start(self, states: np.ndarray) -> np.ndarray:
        states = np.ascontiguousarray(states, dtype=np.uint8)
        out = np.zeros((states.shape[0], START_WORDS), dtype=np.int64)
        self.lib.start(_ptr(states), states.shape[0], _ptr(out))
        return out

    def clone(self, states: np.ndarray, ids: np.ndarray) -> np.ndarray:
        states = np.ascontiguousarray(states, dtype=np.uint8)
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        out = np.zeros((ids.size, STATE_BYTES), dtype=np.uint8)
        self.lib.clone_indexed(_ptr(states), _ptr(ids), ids.size, states.shape[0],
                                        _ptr(out))
        return out

    def branch(self, states: np.ndarray, ids: np.ndarray, actions: np.ndarray):
        states = np.ascontiguousarray(states, dtype=np.uint8)
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        actions = np.ascontiguousarray(actions, dtype=np.int64)
        n = ids.size
        children = np.zeros((n, STATE_BYTES), dtype=np.uint8)
        reward = np.zeros(n, dtype=np.float32)
        done = np.zeros(n, dtype=np.uint8)
        nagari = np.zeros(n, dtype=np.uint8)
        status = np.zeros(n, dtype=np.int16)
        committed = np.zeros(n, dtype=np.uint8)
        self.lib.branch_indexed(_ptr(states), _ptr(ids), _ptr(actions), n,
                                         states.shape[0], _ptr(children), _ptr(reward),
                                         _ptr(done), _ptr(nagari), _ptr(status),
                                         _ptr(committed))
        return (children, reward, done.astype(bool), nagari.astype(bool), status,
                committed.astype(bool))

    def hands(self, states: np.ndarray, ids: np.ndarray) -> np.ndarray:
        states = np.ascontiguousarray(states, dtype=np.uint8)
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        out = np.zeros((ids.size, 2), dtype=np.int64)
        self.lib.hands_indexed(_ptr(states), _ptr(ids), ids.size, states.shape[0],
                                        _ptr(out))
        return out

    def stock(self, states: np.ndarray, ids: np.ndarray) -> np.ndarray:
        states = np.ascontiguousarray(states, dtype=np.uint8)
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        out = np.zeros(ids.size, dtype=np.int64)
        self.lib.stock_indexed(_ptr(states), _ptr(ids), ids.size, states.shape[0],
                                        _ptr(out))
        return out

    def reward0(self, row: np.ndarray) -> int:
        row = np.ascontiguousarray(row, dtype=np.uint8)
        return int(self.lib.reward0(_ptr(row)))

    # -- whole random-policy games and branch work -----------------------------------
    def play_random(self, base_seed: int, n: int, threads: int = 1, record_games: int = 0,
                    record_cap: int = 64, outputs: bool = True):
        digest = np.zeros(n, dtype=np.uint64) if outputs else None
        steps = np.zeros(n, dtype=np.int32) if outputs else None
        reward = np.zeros(n, dtype=np.int64) if outputs else None
        records = None
        if record_games:
            records = np.zeros((record_games, record_cap, self.record_bytes), dtype=np.uint8)
        total = self.lib.play_random(ctypes.c_uint64(base_seed & (2**64 - 1)), n,
                                              threads, _ptr(digest), _ptr(steps), _ptr(reward),
                                              _ptr(records), record_games, record_cap)
        return digest, steps, reward, records, int(total)

    def branch_work(self, roots: np.ndarray, ids: np.ndarray, actions: np.ndarray,
                    threads: int, observe: bool) -> int:
        roots = np.ascontiguousarray(roots, dtype=np.uint8)
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        actions = np.ascontiguousarray(actions, dtype=np.int64)
        return int(self.lib.branch_work(_ptr(roots), _ptr(ids), _ptr(actions), ids.size,
                                                 threads, int(observe)))


    def rollout_canonical(self, seeds: np.ndarray, first: np.ndarray, max_actions: int = 128,
                          threads: int | None = None, explicit: bool = False) -> np.ndarray:
        """The canonical whole-game driver (rollout_canonical_torch50, torch50.h:598-619;
        explicit=True on the reference build: rollout_canonical50, rollout50.h:616-703)
        from seeds[i] / first[i]: int64 [n, 5] digest words (CANONICAL_FIELDS)."""
        seeds = np.ascontiguousarray(seeds, dtype=np.int64)
        first = np.ascontiguousarray(first, dtype=np.int64)
        out = np.zeros((seeds.size, 5), dtype=np.int64)
        threads = threads if threads is not None else min(os.cpu_count() or 1, 16)
        self.lib.rollout_canonical(_ptr(seeds), _ptr(first), seeds.size, max_actions, threads,
                                   int(explicit), _ptr(out))
        return out


# Digest words of a canonical rollout: (word, shift, bits) of each field.
CANONICAL_FIELDS = {
    "final_points": (0, 0, 64), "reward0": (1, 0, 64),
    "actions": (2, 0, 16), "turns": (2, 16, 16), "bonus_actions": (2, 32, 16),
    "special_actions": (2, 48, 16), "go_actions": (3, 0, 16), "end": (3, 16, 8),
    "action_status": (3, 24, 8), "terminal_reason": (3, 32, 8), "winner": (3, 40, 8),
    "next_round_multiplier": (3, 48, 8), "choice_actions": (4, 0, 16),
    "resolve_choices": (4, 16, 16), "pi_choices": (4, 32, 16),
}


def canonical_field(words: np.ndarray, name: str) -> np.ndarray:
    """One field of int64 [n, 5] canonical digest words."""
    w, shift, bits = CANONICAL_FIELDS[name]
    col = words[:, w]
    if bits == 64:
        return col
    return ((col.view(np.uint64) >> np.uint64(shift)) & np.uint64((1 << bits) - 1)).astype(np.int64)


# -- the C1 random-policy protocol, in numpy (shared by tests and the bench) ----------
MASK64 = (1 << 64) - 1


def splitmix_first(seed: int) -> int:
    """SplitMix64(seed).next_u64() (reference include/cugo/core/rng.h:17-22); 0 -> 1."""
    z = (seed + 0x9E3779B97F4A7C15) & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    z = z ^ (z >> 31)
    return z if z != 0 else 1


def xorshift_batch(state: np.ndarray) -> np.ndarray:
    """One xorshift64 (13, 7, 17) step on a uint64 array, in place; returns the outputs."""
    state ^= state << np.uint64(13)
    state ^= state >> np.uint64(7)
    state ^= state << np.uint64(17)
    return state.copy()


def sample_actions(legal: np.ndarray, sampler: np.ndarray, active: np.ndarray) -> np.ndarray:
    """legal[i] ascending list [xorshift(sampler[i]) % count] for active rows with a legal
    action, -1 otherwise; advances sampler only for those rows."""
    n = legal.shape[0]
    actions = np.full(n, -1, dtype=np.int64)
    counts = legal.sum(axis=1)
    rows = np.nonzero(active & (counts > 0))[0]
    if rows.size:
        sub = sampler[rows].copy()
        draws = xorshift_batch(sub)
        sampler[rows] = sub
        picks = (draws % counts[rows].astype(np.uint64)).astype(np.int64)
        cums = np.cumsum(legal[rows], axis=1)
        actions[rows] = np.argmax(cums > picks[:, None], axis=1)
    return actions


FNV_OFFSET = np.uint64(0xCBF29CE484222325)
FNV_PRIME = np.uint64(0x100000001B3)


def fnv_update(h: np.ndarray, records: np.ndarray) -> np.ndarray:
    """FNV-1a over each row of a uint8 [n, k] array, continuing digests h [n]."""
    h = h.copy()
    for col in range(records.shape[1]):
        h ^= records[:, col].astype(np.uint64)
        h *= FNV_PRIME
    return h


def step_record(features, legal, player, done, status, actions, reward, sdone, nagari,
                sstatus, committed, events) -> np.ndarray:
    """The per-decision record of cugo_ref_play_random as a uint8 [n, 3152] array."""
    n = features.shape[0]
    parts = [
        np.ascontiguousarray(features, dtype=np.float32).view(np.uint8).reshape(n, -1),
        legal.astype(np.uint8).reshape(n, -1),
        player.astype(np.uint8).reshape(n, 1),
        done.astype(np.uint8).reshape(n, 1),
        status.astype(np.int16).view(np.uint8).reshape(n, 2),
        actions.astype(np.int64).view(np.uint8).reshape(n, 8),
        reward.astype(np.float32).view(np.uint8).reshape(n, 4),
        sdone.astype(np.uint8).reshape(n, 1),
        nagari.astype(np.uint8).reshape(n, 1),
        sstatus.astype(np.int16).view(np.uint8).reshape(n, 2),
        committed.astype(np.uint8).reshape(n, 1),
        np.ascontiguousarray(events, dtype=np.int64).view(np.uint8).reshape(n, -1),
    ]
    return np.concatenate(parts, axis=1)


# Byte ranges of a row that hold no field (zero in every row the engines write).
PADDING = ((78, 80), (90, 96), (103, 104), (116, 120), (125, 126), (130, 136), (153, 160),
           (197, 200), (220, 224), (241, 248))


class OracleRules:
    """Rule-level entry points of the oracle (oracle/matgo/matgo.c) for the reference's
    known-answer tests: score_captured, go_adjusted_score50 and settle_terminal50."""

    def __init__(self, path: Path | str = ORACLE_LIB) -> None:
        lib = ctypes.CDLL(str(path))
        lib.cugo_oracle_score.argtypes = [ctypes.c_uint64, ctypes.c_int, _P]
        lib.cugo_oracle_score.restype = None
        lib.cugo_oracle_go_points.argtypes = [ctypes.c_uint8, ctypes.c_uint8]
        lib.cugo_oracle_go_points.restype = ctypes.c_uint64
        lib.cugo_oracle_settle.argtypes = [_P, _P]
        lib.cugo_oracle_settle.restype = None
        self.lib = lib

    FIELDS = ("bright_count", "animal_count", "ribbon_count", "pi_units", "bright_points",
              "animal_points", "ribbon_points", "pi_points", "flags", "total_points")

    def score(self, cards: int, gukjin_as_pi: bool = False) -> dict:
        out = np.zeros(10, dtype=np.uint8)
        self.lib.cugo_oracle_score(ctypes.c_uint64(cards), int(gukjin_as_pi), _ptr(out))
        return dict(zip(self.FIELDS, (int(v) for v in out)))

    def go_points(self, base: int, go_count: int) -> int:
        return int(self.lib.cugo_oracle_go_points(base, go_count))

    def settle(self, row: np.ndarray) -> dict:
        row = np.ascontiguousarray(row, dtype=np.uint8)
        out = np.zeros(4, dtype=np.int64)
        self.lib.cugo_oracle_settle(_ptr(row), _ptr(out))
        return {"status": int(out[0]), "winner": int(out[1]), "final_points": int(out[2]),
                "side0": int(out[3])}
