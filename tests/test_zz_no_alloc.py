"""The allocation-free entry point cugo_play_random_noalloc, called through the C ABI.

It must give, bit for bit, what the existing entry points give on the same inputs:
cugo_refill_spares on fresh spares (2 slots) and cugo_play_random (through the
extension's refill_spares and play_random): the eleven outputs of the last step, the
rows, generations and samplers.  Two calls in a row on one device share the library's
static spares, the second on a smaller batch; a batch above the limit is refused with
CUGO_ERROR_SCRATCH_LIMIT before anything is launched.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests.conftest import REPO, announce

pytestmark = pytest.mark.gpu

DEV = "cuda"
SCRATCH_LIMIT_ERROR = -27  # CUGO_ERROR_SCRATCH_LIMIT
MAX_ROWS = 65536  # CUGO_NOALLOC_MAX_ROWS


def _noalloc_fn():
    lib = ctypes.CDLL(str(REPO / "cugo_amd" / "libcugo_hip.so"))
    fn = lib.cugo_play_random_noalloc
    p, i64 = ctypes.c_void_p, ctypes.c_int64
    fn.argtypes = [p, i64, p, p, p, p, p, p, p, p, p, p, p, p, ctypes.c_uint64, i64, p, i64, p]
    fn.restype = ctypes.c_int
    return fn


def _games(ext, n: int, base: int):
    seeds = (np.uint64(base) + np.arange(n, dtype=np.uint64)).view(np.int64)
    states = ext.create(torch.from_numpy(seeds).to(DEV),
                        torch.from_numpy(np.arange(n, dtype=np.int64) & 1).to(DEV))
    gen = torch.zeros(n, dtype=torch.int32, device=DEV)
    return states, gen, ext.seed_samplers(n, base, gen)


def _outputs(n: int):
    def e(*shape, dtype):
        return torch.empty(shape, dtype=dtype, device=DEV)
    return [e(n, 720, dtype=torch.float32), e(n, 179, dtype=torch.bool), e(n, dtype=torch.uint8),
            e(n, dtype=torch.bool), e(n, dtype=torch.int16), e(n, dtype=torch.int64),
            e(n, dtype=torch.float32), e(n, dtype=torch.bool), e(n, dtype=torch.bool),
            e(n, dtype=torch.int16), e(n, dtype=torch.bool)]


def _call(fn, states, sampler, out, base, gen, steps, n=None) -> int:
    n = states.shape[0] if n is None else n
    stream = torch.cuda.current_stream().cuda_stream
    return fn(states.data_ptr(), n, sampler.data_ptr(), *(t.data_ptr() for t in out),
              ctypes.c_uint64(base & (2**64 - 1)), states.shape[0], gen.data_ptr(), steps,
              ctypes.c_void_p(stream))


def test_noalloc_play_random_matches_play_random(ext):
    fn = _noalloc_fn()
    for call, (n, steps, blocks) in enumerate([(65536, 32, 3), (6002, 7, 4)]):
        announce(f"play_random_noalloc call {call}: n={n}, steps={steps} x {blocks}")
        base = 0x243F6A8885A308D3 + 977 * call
        a, gen_a, smp_a = _games(ext, n, base)
        b, gen_b, smp_b = a.clone(), gen_a.clone(), smp_a.clone()
        spares = torch.zeros((2 * n, 248), dtype=torch.uint8, device=DEV)
        spare_gen = torch.zeros(2 * n, dtype=torch.int32, device=DEV)
        for block in range(blocks):
            ext.refill_spares(spares, spare_gen, gen_a, base)
            want = ext.play_random(a, smp_a, base, gen_a, spares, spare_gen, steps=steps)
            got = _outputs(n)
            rc = _call(fn, b, smp_b, got, base, gen_b, steps)
            torch.cuda.synchronize()
            assert rc == 0, rc
            for j, (x, y) in enumerate(zip(want, got)):
                assert torch.equal(x, y), (call, block, j)
            assert torch.equal(a, b), (call, block)
            assert torch.equal(gen_a, gen_b) and torch.equal(smp_a, smp_b), (call, block)
        assert int(gen_b.sum().item()) > n // 2  # finished games took spares and deals


def test_noalloc_refuses_batches_above_its_scratch(ext):
    announce("play_random_noalloc size limit")
    fn = _noalloc_fn()
    n = MAX_ROWS + 1
    states, gen, smp = _games(ext, n, 12345)
    before = states.clone()
    out = _outputs(n)
    rc = _call(fn, states, smp, out, 12345, gen, 4)
    torch.cuda.synchronize()
    assert rc == SCRATCH_LIMIT_ERROR
    assert torch.equal(states, before) and int(gen.sum().item()) == 0
    assert _call(fn, states, smp, out, 12345, gen, 0, n=16) == -22  # steps < 1
