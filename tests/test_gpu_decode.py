"""GPU parity of the HIP decode attention (cugo_decode_attention / _append) against the
reference's matmul formulation (python/cugo_seq_attention50.py:58-62, restated in
oracle/decode_ref.py) and the float64 brute force.

Tolerances: relative Frobenius error <= 1e-2 against the matmul path in bf16 (the
north-star bar; the matmul path itself rounds scores and probabilities to bf16), and
<= 4e-3 against the float64 definition (bf16 output rounding is 2^-9 relative).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cugo_amd.cugo_seq_attention50 import (decode_attention, decode_attention_append,
                                           decode_order)
from oracle.decode_ref import brute_force, matmul_path
from oracle.seq_ref import reference_cached_step
from tests.conftest import announce

pytestmark = pytest.mark.gpu

DEV = "cuda"


def rel_err(got: torch.Tensor, want) -> float:
    got = got.double().cpu()
    want = torch.as_tensor(want).double().cpu()
    return float(torch.linalg.vector_norm(got - want) / torch.linalg.vector_norm(want))


def make_case(n, rows, heads, slots, dh, seed, qdt=torch.bfloat16, kvdt=torch.bfloat16,
              qscale=0.5, kscale=0.5):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = (torch.randn(n, heads, dh, generator=g) * qscale).to(qdt).to(DEV)
    k = (torch.randn(rows, heads, slots, dh, generator=g) * kscale).to(kvdt).to(DEV)
    v = torch.randn(rows, heads, slots, dh, generator=g).to(kvdt).to(DEV)
    return q, k, v


def test_small_shapes_against_float64(ext):
    announce("decode small shapes vs float64")
    for dh, kvdt, qdt in ((32, torch.bfloat16, torch.bfloat16), (16, torch.bfloat16, torch.bfloat16),
                          (64, torch.bfloat16, torch.bfloat16), (128, torch.bfloat16, torch.bfloat16),
                          (32, torch.bfloat16, torch.float32), (32, torch.float16, torch.float16),
                          (32, torch.float32, torch.float32), (64, torch.float32, torch.bfloat16)):
        n, rows, heads, slots = 37, 23, 8, 77
        q, k, v = make_case(n, rows, heads, slots, dh, seed=dh + 3 * n, qdt=qdt, kvdt=kvdt)
        g = np.random.default_rng(dh)
        row_ids = torch.from_numpy(g.integers(0, rows, n)).to(DEV)
        pos = torch.from_numpy(g.integers(0, slots, n)).to(DEV)
        pos[:4] = torch.tensor([0, slots - 1, slots + 5, 63], device=DEV)
        out = decode_attention(q, k, v, pos, rows=row_ids)
        assert out.dtype == q.dtype and out.shape == q.shape
        want = brute_force(q.float().cpu().numpy(), k.float().cpu().numpy(),
                           v.float().cpu().numpy(), pos.cpu().numpy(), row_ids.cpu().numpy())
        tol = 4e-3 if qdt == torch.bfloat16 else 1e-5 if qdt == torch.float32 else 1e-3
        err = rel_err(out, want)
        assert err <= tol, (dh, kvdt, qdt, err)


def test_short_caches_every_head_grouping(ext):
    """Short caches are served with several heads per wavefront (1, 2, 4 or 8, chosen from
    the slot count and the heads): every grouping, plain and fused-append, against float64."""
    announce("decode short caches, grouped heads")
    for dh, kvdt, qdt in ((32, torch.bfloat16, torch.bfloat16), (64, torch.bfloat16, torch.bfloat16),
                          (16, torch.bfloat16, torch.bfloat16), (32, torch.float32, torch.float32)):
        for heads in (1, 2, 4, 8, 16):
            for slots in (5, 16, 33, 50):
                n, rows = 9, 11
                seed = dh * 1000 + heads * 100 + slots
                q, k, v = make_case(n, rows, heads, slots, dh, seed=seed, qdt=qdt, kvdt=kvdt)
                g = np.random.default_rng(seed)
                row_ids = torch.from_numpy(g.permutation(rows)[:n]).to(DEV)
                pos = torch.from_numpy(g.integers(0, slots, n)).to(DEV)
                pos[:2] = torch.tensor([0, slots - 1], device=DEV)
                tol = 4e-3 if qdt == torch.bfloat16 else 1e-5
                out = decode_attention(q, k, v, pos, rows=row_ids)
                want = brute_force(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                   v.float().cpu().numpy(), pos.cpu().numpy(),
                                   row_ids.cpu().numpy())
                assert rel_err(out, want) <= tol, (dh, heads, slots)
                kn = (q * 0.5).to(kvdt)
                vn = (q * -0.25).to(kvdt)
                k2, v2 = k.clone(), v.clone()
                out2 = decode_attention_append(q, kn, vn, k2, v2, pos, rows=row_ids)
                k3, v3 = k.clone(), v.clone()
                k3[row_ids, :, pos] = kn
                v3[row_ids, :, pos] = vn
                assert torch.equal(k2, k3) and torch.equal(v2, v3), (dh, heads, slots)
                want2 = brute_force(q.float().cpu().numpy(), k3.float().cpu().numpy(),
                                    v3.float().cpu().numpy(), pos.cpu().numpy(),
                                    row_ids.cpu().numpy())
                assert rel_err(out2, want2) <= tol, (dh, heads, slots, "append")


def test_strided_rows_read_in_place(ext):
    """q, k_new and v_new as column slices of one packed [n, 3 * heads * dh] projection
    (what cached_step passes): results and cache writes identical to contiguous copies."""
    announce("decode strided q / k_new / v_new")
    n, rows, heads, slots, dh = 300, 512, 8, 50, 32
    _, k, v = make_case(n, rows, heads, slots, dh, seed=21)
    g = torch.Generator(device="cpu").manual_seed(22)
    qkv = (torch.randn(n, 3 * heads * dh, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    q, kn, vn = (t.reshape(n, heads, dh) for t in qkv.chunk(3, -1))
    assert not q.is_contiguous()
    row_ids = torch.from_numpy(np.random.default_rng(23).permutation(rows)[:n]).to(DEV)
    pos = torch.from_numpy(np.random.default_rng(24).integers(0, slots, n)).to(DEV)
    k1, v1, k2, v2 = k.clone(), v.clone(), k.clone(), v.clone()
    a = decode_attention_append(q, kn, vn, k1, v1, pos, rows=row_ids)
    b = decode_attention_append(q.contiguous(), kn.contiguous(), vn.contiguous(), k2, v2, pos,
                                rows=row_ids)
    assert torch.equal(a, b) and torch.equal(k1, k2) and torch.equal(v1, v2)
    assert torch.equal(decode_attention(q, k1, v1, pos, rows=row_ids),
                       decode_attention(q.contiguous(), k1, v1, pos, rows=row_ids))


def test_reference_shape_against_matmul_path(ext):
    """The reference's cache: [2 x 4,096 rows, 8 heads, 50 slots, 32] bf16, 4,096 queries
    on distinct random rows, ragged pos in [0, 49]."""
    announce("decode reference shape vs matmul path")
    q, k, v = make_case(4096, 8192, 8, 50, 32, seed=5)
    g = np.random.default_rng(6)
    rows = torch.from_numpy(g.permutation(8192)[:4096]).to(DEV)
    pos = torch.from_numpy(g.integers(0, 50, 4096)).to(DEV)
    out = decode_attention(q, k, v, pos, rows=rows)
    want = matmul_path(q, k, v, pos, rows)
    assert rel_err(out, want.float()) <= 1e-2
    # no rows argument: row i
    out0 = decode_attention(q, k[:4096].contiguous(), v[:4096].contiguous(), pos)
    want0 = matmul_path(q, k[:4096], v[:4096], pos)
    assert rel_err(out0, want0.float()) <= 1e-2


def test_320_slot_cache_against_matmul_path(ext):
    """One layer of the 320-slot cache [4,096, 8, 320, 32] bf16 with ragged pos up to 319."""
    announce("decode 320-slot cache vs matmul path")
    q, k, v = make_case(4096, 4096, 8, 320, 32, seed=7)
    g = np.random.default_rng(8)
    pos = torch.from_numpy(g.integers(0, 320, 4096)).to(DEV)
    pos[:3] = torch.tensor([0, 319, 255], device=DEV)
    out = decode_attention(q, k, v, pos)
    want = matmul_path(q, k, v, pos)
    assert rel_err(out, want.float()) <= 1e-2
    # per-query check as well: no query may be far off even if the aggregate is close
    per = ((out.float() - want.float()).norm(dim=(1, 2)) / want.float().norm(dim=(1, 2)))
    assert float(per.max()) <= 2e-2


def test_append_equals_index_put_then_decode(ext):
    announce("decode append vs index_put_ + decode")
    n, rows, heads, slots, dh = 1000, 2048, 8, 50, 32
    q, k, v = make_case(n, rows, heads, slots, dh, seed=9)
    g = torch.Generator(device="cpu").manual_seed(10)
    k_new = torch.randn(n, heads, dh, generator=g).to(torch.bfloat16).to(DEV)
    v_new = torch.randn(n, heads, dh, generator=g).to(torch.bfloat16).to(DEV)
    row_ids = torch.from_numpy(np.random.default_rng(11).permutation(rows)[:n]).to(DEV)
    pos = torch.from_numpy(np.random.default_rng(12).integers(0, slots, n)).to(DEV)
    pos[:2] = torch.tensor([0, slots - 1], device=DEV)
    k1, v1 = k.clone(), v.clone()
    flat_rows = (row_ids.view(n, 1) * heads + torch.arange(heads, device=DEV).view(1, heads)).flatten()
    flat_pos = pos.repeat_interleave(heads)
    k1.view(-1, slots, dh).index_put_((flat_rows, flat_pos), k_new.reshape(n * heads, dh))
    v1.view(-1, slots, dh).index_put_((flat_rows, flat_pos), v_new.reshape(n * heads, dh))
    want = decode_attention(q, k1, v1, pos, rows=row_ids)
    k2, v2 = k.clone(), v.clone()
    got = decode_attention_append(q, k_new, v_new, k2, v2, pos, rows=row_ids)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    assert rel_err(got, want.float()) <= 2e-3
    assert rel_err(got, matmul_path(q, k1, v1, pos, row_ids).float()) <= 1e-2


def test_kv_append_equals_index_put(ext):
    """kv_append == index_put_ of k_new / v_new at slot min(pos, slots - 1) of each row
    (the append of decode_attention_append without its attention), with strided inputs
    (columns of a packed projection), skipped tokens (pos < 0) and rows outside the cache
    writing nothing."""
    announce("kv_append vs index_put_")
    n, rows, heads, slots, dh = 1000, 2048, 8, 50, 32
    _, k, v = make_case(n, rows, heads, slots, dh, seed=19)
    g = torch.Generator(device="cpu").manual_seed(20)
    packed = torch.randn(n, 3, heads, dh, generator=g).to(torch.bfloat16).to(DEV)
    k_new, v_new = packed[:, 1], packed[:, 2]
    row_ids = torch.from_numpy(np.random.default_rng(21).permutation(rows)[:n]).to(DEV)
    pos = torch.from_numpy(np.random.default_rng(22).integers(0, slots + 3, n)).to(DEV)
    pos[:3] = torch.tensor([-1, slots + 9, 0], device=DEV)
    row_ids[3] = rows + 5
    want_k, want_v = k.clone(), v.clone()
    keep = (pos >= 0) & (row_ids < rows)
    at = pos.clamp_max(slots - 1)
    flat_rows = (row_ids[keep].view(-1, 1) * heads + torch.arange(heads, device=DEV)).flatten()
    flat_pos = at[keep].repeat_interleave(heads)
    want_k.view(-1, slots, dh).index_put_((flat_rows, flat_pos), k_new[keep].reshape(-1, dh))
    want_v.view(-1, slots, dh).index_put_((flat_rows, flat_pos), v_new[keep].reshape(-1, dh))
    ext.kv_append(k_new, v_new, k, v, pos, row_ids)
    assert torch.equal(k, want_k) and torch.equal(v, want_v)


def test_nan_and_clamp_semantics(ext):
    announce("decode NaN / clamp semantics")
    q, k, v = make_case(6, 4, 8, 10, 32, seed=13)
    rows = torch.tensor([0, 1, 2, 3, 4, -1], device=DEV)
    pos = torch.tensor([-1, 3, 9, 50, 2, 2], device=DEV)
    out = decode_attention(q, k, v, pos, rows=rows).float()
    assert torch.isnan(out[0]).all() and torch.isnan(out[4]).all() and torch.isnan(out[5]).all()
    assert not torch.isnan(out[1:4]).any()
    clamp = decode_attention(q[3:4], k, v, torch.tensor([9], device=DEV), rows=rows[3:4])
    assert torch.equal(out[3].to(torch.bfloat16), clamp[0])
    empty = decode_attention(q[:0], k, v, pos[:0], rows=rows[:0])
    assert empty.shape == (0, 8, 32)


def test_argument_errors(ext):
    announce("decode argument errors")
    q, k, v = make_case(4, 4, 8, 10, 32, seed=14)
    pos = torch.zeros(4, dtype=torch.int64, device=DEV)
    with pytest.raises(RuntimeError):
        decode_attention(q, k[:, :4].contiguous(), v[:, :4].contiguous(), pos)  # heads mismatch
    with pytest.raises(RuntimeError):
        decode_attention(q, k.transpose(1, 2), v.transpose(1, 2), pos)  # not contiguous
    with pytest.raises(RuntimeError):
        decode_attention(q, k, v, pos.int())
    with pytest.raises(RuntimeError):
        decode_attention(q.cpu(), k, v, pos)
    q48, k48, v48 = make_case(2, 2, 2, 4, 48, seed=15)
    with pytest.raises(RuntimeError):
        decode_attention(q48, k48, v48, pos[:2])  # dh = 48 is not supported


@pytest.mark.parametrize("slots", [320, 10_000])
def test_decode_order_is_longest_first(ext, slots):
    """decode_order: a permutation of the queries, non-increasing in min(pos, slots - 1)
    (negative pos last), exactly below 4,096 slots and by bins of 2^s lengths above
    (10,000 slots: s = 2)."""
    announce(f"decode_order, {slots} slots")
    g = np.random.default_rng(slots)
    n = 5000
    pos = torch.from_numpy(g.integers(-3, slots + 40, n)).to(DEV)
    order = decode_order(pos, slots)
    assert order.dtype == torch.int32 and order.shape == (n,)
    o = order.long().cpu()
    assert torch.equal(o.sort().values, torch.arange(n))
    clamped = pos.cpu().clamp(-1, slots - 1)
    shift = 0 if slots < 4096 else 2
    key = (slots - 1 - clamped[o]) >> shift
    assert bool((key[1:] >= key[:-1]).all())
    assert decode_order(pos[:0], slots).shape == (0,)
    assert int(decode_order(pos[:1], slots)[0]) == 0


@pytest.mark.parametrize("slots", [320, 50])
def test_decode_order_changes_no_result(ext, slots):
    """The same queries served in another order (decode_order's, a reversal, a random
    permutation) give bit-identical outputs and cache writes, with and without the append;
    an order entry outside [0, n) leaves its query's output unwritten.  4,096 queries on
    ragged rows: more workgroups than the chip holds at once."""
    announce(f"decode order invariance, {slots}-slot cache")
    n, rows, heads, dh = 4096, 4096, 8, 32
    q, k, v = make_case(n, rows, heads, slots, dh, seed=31 + slots)
    g = np.random.default_rng(32)
    row_ids = torch.from_numpy(g.permutation(rows)).to(DEV)
    pos = torch.from_numpy(g.integers(0, slots, n)).to(DEV)
    pos[:3] = torch.tensor([-1, slots + 7, 0], device=DEV)
    k_new = (torch.randn(n, heads, dh, generator=torch.Generator().manual_seed(33)) * 0.5).to(
        torch.bfloat16).to(DEV)
    v_new = k_new.flip(0).contiguous()
    want = decode_attention(q, k, v, pos, rows=row_ids)
    k0, v0 = k.clone(), v.clone()
    want_app = decode_attention_append(q, k_new, v_new, k0, v0, pos, rows=row_ids)
    orders = [decode_order(pos, slots), torch.arange(n - 1, -1, -1, device=DEV, dtype=torch.int32),
              torch.from_numpy(g.permutation(n).astype(np.int32)).to(DEV)]
    for order in orders:
        got = decode_attention(q, k, v, pos, rows=row_ids, order=order)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        k1, v1 = k.clone(), v.clone()
        got = decode_attention_append(q, k_new, v_new, k1, v1, pos, rows=row_ids, order=order)
        assert torch.equal(got.view(torch.int16), want_app.view(torch.int16))
        assert torch.equal(k1, k0) and torch.equal(v1, v0)
    order = orders[2].clone()
    skipped = int(order[17])
    order[17] = -1
    out = torch.full_like(q, 3.0)
    decode_attention_append(q, k_new, v_new, k.clone(), v.clone(), pos, rows=row_ids, out=out,
                            order=order)
    assert bool((out[skipped] == 3.0).all())
    keep = torch.arange(n, device=DEV) != skipped
    assert torch.equal(out[keep].view(torch.int16), want_app[keep].view(torch.int16))
    with pytest.raises(RuntimeError):
        decode_attention(q, k, v, pos, rows=row_ids, order=order.long())
    with pytest.raises(RuntimeError):
        decode_attention(q, k, v, pos, rows=row_ids, order=order[:-1])


def _layered_model(layers=4, d=256, heads=8, seed=0):
    torch.manual_seed(seed)
    layer = torch.nn.TransformerEncoderLayer(d, heads, 4 * d, dropout=0.0, activation="gelu",
                                             batch_first=True, norm_first=True)
    enc = torch.nn.TransformerEncoder(layer, layers, enable_nested_tensor=False)
    model = torch.nn.Module()
    model.encoder = enc
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0.0, 0.02)
    return model.to(DEV).to(torch.bfloat16).eval()


def test_cached_step_matches_reference_and_replays_in_a_graph(ext):
    """Four steps of the 4-layer d256 policy decode through the fused HIP step and the
    reference formulation; then the fused step captured in a HIP graph and replayed."""
    announce("decode cached_step vs reference, graph replay")
    from cugo_amd.seq_decode import KVCache, cached_step

    model = _layered_model()
    rows_n, n = 512, 256
    ca = KVCache(4, rows_n, 8, 256, 50, torch.device(DEV))
    cb = KVCache(4, rows_n, 8, 256, 50, torch.device(DEV))
    g = torch.Generator(device="cpu").manual_seed(16)
    with torch.no_grad():
        for step in range(4):
            rows = torch.randperm(rows_n, generator=g)[:n].to(DEV)
            x = (torch.randn(n, 256, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
            ha = cached_step(model, ca, x, rows=rows)
            hb = reference_cached_step(model, cb, x, rows)
            assert rel_err(ha, hb.float()) <= 1e-2, step
            ca.length.index_add_(0, rows, torch.ones_like(rows))
            cb.length.index_add_(0, rows, torch.ones_like(rows))
        assert rel_err(ca.k.float(), cb.k.float()) <= 1e-2

        rows = torch.randperm(rows_n, generator=g)[:n].to(DEV)
        x = (torch.randn(n, 256, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
        k0, v0 = ca.k.clone(), ca.v.clone()
        eager = cached_step(model, ca, x, rows=rows)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            cached_step(model, ca, x, rows=rows)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = cached_step(model, ca, x, rows=rows)
        for _ in range(3):
            ca.k.copy_(k0)
            ca.v.copy_(v0)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert rel_err(out, eager.float()) <= 1e-3


def _event_counts(ext, games: int, base: int) -> torch.Tensor:
    """Committed events of each of `games` seeded random-policy games (seed base + j,
    first j & 1), played to the end on the HIP engine."""
    idx = torch.arange(games, dtype=torch.int64, device=DEV)
    states = ext.create(idx + base, idx & 1)
    sampler = ext.seed_samplers(games, base, torch.zeros(games, dtype=torch.int32, device=DEV))
    count = torch.zeros(games, dtype=torch.int64, device=DEV)
    for _ in range(128):
        _, legal, _, done, _ = ext.observe(states)
        if bool(done.all()):
            return count
        out = ext.step_events_indexed(states, idx, ext.sample_uniform(legal, sampler))
        count += (out[4] & ~done).long()
    raise AssertionError("random-policy games did not finish")


@pytest.mark.parametrize("lengths", ["stress", "full", "natural"])
def test_cached_step_full_cache_with_game_lengths(ext, lengths):
    """The sequence policy's step at its full cache shape: 4 layers, d 256, 8 heads of 32,
    cache [4, 4,096, 8, 320, 32] bf16.  Row lengths come from seeded random-policy games,
    as the bench draws them (bench.decode_lengths): "stress" concatenates consecutive
    games' token logs (each game's opening token and events) until a per-row target
    uniform in [1, 320] is reached, "full" while they fit below 320 slots, "natural"
    holds one game.  Two steps of the fused HIP step against the reference formulation
    (index_put_ + the matmul decode path, oracle/seq_ref.py) on identical caches: hidden
    states within 1e-2 relative, and the appended key/value slots within 1e-2."""
    from bench import decode_lengths
    from cugo_amd.seq_decode import KVCache, cached_step

    announce(f"cached_step full cache [4, 4096, 8, 320, 32], {lengths} lengths")
    rows, slots, per_row = 4096, 320, 24
    ev = _event_counts(ext, rows * per_row, 0x243F6A8885A308D3 + 0xDEC0DE).view(per_row, rows)
    length = decode_lengths(torch, ev, slots, seed=0xC5)[lengths]
    assert int(length.max()) <= slots - 2 and int(length.min()) >= 1
    mean = float(length.float().mean())
    expect = {"stress": (140, 200), "full": (250, 318), "natural": (10, 40)}[lengths]
    assert expect[0] < mean < expect[1], mean
    model = _layered_model()
    ca = KVCache(4, rows, 8, 256, slots, torch.device(DEV))
    cb = KVCache(4, rows, 8, 256, slots, torch.device(DEV))
    g = torch.Generator(device=DEV).manual_seed(21)
    for t in (ca.k, ca.v):
        t.copy_((torch.randn(t.shape, generator=g, device=DEV) * 0.5).to(t.dtype))
    cb.k.copy_(ca.k)
    cb.v.copy_(ca.v)
    ca.length.copy_(length)
    cb.length.copy_(length)
    ids = torch.arange(rows, device=DEV)
    with torch.no_grad():
        for step in range(2):
            x = (torch.randn(rows, 256, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
            ha = cached_step(model, ca, x)
            hb = reference_cached_step(model, cb, x, ids)
            assert rel_err(ha, hb.float()) <= 1e-2, step
            at = ca.length.clamp_max(slots - 1)
            for layer in range(4):
                for a, b in ((ca.k, cb.k), (ca.v, cb.v)):
                    new_a = a[layer, ids, :, at]
                    new_b = b[layer, ids, :, at]
                    assert rel_err(new_a, new_b.float()) <= 1e-2, (step, layer)
            ca.length += 1
            cb.length += 1
