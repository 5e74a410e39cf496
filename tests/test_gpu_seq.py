"""GPU parity of the sequence-policy self-play step.

Event/opening token kernels against the oracle's token vectors (oracle/seq_ref.py,
pinned in tests/test_cpu_seq_oracle.py) times the Linear in float64 with the reference's
bf16 roundings; the Gumbel-max kernel against the reference's torch lines on the same
uniforms; the HIP-graph self-play step against the reference formulation of the step
(dense tokens, index_put_ + matmul attention), both driven with the same uniforms.
Tolerances: bf16 outputs within 1e-2 relative (Frobenius) with at least 98 % of the
elements bit-identical (a different fp32 summation order can move a bf16 rounding by one
unit); fp32 token outputs within 1e-5 absolute; sampled actions identical.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.seq_ref import (encode_events_np, encode_start_np, gumbel_reference,
                            reference_cached_step, token_reference)
from tests.conftest import announce

pytestmark = pytest.mark.gpu

DEV = "cuda"


def rel_err(got: torch.Tensor, want: torch.Tensor) -> float:
    got, want = got.double(), want.double()
    return float((got - want).norm() / want.norm().clamp_min(1e-30))


def random_events(ext, games: int, seed: int, steps: int = 40):
    """Committed event words (and the counts before them) of seeded random-policy games."""
    idx = torch.arange(games, dtype=torch.int64, device=DEV)
    states = ext.create(idx * 7919 + seed, idx & 1)
    gen = torch.zeros(games, dtype=torch.int32, device=DEV)
    sampler = ext.seed_samplers(games, seed, gen)
    words, counts = [], []
    count = torch.zeros(games, dtype=torch.int64, device=DEV)
    for _ in range(steps):
        _, legal, _, done, _ = ext.observe(states)
        actions = ext.sample_uniform(legal, sampler)
        out = ext.step_events_indexed(states, idx, actions)
        keep = out[4] & ~done
        words.append(out[5][keep])
        counts.append(count[keep])
        count += keep.long()
    return torch.cat(words), torch.cat(counts)


def edge_events() -> torch.Tensor:
    def m(*c):
        return sum(1 << x for x in c)
    rows = [
        [m(49) | (1 << 50), m(0, 1), m(2), m(3), m(4), m(5), m(6), m(7), 0 | (200 << 8)],
        [m(10), m(11, 12, 13), 0, 0, 0, 0, 0, 0, 1 | (3 << 8)],
        [0, 0, 0, 0, 0, 0, 0, 0, 0],
        [(1 << 64) - 1] * 8 + [1 | (11 << 8)],
    ]
    signed = [[w - (1 << 64) if w >= (1 << 63) else w for w in r] for r in rows]
    return torch.tensor(signed, dtype=torch.int64, device=DEV)


def make_weights(in_features: int, d: int, dtype, seed: int):
    g = torch.Generator(device="cpu").manual_seed(seed)
    w = (torch.randn(d, in_features, generator=g) * 0.05).to(dtype).to(DEV)
    b = (torch.randn(d, generator=g) * 0.05).to(dtype).to(DEV)
    pos = (torch.randn(49, d, generator=g) * 0.05).to(dtype).to(DEV)
    tt = (torch.randn(3, d, generator=g) * 0.05).to(dtype).to(DEV)
    return w, b, pos, tt


def check_tokens(got: torch.Tensor, want: torch.Tensor, dtype) -> None:
    if dtype == torch.float32:
        assert float((got - want).abs().max()) <= 1e-5
    else:
        assert rel_err(got, want) <= 1e-2
        same = float((got.view(torch.int16) == want.view(torch.int16)).float().mean())
        assert same >= 0.98, same


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 256), (torch.float32, 64),
                                     (torch.bfloat16, 1024)])
def test_event_tokens_against_oracle(ext, dtype, d):
    announce(f"event_tokens {dtype} d={d}")
    words, counts = random_events(ext, 256, 0xE1)
    words = torch.cat((words, edge_events()))
    n = words.shape[0]
    index = torch.cat((counts, torch.tensor([-1, 0, 47, 100], device=DEV)))
    for seat_value in (0, 1):
        seat = torch.full((n,), seat_value, dtype=torch.int64, device=DEV)
        w, b, pos, tt = make_weights(414, d, dtype, seed=seat_value + d)
        got = ext.event_tokens(words, seat, index, w.t().contiguous(), b, pos, tt)
        tok = encode_events_np(words.cpu().numpy(), seat.cpu().numpy())
        p = (1 + index.clamp(max=47)).clamp(min=0)
        want = token_reference(tok, w, b, pos[p], tt[1].expand(n, d))
        check_tokens(got, want, dtype)
        # with the first layer's norm1 in the same launch: add_layernorm's bits
        nw = (torch.randn(d, generator=torch.Generator().manual_seed(d)) * 0.3 + 1.0).to(dtype).to(DEV)
        nb = (torch.randn(d, generator=torch.Generator().manual_seed(d + 1)) * 0.1).to(dtype).to(DEV)
        ln = torch.full((n, d), float("nan"), dtype=dtype, device=DEV)
        got_n = ext.event_tokens(words, seat, index, w.t().contiguous(), b, pos, tt,
                                 ln_weight=nw, ln_bias=nb, eps=1e-5, ln_out=ln)
        assert torch.equal(got_n, got)
        assert torch.equal(ln, ext.add_layernorm(got, None, nw, nb, 1e-5)[1])
    # each event read once for both seats (rows r and r + n share event r)
    seats2 = torch.cat((torch.zeros(n, dtype=torch.int64, device=DEV),
                        torch.ones(n, dtype=torch.int64, device=DEV)))
    wt = w.t().contiguous()
    got2 = ext.event_tokens(words, seats2, index, wt, b, pos, tt)
    want2 = ext.event_tokens(words.repeat(2, 1), seats2, index.repeat(2), wt, b, pos, tt)
    assert torch.equal(got2, want2)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 256), (torch.float32, 128)])
def test_start_tokens_against_oracle(ext, dtype, d):
    announce(f"start_tokens {dtype} d={d}")
    n = 600
    idx = torch.arange(n, dtype=torch.int64, device=DEV)
    states = ext.create(idx * 104729 + 0x5EED, idx & 1)
    start = ext.start(states)
    w, b, pos, tt = make_weights(274, d, dtype, seed=7)
    for seat_value in (0, 1):
        seat = torch.full((n,), seat_value, dtype=torch.int64, device=DEV)
        got = ext.start_tokens(start, seat, w.t().contiguous(), b, pos, tt)
        tok = encode_start_np(start.cpu().numpy(), seat.cpu().numpy())
        want = token_reference(tok, w, b, pos[0].expand(n, d), tt[0].expand(n, d))
        check_tokens(got, want, dtype)


def test_token_argument_errors(ext):
    announce("token argument errors")
    words = torch.zeros((4, 9), dtype=torch.int64, device=DEV)
    seat = torch.zeros(4, dtype=torch.int64, device=DEV)
    w, b, pos, tt = make_weights(414, 256, torch.bfloat16, 0)
    with pytest.raises(RuntimeError):
        ext.event_tokens(words, seat, seat, w, b, pos, tt)  # not transposed
    with pytest.raises(RuntimeError):
        ext.event_tokens(words, seat[:3], seat, w.t().contiguous(), b, pos, tt)
    w2, b2, pos2, tt2 = make_weights(414, 96, torch.bfloat16, 0)
    with pytest.raises(RuntimeError):
        ext.event_tokens(words, seat, seat, w2.t().contiguous(), b2, pos2, tt2)  # d = 96
    out = ext.event_tokens(words[:0], seat[:0], seat[:0], w.t().contiguous(), b, pos, tt)
    assert out.shape == (0, 256)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 256), (torch.float32, 512),
                                     (torch.bfloat16, 64)])
def test_add_layernorm_matches_torch(ext, dtype, d):
    """x + y rounded as torch's add, then nn.LayerNorm of it (and of x alone)."""
    announce(f"add_layernorm {dtype} d={d}")
    g = torch.Generator(device="cpu").manual_seed(d)
    n = 3001
    x = (torch.randn(n, d, generator=g) * 2.0 + 0.5).to(dtype).to(DEV)
    y = torch.randn(n, d, generator=g).to(dtype).to(DEV)
    norm = torch.nn.LayerNorm(d).to(DEV).to(dtype)
    with torch.no_grad():
        norm.weight.copy_((torch.randn(d, generator=g) * 0.3 + 1.0).to(dtype))
        norm.bias.copy_((torch.randn(d, generator=g) * 0.1).to(dtype))
        xs, ln = ext.add_layernorm(x, y, norm.weight, norm.bias, norm.eps)
        assert torch.equal(xs, x + y)
        want = norm(x + y)
        x0, ln0 = ext.add_layernorm(x, None, norm.weight, norm.bias, norm.eps)
        assert x0.data_ptr() == x.data_ptr()
        want0 = norm(x)
    for got, ref in ((ln, want), (ln0, want0)):
        if dtype == torch.float32:
            assert float((got - ref).abs().max()) <= 1e-4
        else:
            assert rel_err(got, ref) <= 1e-2
            same = float((got.view(torch.int16) == ref.view(torch.int16)).float().mean())
            assert same >= 0.98, same


@pytest.mark.parametrize("m,n,k", [(4096, 768, 256), (8192, 1024, 256), (4096, 256, 1024),
                                   (1001, 260, 128), (1, 4, 64), (70, 1028, 512),
                                   (4096, 179, 256), (33, 7, 64)])
def test_linear_matches_float64(ext, m, n, k):
    """`linear` against the float64 product of the same bf16 operands, + bias, rounded to
    bf16: every element within the bound of an fp32 sum of k products (k 2^-24 times the
    sum of their magnitudes) rounded to bf16 (one unit), 98 % bit-identical; its GELU
    form equals torch's F.gelu of its plain form bit for bit; every workgroup tile gives
    identical bits (the same K order); with a residual, torch's bf16 add of the two; a
    row-strided x, no bias, the packed-weight cache (rebuilt in place when the weight
    changes), and the shape checks.  An n that is not a multiple of 4 (the head's 179
    logits) gives the first n columns of the same product over the zero-padded weight,
    and takes no residual."""
    from cugo_amd.seq_decode import linear, packed_weight

    announce(f"linear m={m} n={n} k={k}")
    g = torch.Generator(device="cpu").manual_seed(m + n + k)
    x = (torch.randn(m, k, generator=g)).to(torch.bfloat16).to(DEV)
    w = (torch.randn(n, k, generator=g) * k ** -0.5).to(torch.bfloat16).to(DEV)
    b = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    wp = ext.mlp_pack_weight(w, (n + 15) // 16 * 16, k)

    def check(got, bias):
        exact = x.double() @ w.double().T
        mag = x.double().abs() @ w.double().abs().T
        if bias is not None:
            exact = exact + bias.double()
            mag = mag + bias.double().abs()
        delta = mag * (k + 1) * 2.0 ** -24
        excess = (got.double() - exact).abs() - (exact.abs() * 2.0 ** -7 + 2 * delta)
        assert float(excess.max()) <= 0.0, (int((excess > 0).sum()), float(excess.max()))
        want = exact.to(torch.bfloat16)
        same = float((got.view(torch.int16) == want.view(torch.int16)).float().mean())
        assert same >= 0.98, same

    got = ext.linear(x, wp, n, b)
    assert got.shape == (m, n) and got.dtype == torch.bfloat16
    check(got, b)
    assert torch.equal(ext.linear(x, wp, n, b, gelu=True), torch.nn.functional.gelu(got))
    for tile, rows in ((1, 32), (2, 64), (3, 64), (4, 128), (5, 64), (6, 128), (7, 32)):
        if rows * k * 2 <= 160 * 1024:  # the X panel fits the LDS
            assert torch.equal(ext.linear(x, wp, n, b, tile=tile), got), tile
        else:
            with pytest.raises(RuntimeError):
                ext.linear(x, wp, n, b, tile=tile)
    check(ext.linear(x, wp, n, None), None)
    r = torch.randn(m, n, generator=g).to(torch.bfloat16).to(DEV)  # residual, torch's bf16 add
    if n % 4 != 0:
        n16 = (n + 15) // 16 * 16
        b16 = torch.zeros(n16, dtype=torch.bfloat16, device=DEV)
        b16[:n] = b
        assert torch.equal(ext.linear(x, wp, n16, b16)[:, :n], got)
        assert torch.equal(linear(x, w, b), got)
        with pytest.raises(RuntimeError):  # a residual needs n % 4 == 0
            ext.linear(x, wp, n, b, residual=r)
        return
    assert torch.equal(ext.linear(x, wp, n, b, residual=r), r + got)
    assert torch.equal(ext.linear(x, wp, n, b, gelu=True, residual=r),
                       r + torch.nn.functional.gelu(got))
    row = r[-1].contiguous()  # one row added to every row (the query token's + token_type)
    into = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    assert ext.linear(x, wp, n, b, residual=row, out=into).data_ptr() == into.data_ptr()
    assert torch.equal(into, got + row)
    wide = torch.zeros(m, k + 40, dtype=torch.bfloat16, device=DEV)
    wide[:, 8:8 + k] = x
    assert torch.equal(ext.linear(wide[:, 8:8 + k], wp, n, b), got)
    # the module-level wrapper packs the weight once and repacks it when it changes
    assert torch.equal(linear(x, w, b), got)
    assert torch.equal(linear(x, w, b, residual=r), r + got)
    p0 = packed_weight(w)
    assert torch.equal(p0, wp) and packed_weight(w) is p0
    w.mul_(-1.0)
    assert packed_weight(w) is p0 and torch.equal(linear(x, w, b), ext.linear(x, p0, n, b))
    assert torch.equal(p0, ext.mlp_pack_weight(w, (n + 15) // 16 * 16, k))
    if m == 1:
        with pytest.raises(RuntimeError):  # k = 96 is not a supported depth
            ext.linear(torch.zeros(4, 96, dtype=torch.bfloat16, device=DEV),
                       ext.mlp_pack_weight(torch.zeros(4, 96, dtype=torch.bfloat16,
                                                       device=DEV), 16, 96), 4)
        with pytest.raises(RuntimeError):  # packed size does not match n
            ext.linear(x, wp, n + 16, None)
        with pytest.raises(RuntimeError):
            ext.linear(x, wp, n, b, tile=8)


def test_linear_on_a_zero_padded_input(ext):
    """The query MLP's first layer (K = 899) on prepare's zero-padded 1,024-column rows:
    the wrapper packs the weight with zero columns to 1,024, so the result equals the
    kernel on the explicitly padded weight bit for bit, and torch's F.gelu(F.linear) on
    the unpadded input within the bf16 bar; an unpadded 899-column input falls back to
    torch."""
    from cugo_amd.seq_decode import linear

    announce("linear on a zero-padded input (899 of 1,024 columns)")
    g = torch.Generator(device="cpu").manual_seed(899)
    x = torch.randn(1000, 899, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(512, 899, generator=g) * 0.03).to(torch.bfloat16).to(DEV)
    b = (torch.randn(512, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    xpad = torch.zeros(1000, 1024, dtype=torch.bfloat16, device=DEV)
    xpad[:, :899] = x
    wpad = torch.zeros(512, 1024, dtype=torch.bfloat16, device=DEV)
    wpad[:, :899] = w
    got = linear(xpad, w, b, gelu=True)
    assert torch.equal(got, ext.linear(xpad, ext.mlp_pack_weight(wpad, 512, 1024), 512, b,
                                       gelu=True))
    want = torch.nn.functional.gelu(torch.nn.functional.linear(x, w, b))
    assert rel_err(got, want) <= 1e-2
    same = float((got.view(torch.int16) == want.view(torch.int16)).float().mean())
    assert same >= 0.98, same
    assert torch.equal(linear(x, w, b, gelu=True), want)


@pytest.mark.parametrize("m,k", [(4096, 256), (8192, 1024), (1001, 256), (1, 64)])
def test_linear_add_layernorm_equals_its_two_launches(ext, m, k):
    """linear_add_layernorm == add_layernorm(res, linear(x)) bit for bit (x_out and ln),
    with and without bias, on every tile; with one residual row for every row (the query
    token's + token_type[2]) == linear with that residual, then add_layernorm; into given
    output tensors; within torch's bf16 LayerNorm tolerance of the torch ops; the
    module-level wrapper; only 256-wide rows."""
    from cugo_amd.seq_decode import linear_add_norm

    announce(f"linear_add_layernorm m={m} k={k}")
    g = torch.Generator(device="cpu").manual_seed(m * 7 + k)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(256, k, generator=g) * k ** -0.5).to(torch.bfloat16).to(DEV)
    b = (torch.randn(256, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    res = (torch.randn(m, 256, generator=g) * 2.0).to(torch.bfloat16).to(DEV)
    norm = torch.nn.LayerNorm(256).to(DEV).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_((torch.randn(256, generator=g) * 0.3 + 1.0).to(torch.bfloat16))
        norm.bias.copy_((torch.randn(256, generator=g) * 0.1).to(torch.bfloat16))
        wp = ext.mlp_pack_weight(w, 256, k)
        for bias in (b, None):
            xo, ln = ext.linear_add_layernorm(x, wp, bias, res, norm.weight, norm.bias, norm.eps)
            y = ext.linear(x, wp, 256, bias)
            want_x, want_ln = ext.add_layernorm(res, y, norm.weight, norm.bias, norm.eps)
            assert torch.equal(xo, want_x) and torch.equal(ln, want_ln)
        xo, ln = ext.linear_add_layernorm(x, wp, b, res, norm.weight, norm.bias, norm.eps)
        for tile, rows in ((1, 32), (2, 32), (3, 16), (4, 64)):
            if rows * k * 2 > 160 * 1024:  # the X panel does not fit the LDS
                continue
            got = ext.linear_add_layernorm(x, wp, b, res, norm.weight, norm.bias, norm.eps,
                                           tile=tile)
            assert torch.equal(got[0], xo) and torch.equal(got[1], ln), tile
        assert rel_err(ln, norm(res + torch.nn.functional.linear(x, w, b))) <= 1e-2
        got = linear_add_norm(x, w, b, res, norm)
        assert torch.equal(got[0], xo) and torch.equal(got[1], ln)
        row = res[-1].contiguous()  # one residual row for all
        into = torch.full((m, 256), float("nan"), dtype=torch.bfloat16, device=DEV)
        ln_into = torch.full((m, 256), float("nan"), dtype=torch.bfloat16, device=DEV)
        bx, bln = ext.linear_add_layernorm(x, wp, b, row, norm.weight, norm.bias, norm.eps,
                                           out=into, ln_out=ln_into)
        assert bx.data_ptr() == into.data_ptr() and bln.data_ptr() == ln_into.data_ptr()
        want_x = ext.linear(x, wp, 256, b, residual=row)
        want_ln = ext.add_layernorm(want_x, None, norm.weight, norm.bias, norm.eps)[1]
        assert torch.equal(into, want_x) and torch.equal(ln_into, want_ln)
        if m == 1:
            with pytest.raises(RuntimeError):  # only 256-wide rows
                ext.linear_add_layernorm(x, ext.mlp_pack_weight(w[:128].contiguous(), 128, k),
                                         None, res, norm.weight, norm.bias, norm.eps)


@pytest.mark.parametrize("m", [0, 1, 37, 4096 + 5, 12288])
def test_ffn_equals_its_two_launches(ext, m):
    """ffn (linear1 + GELU + linear2 + residual add + next LayerNorm in one launch) ==
    linear(gelu=True) then linear_add_layernorm, bit for bit (x_out and ln), on every row
    tile; without the norm == linear(gelu=True) then linear with the residual; in place
    (x_out over x); and within bf16 tolerance of the torch layer; through the module-level
    feed_forward of a torch encoder layer."""
    from cugo_amd.seq_decode import feed_forward

    announce(f"ffn m={m}")
    g = torch.Generator(device="cpu").manual_seed(m + 3)
    h = torch.randn(m, 256, generator=g).to(torch.bfloat16).to(DEV)
    x = (torch.randn(m, 256, generator=g) * 2.0).to(torch.bfloat16).to(DEV)
    w1 = (torch.randn(1024, 256, generator=g) * 256 ** -0.5).to(torch.bfloat16).to(DEV)
    b1 = (torch.randn(1024, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    w2 = (torch.randn(256, 1024, generator=g) * 1024 ** -0.5).to(torch.bfloat16).to(DEV)
    b2 = (torch.randn(256, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    norm = torch.nn.LayerNorm(256).to(DEV).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_((torch.randn(256, generator=g) * 0.3 + 1.0).to(torch.bfloat16))
        norm.bias.copy_((torch.randn(256, generator=g) * 0.1).to(torch.bfloat16))
        w1p, w2p = ext.mlp_pack_weight(w1, 1024, 256), ext.mlp_pack_weight(w2, 256, 1024)
        u = ext.linear(h, w1p, 1024, b1, True)
        want_x, want_ln = ext.linear_add_layernorm(u, w2p, b2, x, norm.weight, norm.bias, norm.eps)
        want_plain = ext.linear(u, w2p, 256, b2, False, residual=x)
        for rows in (0, 16, 32, 48, 64):
            xo, ln = ext.ffn(h, x, w1p, b1, w2p, b2, norm.weight, norm.bias, norm.eps, rows)
            assert torch.equal(xo, want_x) and torch.equal(ln, want_ln), rows
            plain, empty = ext.ffn(h, x, w1p, b1, w2p, b2, rows=rows)
            assert torch.equal(plain, want_plain) and empty.numel() == 0, rows
        inplace = x.clone()
        got = ext.ffn(h, inplace, w1p, b1, w2p, b2, norm.weight, norm.bias, norm.eps,
                      out=inplace)
        assert got[0].data_ptr() == inplace.data_ptr() and torch.equal(inplace, want_x)
        # the torch layer, float32 from the same bf16 values
        ref_u = torch.nn.functional.gelu(h.float() @ w1.float().T + b1.float())
        ref_x = x.float() + ref_u @ w2.float().T + b2.float()
        assert rel_err(want_x, ref_x) <= 1e-2
        # the module-level form on a torch encoder layer's parameters
        layer = torch.nn.TransformerEncoderLayer(256, 8, 1024, dropout=0.0, activation="gelu",
                                                 batch_first=True, norm_first=True)
        layer = layer.to(DEV).to(torch.bfloat16)
        layer.linear1.weight.copy_(w1)
        layer.linear1.bias.copy_(b1)
        layer.linear2.weight.copy_(w2)
        layer.linear2.bias.copy_(b2)
        fx, fln = feed_forward(layer, h, x, norm)
        assert torch.equal(fx, want_x) and torch.equal(fln, want_ln)
        assert torch.equal(feed_forward(layer, h, x), want_plain)


@pytest.mark.parametrize("m", [0, 1, 37, 4096 + 5, 12288, 16384])
def test_out_proj_ffn_equals_its_launches(ext, m):
    """out_proj_ffn (out_proj + residual add + norm2, then the feed-forward, one launch) ==
    linear_add_layernorm (out_proj, norm2) then ffn, bit for bit (x_out and ln), on every
    row tile, with and without the next norm, in place (x_out over x), on an attention
    output with a row stride (a view of a wider buffer); and through attention_tail of a
    torch encoder layer, against linear_add_norm + feed_forward; within bf16 tolerance of
    the torch layer in float32."""
    from cugo_amd.seq_decode import attention_tail, feed_forward, linear_add_norm

    announce(f"out_proj_ffn m={m}")
    g = torch.Generator(device="cpu").manual_seed(m + 11)
    wide = torch.randn(m, 264, generator=g).to(torch.bfloat16).to(DEV)
    att = wide[:, :256]  # row stride 264
    x = (torch.randn(m, 256, generator=g) * 2.0).to(torch.bfloat16).to(DEV)
    layer = torch.nn.TransformerEncoderLayer(256, 8, 1024, dropout=0.0, activation="gelu",
                                             batch_first=True, norm_first=True)
    layer = layer.to(DEV).to(torch.bfloat16)
    nxt = torch.nn.LayerNorm(256).to(DEV).to(torch.bfloat16)
    with torch.no_grad():
        for norm in (layer.norm2, nxt):
            norm.weight.copy_((torch.randn(256, generator=g) * 0.3 + 1.0).to(torch.bfloat16))
            norm.bias.copy_((torch.randn(256, generator=g) * 0.1).to(torch.bfloat16))
        for lin in (layer.self_attn.out_proj, layer.linear1, layer.linear2):
            lin.bias.copy_((torch.randn(lin.bias.shape, generator=g) * 0.1).to(torch.bfloat16))
        op, n2, l1, l2 = layer.self_attn.out_proj, layer.norm2, layer.linear1, layer.linear2
        wop = ext.mlp_pack_weight(op.weight.contiguous(), 256, 256)
        w1p = ext.mlp_pack_weight(l1.weight.contiguous(), 1024, 256)
        w2p = ext.mlp_pack_weight(l2.weight.contiguous(), 256, 1024)
        x1, h = ext.linear_add_layernorm(att, wop, op.bias, x, n2.weight, n2.bias, n2.eps)
        want_x, want_ln = ext.ffn(h, x1, w1p, l1.bias, w2p, l2.bias, nxt.weight, nxt.bias,
                                  nxt.eps)
        want_plain, _ = ext.ffn(h, x1, w1p, l1.bias, w2p, l2.bias)
        args = (wop, op.bias, n2.weight, n2.bias, n2.eps, w1p, l1.bias, w2p, l2.bias)
        for rows in (0, 16, 32, 48, 64):
            xo, ln = ext.out_proj_ffn(att, x, *args, nxt.weight, nxt.bias, nxt.eps, rows)
            assert torch.equal(xo, want_x) and torch.equal(ln, want_ln), rows
            plain, empty = ext.out_proj_ffn(att, x, *args, rows=rows)
            assert torch.equal(plain, want_plain) and empty.numel() == 0, rows
        inplace = x.clone()
        got = ext.out_proj_ffn(att, inplace, *args, nxt.weight, nxt.bias, nxt.eps, out=inplace)
        assert got[0].data_ptr() == inplace.data_ptr() and torch.equal(inplace, want_x)
        tx, tln = attention_tail(layer, att, x, nxt)
        assert torch.equal(tx, want_x) and torch.equal(tln, want_ln)
        assert torch.equal(attention_tail(layer, att, x), want_plain)
        # the two-launch path gives the same bits
        sx, sh = linear_add_norm(att, op.weight, op.bias, x, n2)
        assert torch.equal(feed_forward(layer, sh, sx, nxt)[0], want_x)
        # the torch layer in float32 from the same bf16 values
        f = {k: v.float() for k, v in layer.state_dict().items()}
        r1 = x.float() + att.float() @ f["self_attn.out_proj.weight"].T + f["self_attn.out_proj.bias"]
        rh = torch.nn.functional.layer_norm(r1, (256,), f["norm2.weight"], f["norm2.bias"], n2.eps)
        ru = torch.nn.functional.gelu(rh @ f["linear1.weight"].T + f["linear1.bias"])
        ref_x = r1 + ru @ f["linear2.weight"].T + f["linear2.bias"]
        assert rel_err(want_x, ref_x) <= 1e-2


def test_gumbel_sample_matches_reference(ext):
    announce("gumbel_sample")
    g = torch.Generator(device=DEV).manual_seed(3)
    n, a = 3000, 179
    logits = torch.randn(n, a, generator=g, device=DEV) * 3.0
    legal = torch.rand(n, a, generator=g, device=DEV) < 0.1
    legal[:5] = False              # no legal action: every entry masked
    legal[5:10] = True
    u = torch.rand(n, a, generator=g, device=DEV)
    u[10, :] = 0.0                 # clamps to 1e-20
    u[11, 17] = 1.0                # -log(-log(1)) = +inf picks action 17
    u[2, 30] = 1.0                 # also where no action is legal: -1e30 + inf = inf
    logits[12, :] = 0.5            # ties among equal scores pick the first index
    u[12, :] = 0.5
    actions, logp = ext.gumbel_sample(logits, legal, u)
    want_a, want_lp = gumbel_reference(logits, legal, u)
    assert torch.equal(actions, want_a)
    assert int(actions[11]) == 17 and int(actions[2]) == 30 and int(actions[3]) == 0
    assert float((logp - want_lp).abs().max()) <= 1e-5
    # bf16 logits read as the reference's .float()
    lb = logits.to(torch.bfloat16)
    actions, logp = ext.gumbel_sample(lb, legal, u)
    want_a, want_lp = gumbel_reference(lb.float(), legal, u)
    assert torch.equal(actions, want_a)
    assert float((logp - want_lp).abs().max()) <= 1e-5
    # other action counts: one lane group short of full (33), the 16-lane form's limit
    # (192) and beyond it (250, one row per wavefront), at a partial last block
    for width in (33, 192, 250):
        lg = torch.randn(1001, width, generator=g, device=DEV)
        ok = torch.rand(1001, width, generator=g, device=DEV) < 0.2
        ok[:3] = False
        un = torch.rand(1001, width, generator=g, device=DEV)
        un[1, width - 1] = 1.0
        got_a, got_lp = ext.gumbel_sample(lg, ok, un)
        want_a, want_lp = gumbel_reference(lg, ok, un)
        assert torch.equal(got_a, want_a), width
        assert float((got_lp - want_lp).abs().max()) <= 1e-5, width
        assert int(got_a[1]) == width - 1
        greedy = ext.masked_argmax(lg, ok)
        assert torch.equal(greedy, lg.masked_fill(~ok, -1.0e30).argmax(1)), width


def _policy(d=256, layers=4, heads=8, seed=0, mode="hybrid"):
    from cugo_amd.seq_selfplay import SeqPolicy

    torch.manual_seed(seed)
    p = SeqPolicy(mode=mode, d_model=d, layers=layers, heads=heads)
    with torch.no_grad():
        for prm in p.parameters():
            prm.normal_(0.0, 0.02)
    return p.to(DEV).to(torch.bfloat16).eval()


@pytest.mark.parametrize("w", [4096, 333])
def test_pair_step_pruned_equals_full(ext, w):
    """cached_step_pair with the event rows' last layer pruned (their key and value
    appended by kv_append, no attention, out_proj or feed-forward for them) against the
    full pass: the queries' hidden states and their final norm bit for bit, and every
    cache slot of every layer; events skipped on some rows, the queries on one of their
    game's two seat rows (self-play's layout), some queries skipped."""
    from cugo_amd.seq_decode import cached_step_pair
    from cugo_amd.seq_selfplay import policy_cache

    announce(f"pair step pruned vs full (w={w})")
    policy = _policy(seed=3)
    g = torch.Generator(device=DEV).manual_seed(w)
    ca = policy_cache(policy, 2 * w, DEV)
    for t in (ca.k, ca.v):
        t.copy_((torch.randn(t.shape, generator=g, device=DEV) * 0.5).to(t.dtype))
    cb_k, cb_v = ca.k.clone(), ca.v.clone()
    length = torch.randint(0, 40, (2 * w,), generator=g, device=DEV)
    pos_a = torch.where(torch.rand(2 * w, generator=g, device=DEV) < 0.2, -1, length)
    seat = torch.randint(0, 2, (w,), generator=g, device=DEV)
    rows_b = torch.arange(w, device=DEV) + w * seat
    pos_b = torch.where(torch.rand(w, generator=g, device=DEV) < 0.1, -1,
                        length[rows_b] + (pos_a[rows_b] >= 0).long())
    x = (torch.randn(3 * w, 256, generator=g, device=DEV) * 0.5).to(torch.bfloat16)
    with torch.no_grad():
        h1, n1 = cached_step_pair(policy, ca, x, 2 * w, pos_a, pos_b, rows_b,
                                  final_norm=policy.norm)
        ca.k, cb_k = cb_k, ca.k  # the full pass on the untouched copy
        ca.v, cb_v = cb_v, ca.v
        h2, n2 = cached_step_pair(policy, ca, x, 2 * w, pos_a, pos_b, rows_b,
                                  final_norm=policy.norm, prune=False)
    assert h1.shape == (w, 256)
    live = pos_b >= 0
    assert torch.equal(h1[live].view(torch.int16), h2[live].view(torch.int16))
    assert torch.equal(n1[live].view(torch.int16), n2[live].view(torch.int16))
    assert torch.equal(cb_k.view(torch.int16), ca.k.view(torch.int16))
    assert torch.equal(cb_v.view(torch.int16), ca.v.view(torch.int16))


def _reference_step(policy, ref, actions_from=None):
    """One WaveCollector step (cugo_seq_selfplay50.py:108-163, no pool) in the reference
    formulation: dense tokens from the oracle, index_put_ + matmul attention, the torch
    sampling and bookkeeping lines.  `ref` holds the reference copy's tensors; with
    actions_from the engine is stepped with those actions (teacher forcing) after
    sampling its own.  Returns (sampled actions, their logp, logits, active games)."""
    ext, w, ids = ref["ext"], ref["w"], ref["ids"]
    p, opp = ref["p"], ref["opp"]
    features, legal, players, done, status = ext.observe_indexed(ref["states"], ids)
    active = ~done
    ref["bad"] += (active & ((status != 0) | ~legal.any(1))).sum()
    player = players.long()
    kept = features if policy.mode == "hybrid" else features.index_select(1, policy.context_index)
    dt = policy.event_in.weight.dtype
    # cugo_seq50.py:166-180 in torch ops
    q = policy.query_in(torch.cat((kept.to(dt), legal.to(dt)), -1)) + policy.token_type[2]
    hidden = reference_cached_step(policy, ref["cache"], q, (player & 1) * w + ids)
    logits = policy.head(policy.norm(hidden)).float()  # cugo_seq50.py:187-189, torch ops
    learner_move = torch.ones_like(active)
    if p:
        pids = torch.arange(p, device=DEV)
        opp_q = opp.query_in(torch.cat((kept[:p].to(dt), legal[:p].to(dt)), -1)) + opp.token_type[2]
        opp_h = reference_cached_step(opp, ref["opp_cache"], opp_q, pids)
        opp_logits = opp.head(opp.norm(opp_h)).float()
        opp_move = player[:p] != ref["learner_seat"][:p]
        logits = torch.cat((torch.where(opp_move.unsqueeze(1), opp_logits, logits[:p]), logits[p:]))
        learner_move = torch.cat((~opp_move, learner_move[p:]))
    actions, logp = gumbel_reference(logits, legal, ref["noise"])
    used = actions if actions_from is None else actions_from
    hands = ext.hands_indexed(ref["states"], ids)
    stock = ext.stock_indexed(ref["states"], ids)
    stop = torch.round(torch.exp2(12.0 * features[:, 471].float()) - 1.0).long()
    rec = ref["rec"]
    rec["features"].append(kept.to(torch.bfloat16))
    rec["legal"].append(legal)
    rec["seat"].append(player)
    rec["count"].append(ref["count"].clone())
    rec["opp_hand"].append(hands.gather(1, (1 - player).unsqueeze(1)).squeeze(1))
    rec["stock"].append(stock)
    rec["stop_points"].append(stop)
    rec["valid"].append(active & learner_move)
    reward0, new_done, nagari, step_status, committed, events = ext.step_events_indexed(
        ref["states"], ids, used)
    ref["bad"] += (active & (step_status != 0)).sum()
    finished_now = active & new_done
    ref["final_reward0"].copy_(torch.where(finished_now, reward0, ref["final_reward0"]))
    ref["final_nagari"] |= finished_now & nagari
    ref["finished"] |= finished_now
    commit = active & committed
    slot = ref["count"].clamp_max(47)
    ref["events"].index_put_((ids, slot),
                             torch.where(commit.unsqueeze(1), events, ref["events"][ids, slot]))
    seats2 = torch.cat((torch.zeros(w, dtype=torch.int64, device=DEV),
                        torch.ones(w, dtype=torch.int64, device=DEV)))
    tok = encode_events_np(events.repeat(2, 1).cpu().numpy(), seats2.cpu().numpy())
    index = ref["count"].repeat(2)
    pos_idx = 1 + index.clamp(max=47)
    x = token_reference(tok, policy.event_in.weight, policy.event_in.bias, policy.position[pos_idx],
                        policy.token_type[1].expand(2 * w, -1))
    reference_cached_step(policy, ref["cache"], x, torch.arange(2 * w, device=DEV))
    if p:
        opp_seat = 1 - ref["learner_seat"][:p]
        tok = encode_events_np(events[:p].cpu().numpy(), opp_seat.cpu().numpy())
        pp = 1 + ref["count"][:p].clamp(max=47)
        xo = token_reference(tok, opp.event_in.weight, opp.event_in.bias, opp.position[pp],
                             opp.token_type[1].expand(p, -1))
        reference_cached_step(opp, ref["opp_cache"], xo, torch.arange(p, device=DEV))
        ref["opp_cache"].length += commit[:p].long()
    ref["cache"].length += commit.repeat(2).long()
    ref["count"] += commit.long()
    return actions, logp, logits, active


@pytest.mark.parametrize("mode,pool", [("hybrid", False), ("events", True)])
def test_selfplay_step_matches_reference_formulation(ext, mode, pool):
    """The captured self-play step against the reference formulation for a wave of 256
    games: identical engine trajectories (the reference copy replays the wave's actions),
    logits within 1e-2 relative, the same sampled action for at least 99 % of the
    decisions, identical records (features, mask, seat, count, opponent hand, stock, stop
    points, valid), event logs, counts, cache lengths, finished flags, final rewards and
    bad counts, and caches whose first layer agrees within 1e-2 (deeper layers 2e-2)."""
    announce(f"selfplay step vs reference formulation ({mode}, pool={pool})")
    from cugo_amd.seq_selfplay import SelfPlayWave, make_seeds, policy_cache

    policy = _policy(mode=mode)
    w = 256
    p = 96 if pool else 0
    opp = _policy(seed=7, mode=mode) if pool else None
    wave = SelfPlayWave(ext, policy, w, max_steps=64, opponent=opp, pool_games=p)
    wave.noise = torch.zeros((w, 179), device=DEV)
    g = torch.Generator(device=DEV).manual_seed(11)
    names = ("features", "legal", "seat", "count", "opp_hand", "stock", "stop_points", "valid")
    with torch.no_grad():
        wave.capture(pool)
        seeds, first = make_seeds(w, 12345, DEV)
        learner = torch.randint(2, (w,), generator=torch.Generator(device=DEV).manual_seed(3),
                                device=DEV)
        wave.reset(seeds, first, learner, pool)
        states = ext.create(seeds, first)
        ref = {"ext": ext, "w": w, "ids": torch.arange(w, device=DEV), "states": states,
               "p": p, "opp": opp, "learner_seat": learner,
               "opp_cache": policy_cache(opp, max(1, p), DEV) if pool else None,
               "cache": policy_cache(policy, 2 * w, DEV),
               "count": torch.zeros(w, dtype=torch.int64, device=DEV), "noise": wave.noise,
               "bad": torch.zeros((), dtype=torch.int64, device=DEV),
               "events": torch.zeros((w, 48, 9), dtype=torch.int64, device=DEV),
               "final_reward0": torch.zeros(w, device=DEV),
               "final_nagari": torch.zeros(w, dtype=torch.bool, device=DEV),
               "finished": ext.observe_indexed(states, torch.arange(w, device=DEV))[3].clone(),
               "rec": {k: [] for k in names}}
        start = ext.start(ref["states"])
        seats2 = torch.cat((torch.zeros(w, dtype=torch.int64, device=DEV),
                            torch.ones(w, dtype=torch.int64, device=DEV)))
        tok = encode_start_np(start.repeat(2, 1).cpu().numpy(), seats2.cpu().numpy())
        x0 = token_reference(tok, policy.start_in.weight, policy.start_in.bias,
                             policy.position[0].expand(2 * w, -1),
                             policy.token_type[0].expand(2 * w, -1))
        reference_cached_step(policy, ref["cache"], x0, torch.arange(2 * w, device=DEV))
        ref["cache"].length.fill_(1)
        if pool:
            tok = encode_start_np(start[:p].cpu().numpy(), (1 - learner[:p]).cpu().numpy())
            xo = token_reference(tok, opp.start_in.weight, opp.start_in.bias,
                                 opp.position[0].expand(p, -1), opp.token_type[0].expand(p, -1))
            reference_cached_step(opp, ref["opp_cache"], xo, torch.arange(p, device=DEV))
            ref["opp_cache"].length.fill_(1)
        agree = total = 0
        steps = 0
        for step in range(40):
            wave.noise.copy_(torch.rand((w, 179), generator=g, device=DEV))
            wave.graph.replay()
            steps += 1
            actions = wave.rec_long["actions"][step]
            a_ref, lp_ref, logits_ref, live = _reference_step(policy, ref, actions_from=actions)
            # finished games' rows are skipped by the HIP step (NaN logits nothing reads)
            assert rel_err(wave.logits[live], logits_ref[live]) <= 1e-2, step
            own = torch.arange(w, device=DEV) >= p  # rows the frozen opponent never reads
            assert bool(torch.isnan(wave.logits[~live & own]).all()), step
            same = actions == a_ref
            agree += int(same.sum())
            total += w
            lp = wave.rec_logp[step]
            assert float((lp - lp_ref)[same].abs().max()) <= 5e-2, step
            assert torch.equal(wave.states, ref["states"]), step
            assert torch.equal(wave.count, ref["count"]), step
            assert torch.equal(wave.cache.length, ref["cache"].length), step
            if pool:
                assert torch.equal(wave.opp_cache.length, ref["opp_cache"].length), step
            assert torch.equal(wave.events, ref["events"]), step
            assert torch.equal(wave.finished, ref["finished"]), step
            assert torch.equal(wave.final_nagari, ref["final_nagari"]), step
            assert torch.equal(wave.final_reward0, ref["final_reward0"]), step
            assert int(wave.bad) == int(ref["bad"]), step
            assert int(wave.step_index[1]) == steps  # the next step's index
            if bool(wave.finished.all()):
                break
        assert agree >= 0.99 * total, (agree, total)
        recs = {"features": wave.rec_features, "legal": wave.rec_legal,
                "seat": wave.rec_long["seat"], "count": wave.rec_long["count"],
                "opp_hand": wave.rec_long["opp_hand"], "stock": wave.rec_long["stock"],
                "stop_points": wave.rec_long["stop_points"], "valid": wave.rec_valid}
        for name in names:
            want = torch.stack(ref["rec"][name])
            assert torch.equal(recs[name][:steps], want), name
        # The last step's event tokens wait for the next step's queries: flush them.
        # Live slots only (below each row's length): slots past it still hold keys of
        # the games played while capturing, which no query reads.  Layer 0's keys come
        # from the tokens alone; deeper layers also carry the reference's bf16 rounding
        # of attention scores and probabilities (the HIP decode keeps them in fp32).
        wave.flush()
        live = (torch.arange(wave.cache.slots, device=DEV).view(1, -1)
                < wave.cache.length.view(-1, 1)).view(1, -1, 1, wave.cache.slots, 1)
        errs = [rel_err((wave.cache.k[i] * live[0]).float(), (ref["cache"].k[i] * live[0]).float())
                for i in range(wave.cache.k.shape[0])]
        assert errs[0] <= 1e-2, errs
        assert max(errs) <= 2e-2, errs


def test_prepare_reads_the_stock_words_itself(ext):
    """SelfPlayState.prepare with stock None (the self-play step's form) records the words
    stock_indexed gives for the same rows, and writes the same query input, rows and slots
    as with stock_indexed's tensor passed in."""
    announce("selfplay prepare: stock words from the state rows")
    from cugo_amd.seq_selfplay import SelfPlayWave, make_seeds

    policy = _policy()
    w = 300
    wave = SelfPlayWave(ext, policy, w, max_steps=8)
    seeds, first = make_seeds(w, 77, DEV)
    with torch.no_grad():
        wave.reset(seeds, first, torch.zeros(w, dtype=torch.int64, device=DEV))
        # a few steps in, so the stock and its draws differ from the deal's
        for _ in range(3):
            wave.step()
        step = int(wave.step_index[1])
        native = wave.native[False]
        obs = ext.observe_indexed(wave.states, wave.ids)
        stock = ext.stock_indexed(wave.states, wave.ids)
        dt = policy.event_in.weight.dtype
        given = native.prepare(wave.states, *obs, stock, dt, wave.q_stride)
        rec_given = wave.rec_long["stock"][step].clone()
        wave.rec_long["stock"][step].zero_()
        read = native.prepare(wave.states, *obs, None, dt, wave.q_stride)
        rec_read = wave.rec_long["stock"][step].clone()
    assert torch.equal(rec_given, stock) and torch.equal(rec_read, stock)
    for x, y in zip(given, read):
        assert torch.equal(x, y)


@pytest.mark.parametrize("pool", [False, True])
def test_selfplay_graph_replays_equal_eager_steps(ext, pool):
    """Replays of the captured step == eager step() calls from the same start (same
    uniforms), repeated with eager work and synchronisations in between."""
    announce(f"selfplay graph replay vs eager (pool={pool})")
    from cugo_amd.seq_selfplay import SelfPlayWave, make_seeds

    policy = _policy(seed=1)
    w = 128
    opp = _policy(seed=9) if pool else None
    wave = SelfPlayWave(ext, policy, w, max_steps=64, opponent=opp, pool_games=40 if pool else 0)
    wave.noise = torch.zeros((w, 179), device=DEV)
    g = torch.Generator(device=DEV).manual_seed(5)
    noises = [torch.rand((w, 179), generator=g, device=DEV) for _ in range(12)]
    seeds, first = make_seeds(w, 777, DEV)
    learner = (torch.arange(w, device=DEV) % 3 == 0).long()
    runs = []
    with torch.no_grad():
        wave.capture(pool)
        for mode in ("eager", "graph", "graph"):
            wave.reset(seeds, first, learner, pool)
            for k in range(12):
                wave.noise.copy_(noises[k])
                if mode == "eager":
                    wave.step(pool)
                else:
                    wave.graph.replay()
                torch.cuda.synchronize()
            runs.append([t.clone() for t in (wave.states, wave.events, wave.count,
                                              wave.rec_long["actions"], wave.rec_logp,
                                              wave.cache.length, wave.cache.k, wave.rec_valid)]
                        + ([wave.opp_cache.k.clone(), wave.opp_cache.length.clone()] if pool
                           else []))
    for a, b in zip(runs[0], runs[1]):
        assert torch.equal(a, b)
    for a, b in zip(runs[1], runs[2]):
        assert torch.equal(a, b)


def test_selfplay_wave_plays_to_the_end(ext):
    """A wave with the default noise (Philox uniforms drawn in the sampling kernel) plays
    to the end with only legal actions; the noise epoch advances once a step."""
    announce("selfplay wave to the end")
    from cugo_amd.seq_selfplay import SelfPlayWave, make_seeds

    policy = _policy(seed=2)
    w = 512
    wave = SelfPlayWave(ext, policy, w, max_steps=64)
    seeds, first = make_seeds(w, 4242, DEV)
    with torch.no_grad():
        wave.capture()
        epoch0 = int(wave.noise_epoch)
        steps = wave.play(seeds, first, torch.zeros(w, dtype=torch.int64, device=DEV))
    # the Philox noise's epoch advanced once per replayed step (fresh uniforms each step)
    assert int(wave.noise_epoch) - epoch0 == steps
    assert 16 <= steps <= 64
    assert bool(wave.finished.all())
    assert int(wave.bad) == 0
    assert int(wave.count.max()) <= 48
    # every recorded action was legal where the row was still playing
    valid = wave.rec_valid[:steps]
    acts = wave.rec_long["actions"][:steps]
    legal = wave.rec_legal[:steps]
    picked = legal.gather(2, acts.unsqueeze(2)).squeeze(2)
    assert bool(picked[valid].all())


def test_selfplay_collect_with_pool(ext):
    """collect() over two waves with a frozen opponent loaded in place: outcomes for every
    game, the learner's decisions only (none on the opponent's moves in pool games), the
    event logs, and the opponent's new weights reach the captured step."""
    announce("selfplay collect")
    from cugo_amd.seq_selfplay import SelfPlayWave

    policy = _policy(seed=3)
    opp = _policy(seed=4)
    w, p = 256, 64
    wave = SelfPlayWave(ext, policy, w, max_steps=64, opponent=opp, pool_games=p)
    other = _policy(seed=5).state_dict()
    torch.manual_seed(0)
    out = wave.collect(2 * w, seed_offset=1000, opponent_state=other)
    assert out["vs_pool"].sum().item() == 2 * p
    assert out["final_reward0"].shape == (2 * w,) and out["steps"] >= 16
    dec = out["decisions"]
    n = dec["actions"].numel()
    assert all(v.shape[0] == n for v in dec.values())
    assert dec["features"].shape[1] == 720
    # no recorded decision of a pool game is the opponent's
    pool_rows = dec["env_ids"] % w < p
    seat_of = out["learner_seat"][dec["env_ids"]]
    assert bool((dec["seat"][pool_rows] == seat_of[pool_rows]).all())
    assert int(out["log"]["count"].max()) <= 48
    w_t = wave.opponent._weight_t("event_in")
    assert torch.equal(w_t, other["event_in.weight"].t().to(w_t.dtype))


def test_empty_batches_of_the_step_ops(ext):
    """Every operation of the sequence policy's step and of the paired evaluation takes a
    batch of no rows: no error, empty outputs of the right shape, nothing written."""
    announce("empty batches")
    bf, i64, u8 = torch.bfloat16, torch.int64, torch.bool
    z = lambda *shape, dtype=bf: torch.zeros(shape, dtype=dtype, device=DEV)  # noqa: E731
    w = (torch.randn(256, 256) * 0.05).to(bf).to(DEV)
    wp = ext.mlp_pack_weight(w, 256, 256)
    w179 = ext.mlp_pack_weight(w[:179].contiguous(), 192, 256)
    b, ones = z(256), torch.ones(256, dtype=bf, device=DEV)
    x = z(0, 256)
    assert ext.linear(x, wp, 256, b, True).shape == (0, 256)
    assert ext.linear(x, wp, 256, b, residual=z(0, 256)).shape == (0, 256)
    assert ext.linear(x, w179, 179, b[:179]).shape == (0, 179)
    xo, ln = ext.linear_add_layernorm(x, wp, b, z(0, 256), ones, b, 1e-5)
    assert xo.shape == (0, 256) and ln.shape == (0, 256)
    xo, ln = ext.linear_add_layernorm(x, wp, b, b, ones, b, 1e-5)  # one residual row for all
    assert xo.shape == (0, 256) and ln.shape == (0, 256)
    assert ext.add_layernorm(x, x, ones, b, 1e-5)[1].shape == (0, 256)
    pos = torch.zeros(0, dtype=i64, device=DEV)
    keys, values = z(4, 8, 16, 32), z(4, 8, 16, 32)
    q = z(0, 8, 32)
    assert ext.decode_attention_append(q, q, q, keys, values, pos).shape == (0, 8, 32)
    ext.kv_append(q, q, keys, values, pos)
    assert not bool(keys.any()) and not bool(values.any())
    logits, legal = z(0, 179), z(0, 179, dtype=u8)
    assert ext.masked_argmax(logits, legal).shape == (0,)
    acts, logp = ext.gumbel_sample(logits.float(), legal, z(0, 179, dtype=torch.float32))
    assert acts.shape == (0,) and logp.shape == (0,)
    epoch = torch.zeros(1, dtype=i64, device=DEV)
    acts, logp = ext.gumbel_sample_philox(logits, legal, 7, epoch, 0)
    assert acts.shape == (0,) and logp.shape == (0,)
    q_in = z(0, 1024)
    ext.query_input(z(0, 720, dtype=torch.float32), legal, None, q_in)
    wt = (torch.randn(274, 256) * 0.05).to(bf).to(DEV)
    assert ext.start_tokens(z(0, 8, dtype=i64), pos, wt, b, z(49, 256), z(3, 256)).shape == (0, 256)
    ext.paired_movers(z(0, dtype=torch.uint8), pos, pos)
    flags = z(0, dtype=u8)
    ext.paired_events(flags, z(0, dtype=torch.int16), flags, flags, pos, pos, pos, pos)
