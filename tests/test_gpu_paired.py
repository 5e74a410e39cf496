"""Paired evaluation (python/cugo_eval50.py:137-361) on the HIP engine.

Pinned end to end against the oracle engine: two policies whose greedy choice is known
in closed form (the first legal action, the last legal action: a zero-weight Linear with
a descending or ascending bias) play the duplicated deals on the CPU oracle, and every
summary field must equal what those games give.  Self-play of one policy on both seats
of a pair plays the same game twice, so every pair scores 0.  The greedy kernel is
checked against torch's masked argmax.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.conftest import announce

pytestmark = pytest.mark.gpu

DEV = "cuda"


def fixed_choice(last: bool) -> torch.nn.Module:
    """Logits that do not depend on the state: argmax over the legal mask picks the first
    (or the last) legal action."""
    lin = torch.nn.Linear(720, 179)
    with torch.no_grad():
        lin.weight.zero_()
        order = torch.arange(179, dtype=torch.float32)
        lin.bias.copy_(order if last else -order)
    return lin.to(DEV)


def test_masked_argmax_matches_torch(ext):
    announce("masked_argmax")
    g = torch.Generator(device=DEV).manual_seed(9)
    logits = torch.randn(5000, 179, generator=g, device=DEV)
    legal = torch.rand(5000, 179, generator=g, device=DEV) < 0.2
    legal[:3] = False
    logits[3:6] = 1.0  # ties: the first legal index
    want = logits.masked_fill(~legal, -1.0e30).argmax(1)
    assert torch.equal(ext.masked_argmax(logits, legal), want)
    lb = logits.to(torch.bfloat16)
    want_b = lb.float().masked_fill(~legal, -1.0e30).argmax(1)
    assert torch.equal(ext.masked_argmax(lb, legal), want_b)


def oracle_games(ref, seeds, first, a_seat, choose):
    """Plays every game to the end on the oracle with A = choose[0], B = choose[1]
    (functions legal row -> action); returns final reward0, nagari, excluded, steps."""
    n = seeds.size
    states = ref.create(seeds, first)
    reward = np.zeros(n, dtype=np.float32)
    nagari = np.zeros(n, dtype=bool)
    excluded = np.zeros(n, dtype=bool)
    ids = np.arange(n)
    steps = 0
    for step in range(200):
        if ids.size == 0:
            break
        _, legal, player, done, status = ref.observe(states, ids)
        assert (status == 0).all()
        if step == 0:
            excluded[ids[done]] = True
            keep = ~done
            ids, legal, player = ids[keep], legal[keep], player[keep]
            if ids.size == 0:
                break
        steps += 1
        acts = np.array([choose[0 if p == s else 1](row)
                         for row, p, s in zip(legal, player, a_seat[ids])])
        r, d, nag, st, _ = ref.step(states, acts, ids)
        assert (st == 0).all()
        ended = d
        reward[ids] = np.where(ended, r, 0.0)
        nagari[ids] = ended & nag
        ids = ids[~d]
    return reward, nagari, excluded, steps


def test_paired_eval_against_oracle_games(ext, ref):
    announce("paired eval vs oracle games")
    from cugo_amd.paired_eval import evaluate_paired
    from cugo_amd.seq_selfplay import make_seeds

    pairs = 200
    got = evaluate_paired(ext, fixed_choice(False), fixed_choice(True), pairs, seed_offset=900,
                          max_steps=128, use_amp=False)
    seeds, first = make_seeds(pairs, 900, "cpu")
    seeds = np.tile(seeds.numpy(), 2)
    first = np.tile(first.numpy(), 2)
    a_seat = (np.arange(2 * pairs) >= pairs).astype(np.int64)
    first_legal = lambda row: int(np.flatnonzero(row)[0])   # noqa: E731
    last_legal = lambda row: int(np.flatnonzero(row)[-1])   # noqa: E731
    reward, nagari, excluded, steps = oracle_games(ref, seeds, first, a_seat,
                                                   (first_legal, last_legal))
    score = np.where(a_seat == 0, reward, -reward)
    s0, s1 = score[:pairs], score[pairs:]
    v0, v1 = ~excluded[:pairs], ~excluded[pairs:]
    pair = (s0 + s1) * 0.5
    both = v0 & v1
    wdl = lambda x: (int((x > 0).sum()), int((x < 0).sum()), int((x == 0).sum()))  # noqa: E731
    assert got.decision_steps == steps
    assert (got.evaluated_pairs, got.evaluated_games, got.predecision_excluded) == (
        int(both.sum()), int((~excluded).sum()), int(excluded.sum()))
    assert (got.a_wins, got.b_wins, got.draws) == wdl(score[~excluded])
    assert (got.a_p0_wins, got.a_p0_losses, got.a_p0_draws) == wdl(s0[v0])
    assert (got.a_p1_wins, got.a_p1_losses, got.a_p1_draws) == wdl(s1[v1])
    assert (got.pair_wins, got.pair_losses, got.pair_draws) == wdl(pair[both])
    assert (got.terminal, got.nagari) == (int((~nagari).sum()), int(nagari.sum()))
    assert got.mean_pair_score_a == pytest.approx(float(pair[both].mean()), rel=1e-6, abs=1e-6)
    assert got.mean_score_a == pytest.approx(float(score[~excluded].mean()), rel=1e-6, abs=1e-6)
    assert got.pair_score_std == pytest.approx(float(pair[both].std(ddof=1)), rel=1e-5)


def test_paired_self_play_scores_zero(ext):
    announce("paired self-play")
    from cugo_amd.paired_eval import evaluate_paired

    torch.manual_seed(4)
    model = torch.nn.Sequential(torch.nn.Linear(720, 128), torch.nn.ReLU(),
                                torch.nn.Linear(128, 179)).to(DEV)
    got = evaluate_paired(ext, model, model, 500, seed_offset=17, max_steps=128, use_amp=False)
    assert got.mean_pair_score_a == 0.0 and got.pair_draws == got.evaluated_pairs
    assert (got.a_p0_wins, got.a_p0_losses) == (got.a_p1_losses, got.a_p1_wins)
    assert got.games == 1000 and got.seconds > 0
    # sampling from the softmax plays, too (its outcome depends on torch's RNG)
    s = evaluate_paired(ext, model, model, 100, seed_offset=3, max_steps=128, use_amp=True,
                        sample_a=True, sample_b=True)
    assert s.a_wins + s.b_wins + s.draws == s.evaluated_games


def test_paired_eval_graph_equals_eager(ext):
    """The captured step and the eager one play the same games: identical summaries (all
    fields but the time) for two different MLP policies under fp16 autocast; the Linear
    weights cast to fp16 once give autocast's own outputs bit for bit."""
    announce("paired eval: graph replay vs eager steps")
    from dataclasses import asdict

    from cugo_amd.paired_eval import evaluate_paired

    def mlp(seed):
        torch.manual_seed(seed)
        return torch.nn.Sequential(torch.nn.Linear(720, 256), torch.nn.ReLU(),
                                   torch.nn.Linear(256, 179)).to(DEV)

    a, b = mlp(5), mlp(6)
    # the fp16 copy of the Linear weights computes what autocast computes, bit for bit
    from cugo_amd.paired_eval import _half_linears

    x = torch.randn(1000, 720, device=DEV)
    with torch.no_grad(), torch.autocast(device_type="cuda", dtype=torch.float16):
        assert torch.equal(_half_linears(a)(x), a(x))
    runs = [asdict(evaluate_paired(ext, a, b, 300, seed_offset=41, max_steps=128, use_amp=True,
                                   graph=g)) for g in (True, False, True)]
    for r in runs:
        r.pop("seconds")
    assert runs[0] == runs[1] == runs[2]
    assert runs[0]["evaluated_games"] > 0 and runs[0]["decision_steps"] > 10


def _seq_policy(seed: int, mode: str):
    from cugo_amd.seq_selfplay import SeqPolicy

    torch.manual_seed(seed)
    p = SeqPolicy(mode=mode)
    with torch.no_grad():
        for prm in p.parameters():
            prm.normal_(0.0, 0.05)
    return p.to(DEV).to(torch.bfloat16).eval()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kept", ["all", "some"])
def test_query_input_equals_concat(ext, dtype, kept):
    """query_input's rows equal torch's concat of the kept feature columns and the legal
    mask, cast to the policy dtype, with the padding zeroed (the rows start as garbage)."""
    announce(f"query_input {kept} {dtype}")
    g = torch.Generator(device="cpu").manual_seed(5)
    n = 3001
    features = torch.randn((n, 720), generator=g).to(DEV)
    legal = (torch.rand((n, 179), generator=g) < 0.3).to(DEV)
    cols = None
    if kept == "some":
        cols = torch.randperm(720, generator=g)[:433].sort().values.to(torch.int32).to(DEV)
    width = 720 if cols is None else cols.numel()
    stride = 1024 if cols is None else 640
    q_in = torch.full((n, stride), 7.0, dtype=dtype, device=DEV)
    ext.query_input(features, legal, cols, q_in)
    kept_f = features if cols is None else features.index_select(1, cols.long())
    want = torch.zeros((n, stride), dtype=dtype, device=DEV)
    want[:, :width] = kept_f.to(dtype)
    want[:, width:width + 179] = legal.to(dtype)
    torch.cuda.synchronize()
    assert torch.equal(q_in.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                       want.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))


def _summary(pairs, reward, nagari, excluded, steps):
    """EvalSummary's fields (cugo_eval50.py:287-361) from finished games, in numpy."""
    n = 2 * pairs
    a_seat = (np.arange(n) >= pairs).astype(np.int64)
    score = np.where(a_seat == 0, reward, -reward).astype(np.float32)
    s0, s1 = score[:pairs], score[pairs:]
    v0, v1 = ~excluded[:pairs], ~excluded[pairs:]
    both = v0 & v1
    pair = ((s0 + s1) * np.float32(0.5))[both]
    wdl = lambda x: (int((x > 0).sum()), int((x < 0).sum()), int((x == 0).sum()))  # noqa: E731
    std = float(pair.std(ddof=1)) if both.sum() > 1 else 0.0
    return {"evaluated_pairs": int(both.sum()), "evaluated_games": int((~excluded).sum()),
            "predecision_excluded": int(excluded.sum()),
            "wdl": wdl(score[~excluded]), "p0": wdl(s0[v0]), "p1": wdl(s1[v1]),
            "pair": wdl(pair), "terminal": int((~nagari).sum()), "nagari": int(nagari.sum()),
            "decision_steps": steps, "mean_pair": float(pair.mean()) if pair.size else 0.0,
            "mean_score": float(score[~excluded].mean()), "pair_std": std}


def _assert_summary(got, want):
    assert got.decision_steps == want["decision_steps"]
    assert (got.evaluated_pairs, got.evaluated_games, got.predecision_excluded) == (
        want["evaluated_pairs"], want["evaluated_games"], want["predecision_excluded"])
    assert (got.a_wins, got.b_wins, got.draws) == want["wdl"]
    assert (got.a_p0_wins, got.a_p0_losses, got.a_p0_draws) == want["p0"]
    assert (got.a_p1_wins, got.a_p1_losses, got.a_p1_draws) == want["p1"]
    assert (got.pair_wins, got.pair_losses, got.pair_draws) == want["pair"]
    assert (got.terminal, got.nagari) == (want["terminal"], want["nagari"])
    assert got.mean_pair_score_a == pytest.approx(want["mean_pair"], rel=1e-6, abs=1e-6)
    assert got.mean_score_a == pytest.approx(want["mean_score"], rel=1e-6, abs=1e-6)
    assert got.pair_score_std == pytest.approx(want["pair_std"], rel=1e-5, abs=1e-6)


@pytest.mark.parametrize("mode_b", ["events", "mlp"])
def test_paired_sequence_policies_match_reference_formulation(ext, ref, mode_b):
    """Sequence policies in paired evaluation (cugo_eval50.py:137-361 with a History,
    :169, :258-263) against the reference formulation, teacher-forced: the oracle engine
    plays the evaluation's own actions (dropping finished games, as the reference does)
    while the reference formulation keeps, for each sequence policy, a KV cache per game
    of dense tokens (oracle/seq_ref.py: the opening and the events from the policy's seat,
    positions 1 + count) run through reference_cached_step (index_put_ + the matmul
    decode, pinned on the CPU against the full causal forward) and the readout in torch
    ops, and takes the masked argmax for the mover.  Every decision's action must be that
    argmax, or lie within the two formulations' logit discrepancy of it (a bf16 near-tie;
    at most 1 % of the decisions); the logits agree within 2e-2; and every summary field
    equals the one those games give.  Model A is a hybrid-mode SeqPolicy; model B an
    events-mode one, or a features-only MLP (one history kept)."""
    from oracle.seq_ref import (encode_events_np, encode_start_np, reference_cached_step,
                                token_reference)
    from cugo_amd.paired_eval import evaluate_paired
    from cugo_amd.seq_selfplay import make_seeds, policy_cache

    announce(f"paired eval: sequence policies vs reference formulation (B: {mode_b})")
    pairs = 192
    n = 2 * pairs
    model_a = _seq_policy(1, "hybrid")
    if mode_b == "mlp":
        torch.manual_seed(8)
        model_b = torch.nn.Sequential(torch.nn.Linear(720, 256), torch.nn.ReLU(),
                                      torch.nn.Linear(256, 179)).to(DEV)
    else:
        model_b = _seq_policy(2, mode_b)
    trace: list = []
    got = evaluate_paired(ext, model_a, model_b, pairs, seed_offset=77, max_steps=128,
                          use_amp=True, trace=trace)

    seeds, first = make_seeds(pairs, 77, "cpu")
    seeds, first = np.tile(seeds.numpy(), 2), np.tile(first.numpy(), 2)
    a_seat = (np.arange(n) >= pairs).astype(np.int64)
    states = ref.create(seeds, first)
    start = ref.start(states)
    models = [(model_a, a_seat), (model_b, 1 - a_seat)]
    seq = [hasattr(m, "query_in") for m, _ in models]
    caches = [policy_cache(m, n, DEV) if s else None for (m, _), s in zip(models, seq)]
    rows_all = torch.arange(n, device=DEV)
    with torch.no_grad():
        for (m, seat), cache in zip(models, caches):
            if cache is None:
                continue
            x0 = token_reference(encode_start_np(start, seat), m.start_in.weight,
                                 m.start_in.bias, m.position[0].expand(n, -1),
                                 m.token_type[0].expand(n, -1))
            reference_cached_step(m, cache, x0, rows_all)
            cache.length.fill_(1)
    count = np.zeros(n, dtype=np.int64)
    reward = np.zeros(n, dtype=np.float32)
    nagari = np.zeros(n, dtype=bool)
    excluded = np.zeros(n, dtype=bool)
    ids = np.arange(n)
    decisions = flips = steps = 0
    worst = 0.0
    with torch.no_grad():
        for k in range(128):
            if ids.size == 0:
                break
            f, legal, player, done, status = ref.observe(states, ids)
            assert (status == 0).all()
            if k == 0:
                excluded[ids[done]] = True
                keep = ~done
                ids, f, legal, player = ids[keep], f[keep], legal[keep], player[keep]
                if ids.size == 0:
                    break
            assert k < len(trace), "the evaluation stopped before the reference games ended"
            steps += 1
            hip = trace[k]["actions"].cpu().numpy()[ids]
            mover_is_a = player.astype(np.int64) == a_seat[ids]
            legal_t = torch.from_numpy(legal.astype(bool)).to(DEV)
            for j, ((m, seat), cache) in enumerate(zip(models, caches)):
                sel = np.nonzero(mover_is_a if j == 0 else ~mover_is_a)[0]
                if sel.size == 0:
                    continue
                ft = torch.from_numpy(f[sel]).to(DEV)
                lt = legal_t[sel]
                if cache is None:
                    with torch.autocast(device_type="cuda", dtype=torch.float16):
                        logits = m(ft).float()
                else:
                    kept = ft if m.mode == "hybrid" else ft.index_select(1, m.context_index)
                    dt = m.event_in.weight.dtype
                    q = m.query_in(torch.cat((kept.to(dt), lt.to(dt)), -1)) + m.token_type[2]
                    rows = torch.from_numpy(ids[sel]).to(DEV)
                    h = reference_cached_step(m, cache, q, rows)
                    logits = m.head(m.norm(h)).float()
                masked = logits.masked_fill(~lt, -1.0e30)
                want = masked.argmax(1).cpu().numpy()
                got_logits = trace[k][("logits_a", "logits_b")[j]].float()[
                    torch.from_numpy(ids[sel]).to(DEV)]
                diff = (got_logits - logits).abs().masked_fill(~lt, 0.0).amax(1)
                worst = max(worst, float((got_logits - logits)[lt].norm() / logits[lt].norm()))
                mine = hip[sel]
                decisions += sel.size
                for r in np.nonzero(mine != want)[0]:
                    gap = float(masked[r].max() - masked[r, int(mine[r])])
                    assert legal[sel[r], mine[r]], f"illegal action at step {k}"
                    assert gap <= 2 * float(diff[r]) + 1e-6, (k, int(ids[sel[r]]), gap)
                    flips += 1
            rew, d, nag, st, com, ev = ref.step(states, hip, ids, events=True)
            assert (st == 0).all()
            keep_ev = np.nonzero(com)[0]
            for (m, seat), cache in zip(models, caches):
                if cache is None or keep_ev.size == 0:
                    continue
                g = ids[keep_ev]
                tok = encode_events_np(ev[keep_ev], seat[g])
                pos_idx = torch.from_numpy(1 + np.minimum(count[g], 47)).to(DEV)
                x = token_reference(tok, m.event_in.weight, m.event_in.bias,
                                    m.position[pos_idx], m.token_type[1].expand(g.size, -1))
                rows = torch.from_numpy(g).to(DEV)
                reference_cached_step(m, cache, x, rows)
                cache.length.index_add_(0, rows, torch.ones_like(rows))
            count[ids[keep_ev]] += 1
            reward[ids] = np.where(d, rew, 0.0)
            nagari[ids] = d & nag
            ids = ids[~d]
    assert ids.size == 0
    assert worst <= 2e-2, worst
    assert flips <= 0.01 * decisions, (flips, decisions)
    _assert_summary(got, _summary(pairs, reward, nagari, excluded, steps))
    print(f"decisions {decisions}, near-tie flips {flips}, logits rel err {worst:.2e}",
          flush=True)


def test_paired_sequence_self_play_scores_zero(ext):
    """One sequence policy on both seats plays each pair's two games identically: every pair
    scores 0 (the two caches of a game hold the two seats' views, computed row by row)."""
    announce("paired eval: sequence policy self-play")
    from cugo_amd.paired_eval import evaluate_paired

    model = _seq_policy(5, "hybrid")
    got = evaluate_paired(ext, model, model, 300, seed_offset=5, max_steps=128, use_amp=True)
    assert got.mean_pair_score_a == 0.0 and got.pair_draws == got.evaluated_pairs
    assert (got.a_p0_wins, got.a_p0_losses) == (got.a_p1_losses, got.a_p1_wins)
    eager = evaluate_paired(ext, model, model, 300, seed_offset=5, max_steps=128, use_amp=True,
                            graph=False)
    from dataclasses import asdict

    a, b = asdict(got), asdict(eager)
    a.pop("seconds")
    b.pop("seconds")
    assert a == b
