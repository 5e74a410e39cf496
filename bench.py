"""Throughput of the gfx950 Shin Matgo engine on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch B] [--no-cpu] [--no-branch]

Workload (timed, one JSON line on stdout): random-policy self-play on B = 65,536
GPU-resident games.  One step = observe (720 features + 179-way mask for every game)
-> uniform legal sample (per-game xorshift64) -> step -> re-create finished games with
their next seed (pre-dealt in a full-width batch every 32 steps, included in the timing).
`value` = complete games per second over K steps.  Games are dealt from
seed = 0x243F6A8885A308D3 + i (+ B per later game of row i), first = i & 1.

Also reported (not timed into `value`):
  roofline      play_kernel (32 steps a launch, the loop's dominant kernel): algorithmic
                bytes per launch over its duration, HIP events on its stream;
                observe_roofline the same for the observe kernel (248 read + 3,063
                written a row); store_ceiling what a plain fill reaches
  branch        4,096 roots (3-15 seeded random decisions deep) x 256 children:
                branch_indexed (clone + step) and the observation of all children, their
                rooflines, and the same children on the host's cores (reference build)
  canonical     the reference's canonical whole-game driver, 131,072 games a launch:
                complete games/s
  decode        sequence-policy decode over a [4, 4,096, 8, 320, 32] bf16 KV cache:
                tokens/s of the 4-layer step and the HIP decode kernel's HBM fraction
  rollout       MLP PPO self-play rollout, B = 32,768 x 128 steps: env steps/s and the
                engine's share of the wall time
  cpu_baseline  the reference engine (oracle/_ref) on this host's cores, same protocol,
                bounded sample
"""

from __future__ import annotations

import argparse
import contextlib
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

SEED_BASE = 0x243F6A8885A308D3
HBM_PEAK_GBS = 8000.0
# Steps between batched pre-deals of the next games, and steps per play_random launch.  A
# launch's first and last steps run without the overlap of stores and stepping and the
# refill is one launch of create_env's latency, so longer blocks amortise both, while rows
# that finish more often than there are spare slots deal inline.  With two slots: 16 steps
# 97M games/s, 24: 100M, 32: 101M, 48: 99M (one slot: 8: 86M, 16: 95M, 32: 93M).
REFILL = 32
# Pre-dealt next games per row: games last about 20 steps, so a row finishes about 1.6
# times in a block of 32, and a finish with no spare left deals its game inline (the whole
# wavefront waits on create_env); two slots hold the next two games (four: 99M games/s).
SPARE_SLOTS = 2
OBSERVE_BYTES_PER_ROW = 248 + 720 * 4 + 179 + 1 + 1 + 2  # 3,311
# play_random per row: every step writes the observation (2,880 + 179 + 4), the action (8)
# and the step outputs (9); once per launch the state is read and written (2 x 248), the
# sampler word read and written (16) and the generation read and written (8).  A finished
# row's spare (248 B for ~5 % of rows a step) is left out.
PLAY_STEP_BYTES_PER_ROW = 720 * 4 + 179 + 4 + 8 + 9  # 3,080
PLAY_LAUNCH_BYTES_PER_ROW = 2 * 248 + 16 + 8  # 520


def play_bytes_per_row(steps: int) -> int:
    """Algorithmic bytes per row of one play_random launch of `steps` steps."""
    return steps * PLAY_STEP_BYTES_PER_ROW + PLAY_LAUNCH_BYTES_PER_ROW
STEP_BYTES_PER_ROW = 248 + 8 + 248 + 4 + 1 + 1 + 2 + 1  # 513
BRANCH_BYTES_PER_CHILD = 8 + 8 + 248 + 4 + 1 + 1 + 2 + 1  # parent reads hit L2: 273


def measured_traffic(kernel: str, key: str) -> int | None:
    """HBM bytes per launch of `kernel` for workload `key`, from the committed
    rocprofv3 PMC summary (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by what the
    counter reads for a plain copy of known size); None when not measured for this size."""
    path = REPO / "profiles" / "pmc_traffic.json"
    if not path.exists():
        return None
    entry = json.loads(path.read_text()).get(kernel, {}).get(key)
    return None if entry is None else int(entry["bytes"])


@contextlib.contextmanager
def region(name: str):
    """A ROCTx range named `name` around a timed region (torch.cuda.nvtx is ROCTx on
    ROCm), so that a `rocprofv3 --marker-trace --kernel-trace` run can attribute the
    kernels that ran inside it."""
    import torch

    torch.cuda.nvtx.range_push(name)
    try:
        yield
    finally:
        torch.cuda.nvtx.range_pop()


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1024)
    p.add_argument("--warmup", type=int, default=128)
    p.add_argument("--batch", type=int, default=65536)
    p.add_argument("--branch-iters", type=int, default=20)
    p.add_argument("--no-branch", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-decode", action="store_true")
    p.add_argument("--no-canonical", action="store_true")
    p.add_argument("--no-tunable", action="store_true",
                   help="keep hipBLASLt's own GEMM choice (no TunableOp timing)")
    p.add_argument("--no-rollout", action="store_true")
    p.add_argument("--no-selfplay", action="store_true")
    p.add_argument("--no-redeal", action="store_true")
    p.add_argument("--no-paired", action="store_true")
    p.add_argument("--no-published", action="store_true",
                   help="skip the reference's own two published-figure harnesses")
    p.add_argument("--streams", type=int, default=1,
                   help="slices of the batch stepped on their own streams")
    p.add_argument("--no-graph", action="store_true", help="issue the loop eagerly")
    p.add_argument("--two-launch", action="store_true",
                   help="observe_sample and step_reset_spares as two launches per step")
    p.add_argument("--copy-probe", action="store_true",
                   help="also run a plain 1 GiB device copy (calibrates HBM byte counters)")
    p.add_argument("--decode-steps", type=int, default=20)
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--branch-cpu-seconds", type=float, default=3.0,
                   help="per branch CPU baseline (clone + step, and with observe)")
    return p.parse_args()


def random_policy(ext, torch, batch: int, steps: int, warmup: int, streams: int,
                  graph: bool, fused: bool = True) -> dict:
    """The timed loop.  The batch is cut into `streams` contiguous slices (even length),
    each stepped on its own default-priority stream; REFILL steps of every slice form one
    block (the spares refill, then one play_random launch of REFILL steps), captured once
    as a HIP graph and replayed (or issued eagerly with graph=False).
    Every slice deals the same games the unsliced batch would: seed = base + global row +
    batch * generation."""
    dev = torch.device("cuda")
    idx = torch.arange(batch, dtype=torch.int64, device=dev)
    states = ext.create(idx + SEED_BASE, idx & 1)
    gen = torch.zeros(batch, dtype=torch.int32, device=dev)
    sampler = ext.seed_samplers(batch, SEED_BASE, gen)
    # Next games are pre-dealt in full-width batches every REFILL steps; a finished row
    # copies its spare (dealt inline if stale), the same rows reset_done would deal.
    if batch % (2 * streams):
        raise SystemExit("the batch must split into slices of even length")
    width = batch // streams
    spares = [torch.empty((SPARE_SLOTS * width, 248), dtype=torch.uint8, device=dev)
              for _ in range(streams)]
    spare_gen = [torch.zeros(SPARE_SLOTS * width, dtype=torch.int32, device=dev)
                 for _ in range(streams)]
    side = [torch.cuda.Stream() for _ in range(streams)]

    def block(nsteps: int) -> None:
        """nsteps loop steps on every slice; the first one pre-deals the spares."""
        cur = torch.cuda.current_stream()
        for s in side:
            s.wait_stream(cur)
        for k, s in enumerate(side):
            r = slice(k * width, (k + 1) * width)
            st, g, sm, sp, sg = states[r], gen[r], sampler[r], spares[k], spare_gen[k]
            base = SEED_BASE + k * width
            with torch.cuda.stream(s):
                if fused and nsteps:
                    # nsteps x (observe + draw + step + auto-reset) in one launch
                    ext.refill_spares(sp, sg, g, base, batch)
                    ext.play_random(st, sm, base, g, sp, sg, batch, nsteps)
                for t in range(0 if fused else nsteps):
                    if t == 0:
                        ext.refill_spares(sp, sg, g, base, batch)
                    # observe + the random policy's draw from the legal mask, one launch
                    _, _, _, _, _, actions = ext.observe_sample(st, sm)
                    # step + auto-reset of the finished rows from their spares
                    ext.step_reset_spares(st, actions, base, g, sm, sp, sg, batch)
        for s in side:
            cur.wait_stream(s)

    def runner(nsteps: int):
        if not graph or nsteps == 0:
            return lambda: block(nsteps)
        block(nsteps)  # warm the allocator and handles outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            block(nsteps)
        return g.replay

    for _ in range(warmup // REFILL):
        block(REFILL)
    block(warmup % REFILL)
    full, rest = runner(REFILL), runner(steps % REFILL)
    # A graph's first replay carries a one-off cost (about 0.4 ms on this GPU): replay
    # each graph the timed loop uses once here, so the timed steps run at steady state.
    if steps >= REFILL:
        full()
    if steps % REFILL:
        rest()
    torch.cuda.synchronize()
    # Every finished game bumps its row's generation once.
    start_games = int(gen.sum(dtype=torch.int64).item())
    torch.cuda.synchronize()
    with region("c2.loop"):
        t0 = time.perf_counter()
        for _ in range(steps // REFILL):
            full()
        rest()
        torch.cuda.synchronize()
        seconds = time.perf_counter() - t0
    games = int(gen.sum(dtype=torch.int64).item()) - start_games
    # Per-kernel durations: launches captured in a HIP graph and replayed between two
    # events on the stream the replay runs on, so the kernels run back to back (issued
    # eagerly, a launch of the 43 us observe kernel waits on the host's allocation and
    # launch instead).
    stream = torch.cuda.current_stream()

    def graph_of(fn, reps: int):
        fn()  # warm the allocator outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(reps):
                fn()
        return g

    def replay_ms(g, name: str, times: int = 1) -> float:
        total = 0.0
        with region(name):
            for _ in range(times):
                ev = (torch.cuda.Event(enable_timing=True),
                      torch.cuda.Event(enable_timing=True))
                ev[0].record(stream)
                g.replay()
                ev[1].record(stream)
                torch.cuda.synchronize()
                total += ev[0].elapsed_time(ev[1])
        return total

    # The observe kernel alone on the loop's live (mid-game) states, whole batch:
    # 5 replays of 10 launches.
    obs = graph_of(lambda: ext.observe(states), 10)
    observe_ms = replay_ms(obs, "c2.observe", times=5) / 50
    del obs
    # play_random alone (one launch of REFILL steps on the whole batch, as in the loop),
    # continuing the games: 6 back-to-back replays of the loop's block (refill_spares, then
    # the launch) less 6 of refill_spares alone, so that only the first replay's submission
    # falls between the events.
    play_ms = record_ms = None
    if fused and streams == 1:
        def block_once():
            ext.refill_spares(spares[0], spare_gen[0], gen, SEED_BASE, batch)
            ext.play_random(states, sampler, SEED_BASE, gen, spares[0], spare_gen[0], batch,
                            REFILL)

        def six(g, name: str) -> float:
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            with region(name):
                ev[0].record(stream)
                for _ in range(6):
                    g.replay()
                ev[1].record(stream)
                torch.cuda.synchronize()
            return ev[0].elapsed_time(ev[1])

        def block_record():
            ext.refill_spares(spares[0], spare_gen[0], gen, SEED_BASE, batch)
            ext.play_random(states, sampler, SEED_BASE, gen, spares[0], spare_gen[0], batch,
                            REFILL, record=True)

        blocks = graph_of(block_once, 1)
        refills = graph_of(lambda: ext.refill_spares(spares[0], spare_gen[0], gen, SEED_BASE,
                                                     batch), 1)
        play_ms = (six(blocks, "c2.play") - six(refills, "c2.refill")) / 6
        del blocks
        # The same launch with every step's outputs at their own addresses (record mode:
        # 6.4 GB of observations a launch, 25x the GPU's 256 MB last-level cache), so no
        # step's stores can be absorbed by a cache line that the next step overwrites.
        records = graph_of(block_record, 1)
        record_ms = (six(records, "c2.play_record") - six(refills, "c2.refill")) / 6
        del records, refills
    return {"seconds": seconds, "games": games, "observe_ms": observe_ms, "play_ms": play_ms,
            "record_ms": record_ms}


def mid_game_roots(ext, torch, n: int, base: int):
    """n games dealt from seed base + i, each played 3-15 seeded random decisions deep (the
    depth drawn from the game's own sampler); returns the rows still running and their
    movers."""
    import numpy as np

    dev = torch.device("cuda")
    idx = torch.arange(n, dtype=torch.int64, device=dev)
    roots = ext.create(idx + base, idx & 1)
    gen = torch.zeros(n, dtype=torch.int32, device=dev)
    sampler = ext.seed_samplers(n, base, gen)
    depth = 3 + (sampler.cpu().numpy().view(np.uint64) % np.uint64(13)).astype(np.int64)
    depth_t = torch.from_numpy(depth).to(dev)
    for d in range(15):
        _, legal, _, done, _ = ext.observe(roots)
        actions = ext.sample_uniform(legal, sampler)
        ext.step_indexed(roots, idx[depth_t > d], actions[depth_t > d])
    _, _, player, done, status = ext.observe(roots)
    live = torch.nonzero(~done & (status == 0)).flatten()
    return roots.index_select(0, live).contiguous(), player.long().index_select(0, live)


# Host threads for the CPU baselines: one per core this process may run on, at most 16
# (the host cores that go with one GPU on the MI355X boxes this runs on: each of a node's
# GPUs has a 16-core share of the host, however many cores the OS reports).
CPU_THREAD_CAP = 16


def host_cores() -> dict:
    """The host the CPU baselines run on: the OS's core count, the cores this process may
    run on (its affinity), the CPU model, and the threads used (the affinity count, capped
    at CPU_THREAD_CAP)."""
    count = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = count
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    threads = max(1, min(affinity, CPU_THREAD_CAP))
    return {"threads": threads, "os_cpu_count": count, "affinity_cores": affinity,
            "cpu_model": model, "thread_cap": CPU_THREAD_CAP,
            "cap_reason": "16 host cores go with each GPU of the node"}


def branch_cpu_baseline(roots, parent, actions, seconds: float) -> dict:
    """The same children on the host's cores: the reference engine's own build
    (oracle/_ref; the oracle's C restatement where it is absent) clones each child's root
    and steps it (branch_indexed), then also observes the child (branch + observe), one
    child per task on a thread pool, repeated over the whole 1,048,576-child batch until
    `seconds` have passed.  The CPU writes no child rows or observations to memory, so it
    does less memory work per child than the GPU."""
    from oracle.ref import REF_LIB, RefEngine

    reference = REF_LIB.exists()
    ref = RefEngine(reference=reference)
    host = host_cores()
    threads = host["threads"]
    r, ids, acts = (t.cpu().numpy() for t in (roots, parent, actions))
    out = {"cores": threads, "kind": "reference" if reference else "port", "host": host}
    for name, observe in (("branch", False), ("branch_observe", True)):
        reps, dt = 0, 0.0
        t0 = time.perf_counter()
        while dt < seconds:
            ref.branch_work(r, ids, acts, threads, observe)
            reps += 1
            dt = time.perf_counter() - t0
        out[name] = {"value": round(reps * ids.size / dt, 1), "unit": "children/s",
                     "sample": f"{reps} x {ids.size} children in {dt:.1f} s"}
    return out


def branch_workload(ext, torch, iters: int, cpu_seconds: float | None) -> dict:
    """4,096 roots from seeded random play of 3-15 decisions; child k of a root takes
    legal[k] while k < count, then legal[xorshift % count]."""
    dev = torch.device("cuda")
    roots_n, fan = 4096, 256
    # live roots only (a root may have finished early); children cycle over them
    roots, _ = mid_game_roots(ext, torch, roots_n, SEED_BASE + 0x5EED)
    _, legal, _, _, _ = ext.observe(roots)
    n_live = roots.shape[0]
    parent = (torch.arange(roots_n * fan, device=dev) // fan) % n_live
    k = torch.arange(roots_n * fan, device=dev) % fan
    lg = legal.index_select(0, parent)
    counts = lg.sum(1)
    x = (torch.arange(roots_n * fan, device=dev) * 0x9E3779B97F4A7C15 + 1) & ((1 << 62) - 1)
    pick = torch.where(k < counts, k, x % counts)
    actions = torch.argmax((lg.cumsum(1) > pick[:, None]).to(torch.int8), dim=1)
    parent, actions = parent.contiguous(), actions.contiguous()
    children = ext.branch_indexed(roots, parent, actions)[0]
    ext.observe(children)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    stream = torch.cuda.current_stream()
    with region("c3.branch"):
        ev[0].record(stream)
        for _ in range(iters):
            children = ext.branch_indexed(roots, parent, actions)[0]
        ev[1].record(stream)
        torch.cuda.synchronize()
    ev.append(torch.cuda.Event(enable_timing=True))
    with region("c3.observe"):
        ev[3].record(stream)
        for _ in range(iters):
            ext.observe(children)
        ev[2].record(stream)
        torch.cuda.synchronize()
    branch_ms = ev[0].elapsed_time(ev[1]) / iters
    observe_ms = ev[3].elapsed_time(ev[2]) / iters
    # the same children branched and observed by one launch (branch_observe_indexed)
    del children
    out = ext.branch_observe_indexed(roots, parent, actions)
    del out
    torch.cuda.synchronize()
    with region("c3.branch_observe"):
        ev[0].record(stream)
        for _ in range(iters):
            out = ext.branch_observe_indexed(roots, parent, actions)
            del out
        ev[1].record(stream)
        torch.cuda.synchronize()
    fused_ms = ev[0].elapsed_time(ev[1]) / iters
    n = roots_n * fan
    branch_gbs = n * BRANCH_BYTES_PER_CHILD / (branch_ms * 1e-3) / 1e9
    fused_per_child = BRANCH_BYTES_PER_CHILD + OBSERVE_BYTES_PER_ROW - 248
    fused_gbs = n * fused_per_child / (fused_ms * 1e-3) / 1e9
    out = {
        "children": n,
        "live_roots": int(n_live),
        "branch_ms": round(branch_ms, 4),
        "branches_per_s": n / (branch_ms * 1e-3),
        "branch_gbs": branch_gbs,
        "observe_children_ms": round(observe_ms, 4),
        "branch_observe_per_s": n / ((branch_ms + observe_ms) * 1e-3),
        "branch_observe_fused_ms": round(fused_ms, 4),
        "branch_observe_fused_per_s": n / (fused_ms * 1e-3),
        "branch_observe_fused_gbs": fused_gbs,
        # branch_indexed: 8 (id) + 8 (action) + 248 (child) + 9 (step outputs) B a child,
        # the parents read from L2.  branch_observe_indexed: that plus the child's
        # observation (2,880 + 179 + 1 + 1 + 2 B) and no child read-back.
        "roofline": {"kernel": "branch_kernel (branch_indexed)", "bound": "hbm",
                     "achieved": round(branch_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(branch_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("branch_kernel", str(n)),
                     "bytes_per_child": BRANCH_BYTES_PER_CHILD,
                     "avg_launch_ms": round(branch_ms, 4)},
        "observe_roofline": {"kernel": "branch_observe_kernel (branch_observe_indexed)",
                             "bound": "hbm", "achieved": round(fused_gbs, 2),
                             "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(fused_gbs / HBM_PEAK_GBS, 4),
                             "traffic": measured_traffic("branch_observe_kernel", str(n)),
                             "bytes_per_child": fused_per_child,
                             "avg_launch_ms": round(fused_ms, 4)},
    }
    if cpu_seconds:
        out["cpu_baseline"] = branch_cpu_baseline(roots, parent, actions, cpu_seconds)
    return out


def event_lengths(ext, torch, games: int, base_seed: int) -> "torch.Tensor":
    """Committed events per game of `games` seeded random-policy games (seed = base + j,
    first = j & 1), played to the end on the GPU engine."""
    dev = torch.device("cuda")
    idx = torch.arange(games, dtype=torch.int64, device=dev)
    states = ext.create(idx + base_seed, idx & 1)
    gen = torch.zeros(games, dtype=torch.int32, device=dev)
    sampler = ext.seed_samplers(games, base_seed, gen)
    count = torch.zeros(games, dtype=torch.int64, device=dev)
    for _ in range(128):
        _, legal, _, done, _ = ext.observe(states)
        if bool(done.all()):
            break
        actions = ext.sample_uniform(legal, sampler)
        out = ext.step_events_indexed(states, idx, actions)
        count += (out[4] & ~done).long()
    return count


def canonical_workload(ext, torch, games: int = 131072, iters: int = 8) -> dict:
    """The reference's canonical whole-game driver (rollout_canonical_torch50; its GPU
    bench times 131,072 games a launch, tests/cuda_rollout50_bench.cu:22-33, 111):
    seeds 0xBB67AE8584CAA73B + i * 0x9E3779B97F4A7C15, first = i & 1, one game per lane
    played to the end in registers.  Complete games/s over `iters` launches (HIP events)
    at that size and at 8x it, and the HBM roofline of its 56 bytes a game (seed, first,
    five digest words) at the reference's size."""
    dev = torch.device("cuda")
    stream = torch.cuda.current_stream()

    def timed(n: int):
        i = torch.arange(n, dtype=torch.int64, device=dev)
        seeds = i * -7046029254386353131 + (0xBB67AE8584CAA73B - (1 << 64))
        first = i & 1
        ext.rollout_canonical(seeds, first)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with region(f"a16.canonical_{n}"):
            e0.record(stream)
            for _ in range(iters):
                digest = ext.rollout_canonical(seeds, first)
            e1.record(stream)
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters, digest

    ms, digest = timed(games)
    big_ms, _ = timed(8 * games)
    actions = ((digest[:, 2] & 0xFFFF).sum()).item()
    gbs = games * 56 / (ms * 1e-3) / 1e9
    return {"games_per_s": round(games / (ms * 1e-3), 1), "launch_ms": round(ms, 4),
            "games": games, "primary_actions_per_game": round(actions / games, 2),
            "games_per_s_8x": round(8 * games / (big_ms * 1e-3), 1),
            "launch_ms_8x": round(big_ms, 4),
            "roofline": {"kernel": "canonical_kernel", "bound": "hbm", "achieved": round(gbs, 2),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 6),
                         "traffic": measured_traffic("canonical_kernel", str(games)),
                         "bytes_per_game": 56, "avg_launch_ms": round(ms, 4),
                         "bound_note": "HBM is not what bounds it: VALU issue is (SQ counters: "
                                       "VALU busy 0.67 at 131,072 games, 0.78 at 1,048,576)"}}


def decode_lengths(torch, events: "torch.Tensor", slots: int, seed: int) -> dict:
    """Cache row lengths from per-game event counts `events` [games per row, rows] (game k
    of row i is seeded game i + rows * k): each game adds its opening token and its events.
    "stress": games are concatenated until a per-row target drawn uniformly from
    [1, slots] (torch generator seeded with `seed`) is reached; "full": as many games as
    fit below `slots` - 1; "natural": one game.  Every length is clamped to `slots` - 2, so
    that a row can take two more tokens."""
    total = torch.cumsum(events + 1, 0)
    cap = slots - 2
    natural = total[0].clamp_max(cap)
    gen = torch.Generator(device=events.device).manual_seed(seed)
    target = torch.randint(1, slots + 1, (events.shape[1],), generator=gen,
                           device=events.device)
    reached = total >= target
    first = torch.where(reached.any(0), reached.int().argmax(0),
                        torch.full_like(target, events.shape[0] - 1))
    stress = total.gather(0, first[None]).squeeze(0).clamp_max(cap)
    full = torch.where(total <= cap, total, torch.zeros_like(total)).max(0).values
    full = torch.where(full == 0, natural, full)
    return {"stress": stress, "full": full, "natural": natural}


def decode_workload(ext, torch, steps: int, rows: int = 4096, slots: int = 320) -> dict:
    """Sequence-policy decode: a 4-layer causal transformer (d_model 256, 8 heads of 32,
    GELU MLP 1024, pre-norm, bf16, N(0, 0.02) weights from seed 0) runs one query token
    per cache row through `cached_step` (per layer: in-projection GEMM -> KV append fused
    with the HIP decode attention -> out-projection and MLP GEMMs).  KV cache
    [4, 4,096, 8, 320, 32] bf16.  Row lengths come from seeded random-policy games: row i
    concatenates the event logs of games i, i + 4,096, i + 8,192, ... (one opening token
    plus each game's events) until a per-row target drawn uniformly from [1, 320] is
    reached ("stress", mean pos ~170), or while they fit below 320 slots ("full", pos
    ~300), or holds one game (the reference's 50-slot regime, "natural").  The step takes
    the queries longest first (`decode_order`, one launch a step for its 4 layers); the
    decode kernel alone is timed over the 4 layers' caches in turn (as the step reads
    them) with that order, in index order, and on one layer's cache."""
    from torch import nn

    from cugo_amd.seq_decode import KVCache, order_pays, cached_step
    from cugo_amd.cugo_seq_attention50 import decode_attention_append, decode_order

    dev = torch.device("cuda")
    layers, d, heads = 4, 256, 8
    dh = d // heads
    torch.manual_seed(0)
    layer = nn.TransformerEncoderLayer(d, heads, 4 * d, dropout=0.0, activation="gelu",
                                       batch_first=True, norm_first=True)
    model = nn.Module()
    model.encoder = nn.TransformerEncoder(layer, layers, enable_nested_tensor=False)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0.0, 0.02)
    model = model.to(dev).to(torch.bfloat16).eval()

    per_row = 24
    ev = event_lengths(ext, torch, rows * per_row, SEED_BASE + 0xDEC0DE).view(per_row, rows)
    lengths = decode_lengths(torch, ev, slots, seed=0xC5)

    cache = KVCache(layers, rows, heads, d, slots, dev)
    gen = torch.Generator(device=dev).manual_seed(1)
    for t in (cache.k, cache.v):
        t.copy_((torch.randn(t.shape, generator=gen, device=dev) * 0.5).to(t.dtype))
    x = (torch.randn(rows, d, generator=gen, device=dev) * 0.5).to(torch.bfloat16)
    out = {}
    stream = torch.cuda.current_stream()
    with torch.no_grad():
        for name in ("stress", "full", "natural"):
            cache.length.copy_(lengths[name])
            for _ in range(3):
                cached_step(model, cache, x)
            torch.cuda.synchronize()
            with region(f"c5.step_{name}"):
                t0 = time.perf_counter()
                for _ in range(steps):
                    cached_step(model, cache, x)
                torch.cuda.synchronize()
                step_s = (time.perf_counter() - t0) / steps
            # The decode kernel alone, same call as inside the step: the layers' caches in
            # turn, as the step reads them (a burst on one layer's cache also times how much
            # of a launch's reads the last-level cache keeps from the launch before), with
            # the step's query order (longest first, one order launch a step for 4 layers).
            q = (torch.randn(rows, heads, dh, generator=gen, device=dev) * 0.5).to(torch.bfloat16)
            kn, vn = q.clone(), q.clone()
            pos = lengths[name].clamp_max(slots - 1)
            order = decode_order(pos, slots) if order_pays(rows, slots) else None
            reps = 52

            def burst(label, order, layer_of=lambda r: r % layers):
                for r in range(4):
                    decode_attention_append(q, kn, vn, cache.k[layer_of(r)],
                                            cache.v[layer_of(r)], pos, order=order)
                ev0 = torch.cuda.Event(enable_timing=True)
                ev1 = torch.cuda.Event(enable_timing=True)
                with region(label):
                    ev0.record(stream)
                    for r in range(reps):
                        decode_attention_append(q, kn, vn, cache.k[layer_of(r)],
                                                cache.v[layer_of(r)], pos, order=order)
                    ev1.record(stream)
                    torch.cuda.synchronize()
                return ev0.elapsed_time(ev1) / reps

            kernel_ms = burst(f"c5.decode_{name}", order)
            one_layer_ms = burst(f"c5.decode_{name}_one_layer", order, lambda r: 0)
            unordered_ms = burst(f"c5.decode_{name}_unordered", None) if order is not None else None
            order_ms = None
            if order is not None:
                ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                ev0.record(stream)
                for _ in range(reps):
                    decode_order(pos, slots)
                ev1.record(stream)
                torch.cuda.synchronize()
                order_ms = ev0.elapsed_time(ev1) / reps
            # cache reads (slots < pos; slot pos comes from registers) + q, k_new, v_new
            # reads + k/v slot writes + out writes + pos
            row_bytes = heads * dh * 2
            nbytes = int(pos.sum()) * row_bytes * 2 + rows * row_bytes * 6 + rows * 8
            gbs = nbytes / (kernel_ms * 1e-3) / 1e9
            traffic = measured_traffic("decode_kernel", f"{rows} {name}")
            out[name] = {"tokens_per_s": round(rows / step_s, 1),
                         "roofline": {"kernel": "decode_kernel", "bound": "hbm",
                                      "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                                      "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                                      "traffic": traffic},
                         "step_ms": round(step_s * 1e3, 4),
                         "mean_pos": round(float(pos.float().mean()), 2),
                         "max_pos": int(pos.max()),
                         "decode_kernel_ms": round(kernel_ms, 4),
                         "decode_kernel_ms_one_layer": round(one_layer_ms, 4),
                         "decode_kernel_ms_index_order": (round(unordered_ms, 4)
                                                          if unordered_ms is not None else None),
                         "order_ms": round(order_ms, 4) if order_ms is not None else None,
                         "decode_bytes": nbytes,
                         }
    out["cache"] = [layers, rows, heads, slots, dh]
    return out


def selfplay_workload(ext, torch, wave: int = 4096, waves: int = 3) -> dict:
    """Event-sequence policy self-play (the reference's WaveCollector step): a 4-layer d256
    SeqPolicy (8 heads of 32, bf16, N(0, 0.02) weights from seed 0) plays waves of `wave`
    games to the end; each decision step (observe, query token, cached decode over the
    [4, 2 * wave, 8, 50, 32] bf16 cache, readout, Gumbel-max, engine step with events, one
    event token per seat appended) is one HIP-graph replay.  Reports complete games/s,
    decision steps/s and tokens/s (three tokens per game per step: the query and two
    event tokens), with the same step issued eagerly for comparison."""
    from cugo_amd.seq_selfplay import SelfPlayWave, SeqPolicy, make_seeds

    dev = torch.device("cuda")
    torch.manual_seed(0)
    policy = SeqPolicy(d_model=256, layers=4, heads=8)
    with torch.no_grad():
        for prm in policy.parameters():
            prm.normal_(0.0, 0.02)
    policy = policy.to(dev).to(torch.bfloat16).eval()
    sp = SelfPlayWave(ext, policy, wave, max_steps=64)
    learner = torch.zeros(wave, dtype=torch.int64, device=dev)
    seeds, first = make_seeds(wave, 0, dev)
    sp.play(seeds, first, learner)  # capture + one warm wave
    torch.cuda.synchronize()
    with region("f1.selfplay"):
        t0 = time.perf_counter()
        steps = 0
        for k in range(waves):
            seeds, first = make_seeds(wave, (k + 1) * wave, dev)
            steps += sp.play(seeds, first, learner)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    # one step: graph replay vs eager, same state
    reps = 16
    sp.reset(seeds, first, learner)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(reps):
        sp.graph.replay()
    torch.cuda.synchronize()
    graph_ms = (time.perf_counter() - t1) / reps * 1e3
    sp.reset(seeds, first, learner)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(reps):
        sp.step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t1) / reps * 1e3
    # the step's largest launch on its own: a layer's feed-forward half (ffn: linear1,
    # GELU, linear2, the residual add and the next norm) over the paired pass's 3 w rows
    # (events of both seats and the queries), HIP events around 20 launches; beside it the
    # two launches it replaces (linear + GELU, linear_add_layernorm)
    from cugo_amd.seq_decode import feed_forward, linear, linear_add_norm

    layer, nxt = policy.encoder.layers[0], policy.encoder.layers[1].norm1
    m = 3 * wave
    h = torch.randn(m, 256, device=dev).to(torch.bfloat16)
    x = torch.randn(m, 256, device=dev).to(torch.bfloat16)
    stream = torch.cuda.current_stream()

    def launch_us(fn, name: str) -> float:
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with region(name):
            e0.record(stream)
            for _ in range(20):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / 20

    ffn_us = launch_us(lambda: feed_forward(layer, h, x, nxt), "f1.ffn")
    u = linear(h, layer.linear1.weight, layer.linear1.bias, gelu=True)
    two_us = (launch_us(lambda: linear(h, layer.linear1.weight, layer.linear1.bias, gelu=True),
                        "f1.linear1")
              + launch_us(lambda: linear_add_norm(u, layer.linear2.weight, layer.linear2.bias, x,
                                                  nxt), "f1.linear2"))
    ffn_flops = 2 * m * (256 * 1024 + 1024 * 256)
    ffn_hbm = 2 * (4 * m * 256 + 2 * 256 * 1024 + 1024 + 3 * 256)
    rows_wg = 48 if m == 12288 else None
    wgs = (m + 47) // 48 if rows_wg else None
    return {"games_per_s": round(wave * waves / wall, 1),
            "ffn_roofline": {
                "kernel": f"ffn_kernel (linear1 + GELU + linear2 + residual + LayerNorm, {m} "
                          "rows, 256 -> 1024 -> 256, bf16)",
                "bound": "mfma", "achieved": round(ffn_flops / ffn_us / 1e6, 1),
                "peak": 2500.0, "unit": "TFLOP/s",
                "frac": round(ffn_flops / ffn_us / 1e6 / 2500.0, 4), "traffic": None,
                "us_per_launch": round(ffn_us, 2),
                "two_launch_us": round(two_us, 2),
                "hbm_gbs": round(ffn_hbm / ffn_us / 1e3, 1),
                # every workgroup streams all of W1 and W2 (1 MiB) through its CU's L1
                "l1_weight_gbs": (round(wgs * (1 << 20) / ffn_us / 1e3, 1) if wgs else None),
                "workgroups": wgs},
            "steps_per_wave": round(steps / waves, 2),
            "decision_steps_per_s": round(wave * steps / wall, 1),
            "tokens_per_s": round(3 * wave * steps / wall, 1),
            "step_ms_graph": round(graph_ms, 4), "step_ms_eager": round(eager_ms, 4),
            "wave": wave, "cache": [4, 2 * wave, 8, 50, 32], "dtype": "bf16"}


def redeal_workload(ext, torch, rows: int = 4096, worlds: int = 8) -> dict:
    """Redealt worlds (the reference's redeal_worlds): 4,096 mid-game rows from seeded
    random play (3-15 decisions deep), 8 worlds each, every world redealt until the
    observer's features and mask match (8 tries); plus the redeal kernel alone on all
    32,768 copies."""
    from cugo_amd.redeal import redeal, redeal_worlds

    dev = torch.device("cuda")
    roots, players = mid_game_roots(ext, torch, rows, SEED_BASE + 0x5EA1)
    env_rows = torch.arange(roots.shape[0], device=dev)
    torch.manual_seed(0)
    redeal_worlds(ext, roots, env_rows, players, worlds)
    torch.cuda.synchronize()
    reps = 5
    with region("f3.redeal_worlds"):
        t0 = time.perf_counter()
        for _ in range(reps):
            out = redeal_worlds(ext, roots, env_rows, players, worlds)
        torch.cuda.synchronize()
        worlds_s = (time.perf_counter() - t0) / reps
    copies = roots.repeat(worlds, 1)
    seats = players.repeat(worlds)
    keys = torch.rand(copies.shape[0], 50, device=dev)
    rng = torch.randint(-2**62, 2**62, (copies.shape[0],), device=dev)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ext.redeal(copies, seats, keys, rng)
    with region("f3.redeal_kernel"):
        e0.record(stream)
        for _ in range(20):
            ext.redeal(copies, seats, keys, rng)
        e1.record(stream)
        torch.cuda.synchronize()
    kernel_ms = e0.elapsed_time(e1) / 20
    changed = float((out.view(torch.int64)[:, 3] != roots.repeat(worlds, 1).view(torch.int64)[:, 3])
                    .float().mean())
    return {"worlds_per_s": round(out.shape[0] / worlds_s, 1),
            "redeal_worlds_ms": round(worlds_s * 1e3, 3),
            "redeal_kernel_ms": round(kernel_ms, 4),
            "redealt_fraction": round(changed, 4), "rows": int(roots.shape[0]), "worlds": worlds}


def paired_workload(ext, torch, pairs: int = 4096) -> dict:
    """Paired evaluation (the reference's evaluate_paired): 4,096 deals played twice with
    the seats swapped, two 3x512 residual MLP policies (fp32 weights, fp16 autocast, random
    N(0, 0.02) init), greedy actions; complete games/s."""
    from torch import nn

    from cugo_amd.paired_eval import evaluate_paired

    dev = torch.device("cuda")

    class Block(nn.Module):
        def __init__(self, d: int) -> None:
            super().__init__()
            self.norm = nn.LayerNorm(d)
            self.fc1 = nn.Linear(d, d)
            self.fc2 = nn.Linear(d, d)

        def forward(self, h):
            return h + self.fc2(torch.relu(self.fc1(self.norm(h))))

    def actor(seed: int) -> nn.Module:
        torch.manual_seed(seed)
        m = nn.Sequential(nn.Linear(720, 512), Block(512), Block(512), Block(512),
                          nn.LayerNorm(512), nn.Linear(512, 179))
        with torch.no_grad():
            for prm in m.parameters():
                prm.normal_(0.0, 0.02)
        return m.to(dev)

    a, b = actor(1), actor(2)
    evaluate_paired(ext, a, b, 256, seed_offset=0, max_steps=128, use_amp=True)  # warm
    with region("f4.paired"):
        s = evaluate_paired(ext, a, b, pairs, seed_offset=1 << 20, max_steps=128,
                            use_amp=True)
    return {"games_per_s": round(s.games / s.seconds, 1), "seconds": round(s.seconds, 4),
            "decision_steps": s.decision_steps, "pairs": pairs,
            "mean_pair_score_a": round(s.mean_pair_score_a, 4)}


def paired_seq_workload(ext, torch, pairs: int = 4096) -> dict:
    """Paired evaluation of two sequence policies (evaluate_paired with a History,
    cugo_eval50.py:169): 4,096 deals played twice with the seats swapped, two hybrid-mode
    4-layer d256 SeqPolicy models (fp32 weights from N(0, 0.02), seeds 1 and 2, run in bf16
    as use_amp does), greedy actions; complete games/s."""
    from cugo_amd.paired_eval import evaluate_paired
    from cugo_amd.seq_selfplay import SeqPolicy

    dev = torch.device("cuda")

    def policy(seed: int):
        torch.manual_seed(seed)
        m = SeqPolicy("hybrid")
        with torch.no_grad():
            for prm in m.parameters():
                prm.normal_(0.0, 0.02)
        return m.to(dev).eval()

    a, b = policy(1), policy(2)
    evaluate_paired(ext, a, b, 256, seed_offset=0, max_steps=128, use_amp=True)  # warm
    with region("f4.paired_seq"):
        s = evaluate_paired(ext, a, b, pairs, seed_offset=1 << 20, max_steps=128,
                            use_amp=True)
    return {"games_per_s": round(s.games / s.seconds, 1), "seconds": round(s.seconds, 4),
            "decision_steps": s.decision_steps, "pairs": pairs,
            "ms_per_decision_step": round(1e3 * s.seconds / max(1, s.decision_steps), 4),
            "mean_pair_score_a": round(s.mean_pair_score_a, 4)}


PUBLISHED_GAMES_PER_S = 100_000.0      # README.md:22-23, torch50_smoke.py on one RTX 5080
PUBLISHED_BRANCHES_PER_S = 100_000_000.0  # README.md:23, branch50_smoke.py on one RTX 5080


def published_smoke_workload(ext, torch, batch: int = 32768, iters: int = 3,
                             max_steps: int = 128) -> dict:
    """The workload of the reference's published games/s figure (torch50_smoke.py:62-134,
    run_games): each batch of B = 32,768 games is dealt from make_seeds(B, offset) and
    played to the end by PpoActor(256, blocks=1, norm="none") in fp16 (seed 12345: Linear
    720 -> 256, one residual block x + fc2(SiLU(fc1(x))) with fc2 zero-initialised, then
    out(SiLU(h)) with out zero-initialised) and the masked argmax; every step observes and
    steps all B games.  Timed as the reference times it: a warm-up batch, then `iters`
    batches (offsets 2,000,000 + i B), games/s = B / seconds per batch, their mean.  Here a
    step is one HIP-graph replay (observe -> the model's GEMMs -> masked argmax -> the
    status checks on the device -> step) and the host reads the all-done flag one step
    behind instead of synchronising on every step's checks."""
    from torch import nn
    from torch.nn import functional as F

    from cugo_amd.seq_selfplay import make_seeds

    dev = torch.device("cuda")

    class SmokeActor(nn.Module):
        """PpoActor(256, blocks=1, norm="none") (cugo_ppo_nets50.py:22-64)."""

        def __init__(self, hidden: int = 256) -> None:
            super().__init__()
            self.inp = nn.Linear(720, hidden)
            self.fc1 = nn.Linear(hidden, hidden)
            self.fc2 = nn.Linear(hidden, hidden)
            self.out = nn.Linear(hidden, 179)
            for lin in (self.fc2, self.out):
                nn.init.zeros_(lin.weight)
                nn.init.zeros_(lin.bias)

        def forward(self, x):
            h = self.inp(x)
            h = h + self.fc2(F.silu(self.fc1(h)))
            return self.out(F.silu(h))

    torch.manual_seed(12345)
    torch.cuda.manual_seed_all(12345)
    model = SmokeActor().to(dev).half().eval()
    states = torch.empty((batch, 248), dtype=torch.uint8, device=dev)
    a_seat = torch.zeros(batch, dtype=torch.int64, device=dev)
    active = torch.zeros(batch, dtype=torch.bool, device=dev)
    final_reward = torch.zeros(batch, device=dev)
    final_nagari = torch.zeros(batch, dtype=torch.bool, device=dev)
    bad = torch.zeros(3, dtype=torch.int64, device=dev)
    steps = torch.zeros(1, dtype=torch.int64, device=dev)
    any_active = torch.zeros(1, dtype=torch.int32, device=dev)
    playing = torch.zeros(1, dtype=torch.int32, device=dev)  # 1 while a game is left
    flags = torch.zeros(2, dtype=torch.int32, pin_memory=True)

    def step() -> None:
        features, legal, players, done, status = ext.observe(states)
        logits = model(features.to(torch.float16))
        actions = ext.masked_argmax(logits.float(), legal)
        actions = ext.paired_select(active, status, done, legal.any(1), players, a_seat,
                                    actions, actions, bad, any_active, playing)
        reward, new_done, nagari, step_status, _ = ext.step(states, actions)
        ext.paired_update(active, step_status, new_done, reward, nagari, final_reward,
                          final_nagari, bad, any_active, steps, playing)

    def deal(offset: int) -> None:
        seeds, first = make_seeds(batch, offset, dev)
        states.copy_(ext.create(seeds, first))
        done = ext.observe(states)[3]
        active.copy_(~done)
        final_reward.zero_()
        final_nagari.zero_()

    def run(offset: int, replay) -> tuple[float, int]:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        deal(offset)
        stream = torch.cuda.current_stream()
        behind = None
        for k in range(max_steps):
            replay()
            flags[k & 1].copy_(playing[0], non_blocking=True)
            queued = (torch.cuda.Event(), k & 1, k + 1)
            queued[0].record(stream)
            if behind is not None:
                behind[0].synchronize()
                if not int(flags[behind[1]]):
                    break
            behind = queued
        else:
            raise RuntimeError(f"not all games finished within {max_steps} decision steps")
        torch.cuda.synchronize()
        return time.perf_counter() - t0, behind[2]

    with torch.inference_mode():
        deal(0)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
            step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        run(1_000_000, graph.replay)  # warm-up batch
        bad.zero_()
        seconds, step_counts = [], []
        with region("published.smoke"):
            for i in range(iters):
                dt, n_steps = run(2_000_000 + i * batch, graph.replay)
                seconds.append(dt)
                step_counts.append(n_steps)
    problems = [int(x) for x in bad.tolist()]
    if any(problems):
        raise RuntimeError(f"observe/legal/step checks failed: {problems}")
    mean_s = sum(seconds) / len(seconds)
    gps = batch / mean_s
    return {"games_per_s": round(gps, 1), "best_games_per_s": round(batch / min(seconds), 1),
            "mean_ms_per_batch": round(1e3 * mean_s, 4), "batch": batch, "iters": iters,
            "decision_steps": step_counts,
            "published_games_per_s": PUBLISHED_GAMES_PER_S,
            "vs_published": round(gps / PUBLISHED_GAMES_PER_S, 2),
            "published_on": "1x RTX 5080 (README.md:22-23)",
            "model": "PpoActor(256, blocks=1, norm=none) fp16, masked argmax"}


def published_branch_workload(ext, torch, batch: int = 262144, parents_n: int = 4096,
                              warmup: int = 5, iters: int = 20) -> dict:
    """The workload of the reference's published branches/s figure (branch50_smoke.py:
    68-191): 4,096 games dealt from make_seeds, each stepped once with its first legal
    action, the live ones kept as parents; 262,144 children, child j of parent j mod P,
    each taking its parent's first legal action; branch_indexed timed over 20 calls after
    5, branches/s = children x calls / seconds."""
    from cugo_amd.seq_selfplay import make_seeds

    dev = torch.device("cuda")

    def live(rows):
        _, legal, _, done, status = ext.observe(rows)
        keep = torch.nonzero(~done & (status == 0)).flatten()
        return rows.index_select(0, keep).contiguous(), legal.index_select(0, keep)

    parents, legal = live(ext.create(*make_seeds(parents_n, 0, dev)))
    ext.step(parents, legal.to(torch.int64).argmax(1))
    parents, legal = live(parents)
    n_parents = parents.shape[0]
    ids = torch.arange(batch, dtype=torch.int64, device=dev).remainder(n_parents)
    actions = legal.to(torch.int64).argmax(1).index_select(0, ids)
    for _ in range(warmup):
        ext.branch_indexed(parents, ids, actions)
    torch.cuda.synchronize()
    with region("published.branch"):
        t0 = time.perf_counter()
        for _ in range(iters):
            ext.branch_indexed(parents, ids, actions)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
    rate = batch * iters / dt
    return {"branches_per_s": round(rate, 1), "ms_per_call": round(1e3 * dt / iters, 4),
            "children": batch, "parents": int(n_parents), "iters": iters,
            "published_branches_per_s": PUBLISHED_BRANCHES_PER_S,
            "vs_published": round(rate / PUBLISHED_BRANCHES_PER_S, 2),
            "published_on": "1x RTX 5080 (README.md:23)"}


def engine_traffic(batch: int, fused: bool) -> int | None:
    """HBM bytes of one engine step of the rollout from the committed counter summary: the
    fused step + observation (bf16 features) and a 32nd of the spares' refill, or observe
    with the draw and the step with auto-reset for an actor the one-launch forward does
    not serve."""
    if fused:
        parts = [measured_traffic("step_observe_kernel", str(batch)),
                 measured_traffic("refill_kernel", str(batch))]
    else:
        parts = [measured_traffic("observe_sample_kernel", str(batch)),
                 measured_traffic("step_reset_spares_kernel", str(batch)),
                 measured_traffic("refill_kernel", str(batch))]
    if None in parts:
        return None
    return sum(parts[:-1]) + parts[-1] // 32


ROLLOUT_BASE = SEED_BASE + 0xC4  # the MLP rollout's deal seeds


def make_rollout(ext, torch, batch: int = 32768, horizon: int = 128):
    """The MLP rollout the `rollout` leg times: the residual MLP actor (720 -> 512, three
    blocks, bf16, N(0, 0.02) weights from seed 0), B games dealt from ROLLOUT_BASE + i, the
    sampler's Philox key drawn from a generator seeded 1."""
    from cugo_amd.rollout import MlpRollout, ResidualMlpActor

    dev = torch.device("cuda")
    torch.manual_seed(0)
    actor = ResidualMlpActor()
    with torch.no_grad():
        for prm in actor.parameters():
            prm.normal_(0.0, 0.02)
    actor = actor.to(dev).to(torch.bfloat16).eval()
    gen = torch.Generator(device=dev).manual_seed(1)
    return MlpRollout(ext, actor, batch, horizon, ROLLOUT_BASE, generator=gen)


def rollout_workload(ext, torch, batch: int = 32768, horizon: int = 128) -> dict:
    """MLP PPO self-play rollout (cugo_amd/rollout.py): B games, a residual MLP actor
    (720 features -> Linear 512 -> 3 blocks of h + Linear(ReLU(Linear(LayerNorm(h)))) ->
    LayerNorm -> 179 logits and a value head; bf16, N(0, 0.02) weights from seed 0),
    Gumbel-max sampling over the legal actions, a `horizon`-step buffer (bf16 features,
    mask, action, log-prob, value, reward, done), finished games re-dealt from pre-dealt
    spares inside the step.  Reports env steps/s, the engine's and the actor's shares of
    the step time and a roofline for each: the actor's FLOPs over its forward time (the
    one-launch MFMA forward, `mlp_forward`, that the rollout runs) against the bf16 MFMA
    peak, the engine's bytes (the fused step + next observation: the rows read and
    written once, the action, the step outputs and the bf16 observation, 2,136 B a row)
    over its time against HBM.  The rollout runs as one HIP graph per horizon; the shares
    come from graphs of the engine's and the actor's launches alone."""
    from cugo_amd.rollout import fused_forward, mlp_forward, pack_actor

    dev = torch.device("cuda")
    ro = make_rollout(ext, torch, batch, horizon)
    actor = ro.actor
    stream = torch.cuda.current_stream()

    def graph_ms(g, reps: int, name: str) -> float:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with region(name):
            e0.record(stream)
            for _ in range(reps):
                g.replay()
            e1.record(stream)
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    with torch.no_grad():
        ro.capture()  # the whole horizon as one HIP graph
        ro.replay()   # first replay outside the timed region
        torch.cuda.synchronize()
        games0 = ro.games_completed()
        reps = 2
        with region("c4.rollout"):
            t0 = time.perf_counter()
            for _ in range(reps):
                ro.replay()
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
        games = ro.games_completed() - games0
        step_ms = wall * 1e3 / (reps * horizon)
        # The engine's share: its launches alone on a copy of the games, 32 steps in one
        # graph (the spares refilled once), with the uniform legal actions a first eager
        # pass from the same rows drew (they stand in for the actor's): the rollout's fused
        # step + next observation (bf16 features), or observe and step_reset_spares for an
        # actor the one-launch forward does not serve.  Each replay first restores the rows,
        # generations, samplers and spares; a graph of the restore alone is subtracted.
        # The actor's share: its forward pass, the Gumbel-max draw (uniforms from Philox in
        # the kernel) and the buffer writes of one step, one graph.
        start = [t.clone() for t in (ro.states, ro.generation, ro.sampler, ro.spares,
                                     ro.spare_gen)]
        st, g2, smp, sp, sg = (t.clone() for t in start)
        feats = torch.empty((batch, 720), dtype=torch.bfloat16, device=dev)
        legal = ext.observe_bf16(st, feats)[1]
        acts = []
        ext.refill_spares(sp, sg, g2, ROLLOUT_BASE)
        for _ in range(32):
            acts.append(ext.sample_uniform(legal, smp))
            legal = ext.step_observe_spares(st, acts[-1], ROLLOUT_BASE, g2, smp, sp, sg,
                                            feats)[6]

        def engine_block(engine: bool):
            for dst, src in zip((st, g2, smp, sp, sg), start):
                dst.copy_(src)
            if not engine:
                return
            ext.refill_spares(sp, sg, g2, ROLLOUT_BASE)
            for k in range(32):
                if ro.fused_kernel:
                    ext.step_observe_spares(st, acts[k], ROLLOUT_BASE, g2, smp, sp, sg, feats)
                else:
                    ext.step_reset_spares(st, acts[k], ROLLOUT_BASE, g2, smp, sp, sg)
                    ext.observe(st)

        def block_ms(engine: bool, name: str) -> float:
            engine_block(engine)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                engine_block(engine)
            ms = graph_ms(g, 3, name)
            del g
            return ms

        engine_step_ms = (block_ms(True, "c4.engine") - block_ms(False, "c4.restore")) / 32
        del start, st, g2, smp, sp, sg, feats, acts
        ro.observe(0)
        ro.act(0)
        torch.cuda.synchronize()
        ag = torch.cuda.CUDAGraph()
        with torch.cuda.graph(ag):
            ro.act(0)
        actor_step_ms = graph_ms(ag, 10, "c4.actor")
        del ag
        # the forward pass alone, a graph of 20 back-to-back passes on the last step's
        # input (bf16), replayed 3 times: the rollout's one-launch forward, and the
        # layer-by-layer form (hipBLASLt GEMMs + HIP add + LayerNorm) for comparison
        x = ro.buffer.features[horizon - 1]
        packed = ro.packed if ro.fused_kernel else pack_actor(ext, actor)

        def forward_graph(fn) -> "torch.cuda.CUDAGraph":
            fn()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(20):
                    fn()
            return g

        fg = forward_graph(lambda: mlp_forward(ext, packed, x))
        forward_ms = graph_ms(fg, 3, "c4.forward") / 20
        del fg
        lg = forward_graph(lambda: fused_forward(ext, actor, x))
        layered_ms = graph_ms(lg, 3, "c4.forward_layers") / 20
        del lg
    flops_row = actor.flops_per_row()
    tflops = flops_row * batch / (forward_ms * 1e-3) / 1e12
    # fused: the rows read and written once, the action, the step outputs and the bf16
    # observation; else observe (float32 features) and the step, the rows read twice
    engine_row = (STEP_BYTES_PER_ROW + 720 * 2 + 179 + 4 if ro.fused_kernel
                  else OBSERVE_BYTES_PER_ROW + STEP_BYTES_PER_ROW)
    engine_bytes = batch * engine_row
    engine_gbs = engine_bytes / (engine_step_ms * 1e-3) / 1e9
    return {"env_steps_per_s": round(batch * reps * horizon / wall, 1),
            "games_per_s": round(games / wall, 1),
            "step_ms": round(step_ms, 4),
            "engine_share": round(engine_step_ms / step_ms, 4),
            "actor_share": round(actor_step_ms / step_ms, 4),
            "engine_step_ms": round(engine_step_ms, 4), "actor_step_ms": round(actor_step_ms, 4),
            "hip_graph": "one graph per rollout of horizon steps",
            "roofline": {"kernel": "actor_kernel (mlp_forward: the whole actor in one launch)",
                         "bound": "mfma", "achieved": round(tflops, 1), "peak": 2500.0,
                         "unit": "TFLOP/s", "frac": round(tflops / 2500.0, 4),
                         "traffic": (measured_traffic("actor_kernel", str(batch))
                                     if ro.fused_kernel else None),
                         "flops_per_row": flops_row,
                         "avg_forward_ms": round(forward_ms, 4),
                         "layered_forward_ms": round(layered_ms, 4),
                         "layered_tflops": round(flops_row * batch / (layered_ms * 1e-3)
                                                 / 1e12, 1)},
            "engine_roofline": {"kernel": ("step_observe_spares" if ro.fused_kernel
                                           else "observe + step_reset_spares")
                                          + " (+ refill_spares)",
                                "bound": "hbm", "achieved": round(engine_gbs, 2),
                                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(engine_gbs / HBM_PEAK_GBS, 4),
                                "traffic": engine_traffic(batch, ro.fused_kernel),
                                "bytes_per_row_step": engine_row,
                                "ms_per_step": round(engine_step_ms, 4)},
            "games_completed": games,
            "batch": batch, "horizon": horizon, "dtype": "bf16"}


def cpu_baseline(seconds: float) -> dict:
    """The reference engine's own build (oracle/_ref; the oracle's C restatement when that
    is absent) on the host cores, same random-policy protocol (observe + sample +
    step_events per decision), growing the sample to ~`seconds`."""
    from oracle.ref import REF_LIB, SEED_BASE as base, RefEngine

    reference = REF_LIB.exists()
    ref = RefEngine(reference=reference)
    host = host_cores()
    threads = host["threads"]
    n = 4096
    while True:
        t0 = time.perf_counter()
        _, _, _, _, decisions = ref.play_random(base + 10**9, n, threads=threads, outputs=False)
        dt = time.perf_counter() - t0
        if dt >= seconds or n >= 1 << 24:
            break
        n = int(n * min(8.0, max(1.5, seconds / max(dt, 1e-3))))
    return {"value": n / dt, "unit": "games/s", "cores": threads,
            "kind": "reference" if reference else "port",
            "sample": f"{n} random-policy games ({decisions} decisions) in {dt:.1f} s",
            "steps_per_s": decisions / dt, "host": host}


def store_ceiling(torch, ext=None) -> dict:
    """What plain stores reach on this GPU: torch's fill_ of a 192 MiB float32 tensor (about
    the bytes of one observation step at B = 65,536; it fits in the GPU's 256 MB last-level
    cache, as the loop's output buffers do) and of a 4 GiB one (every byte has to reach
    DRAM), 20 launches each timed with events.  The observation kernels are store-bound, so
    these are their practical ceilings below the published 8 TB/s.  With `ext`, also the
    store probe: play_random's observation-row store pattern without the game (65,536 rows
    of 2,880 bytes, 32 steps), over the same rows every step and at distinct rows."""
    stream = torch.cuda.current_stream()

    def fill_gbs(numel: int) -> tuple[float, float]:
        buf = torch.empty(numel, dtype=torch.float32, device="cuda")
        for _ in range(3):
            buf.fill_(1.0)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 20
        with region("ceiling.fill"):
            e0.record(stream)
            for _ in range(reps):
                buf.fill_(1.0)
            e1.record(stream)
            torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        del buf
        return numel * 4 / (ms * 1e-3) / 1e9, ms

    gbs, ms = fill_gbs(48 << 20)
    large_gbs, large_ms = fill_gbs(1 << 30)
    out = {"kernel": "torch fill_, 192 MiB float32", "gbs": round(gbs, 1),
           "avg_launch_ms": round(ms, 4), "large_fill_gbs": round(large_gbs, 1),
           "large_fill": "torch fill_, 4 GiB float32", "large_fill_ms": round(large_ms, 4)}
    if ext is not None:
        rows, row_bytes, steps = 65536, 720 * 4, REFILL
        buf = torch.empty(rows * row_bytes * steps, dtype=torch.uint8, device="cuda")
        probe = {"pattern": f"{rows} rows x {row_bytes} B, {steps} steps, 64 rows a wave, "
                            "4 rows at a time, 1 KiB float4 stores"}
        for name, distinct in (("looped", False), ("distinct", True)):
            for _ in range(2):
                ext.store_probe(buf, rows, row_bytes, steps, distinct)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with region(f"ceiling.store_probe_{name}"):
                e0.record(stream)
                for _ in range(5):
                    ext.store_probe(buf, rows, row_bytes, steps, distinct)
                e1.record(stream)
                torch.cuda.synchronize()
            pms = e0.elapsed_time(e1) / 5
            probe[f"{name}_ms"] = round(pms, 4)
            probe[f"{name}_gbs"] = round(rows * row_bytes * steps / (pms * 1e-3) / 1e9, 1)
        del buf
        out["store_probe"] = probe
    return out


@contextlib.contextmanager
def tuned_gemms(torch, enabled: bool):
    """PyTorch-ROCm TunableOp for a leg whose eager warm-up runs every library GEMM shape
    it then captures into a HIP graph (the rollout leg's layer-by-layer baseline): each
    shape's first call times the library's solutions and the graph keeps the fastest.
    Its results file goes to the temporary directory."""
    tunable = torch.cuda.tunable
    if enabled:
        tunable.set_filename(os.path.join(os.environ.get("TMPDIR", "/tmp"),
                                          "cugo_tunableop_results.csv"))
        tunable.enable(True)
        tunable.tuning_enable(True)
    try:
        yield
    finally:
        if enabled:
            tunable.tuning_enable(False)
            tunable.enable(False)


def main() -> None:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)
    import torch

    from cugo_amd import load_extension

    ext = load_extension()
    if args.copy_probe:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    ceiling = store_ceiling(torch, ext)
    rp = random_policy(ext, torch, args.batch, args.steps, args.warmup, args.streams,
                       not args.no_graph, not args.two_launch)
    games_per_s = rp["games"] / rp["seconds"]
    ms_per_step = 1000.0 * rp["seconds"] / args.steps
    observe_gbs = args.batch * OBSERVE_BYTES_PER_ROW / (rp["observe_ms"] * 1e-3) / 1e9
    observe_roofline = {"kernel": "observe_kernel", "bound": "hbm",
                        "achieved": round(observe_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(observe_gbs / HBM_PEAK_GBS, 4),
                        "traffic": measured_traffic("observe_kernel", str(args.batch)),
                        "bytes_per_row": OBSERVE_BYTES_PER_ROW,
                        "avg_launch_ms": round(rp["observe_ms"], 4),
                        "frac_of_store_ceiling": round(observe_gbs / ceiling["gbs"], 4)}
    if rp["play_ms"] is not None:
        play_bytes = play_bytes_per_row(REFILL)
        play_gbs = args.batch * play_bytes / (rp["play_ms"] * 1e-3) / 1e9
        roofline = {"kernel": "play_kernel", "bound": "hbm",
                    "achieved": round(play_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(play_gbs / HBM_PEAK_GBS, 4),
                    "traffic": measured_traffic("play_kernel", f"{args.batch} x {REFILL}"),
                    "bytes_per_row": play_bytes, "steps_per_launch": REFILL,
                    "avg_launch_ms": round(rp["play_ms"], 4),
                    "ms_per_step": round(rp["play_ms"] / REFILL, 4),
                    "frac_of_store_ceiling": round(play_gbs / ceiling["gbs"], 4),
                    # the same launch writing each step's outputs to distinct addresses
                    "record_avg_launch_ms": round(rp["record_ms"], 4),
                    "record_achieved": round(args.batch * play_bytes
                                             / (rp["record_ms"] * 1e-3) / 1e9, 2),
                    "record_frac_of_large_fill": round(
                        args.batch * play_bytes / (rp["record_ms"] * 1e-3) / 1e9
                        / ceiling["large_fill_gbs"], 4)}
        probe = ceiling.get("store_probe")
        if probe is not None and args.batch == 65536:
            # the time the launch's feature rows alone take to store (the probe), over
            # the launch's time
            roofline["frac_of_store_probe"] = round(probe["looped_ms"] / rp["play_ms"], 4)
            roofline["record_frac_of_store_probe"] = round(
                probe["distinct_ms"] / rp["record_ms"], 4)
    else:
        roofline = observe_roofline
    result = {
        "metric": "complete games/sec (random-policy self-play, B=65536 resident games)",
        "value": round(games_per_s, 1),
        "unit": "games/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic",
        "config": {"workload": "random-policy self-play: observe -> sample -> step -> "
                               "auto-reset, "
                               + (f"one play_random launch per {REFILL} steps (every step's "
                                  "observation written)" if not args.two_launch
                                  else "observe_sample + step_reset_spares per step"),
                   "batch": args.batch, "seed_base": hex(SEED_BASE),
                   "policy": "uniform legal action, per-game xorshift64",
                   "streams": args.streams, "hip_graph": not args.no_graph,
                   "spare_slots": SPARE_SLOTS,
                   "gemm_selection": ("hipBLASLt heuristics" if args.no_tunable else
                                      "PyTorch-ROCm TunableOp for the rollout leg's "
                                      "layer-by-layer baseline (the self-play and decode "
                                      "legs' layers run on this build's kernels)")},
        "kernel_ms_per_step": (round(rp["play_ms"] / REFILL, 4)
                               if rp["play_ms"] is not None else None),
        "steps_per_s": round(args.batch * args.steps / rp["seconds"], 1),
        "games_timed": rp["games"],
        "roofline": roofline,
        "observe_roofline": observe_roofline,
        "store_ceiling": ceiling,
    }
    if not args.no_branch:
        result["branch"] = branch_workload(ext, torch, args.branch_iters,
                                           None if args.no_cpu else args.branch_cpu_seconds)
    if not args.no_canonical:
        result["canonical"] = canonical_workload(ext, torch)
    if not args.no_decode:
        result["decode"] = decode_workload(ext, torch, args.decode_steps)
    if not args.no_selfplay:
        result["selfplay"] = selfplay_workload(ext, torch)
    if not args.no_redeal:
        result["redeal"] = redeal_workload(ext, torch)
    if not args.no_paired:
        result["paired"] = paired_workload(ext, torch)
        result["paired_seq"] = paired_seq_workload(ext, torch)
    if not args.no_published:
        result["published_smoke"] = published_smoke_workload(ext, torch)
        result["published_branch"] = published_branch_workload(ext, torch)
    if not args.no_rollout:
        with tuned_gemms(torch, not args.no_tunable):
            result["rollout"] = rollout_workload(ext, torch)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
