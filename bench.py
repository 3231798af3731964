"""Throughput of the NanoRTS hot path on one MI355X.

Workload: basesWorkers16x16, VERSION_ORIGINAL_FINETUNED, CANCEL_RANDOM,
partial observability, 65536 games, seeded uniform-random legal actions for
both players, auto-reset on done.  One step is one env.step cycle of every
game: legality masks -> sampled actions -> decode -> core.step -> auto-reset
-> symbolic observations of both agents written to HBM.  The timed loop runs
the fused rollout kernel (state resident in LDS for `--chunk` cycles per
launch); the per-call path (masks, sampler and env.step as three launches per
cycle) is timed beside it and reported in `config`.

`--workload seat-workerrush` / `seat-lightrush` measure the learner-vs-bot
configuration instead: basesWorkers16x16, VERSION_ORIGINAL_FINETUNED,
CANCEL_BOTH, max_cycles 3000, 32768 games, player_1 = WorkerRush or LightRush
on the device, player_0 = seeded uniform-random legal actions, full episodes
with auto-reset (the fused seat rollout kernel).

`--workload gridnet` measures the GridNet surface: basesWorkers16x16,
VERSION_ORIGINAL_FINETUNED, CANCEL_RANDOM, 32768 games, one-hot int32 planes
and the packed action mask; per cycle the harness sampler draws every
source cell's row from the last observation's mask and one GridNet step
launch decodes, steps, rewards, resets and observes.

`--workload groups` measures the multi-group core.step: four groups of
16384 games on basesWorkers16x16 (VERSION_ORIGINAL_FINETUNED, CANCEL_RANDOM,
horizons 5000, 4000, 3000 and 2000: one bucket), each cycle stepping every
group on uniformly random Commands (a pool of eight sets held in HBM) with
one nanorts_amd_step_groups launch; one launch per group is timed beside it.

`--workload gow` measures the GardenOfWar64x64 configuration: CANCEL_ALTERNATING,
the slot count without the capacity profile, 4096 games of symbolic
observations in the fused rollout (500 steps by the configuration), and 256
games on the pixel surface (both agents' uint8[1024, 1024, 3] images every
cycle) through the per-call path, reported in `pixel_leg` with the render
kernel's own bandwidth.

Prints one JSON line (rank 0, N=1).
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
MAP = "basesWorkers16x16"
# Untimed cycles every game plays before the warmup and the timed region, so
# that the timed cycles run from mid-game positions (the reference's README
# measures from mid-game positions too), whatever --warmup is.
MIDGAME = 200
SIMDS = 256 * 4  # MI355X: 256 CUs of 4 SIMDs
XCDS = 8
NUM_ENVS = 65536
METRIC = "env-steps/sec (both players) at 16x16 × 65536 envs; % HBM roofline"
SEAT_ENVS = 32768
GRID_ENVS = 32768
GROUP_ENVS = 65536
GROUP_HORIZONS = (5000, 4000, 3000, 2000)


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=("headline", "seat-workerrush", "seat-lightrush", "gridnet", "groups", "gow"),
                    default="headline")
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--envs", type=int, default=None)
    ap.add_argument("--chunk", type=int, default=100, help="cycles per fused launch")
    ap.add_argument("--depth", type=int, default=2, help="observation ring depth in HBM")
    ap.add_argument("--per-call-steps", type=int, default=20)
    ap.add_argument("--cpu-envs", type=int, default=4096)
    ap.add_argument("--cpu-steps", type=int, default=3000)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--pixel-steps", type=int, default=20, help="gow: cycles of the pixel leg")
    ap.add_argument("--one-pass", action="store_true",
                    help="headline: run each launch as one pass on the full LDS block (no two-pass launch)")
    ap.add_argument("--traffic", choices=("auto", "off"), default="auto")
    ap.add_argument("--profile-child", choices=("rollout", "copy", "gridnet", "seat"), default=None,
                    help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.envs is None:
        args.envs = {"headline": NUM_ENVS, "gridnet": GRID_ENVS, "groups": GROUP_ENVS,
                     "gow": GOW_ENVS}.get(args.workload, SEAT_ENVS)
    return args


def state_bytes(bucket) -> int:
    from nanorts_amd.model import STATE_LEAVES, leaf_shape

    total = 0
    for leaf in STATE_LEAVES:
        n = 1
        for d in leaf_shape(leaf, bucket):
            n *= d
        total += n * leaf.dtype.itemsize
    return total + 8 + 4  # environment_root + episode_index


def step_bytes(bucket) -> int:
    """Algorithmic HBM bytes written per env-step by the fused rollout:
    both agents' feature maps and scalars, rewards and the done flag."""
    return 2 * bucket.cell_count * 6 + 2 * 4 * 4 + 2 * 4 + 1


def make_env(envs: int):
    import nanorts_amd
    from nanorts_amd import env as envmod

    game = nanorts_amd.map_name_to_scenario(MAP, conflict_strategy="CANCEL_RANDOM", max_cycles=5000)
    env = nanorts_amd.make("NanoRTS", scenario=game, partial_observability=True, final_observation=False)
    _, state = env.reset(envmod.env_roots(0, envs))
    return game, env, state


# whether the last rollout launch ran two passes (set by run_rollout)
LAST_TWO_PASS = False


def run_rollout(env, state, steps: int, chunk: int, depth: int, step0: int, events=None, two_pass: bool = True):
    """Run `steps` cycles in launches of `chunk`; returns per-launch ms when
    `events` is requested."""
    import torch

    global LAST_TWO_PASS
    done = 0
    times = []
    out = None
    while done < steps:
        n = min(chunk, steps - done)
        if events:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
        out = env.rollout(state, n, (11, 13), step0=step0 + done, record=True, observation_depth=depth,
                          two_pass=two_pass)
        if events:
            b.record()
            times.append((a, b, n))
        done += n
    if out is not None:
        # the first pass ran at least one cycle of some game
        first = out["first_pass_cycles"]
        LAST_TWO_PASS = first is not None and bool((first > 0).any().item())
    return times


def copy_bandwidth() -> float:
    import torch

    n = 1 << 28  # 1 GiB of int32
    src = torch.empty(n, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    reps = 10
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    return 2 * n * 4 * reps / (a.elapsed_time(b) / 1e3) / 1e9


def host_cpu() -> dict:
    """The host's CPU model and core counts, for the CPU baseline's record."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return {"cpu_model": model, "host_cpus": os.cpu_count(), "usable_cpus": usable}


def cpu_baseline(envs: int, steps: int) -> dict:
    """The oracle (plain-C restatement of the reference step, masks and
    encoders) timed on the host cores over a bounded sample."""
    from nanorts_amd import env as envmod
    from nanorts_amd.content import map_name_to_scenario
    from oracle.oracle import Oracle, batch_initial

    game = map_name_to_scenario(MAP, conflict_strategy="CANCEL_RANDOM", max_cycles=5000)
    oracle = Oracle(game)
    state = batch_initial(game, envs, envmod.env_roots(0, envs))
    host = host_cpu()
    threads = max(1, min(host["usable_cpus"], 16))  # one GPU's share of the host cores
    t0 = time.perf_counter()
    used = oracle.rollout(state, (11, 13), 0, steps, True, threads=threads, record=False)["threads"]
    dt = time.perf_counter() - t0
    return {"value": round(envs * steps / dt, 1), "unit": "env-steps/s", "cores": int(used), "kind": "port",
            "sample": f"{envs} games x {steps} cycles of the same workload (oracle rollout: masks, sampler, "
                      f"env.step, auto-reset, partial-observability symbolic obs) on {used} host threads "
                      f"(one GPU's share of the box's cores), {dt:.1f} s", **host}


def child(args) -> None:
    """Short runs under rocprofv3 --pmc (traffic counters)."""
    import torch

    if args.profile_child == "copy":
        n = 1 << 26  # 256 MiB
        src = torch.ones(n, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        return
    if args.profile_child == "seat":
        seat, state = make_seat(args.workload, args.envs)
        for t in range(2):
            seat.rollout(state, args.chunk, (11, 13), step0=t * args.chunk, observation_depth=args.depth)
        torch.cuda.synchronize()
        return
    if args.profile_child == "gridnet":
        g, state, mask = make_gridnet(args.envs)
        for t in range(8):
            out = g.step(state, g.sample_actions(mask, (11, 13), t), donate=True)
            state, mask = out.environment_state, out.observation.action_mask
        torch.cuda.synchronize()
        return
    # the headline's timed launch shape: the mid-game advance, then launches
    # of `chunk` cycles (the caller passes the timed chunk)
    game, env, state = make_env(args.envs)
    run_rollout(env, state, MIDGAME, args.chunk, args.depth, 0, two_pass=not args.one_pass)
    run_rollout(env, state, PMC_LAUNCHES * args.chunk, args.chunk, args.depth, MIDGAME, two_pass=not args.one_pass)
    torch.cuda.synchronize()


PMC_LAUNCHES = 3  # timed-shape launches the headline's profile child runs after the advance


def progress(message: str) -> None:
    """A progress line on stderr (stdout carries only the JSON line)."""
    print(f"bench: {message}", file=sys.stderr, flush=True)


def kernel_base(name: str) -> str:
    """A rocprofv3 kernel name without its argument list."""
    return name.split("(")[0].split()[-1] if name.strip() else ""


def pmc_counters(args, mode: str, kernel, counters: str, chunk: int) -> list[dict[str, float]]:
    """One rocprofv3 --pmc pass over a profile child; per dispatch of the
    kernels named in `kernel` (one name or a tuple; in dispatch order) the
    counter values, the duration in ns and the kernel's name."""
    kernels = (kernel,) if isinstance(kernel, str) else tuple(kernel)
    import csv
    import shutil
    import tempfile

    rocprof = shutil.which("rocprofv3")
    if rocprof is None:
        return []
    progress(f"rocprofv3 --pmc {counters} over the {mode} child")
    out = Path(tempfile.mkdtemp(prefix="nr_pmc_", dir=os.environ.get("TMPDIR", "/tmp")))
    cmd = ["timeout", "-s", "KILL", "120", rocprof, "--pmc", *counters.split(), "-d", str(out), "-o", "pmc",
           "--output-format", "csv", "--", sys.executable, str(ROOT / "bench.py"), "--profile-child", mode,
           "--workload", args.workload, "--envs", str(args.envs), "--chunk", str(chunk), "--depth", str(args.depth)]
    if getattr(args, "one_pass", False):
        cmd.append("--one-pass")
    subprocess.run(cmd, env=dict(os.environ), capture_output=True, text=True, timeout=180)
    rows: dict[int, dict[str, float]] = {}
    for path in out.rglob("*counter_collection.csv"):
        with open(path) as fh:
            for row in csv.DictReader(fh):
                name = row.get("Kernel_Name", "")
                want = (kernel_base(name) in kernels if mode != "copy"
                        else ("copy" in name.lower() or "elementwise" in name.lower()))
                if not want:
                    continue
                rec = rows.setdefault(int(row.get("Dispatch_Id") or len(rows)), {"kernel": kernel_base(name)})
                rec[row["Counter_Name"]] = rec.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
                if row.get("Start_Timestamp") and row.get("End_Timestamp"):
                    rec["duration_ns"] = float(row["End_Timestamp"]) - float(row["Start_Timestamp"])
    shutil.rmtree(out, ignore_errors=True)
    return [rows[k] for k in sorted(rows)]


def _median(values: list[float]) -> float:
    return sorted(values)[len(values) // 2]


# The headline rollout's launch: a first pass (two games per wave, or one)
# and the second pass that follows it on the same stream (or the one pass on
# the full block).  The library picks the first pass by board.
FIRST_PASS_KERNELS = ("k_rollout_pair", "k_rollout_lean")
ROLLOUT_KERNELS = FIRST_PASS_KERNELS + ("k_rollout",)


def first_pass_seen(rows: list[dict[str, float]]) -> str | None:
    """The first-pass kernel that ran in profiled rows, if any."""
    for name in FIRST_PASS_KERNELS:
        if any(r.get("kernel") == name for r in rows):
            return name
    return None


def rollout_kernels(env) -> str:
    """The kernels of one rollout launch, as the library chooses them."""
    first = env.rollout_first_pass()
    return f"k_rollout_{first} + k_rollout (second pass)" if first else "k_rollout"


def per_launch(rows: list[dict[str, float]], counter: str, kernels) -> list[float]:
    """Counter sums per launch of a kernel sequence: a launch opens at each
    dispatch of its first kernel (for the rollout, the first pass that ran)
    and takes the dispatches of the last kernel that follow it (each
    dispatch is its own launch when no opener ran)."""
    kernels = (kernels,) if isinstance(kernels, str) else tuple(kernels)
    openers = [k for k in kernels[:-1] if any(r.get("kernel") == k for r in rows)]
    opener = openers[0] if openers else None
    sums: list[float] = []
    for r in rows:
        if counter not in r:
            continue
        if opener is None or r.get("kernel") == opener or not sums:
            sums.append(r[counter])
        else:
            sums[-1] += r[counter]
    return sums


def pmc_traffic(args, per_launch_steps: int, mode: str = "rollout", kernel=ROLLOUT_KERNELS,
                last: int = 0) -> dict | None:
    """FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of the measured launches of
    `per_launch_steps` cycles (the last `last` launches when set, else every
    one; a launch of several kernels sums them), each scaled by what the
    counter reads for a plain copy of known size."""
    if args.traffic == "off":
        return None
    try:
        copy_bytes = 2 * (1 << 26) * 4  # read + write of the 256 MiB copy
        fetch_copy = [r["FETCH_SIZE"] for r in pmc_counters(args, "copy", "", "FETCH_SIZE", 1) if "FETCH_SIZE" in r]
        write_copy = [r["WRITE_SIZE"] for r in pmc_counters(args, "copy", "", "WRITE_SIZE", 1) if "WRITE_SIZE" in r]
        fetch_rows = pmc_counters(args, mode, kernel, "FETCH_SIZE", per_launch_steps)
        fetch = per_launch(fetch_rows, "FETCH_SIZE", kernel)
        write = per_launch(pmc_counters(args, mode, kernel, "WRITE_SIZE", per_launch_steps), "WRITE_SIZE", kernel)
        if last:
            fetch, write = fetch[-last:], write[-last:]
        if not (fetch_copy and write_copy and fetch and write):
            return None
        # a copy of B bytes fetches B/2 and writes B/2
        f_scale = (copy_bytes / 2) / (_median(fetch_copy) * 1024)
        w_scale = (copy_bytes / 2) / (_median(write_copy) * 1024)
        out = {"fetch_bytes": _median(fetch) * 1024 * f_scale, "write_bytes": _median(write) * 1024 * w_scale,
               "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4), "dispatches": len(fetch),
               "cycles_per_dispatch": per_launch_steps}
        seen = first_pass_seen(fetch_rows)
        if seen:
            out["first_pass"] = seen
        return out
    except Exception:
        return None


def pmc_limiter(args, per_launch_steps: int, last: int) -> dict | None:
    """VALU busy and lane use of the measured launches (one counter pass):
    busy = SQ_ACTIVE_INST_VALU x 4 / SIMDs / GPU cycles of one XCD, lanes =
    SQ_THREAD_CYCLES_VALU / (SQ_ACTIVE_INST_VALU x 64)."""
    if args.traffic == "off":
        return None
    try:
        rows = [r for r in pmc_counters(args, "rollout", ROLLOUT_KERNELS,
                                        "SQ_ACTIVE_INST_VALU SQ_THREAD_CYCLES_VALU GRBM_GUI_ACTIVE", per_launch_steps)
                if "SQ_ACTIVE_INST_VALU" in r and "GRBM_GUI_ACTIVE" in r]
        # the first pass is the launch's dominant kernel when it ran
        main = first_pass_seen(rows) or "k_rollout"
        rows = [r for r in rows if r["kernel"] == main][-last:]
        if not rows:
            return None
        busy, lanes = [], []
        for r in rows:
            gui = r["GRBM_GUI_ACTIVE"]
            # the counter sums its XCDs when it reads more cycles than a
            # 4 GHz clock gives in the dispatch's duration
            if r.get("duration_ns") and gui > 4.0 * r["duration_ns"]:
                gui /= XCDS
            busy.append(r["SQ_ACTIVE_INST_VALU"] * 4 / SIMDS / gui)
            lanes.append(r["SQ_THREAD_CYCLES_VALU"] / (r["SQ_ACTIVE_INST_VALU"] * 64))
        return {"valu_busy": round(_median(busy), 3), "valu_lane_use": round(_median(lanes), 3)}
    except Exception:
        return None


def carry_bytes(bucket) -> int:
    """One env's bot carry (AbstractActions): nine int32 rows, a bool row and
    next_order."""
    return bucket.per_player_capacity * (9 * 4 + 1) + 4


def cpu_seat_baseline(bot_name: str, envs: int, steps: int) -> dict:
    """The oracle's seat loop (masks, the learner's sampler rows, bot act,
    seat step) on one host thread over a bounded sample."""
    from nanorts_amd import env as envmod
    from nanorts_amd.content import map_name_to_scenario
    from oracle.oracle import Oracle, batch_initial, empty_carry

    game = map_name_to_scenario(MAP, max_cycles=3000)
    oracle = Oracle(game)
    state = batch_initial(game, envs, envmod.env_roots(0, envs))
    carry = empty_carry(envs, game.bucket.per_player_capacity)
    strategy = 0 if bot_name == "workerRushAI" else 1
    t0 = time.perf_counter()
    for t in range(steps):
        actions = oracle.sample_actions(oracle.avail_rows(state), (11, 13), t)[:, 0].copy()
        oracle.seat_step(state, carry, strategy, 4, 0, actions, False)
    dt = time.perf_counter() - t0
    return {"value": round(envs * steps / dt, 1), "unit": "env-steps/s", "cores": 1, "kind": "port",
            "sample": f"{envs} games x {steps} cycles of the same workload (oracle: masks, learner sampler, "
                      f"{bot_name} act, seat step, auto-reset, symbolic obs) on 1 host thread, {dt:.1f} s"}


def make_seat(workload: str, envs: int):
    import torch

    import nanorts_amd
    from nanorts_amd import bots
    from nanorts_amd import env as envmod

    torch.cuda.set_device(0)
    bot = bots.workerRushAI if workload == "seat-workerrush" else bots.lightRushAI
    game = nanorts_amd.map_name_to_scenario(MAP, max_cycles=3000)
    seat = bots.SeatEnv(bot, scenario=game, final_observation=False)
    _, state = seat.reset(envmod.env_roots(0, envs))
    return seat, state


def main_seat(args) -> None:
    import torch

    seat, state = make_seat(args.workload, args.envs)
    bot, game = seat.bot, seat.game
    L = args.envs
    chunk = max(1, min(args.chunk, args.steps))

    paired = [False]  # whether the last launch ran the two-games-per-wave first pass

    def run(steps, step0, events):
        done, times = 0, []
        while done < steps:
            n = min(chunk, steps - done)
            if events:
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
            out = seat.rollout(state, n, (11, 13), step0=step0 + done, observation_depth=args.depth)
            if events:
                b.record()
                times.append((a, b, n))
            done += n
        first = out["first_pass_cycles"] if steps else None
        if first is not None:
            paired[0] = bool((first > 0).any().item())
        return times

    run(args.warmup, 0, False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    times = run(args.steps, args.warmup, True)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = [a.elapsed_time(b) for a, b, _ in times]
    full = [ms for (a, b, n), ms in zip(times, launch_ms) if n == chunk] or launch_ms
    avg_launch_s = sum(full) / len(full) / 1e3
    b = game.bucket
    # the kernel keeps the state and the bot's carry in LDS for the launch:
    # both are read and written once per launch, the outputs every cycle
    per_step = step_bytes(b)
    per_launch_bytes = L * (chunk * per_step + 2 * state_bytes(b) + 2 * carry_bytes(b))
    achieved = per_launch_bytes / avg_launch_s / 1e9
    seat_kernels = ("k_seat_rollout_pair", "k_seat_rollout")
    traffic = pmc_traffic(args, chunk, mode="seat", kernel=seat_kernels)
    cpu = None if args.no_cpu else cpu_seat_baseline(bot.name, args.cpu_envs // 4, args.cpu_steps // 15)
    line = {
        "metric": f"env-steps/sec (learner vs {bot.name}) at 16x16 × {L} envs; % HBM roofline",
        "value": round(L * args.steps / wall, 1),
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": "synthetic: player_0 seeded uniform-random legal actions, player_1 the scripted bot, shipped "
                "basesWorkers16x16 map",
        "config": {
            "workload": f"{MAP}, VERSION_ORIGINAL_FINETUNED, CANCEL_BOTH, max_cycles 3000, {L} games, player_1 "
                        f"{bot.name} on the device, full episodes with auto-reset, fused seat rollout {chunk} "
                        f"cycles/launch",
            "games": L, "slots_per_player": b.per_player_capacity,
            "algorithmic_bytes_per_env_step": per_step, "carry_bytes_per_env": carry_bytes(b),
            "state_bytes_per_env": state_bytes(b), "observation_ring_depth": args.depth,
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": None if traffic is None else round(traffic["fetch_bytes"] + traffic["write_bytes"], 1),
            "kernel": "k_seat_rollout_pair + k_seat_rollout (second pass)" if paired[0] else "k_seat_rollout",
            "avg_launch_ms": round(avg_launch_s * 1e3, 4),
            "algorithmic_bytes_per_launch": per_launch_bytes,
        },
        "cpu_baseline": cpu,
    }
    if traffic is not None:
        line["roofline"]["traffic_detail"] = traffic
    print(json.dumps(line))


def gridnet_step_bytes(bucket) -> int:
    """Algorithmic HBM bytes of one GridNet step of one env: the state read
    and written, both players' per-cell actions, the ending state's planes and
    the next observation (one-hot int32 planes, the source mask, the packed
    action mask), the reward components and reward dones, and the four flags
    and the winner."""
    cells = bucket.cell_count
    planes = 2 * cells * 29 * 4
    return 2 * state_bytes(bucket) + 2 * cells * 7 * 4 + 2 * planes + 2 * cells + 2 * cells * 3 * 4 + 48 + 12 + 4 + 4


def cpu_gridnet_baseline(envs: int, steps: int) -> dict:
    """The oracle's GridNet cycle on one host thread over a bounded sample:
    masks and planes from the oracle's legality rows and symbolic maps, the
    harness sampler, decode, core.step keyed by the episode root, rewards,
    auto-reset."""
    import ctypes

    import numpy as np

    from nanorts_amd import env as envmod
    from nanorts_amd.content import map_name_to_scenario
    from oracle.oracle import Oracle, batch_initial, load_library

    game = map_name_to_scenario(MAP, conflict_strategy="CANCEL_RANDOM")
    b = game.bucket
    oracle = Oracle(game)
    lib = load_library()
    L, N, C, H, W = envs, b.neutral_capacity, b.per_player_capacity, b.height, b.width
    state = batch_initial(game, L, envmod.env_roots(0, L))
    widths, offsets = np.asarray((5, 5, 3, 8, 6, 2)), np.asarray((0, 5, 10, 13, 21, 27))

    def observe(st):
        maps = np.minimum(oracle.symbolic(st, False)[0].astype(np.int64), widths - 1)
        planes = np.zeros(maps.shape[:-1] + (29,), np.int32)
        for f in range(6):
            np.put_along_axis(planes, (offsets[f] + maps[..., f])[..., None], 1, axis=-1)
        slot = st["entity_at"].reshape(L, H * W).astype(np.int64)
        s = np.clip(slot, 0, b.entity_capacity - 1)
        owner = np.where(slot >= 0, np.take_along_axis(st["owner"].astype(np.int64), s, 1), -1)
        pending = np.take_along_axis(st["pending_kind"].astype(np.int64), s, 1)
        source = np.stack([(slot >= 0) & (owner == p) & (pending == -1) for p in range(2)], 1)
        rows = oracle.legality_rows(st).reshape(L, 2 * C, 78)
        at = np.take_along_axis(rows, np.clip(slot - N, 0, 2 * C - 1)[..., None], 1)
        return planes, source, source[..., None] & at[:, None]

    def episode_roots(st):
        out = np.zeros((L, 2), np.uint32)
        for l in range(L):
            k = (ctypes.c_uint32 * 2)(*[int(v) for v in st["environment_root"][l]])
            o = (ctypes.c_uint32 * 2)()
            lib.nro_fold_in(k, ctypes.c_uint32(int(st["episode_index"][l])), o)
            out[l] = (o[0], o[1])
        return out

    _, _, mask = observe(state)
    t0 = time.perf_counter()
    for t in range(steps):
        acts = oracle.gridnet_sample_actions(mask, (11, 13), t)
        cmds = oracle.gridnet_decode(state, acts)
        out = oracle.core_step(state, cmds, episode_roots(state))
        observe(state)  # the ending state's planes
        oracle.reset_where_done(state, (out["terminated"] | out["truncated"]).astype(np.uint8))
        _, _, mask = observe(state)
    dt = time.perf_counter() - t0
    return {"value": round(envs * steps / dt, 1), "unit": "env-steps/s", "cores": 1, "kind": "port",
            "sample": f"{envs} games x {steps} cycles of the same workload (oracle: harness sampler, GridNet decode, "
                      f"core.step, planes and masks of the ending and next states, auto-reset) on 1 host thread, "
                      f"{dt:.1f} s"}


def make_gridnet(envs: int):
    import torch

    import nanorts_amd
    from nanorts_amd import env as envmod
    from nanorts_amd import gridnet

    torch.cuda.set_device(0)
    game = nanorts_amd.map_name_to_scenario(MAP, conflict_strategy="CANCEL_RANDOM")
    g = gridnet.GridNet(game, gridnet.prepare(game, mask_form="packed"), device="cuda:0")
    state, obs = g.reset(envmod.env_roots(0, envs))
    return g, state, obs.action_mask


def main_gridnet(args) -> None:
    import torch

    g, state, mask = make_gridnet(args.envs)
    game = g.game
    L = args.envs

    def run(steps, step0, events):
        nonlocal state, mask
        times = []
        for t in range(steps):
            acts = g.sample_actions(mask, (11, 13), step0 + t)
            if events:
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
            out = g.step(state, acts, donate=True)
            if events:
                b.record()
                times.append((a, b))
            state, mask = out.environment_state, out.observation.action_mask
        return times

    run(args.warmup, 0, False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    times = run(args.steps, args.warmup, True)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    avg_launch_s = sum(a.elapsed_time(b) for a, b in times) / len(times) / 1e3
    b = game.bucket
    per_step = gridnet_step_bytes(b)
    achieved = L * per_step / avg_launch_s / 1e9
    traffic = pmc_traffic(args, 1, mode="gridnet", kernel="k_gridnet_step")
    cpu = None if args.no_cpu else cpu_gridnet_baseline(args.cpu_envs // 16, args.cpu_steps // 30)
    line = {
        "metric": f"env-steps/sec (GridNet surface, both players) at 16x16 × {L} envs; % HBM roofline",
        "value": round(L * args.steps / wall, 1),
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": "synthetic: seeded uniform-random legal per-cell actions for both players, shipped basesWorkers16x16 "
                "map",
        "config": {
            "workload": f"{MAP}, VERSION_ORIGINAL_FINETUNED, CANCEL_RANDOM, GridNet surface (one-hot int32 planes, "
                        f"packed action mask), {L} games, max_cycles 5000, auto-reset; per cycle one sampler launch "
                        f"and one GridNet step launch",
            "games": L, "algorithmic_bytes_per_env_step": per_step, "state_bytes_per_env": state_bytes(b),
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": None if traffic is None else round(traffic["fetch_bytes"] + traffic["write_bytes"], 1),
            "kernel": "k_gridnet_step", "avg_launch_ms": round(avg_launch_s * 1e3, 4),
            "algorithmic_bytes_per_launch": L * per_step,
        },
        "cpu_baseline": cpu,
    }
    if traffic is not None:
        line["roofline"]["traffic_detail"] = traffic
    print(json.dumps(line))


def core_step_bytes(bucket) -> int:
    """Algorithmic HBM bytes of one core.step of one env: the state read and
    written, the six int32 Commands fields of 2C positions, and the
    terminated / truncated flags, rewards and admitted event counts."""
    C, T = bucket.per_player_capacity, bucket.unit_type_capacity
    return 2 * state_bytes(bucket) + 6 * 2 * C * 4 + 2 + 8 + 4 * (2 + 2 + 2 * T + 6)


GOW_MAP = "GardenOfWar64x64"
GOW_ENVS = 4096
GOW_PIXEL_ENVS = 256


def main_gow(args) -> None:
    """The GardenOfWar64x64 configuration: CANCEL_ALTERNATING, the slot count
    without the capacity profile, 4096 games of symbolic observations in the
    fused rollout, and 256 games on the pixel surface (uint8[1024, 1024, 3]
    images of both agents each cycle) through the per-call path."""
    import torch

    import nanorts_amd
    from nanorts_amd import env as envmod

    torch.cuda.set_device(0)
    game = nanorts_amd.map_name_to_scenario(GOW_MAP, conflict_strategy="CANCEL_ALTERNATING", capacity_profile=False)
    b = game.bucket
    L = args.envs
    chunk = max(1, min(args.chunk, args.steps))
    env = nanorts_amd.make("NanoRTS", scenario=game, final_observation=False, device="cuda:0")
    _, state = env.reset(envmod.env_roots(0, L))
    run_rollout(env, state, args.warmup, chunk, args.depth, 0)
    torch.cuda.synchronize()
    progress(f"{args.warmup} warmup cycles done")
    t0 = time.perf_counter()
    times = run_rollout(env, state, args.steps, chunk, args.depth, args.warmup, events=True)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = [a.elapsed_time(e) for a, e, _ in times]
    full = [ms for (a, e, n), ms in zip(times, launch_ms) if n == chunk] or launch_ms
    avg_launch_s = sum(full) / len(full) / 1e3
    per_step, sbytes = step_bytes(b), state_bytes(b)
    per_launch_bytes = L * (chunk * per_step + 2 * sbytes)
    achieved = per_launch_bytes / avg_launch_s / 1e9

    # the pixel leg: masks -> sampler -> env.step, whose observation is both
    # agents' images rendered from the step's symbolic maps
    P = GOW_PIXEL_ENVS
    penv = nanorts_amd.make("NanoRTS", scenario=game, surface="pixels", final_observation=False, device="cuda:0")
    _, pstate = penv.reset(envmod.env_roots(1, P))
    image_bytes = 2 * (16 * b.height) * (16 * b.width) * 3

    def pixel_cycles(n, base):
        nonlocal pstate
        for t in range(n):
            words = penv.get_avail_actions(pstate, form="words")
            acts = penv.sample_actions(words, (11, 13), base + t)
            _, pstate, _, _, _ = penv.step(None, pstate, acts, donate=True)

    pixel_cycles(3, 0)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    pixel_cycles(args.pixel_steps, 3)
    torch.cuda.synchronize()
    pixel_rate = P * args.pixel_steps / (time.perf_counter() - t1)
    # the render kernel alone, on symbolic maps of P of the rollout's games
    sym = env.get_obs(state)
    maps_p = torch.stack([sym[a].feature_maps[:P] for a in env.agents], 1).contiguous()
    a_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    penv.pixels_from_maps(maps_p)
    torch.cuda.synchronize()
    a_ev.record()
    reps = 5
    for _ in range(reps):
        penv.pixels_from_maps(maps_p)
    e_ev.record()
    torch.cuda.synchronize()
    render_s = a_ev.elapsed_time(e_ev) / reps / 1e3
    render_gbps = P * image_bytes / render_s / 1e9

    line = {
        "metric": f"env-steps/sec (both players) at {GOW_MAP} x {L} envs (symbolic) + {P} envs (pixels); "
                  "% HBM roofline",
        "value": round(L * args.steps / wall, 1),
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": f"synthetic: seeded uniform-random legal actions from the shipped {GOW_MAP} map",
        "config": {
            "workload": f"{GOW_MAP}, VERSION_ORIGINAL_FINETUNED, CANCEL_ALTERNATING, capacity_profile=False "
                        f"({b.per_player_capacity} slots per player), {L} games symbolic in the fused rollout "
                        f"({chunk} cycles per launch), {P} games on the pixel surface",
            "games": L, "slots_per_player": b.per_player_capacity, "entity_capacity": b.entity_capacity,
            "algorithmic_bytes_per_env_step": per_step, "state_bytes_per_env": sbytes,
            "observation_ring_depth": args.depth,
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None,
            "kernel": rollout_kernels(env), "avg_launch_ms": round(avg_launch_s * 1e3, 4),
            "algorithmic_bytes_per_launch": per_launch_bytes, "cycles_per_launch": chunk,
        },
        "pixel_leg": {
            "games": P, "steps": args.pixel_steps, "env_steps_per_s": round(pixel_rate, 1),
            "image_bytes_per_env_step": image_bytes,
            "render_kernel": "k_pixels_from_maps", "render_ms": round(render_s * 1e3, 4),
            "render_GBps": round(render_gbps, 1), "render_frac": round(render_gbps / HBM_PEAK_GBPS, 4),
        },
        "cpu_baseline": None,
    }
    print(json.dumps(line))


def main_groups(args) -> None:
    import numpy as np
    import torch

    import nanorts_amd
    from nanorts_amd import env as envmod
    from nanorts_amd import groups

    torch.cuda.set_device(0)
    G = len(GROUP_HORIZONS)
    per = args.envs // G
    games = [nanorts_amd.map_name_to_scenario(MAP, conflict_strategy="CANCEL_RANDOM", max_cycles=h)
             for h in GROUP_HORIZONS]
    envs = [nanorts_amd.make("NanoRTS", scenario=g, final_observation=False, device="cuda:0") for g in games]
    states = [env.reset(envmod.env_roots(i, per))[1] for i, env in enumerate(envs)]
    b = games[0].bucket
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(5)
    C, T, cells = b.per_player_capacity, b.unit_type_capacity, b.cell_count

    def commands():
        shape = (per, 2, C)
        draw = lambda lo, hi: torch.randint(lo, hi, shape, generator=gen, device="cuda:0", dtype=torch.int32)
        return {"kind": draw(0, 6), "direction": draw(0, 4), "none_duration": draw(1, 11),
                "target_cell": draw(0, cells), "produced_type": draw(0, T), "request_order": draw(0, 2 * C)}

    pool = [[commands() for _ in range(G)] for _ in range(8)]
    keys = [torch.tensor([[7, i]], dtype=torch.int32, device="cuda:0") for i in range(G)]

    def run(steps, together, events):
        times = []
        for t in range(steps):
            cmds = pool[t % len(pool)]
            reqs = [(keys[i], states[i], cmds[i], envs[i]) for i in range(G)]
            if events:
                a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
            if together:
                groups.step_groups(reqs)
            else:
                for req in reqs:
                    groups.step_groups([req])
            if events:
                e.record()
                times.append((a, e))
        return times

    run(args.warmup, True, False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    times = run(args.steps, True, True)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    avg_launch_s = sum(a.elapsed_time(e) for a, e in times) / len(times) / 1e3
    run(10, False, False)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    run(args.steps, False, False)
    torch.cuda.synchronize()
    apart = G * per * args.steps / (time.perf_counter() - t1)
    per_step = core_step_bytes(b)
    achieved = G * per * per_step / avg_launch_s / 1e9
    line = {
        "metric": f"env-steps/sec (core.step over {G} groups in one launch) at 16x16 × {G * per} envs; % HBM roofline",
        "value": round(G * per * args.steps / wall, 1),
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": "synthetic: uniformly random Commands (a pool of eight sets in HBM), shipped basesWorkers16x16 map",
        "config": {
            "workload": f"{MAP}, VERSION_ORIGINAL_FINETUNED, CANCEL_RANDOM, {G} groups x {per} games, horizons "
                        f"{list(GROUP_HORIZONS)}, one nanorts_amd_step_groups launch per cycle",
            "games": G * per, "groups": G, "algorithmic_bytes_per_env_step": per_step,
            "one_launch_per_group_env_steps_per_s": round(apart, 1),
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": None, "kernel": "k_step_groups",
            "avg_launch_ms": round(avg_launch_s * 1e3, 4), "algorithmic_bytes_per_launch": G * per * per_step,
        },
        "cpu_baseline": None if args.no_cpu else cpu_groups_baseline(args.cpu_envs // 4, args.cpu_steps // 10),
    }
    print(json.dumps(line))


def cpu_groups_baseline(envs: int, steps: int) -> dict:
    """The oracle's core.step on uniformly random Commands, one host thread."""
    import numpy as np

    from nanorts_amd import env as envmod
    from nanorts_amd.content import map_name_to_scenario
    from oracle.oracle import Oracle, batch_initial

    game = map_name_to_scenario(MAP, conflict_strategy="CANCEL_RANDOM")
    b = game.bucket
    oracle = Oracle(game)
    state = batch_initial(game, envs, envmod.env_roots(0, envs))
    rng = np.random.default_rng(5)
    C, T, cells = b.per_player_capacity, b.unit_type_capacity, b.cell_count
    shape = (envs, 2, C)
    pool = [{"kind": rng.integers(0, 6, shape, dtype=np.int32), "direction": rng.integers(0, 4, shape, dtype=np.int32),
             "none_duration": rng.integers(1, 11, shape, dtype=np.int32),
             "target_cell": rng.integers(0, cells, shape, dtype=np.int32),
             "produced_type": rng.integers(0, T, shape, dtype=np.int32),
             "request_order": rng.integers(0, 2 * C, shape, dtype=np.int32)} for _ in range(4)]
    keys = np.tile(np.asarray([[7, 0]], np.uint32), (envs, 1))
    t0 = time.perf_counter()
    for t in range(steps):
        oracle.core_step(state, pool[t % 4], keys)
    dt = time.perf_counter() - t0
    return {"value": round(envs * steps / dt, 1), "unit": "env-steps/s", "cores": 1, "kind": "port",
            "sample": f"{envs} games x {steps} cycles of core.step on uniformly random Commands (oracle) on 1 host "
                      f"thread, {dt:.1f} s"}


def main() -> None:
    args = parse()
    if args.profile_child:
        child(args)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the env path shards by env with no exchange, and this run has no "
              f"multi-GPU configuration (asked for --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)
    if args.workload == "gridnet":
        main_gridnet(args)
        return
    if args.workload == "groups":
        main_groups(args)
        return
    if args.workload == "gow":
        main_gow(args)
        return
    if args.workload != "headline":
        main_seat(args)
        return
    import torch

    torch.cuda.set_device(0)
    game, env, state = make_env(args.envs)
    L = args.envs
    chunk = max(1, min(args.chunk, args.steps))
    # untimed: the mid-game advance, then the warmup
    two = not args.one_pass
    run_rollout(env, state, MIDGAME, chunk, args.depth, 0, two_pass=two)
    run_rollout(env, state, args.warmup, chunk, args.depth, MIDGAME, two_pass=two)
    torch.cuda.synchronize()
    progress(f"{MIDGAME} mid-game + {args.warmup} warmup cycles done")
    # timed region: exactly `steps` cycles
    t0 = time.perf_counter()
    times = run_rollout(env, state, args.steps, chunk, args.depth, MIDGAME + args.warmup, events=True, two_pass=two)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = [a.elapsed_time(b) for a, b, _ in times]
    full = [ms for (a, b, n), ms in zip(times, launch_ms) if n == chunk] or launch_ms
    avg_launch_s = sum(full) / len(full) / 1e3
    value = L * args.steps / wall
    ms_per_step = wall * 1e3 / args.steps

    b = game.bucket
    sbytes = state_bytes(b)
    per_step = step_bytes(b)
    per_launch_bytes = L * (chunk * per_step + 2 * sbytes)
    achieved = per_launch_bytes / avg_launch_s / 1e9

    # per-call path: masks (words) -> sampler -> env.step, 3 launches per cycle
    pc_rate = None
    if args.per_call_steps > 0:
        _, pc_state = env.reset(__import__("nanorts_amd.env", fromlist=["env_roots"]).env_roots(1, L))
        def per_call(n, base):
            nonlocal pc_state
            for t in range(n):
                words = env.get_avail_actions(pc_state, form="words")
                acts = env.sample_actions(words, (11, 13), base + t)
                _, pc_state, _, _, _ = env.step(None, pc_state, acts, donate=True)
        per_call(3, 0)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        per_call(args.per_call_steps, 3)
        torch.cuda.synchronize()
        pc_rate = L * args.per_call_steps / (time.perf_counter() - t1)

    progress(f"timed {args.steps} cycles: {value / 1e6:.1f} M env-steps/s; per-call path "
             f"{0 if pc_rate is None else pc_rate / 1e6:.1f} M")
    bw = copy_bandwidth()
    traffic = pmc_traffic(args, chunk, last=PMC_LAUNCHES)
    limiter = pmc_limiter(args, chunk, PMC_LAUNCHES)
    if not args.no_cpu:
        progress("CPU baseline")
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_envs, args.cpu_steps)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": "synthetic: seeded uniform-random legal actions from the shipped basesWorkers16x16 map",
        "config": {
            "workload": f"{MAP}, VERSION_ORIGINAL_FINETUNED, CANCEL_RANDOM, partial_observability, "
                        f"{L} games, max_cycles 5000, auto-reset, fused rollout {chunk} cycles/launch, timed "
                        f"from cycle {MIDGAME + args.warmup} ({MIDGAME} untimed mid-game cycles + warmup)",
            "games": L, "slots_per_player": b.per_player_capacity, "entity_capacity": b.entity_capacity,
            "per_call_env_steps_per_s": None if pc_rate is None else round(pc_rate, 1),
            "copy_kernel_GBps": round(bw, 1),
            "algorithmic_bytes_per_env_step": per_step,
            "state_bytes_per_env": sbytes,
            "observation_ring_depth": args.depth,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": None if traffic is None else round(traffic["fetch_bytes"] + traffic["write_bytes"], 1),
            "kernel": rollout_kernels(env) if LAST_TWO_PASS else "k_rollout",
            "avg_launch_ms": round(avg_launch_s * 1e3, 4),
            "algorithmic_bytes_per_launch": per_launch_bytes,
            "cycles_per_launch": chunk,
        },
        "cpu_baseline": cpu,
    }
    if traffic is not None:
        line["roofline"]["traffic_detail"] = traffic
    if limiter is not None:
        # "bound" names the roofline the fraction is taken against (the path
        # runs no MFMA); the counters say what limits the kernel below it
        line["roofline"]["limiter"] = {
            **limiter, "hbm_frac": round(achieved / HBM_PEAK_GBPS, 4),
            "verdict": "VALU issue" if limiter["valu_busy"] > 2 * achieved / HBM_PEAK_GBPS else "HBM"}
    print(json.dumps(line))


if __name__ == "__main__":
    main()
