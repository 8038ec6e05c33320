"""Benchmark: env-steps/s (frame-skip 4) of the MI355X batched NROM console.

Workload (one GPU): 65,536 consoles on the
seeded synthetic NROM ROM, RAM observation, frame-skip 4, each console on its
own counter-based pad stream (one uniformly drawn mask per step, held for the
step's 4 frames); done fires when the ROM's countdown byte reaches 0 and the
console auto-resets from one of 8 snapshots captured after 100-800 seeded
warm-up frames (per-env level drawn uniformly); reward = clip(dx, -15, 15) -
0.01 on the ROM's 16-bit x position.  The 4,096-console configuration (no
resets) is timed in the same run and reported under "extra", and so is the
pixel-observation workload: 16,384 consoles on the status-bar variant of the
ROM (sprite-0 timed, IRQ-free mid-frame $2005 writes, so frames start and end
with different scrolls), each step followed by one render of every console's
84x84 gray observation into device memory (100 steps by default; the full
2,000 take ``--pixel-steps 2000``), and the GPU-resident PPO
workload: 8,192 consoles x 128 steps per update on the snapshot/x-delta setup,
RAM MLP policy (12-way action space, Xavier init), GAE and 4 epochs of
minibatch 8,192, with the step kernel's share of the update's wall time; and
the SB3/NumPy host path (``nesle_amd.env.NesleVecEnv`` at 4,096 consoles,
RAM observations copied to host every step).

Timed region: W untimed warm-up steps, synchronize, K timed steps of the
Python-level ``CudaBatch.step_device(actions[k], auto_reset=True)`` loop (the
reference's measurement harness shape), synchronize.  Inputs (ROM, snapshots,
the whole action table) are resident in HBM before timing starts.

Roofline: the step kernel's launches are timed with HIP events on the stream
it runs on.  The binding roof is integer VALU issue: ``roofline`` divides the
VALU lane-ops of one launch (SQ_THREAD_CYCLES_VALU, rocprofv3, committed in
profiles/step_kernel_65536_fs4.md) by the live kernel time and prices them
against 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz = 39.3e12 lane-ops/s; its
``traffic`` is the HBM bytes per launch from the same summary (FETCH_SIZE and
WRITE_SIZE, scaled by a copy-kernel calibration).  ``roofline_hbm`` prices
the algorithmic HBM bytes per env-step (RAM read+write 4,096 + OAM
read+write 512 + registers/PPU/reward scalars 128 + action 1 + reward/done 5
= 4,742 B) against 8 TB/s.  ``by_size`` repeats the figures, with NES
frames/s and the useful-lane fraction, for 4,096 and 65,536 consoles.

Resets while timed: each console's first episode starts at a seeded point of
its level's done countdown, so the timed window holds the steady auto-reset
rate; the dones of the timed steps are summed on the device and reported.
``reset_burst_65536`` times the same step with and without auto-reset on
two batches in the same state: a step of the workload, and burst steps in
which a whole level, or every console, ends its episode.

``cpu_baseline``: the reference's own CPU core (``nesle::Console`` compiled
from the reference sources into oracle/_ref) on the host's cores (the job's
CPU share), consoles split statically over std::threads, on a bounded sample
of the same workload: the first consoles of the 65,536 from their snapshots,
staggered done bytes, pad streams and auto-reset.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from nesle_amd import synthrom  # noqa: E402

ROM_SEED = 2026
ACTION_SEED = 0x5EED
SNAPSHOT_SEED = 77
STAGGER_SEED = 78
NUM_LEVELS = 8
TIME_PENALTY = 0.01
B_STEP = 4742                       # algorithmic HBM bytes per env-step
HBM_PEAK_GBS = 8000.0
VALU_PEAK_LANE_OPS = 256 * 4 * 16 * 2.4e9   # int32 lane-ops/s


PROFILE = ROOT / "profiles" / "step_kernel_65536_fs4.md"


def profile_figure(key: str, num_envs: int) -> float | None:
    """A machine-readable figure (``<key> <envs> <value>``) of the committed
    rocprofv3 summary, or None when the summary has none for this size."""
    if not PROFILE.exists():
        return None
    for line in PROFILE.read_text().splitlines():
        parts = line.split()
        if len(parts) == 3 and parts[0] == key and parts[1] == str(num_envs):
            return float(parts[2])
    return None


def size_figures(run: dict, num_envs: int) -> dict:
    """Throughput and roofline fractions of one batch size: NES frames/s,
    algorithmic and measured (rocprofv3, committed summary) HBM bytes per
    kernel time against the 8 TB/s peak, and the VALU pipe's busy fraction."""
    kernel_s = run["kernel_ms_per_launch"] / 1000.0
    algo = num_envs * B_STEP / kernel_s / 1e9
    traffic = profile_figure("traffic_bytes_per_launch", num_envs)
    measured = traffic / kernel_s / 1e9 if traffic else None
    lane_ops = profile_figure("valu_lane_ops_per_launch", num_envs)
    lanes = consoles_per_wave(num_envs)
    return {
        "num_envs": num_envs,
        "env_steps_per_s": run["env_steps_per_s"],
        "nes_frames_per_s": 4 * run["env_steps_per_s"],
        "kernel_ms_per_launch": run["kernel_ms_per_launch"],
        "emulated_instr_per_s": run["instructions_per_env_step"] * num_envs / kernel_s,
        "hbm_algorithmic_gbs": algo,
        "hbm_algorithmic_frac": algo / HBM_PEAK_GBS,
        "hbm_measured_gbs": measured,
        "hbm_measured_frac": measured / HBM_PEAK_GBS if measured else None,
        "valu_busy_frac": profile_figure("valu_busy", num_envs),
        "valu_lane_ops_frac": lane_ops / kernel_s / VALU_PEAK_LANE_OPS if lane_ops else None,
        "consoles_per_wave": lanes,
        # Lanes without a console run the datapath on a dummy block: only
        # lanes/64 of the VALU lane-ops serve a console.
        "useful_lane_frac": lanes / 64,
        "useful_valu_lane_ops_frac": lane_ops / kernel_s / VALU_PEAK_LANE_OPS * lanes / 64 if lane_ops else None,
    }


def consoles_per_wave(num_envs: int) -> int:
    """Consoles per wave64 of the step kernel's launch: the smallest power of
    two L (at most 64) with 1,024 waves x L >= num_envs (one wave per SIMD)."""
    lanes = 1
    while lanes < 64 and 1024 * lanes < num_envs:
        lanes *= 2
    return lanes


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_snapshots(core, rom: bytes, rng: np.random.Generator) -> tuple[list[bytes], list[int], list[int]]:
    """8 full-state snapshots after seeded warm-up frames (100-800) on the GPU,
    each with its done countdown re-drawn so done fires after 200-2,000 frames."""
    warm = sorted(int(w) for w in rng.integers(100, 801, NUM_LEVELS))
    done_vals = [int(v) for v in rng.integers(25, 251, NUM_LEVELS)]  # decremented every 8th frame
    b = core.CudaBatch(NUM_LEVELS, 1, rom)
    import torch

    slot = 0
    for f in range(warm[-1] + 1):
        while slot < NUM_LEVELS and warm[slot] == f:
            b.snapshot_capture(slot, slot)
            slot += 1
        if slot == NUM_LEVELS:
            break
        acts = torch.from_numpy(synthrom.action_masks(SNAPSHOT_SEED, NUM_LEVELS, f)).cuda()
        b.step_device(acts, auto_reset=False, synchronize=False)
    blobs = []
    for s in range(NUM_LEVELS):
        blob = bytearray(b.snapshot_export(s))
        blob[80 + synthrom.DONE_BYTE] = done_vals[s]
        blobs.append(bytes(blob))
    return blobs, warm, done_vals


def staggered_done(levels: np.ndarray, done_vals: list[int]) -> np.ndarray:
    """Each console's first episode starts at a seeded point of its level's
    countdown: done byte uniform in [1, the level's full count].  Consoles of
    a level then finish at different steps, and any window of steps holds the
    workload's steady reset rate (after a reset a console restarts from its
    level's full count)."""
    full = np.asarray(done_vals, dtype=np.int64)[levels]
    u = np.random.default_rng(STAGGER_SEED).random(levels.size)
    return (1 + np.floor(u * full)).astype(np.uint8)


def reward_spec() -> dict:
    return {"kind": "x_delta", "x_lo": synthrom.X_LO, "x_hi": synthrom.X_HI,
            "done_addr": synthrom.DONE_BYTE, "clip": 15, "time_penalty": TIME_PENALTY}


def run_gpu(core, rom: bytes, num_envs: int, steps: int, warmup: int, snapshots: list[bytes] | None,
            levels: np.ndarray | None, gray84: bool = False, done_init: np.ndarray | None = None) -> dict:
    import torch

    if snapshots is not None:
        batch = core.CudaBatch(num_envs, 4, rom, snapshots, levels, reward=reward_spec())
        if done_init is not None:
            batch.poke_ram_envs(synthrom.DONE_BYTE, done_init)
    else:
        batch = core.CudaBatch(num_envs, 4, rom, reward=reward_spec())
    batch.set_stream(torch.cuda.current_stream().cuda_stream)
    auto_reset = snapshots is not None
    table = torch.from_numpy(synthrom.action_table(ACTION_SEED, num_envs, warmup + steps)).cuda()
    # Dones of the timed steps, summed on the device (one elementwise add per step).
    dones = torch.from_dlpack(batch.last_done_device())
    done_count = torch.zeros(num_envs, dtype=torch.int32, device="cuda")

    def one_step(k: int) -> None:
        batch.step_device(table[k], auto_reset=auto_reset, synchronize=False)
        done_count.add_(dones)
        if gray84:
            batch.render_frames_device(rgb=False, palette=False, gray84=True)

    # The warm-up runs exactly the timed loop's body (every launch of it has
    # run once before timing starts), with the event timing on, whose event
    # objects are created by set_timing.
    batch.set_timing(True)
    for k in range(warmup):
        one_step(k)
    torch.cuda.synchronize()
    done_count.zero_()
    batch.set_timing(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(warmup, warmup + steps):
        one_step(k)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kernel_ms, reset_ms, launches = batch.kernel_timing_split()
    batch.set_timing(False)
    done_total = int(done_count.sum().item())
    # Exact emulated instruction count per env-step from one stats step.
    stats = batch.step_stats(synthrom.action_masks(ACTION_SEED, num_envs, warmup + steps))
    instr = np.asarray(stats["instructions"], dtype=np.float64)
    return {
        "num_envs": num_envs,
        "steps": steps,
        "seconds": elapsed,
        "env_steps_per_s": num_envs * steps / elapsed,
        "ms_per_step": 1000.0 * elapsed / steps,
        "kernel_ms_per_launch": kernel_ms / max(launches, 1),
        "restore_ms_per_launch": reset_ms / max(launches, 1),
        "kernels_ms_per_step": (kernel_ms + reset_ms) / max(launches, 1),
        "kernel_launches": launches,
        "instructions_per_env_step": float(instr.mean()),
        "dones_in_timed_window": done_total,
        "dones_per_step": done_total / steps,
    }


def run_reset_burst(core, rom: bytes, snapshots: list[bytes], levels: np.ndarray, done_vals: list[int],
                    done_init: np.ndarray, warmup: int = 40) -> dict:
    """What auto-reset costs a step, at 65,536 consoles: two batches in the
    same state take the same step, one with auto-reset and one without, and
    their step-kernel times (HIP events, one step per timing window) differ
    only by the resets.  Measured on a step of the benchmark workload itself
    (after ``warmup`` steps), and on burst steps in which every console of
    level 0 (1/8 of the batch), or every console, ends its episode: the ROM
    decrements the done byte in the NMI of every frame whose incremented
    frame counter is a multiple of 8, so poking the frame counter to 7 and
    the done byte to 1 makes the selected consoles done in the first frame
    of the next step (the others get 200)."""
    import torch

    n = levels.size
    pair = []
    for _ in range(2):
        b = core.CudaBatch(n, 4, rom, snapshots, levels, reward=reward_spec())
        b.poke_ram_envs(synthrom.DONE_BYTE, done_init)
        b.set_stream(torch.cuda.current_stream().cuda_stream)
        pair.append(b)
    table = torch.from_numpy(synthrom.action_table(ACTION_SEED, n, warmup + 8)).cuda()
    for k in range(warmup):
        for b in pair:
            b.step_device(table[k], auto_reset=True, synchronize=False)
    torch.cuda.synchronize()
    k = warmup

    def step_both() -> tuple[float, float, int]:
        """(ms with auto-reset, ms without, dones) of the same step; the
        batch without auto-reset then takes the same masked reset."""
        nonlocal k
        ms = []
        for b, ar in zip(pair, (True, False)):
            b.set_timing(True)
            b.step_device(table[k], auto_reset=ar, synchronize=False)
            torch.cuda.synchronize()
            step_ms, reset_ms, _ = b.kernel_timing_split()
            ms.append(step_ms + reset_ms)
            b.set_timing(False)
        dones = torch.from_dlpack(pair[1].last_done_device()).clone()
        pair[1].reset_envs_device(dones)
        k += 1
        return ms[0], ms[1], int(dones.to(torch.int64).sum().item())

    out = {"num_envs": n, "warmup_steps": warmup}
    steady = [step_both() for _ in range(3)]
    out["workload_steps"] = [{"with_reset_ms": a, "without_ms": w, "dones": d} for a, w, d in steady]
    for name, sel in (("level0", levels == 0), ("all", np.ones(n, dtype=bool))):
        vals = np.full(n, 200, dtype=np.uint8)
        vals[sel] = 1
        for b in pair:
            b.poke_ram(synthrom.FRAME_COUNTER, 7)
            b.poke_ram_envs(synthrom.DONE_BYTE, vals)
        a, w, d = step_both()
        assert d == int(sel.sum()), f"burst {name}: {d} dones, expected {int(sel.sum())}"
        out[f"burst_{name}"] = {"with_reset_ms": a, "without_ms": w, "dones": d, "ratio": a / w}
    out["workload_ratio"] = float(np.mean([a / w for a, w, _ in steady]))
    return out


def run_vec_env(rom: bytes, steps: int) -> dict:
    """The SB3/NumPy host path: NesleVecEnv.step with host action indices,
    RAM observations, rewards and dones copied to host NumPy every step,
    auto-reset with terminal observations (12-way action space, episodes cut
    at 500 steps)."""
    from nesle_amd.env import NesleVecEnv

    n = 4096
    env = NesleVecEnv("synthetic.nes", n, frameskip=4, action_space="complex", observation_mode="ram",
                      max_episode_steps=500, rom_bytes=rom)
    env.reset()
    acts = np.random.default_rng(ACTION_SEED).integers(0, 12, (steps + 5, n))
    for k in range(5):
        env.step(acts[k])
    t0 = time.perf_counter()
    for k in range(5, steps + 5):
        env.step(acts[k])
    dt = time.perf_counter() - t0
    return {"num_envs": n, "steps": steps, "seconds": dt, "env_steps_per_s": n * steps / dt,
            "ms_per_step": 1000.0 * dt / steps}


def run_ppo(rom: bytes, snapshots: list[bytes], updates: int) -> dict:
    """GPU-resident PPO on the snapshot/x-delta setup: 8,192 consoles x 128
    steps per update, MLP on RAM, 12-way action space, Xavier init, GAE
    (0.99, 0.95), 4 epochs of minibatch 8,192.  Figures are the last update's
    (the first also pays library warm-up)."""
    from nesle_amd import native_ppo as P

    n = 8192
    reward = {"kind": "x_delta", "x_lo": synthrom.X_LO, "x_hi": synthrom.X_HI,
              "done_addr": synthrom.DONE_BYTE, "clip": 15, "time_penalty": TIME_PENALTY}
    levels = np.random.default_rng(SNAPSHOT_SEED + 1).integers(0, NUM_LEVELS, n)
    cfg = P.NativePPOConfig("synthetic.nes", num_envs=n, total_timesteps=n * 128 * updates, n_steps=128,
                            batch_size=8192, update_epochs=4, frameskip=4, action_space="complex", init="xavier",
                            reward=reward, save_checkpoints=False, seed=1, log_interval=1000,
                            env_to_level=tuple(int(x) for x in levels))
    import contextlib

    with contextlib.redirect_stdout(sys.stderr):   # stdout carries only the result line
        stats = P.train_native_ppo(cfg, rom_bytes=rom, snapshot_bytes=snapshots)
    last = stats["per_update"][-1]
    wall = last["rollout_s"] + last["update_s"]
    return {
        "num_envs": n, "n_steps": 128, "updates": stats["updates"],
        "rollout_s": last["rollout_s"], "update_s": last["update_s"], "emulator_s": last["emulator_s"],
        "env_steps_per_s": n * 128 / wall,
        "rollout_env_steps_per_s": n * 128 / last["rollout_s"],
        "emulator_share": last["emulator_s"] / wall,
        "episodes": stats["log"][-1]["episodes"],
    }


def cpu_share() -> tuple[int, dict]:
    """Threads for the CPU baseline: every CPU this process may run on, unless
    the host grants the job a smaller CPU share through OMP_NUM_THREADS (a
    one-GPU box gives one GPU's job 16 CPUs; threads beyond the share only
    time-slice).  Returns the count and what it was derived from."""
    nproc = os.cpu_count() or 1
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        affinity = nproc
    share = os.environ.get("OMP_NUM_THREADS", "")
    threads = affinity
    if share.isdigit() and 0 < int(share) < affinity:
        threads = int(share)
    return threads, {"nproc": nproc, "affinity": affinity, "omp_num_threads": share or None}


def cpu_baseline(rom: bytes, snaps: list[bytes], levels: np.ndarray, done_init: np.ndarray,
                 target_seconds: float) -> dict | None:
    """The reference's CPU core on the benchmark's own workload: the first
    consoles of the 65,536 (same snapshot levels, staggered done bytes, pad
    streams), auto-reset from the level's snapshot whenever the done byte
    reaches 0, consoles split statically over std::threads."""
    try:
        from oracle import oracle as O
    except Exception as exc:  # pragma: no cover
        log(f"cpu baseline unavailable: {exc}")
        return None
    kind = "reference" if O.ref_available() else "port"
    threads, share = cpu_share()
    envs = 8 * threads
    lv, di = levels[:envs], done_init[:envs]
    # Calibrate on a short run, then size the sample to ~target_seconds.
    secs, _, _, _ = O.run_levels(rom, snaps, lv, di, synthrom.DONE_BYTE, 10, 4, ACTION_SEED, 0, threads, kind=kind)
    steps = max(50, int(target_seconds * envs * 10 / secs / envs))
    secs, _, instr, resets = O.run_levels(rom, snaps, lv, di, synthrom.DONE_BYTE, steps, 4, ACTION_SEED, 0,
                                          threads, kind=kind)
    value = envs * steps / secs
    return {
        "value": value,
        "unit": "env-steps/s",
        "cores": threads,
        "kind": kind,
        "sample": f"consoles 0-{envs - 1} of the 65,536-console workload x {steps} env-steps (frame-skip 4) from "
                  f"their snapshots with the staggered done bytes, auto-reset on done ({resets} resets), same pad "
                  f"streams, {threads} std::threads, {secs:.1f} s",
        "per_core": value / threads,
        "instructions_per_env_step": instr / (envs * steps),
        "cpu_model": _cpu_model(),
        "build": "g++ 11 -O3 -march=x86-64-v3 (oracle/Makefile: built beside the GPU code and shipped with it, "
                 "so the ISA level is fixed rather than -march=native of the machine that runs it)",
        **share,
    }


def _cpu_model() -> str:
    """Model name, family/model/stepping and clock of the host CPU from
    /proc/cpuinfo (some hosts report only the vendor in the model name)."""
    try:
        info = {}
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, value = line.partition(":")
            key = key.strip()
            if key in ("model name", "cpu family", "model", "stepping", "cpu MHz") and key not in info:
                info[key] = value.strip()
        if info:
            return (f"{info.get('model name', '?')} (family {info.get('cpu family', '?')}, model "
                    f"{info.get('model', '?')}, stepping {info.get('stepping', '?')}, {info.get('cpu MHz', '?')} MHz)")
    except OSError:
        pass
    return "unknown"


def run_census(rom: bytes, snaps: list[bytes], levels: np.ndarray | None, done_init: np.ndarray | None,
               num_envs: int, steps: int, warmup: int) -> dict:
    """The step kernel's census (stats mode 3) over ``steps`` steps of a
    workload, after ``warmup`` ordinary steps: per wave-iteration, how often
    a wave takes the rare path and why, the I/O read side path, OAM DMA and
    the presentation capture, active lanes and distinct microcode entries,
    and the shader cycles in the loop, the rare path and the I/O read path.
    With ``snaps`` the 65,536-console workload's snapshot levels, staggered
    done bytes and auto-reset; without, the 4,096-console one (no resets).
    Also times the same steps without the census (HIP events) to relate
    cycles to time."""
    from nesle_amd import abi

    b = abi.Batch(rom, num_envs, 4, reward_kind=abi.REWARD_XDELTA, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI,
                  done_addr=synthrom.DONE_BYTE, clip=15, time_penalty=TIME_PENALTY)
    auto_reset = snaps is not None
    if auto_reset:
        b.set_snapshots(snaps, levels)
        b.poke_ram_envs(synthrom.DONE_BYTE, done_init)
    for k in range(warmup):
        b.set_actions(synthrom.action_masks(ACTION_SEED, num_envs, k))
        b.step(auto_reset=auto_reset)
    totals: dict[str, int] = {}
    ms_plain = []
    for k in range(warmup, warmup + steps):
        b.set_actions(synthrom.action_masks(ACTION_SEED, num_envs, k))
        b.set_timing(True)
        b.step(auto_reset=auto_reset, stats_mode=3)
        b.synchronize()
        census_ms = b.timing()[0]
        for name, value in b.census().items():
            totals[name] = totals.get(name, 0) + value
        totals["census_kernel_us"] = totals.get("census_kernel_us", 0) + int(1000 * census_ms)
        instr = b.host(abi.VIEW_INSTRUCTIONS).astype(np.float64)
        totals["instructions"] = totals.get("instructions", 0) + int(instr.sum())
    # The same number of ordinary steps, timed, for the kernel's plain speed.
    for k in range(warmup + steps, warmup + 2 * steps):
        b.set_actions(synthrom.action_masks(ACTION_SEED, num_envs, k))
        b.set_timing(True)
        b.step(auto_reset=auto_reset)
        b.synchronize()
        ms_plain.append(b.timing()[0])
    b.close()
    it = max(totals["iterations"], 1)
    per_it = {k: totals[k] / it for k in totals if k not in ("waves", "iterations", "census_kernel_us",
                                                             "instructions", "distinct_entries", "distinct_samples")}
    per_it["distinct_entries"] = totals["distinct_entries"] / max(totals["distinct_samples"], 1)
    waves = max(totals["waves"], 1)
    plain_ms = float(np.mean(ms_plain))
    return {
        "num_envs": num_envs, "steps": steps, "warmup": warmup, "totals": totals,
        "per_wave_iteration": per_it,
        "wave_iterations_per_wave_per_step": totals["iterations"] / waves,
        "cycles_per_wave_iteration": totals["cycles_loop"] / it,
        "rare_cycles_per_rare_iteration": totals["cycles_rare"] / max(totals["rare"], 1),
        "io_read_cycles_per_io_iteration": totals["cycles_io_read"] / max(totals["io_read"], 1),
        "census_kernel_ms": totals["census_kernel_us"] / 1000.0 / steps,
        "plain_kernel_ms": plain_ms,
        "instructions_per_env_step": totals["instructions"] / (num_envs * steps),
    }


def copy_calibration(mib: int) -> int:
    """A plain device-to-device copy of known size: each dispatch reads and
    writes exactly ``mib`` MiB, so rocprof's per-dispatch FETCH_SIZE and
    WRITE_SIZE for it give the counters' scale on this GPU."""
    import torch

    src = torch.ones(mib << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": mib << 20, "dispatches": 5}))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--envs", type=int, default=65536)
    ap.add_argument("--small-envs", type=int, default=4096)
    ap.add_argument("--small-steps", type=int, default=200)
    ap.add_argument("--pixel-envs", type=int, default=16384)
    ap.add_argument("--pixel-steps", type=int, default=100)
    ap.add_argument("--vec-steps", type=int, default=50,
                    help="steps of the SB3/NumPy vector env (4,096 consoles, RAM observations on the host; 0 skips)")
    ap.add_argument("--ppo-updates", type=int, default=2,
                    help="PPO updates of 8,192 consoles x 128 steps (the first warms up; 0 skips)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-burst", dest="burst", action="store_false",
                    help="skip the single-step reset-burst timings")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB device-to-device 5 times (scales rocprof FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--census", type=int, default=0, metavar="STEPS",
                    help="only print the step kernel's census (stats mode 3) over STEPS steps of the 65,536- and "
                         "4,096-console workloads")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; the consoles shard trivially "
                                   "across GPUs but no multi-GPU figure is produced (--gpus 1)"}))
        return 2

    import torch

    from nesle_amd import load_cuda_core

    core = load_cuda_core()
    if not torch.cuda.is_available():
        log("no GPU visible")
        return 1
    rom = synthrom.make_rom(ROM_SEED).rom
    rng = np.random.default_rng(SNAPSHOT_SEED)
    log("capturing snapshot bank")
    snaps, warm, done_vals = make_snapshots(core, rom, rng)
    levels = rng.integers(0, NUM_LEVELS, args.envs).astype(np.uint8)
    done_init = staggered_done(levels, done_vals)

    if args.census:
        out = {"census": [run_census(rom, snaps, levels, done_init, args.envs, args.census, args.warmup),
                          run_census(rom, None, None, None, args.small_envs, args.census, max(5, args.warmup // 4))]}
        print(json.dumps(out))
        return 0

    log(f"timing {args.envs} envs x {args.steps} steps (warmup {args.warmup})")
    big = run_gpu(core, rom, args.envs, args.steps, args.warmup, snaps, levels, done_init=done_init)
    log(f"  {big['env_steps_per_s']:.0f} env-steps/s, {big['ms_per_step']:.2f} ms/step: step kernel "
        f"{big['kernel_ms_per_launch']:.2f} ms + restore {big['restore_ms_per_launch']:.3f} ms, "
        f"{big['dones_in_timed_window']} auto-resets while timed")
    burst = None
    if args.burst:
        log("reset bursts: single-step kernel times")
        burst = run_reset_burst(core, rom, snaps, levels, done_vals, done_init)
        log(f"  step with/without auto-reset: workload x{burst['workload_ratio']:.4f}, level burst "
            f"x{burst['burst_level0']['ratio']:.4f}, every console x{burst['burst_all']['ratio']:.4f}")
    log(f"timing {args.small_envs} envs x {args.small_steps} steps (no resets)")
    small = run_gpu(core, rom, args.small_envs, args.small_steps, max(5, args.warmup // 4), None, None)
    log(f"  {small['env_steps_per_s']:.0f} env-steps/s")
    vec = None
    if args.vec_steps > 0:
        log(f"SB3 vector env: 4096 envs x {args.vec_steps} steps, RAM observations to host")
        vec = run_vec_env(rom, args.vec_steps)
        log(f"  {vec['env_steps_per_s']:.0f} env-steps/s")
    ppo = None
    if args.ppo_updates > 0:
        log(f"PPO: 8192 envs x 128 steps, {args.ppo_updates} updates")
        ppo = run_ppo(rom, snaps, args.ppo_updates)
        log(f"  {ppo['env_steps_per_s']:.0f} env-steps/s end to end, emulator share {ppo['emulator_share']:.2f}")
    pixel = None
    if args.pixel_steps > 0:
        log(f"timing {args.pixel_envs} envs x {args.pixel_steps} steps with an 84x84 gray frame per step")
        pixel = run_gpu(core, synthrom.make_rom(ROM_SEED, split=True).rom, args.pixel_envs, args.pixel_steps,
                        max(5, args.warmup // 4), None, None, gray84=True)
        pixel["rom"] = "status-bar variant of the seed-2026 ROM (sprite-0 timed mid-frame $2005 writes)"
        log(f"  {pixel['env_steps_per_s']:.0f} env-steps/s (pixel observations)")

    kernel_s = big["kernel_ms_per_launch"] / 1000.0
    hbm_achieved = args.envs * B_STEP / kernel_s / 1e9
    instr_rate = big["instructions_per_env_step"] * args.envs / kernel_s
    lane_ops = profile_figure("valu_lane_ops_per_launch", args.envs)
    valu_achieved = lane_ops / kernel_s / 1e12 if lane_ops else None
    result = {
        "metric": "env-steps/s (frameskip 4)",
        "value": big["env_steps_per_s"],
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": big["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic (seeded NROM ROM, seeded pad streams)",
        "config": {
            "workload": "65,536 consoles, synthetic NROM ROM seed 2026, RAM obs, frame-skip 4, auto-reset from "
                        "8 snapshots, x-delta reward",
            "num_envs": args.envs,
            "frameskip": 4,
            "snapshot_warmup_frames": warm,
            "done_countdown": done_vals,
        },
        "nes_frames_per_s": 4 * big["env_steps_per_s"],
        "roofline": {
            "bound": "valu",
            "achieved": valu_achieved,
            "peak": VALU_PEAK_LANE_OPS / 1e12,
            "unit": "T int32 lane-ops/s",
            "frac": valu_achieved * 1e12 / VALU_PEAK_LANE_OPS if valu_achieved else None,
            "traffic": profile_figure("traffic_bytes_per_launch", args.envs),
            "source": "achieved = SQ_THREAD_CYCLES_VALU per launch (= SQ_INSTS_VALU x 64 x VALU utilisation, "
                      "rocprofv3, profiles/step_kernel_65536_fs4.md) / step-kernel time per launch (HIP events, "
                      "this run); peak = 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz; traffic = HBM bytes per launch "
                      "(FETCH_SIZE x2.000 + WRITE_SIZE x1.000, same summary)",
            "kernel_ms_per_launch": big["kernel_ms_per_launch"],
            "restore_ms_per_launch": big["restore_ms_per_launch"],
            "window_over_kernels": big["ms_per_step"] / big["kernels_ms_per_step"] - 1.0,
            "emulated_instr_per_s": instr_rate,
            "instructions_per_env_step": big["instructions_per_env_step"],
            "valu_busy_frac": profile_figure("valu_busy", args.envs),
        },
        "roofline_hbm": {
            "achieved": hbm_achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": hbm_achieved / HBM_PEAK_GBS,
            "algorithmic_bytes_per_env_step": B_STEP,
            "measured_bytes_per_env_step": (profile_figure("traffic_bytes_per_launch", args.envs) or 0) / args.envs
            or None,
        },
        "by_size": [size_figures(small, args.small_envs), size_figures(big, args.envs)],
        "extra": {"envs_4096": small, "envs_65536": big, "pixels_16384_gray84": pixel, "ppo_8192x128": ppo,
                  "vec_env_ram_4096": vec, "reset_burst_65536": burst},
    }
    if not args.no_cpu_baseline:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(rom, snaps, levels, done_init, args.cpu_seconds)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
