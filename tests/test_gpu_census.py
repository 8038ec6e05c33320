"""The step kernel's census build (stats mode 3) and the split kernel timing,
on the GPU through the C ABI.

The census build is the step kernel with per-wave ballot counters and shader
clock reads added.  It must leave every console exactly as the plain build
does (RAM, rewards, dones, the whole state of sampled consoles), and its
counters must satisfy what the loop's structure fixes: every wave that runs
the loop leaves it once, from the rare path; a count of wave-iterations with
an event is at most the iterations and at most the lanes with it; on a ROM
without idle loops every counted instruction is one active lane-iteration;
every console crosses at least one timing event per frame and captures its
presentation record once per step.  Both LDS layouts run (4,096 consoles,
all RAM in LDS; 16,384, split).  The timing test checks that the step and
restore kernels are timed apart and that the step kernel's time is what the
single-figure timing reports.
"""

from __future__ import annotations

import numpy as np
import pytest

from nesle_amd import abi, synthrom
from oracle import oracle as O
from tests.helpers import first_diff, masks_for, say, warm_snapshots

pytestmark = pytest.mark.gpu

FRAMESKIP = 4


def _batch(rom: bytes, n: int) -> abi.Batch:
    return abi.Batch(rom, n, FRAMESKIP, reward_kind=abi.REWARD_XDELTA, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI,
                     done_addr=synthrom.DONE_BYTE, clip=15, time_penalty=0.01)


def _check_census(c: dict, n: int, instructions: int, split: bool) -> None:
    it = c["iterations"]
    assert c["waves"] >= 1 and c["exits"] == c["waves"], c
    assert it >= c["waves"] and c["rare"] >= c["exits"], c
    for k in ("rare", "io_read", "dma", "present"):
        assert c[k] <= it, (k, c)
    for k in ("rare_io_write", "rare_side", "rare_idle", "rare_illegal", "rare_timing", "rare_budget",
              "rare_outside", "dma", "present"):
        assert c[k] <= c["rare"], (k, c)
    assert c["rare_only_io_write"] <= c["rare_io_write"] <= c["lanes_io_write"], c
    assert c["rare_timing"] <= c["lanes_timing"], c
    assert c["io_read_slow"] <= c["io_read"] <= c["lanes_io_read"], c
    assert c["io_read_slow"] <= c["lanes_io_read_slow"] <= c["lanes_io_read"], c
    # No idle loop on this ROM: each counted instruction is one active
    # lane-iteration (NMI entries are active iterations that count none).
    assert instructions <= c["active_lanes"] <= 64 * it, (instructions, c)
    assert c["lanes_timing"] >= FRAMESKIP * n, c          # at least the frame end of every frame
    assert c["present"] >= 1 and c["rare_idle"] == 0 and c["rare_illegal"] == 0, c
    assert 0 < c["distinct_samples"] <= it and c["distinct_entries"] <= 64 * c["distinct_samples"], c
    assert c["cycles_io_read"] <= c["cycles_loop"] and c["cycles_rare"] <= c["cycles_loop"], c
    parts = sum(c[k] for k in ("cycles_io_write", "cycles_settle", "cycles_dma", "cycles_present", "cycles_redo"))
    assert parts <= c["cycles_rare"], c
    if split:
        assert c["redo"] == c["rare"] - c["exits"], c      # the decode is redone after rare work that continues
    else:
        assert c["redo"] == 0 and c["cycles_redo"] == 0, c  # all RAM in LDS: decoded at the top of the iteration


@pytest.mark.parametrize("n", [4096, 16384])
def test_census_build_leaves_every_console_as_the_plain_build(n):
    rom = synthrom.make_rom(2026).rom
    say(f"[gpu] census vs plain build: N={n}")
    plain, census = _batch(rom, n), _batch(rom, n)
    for k in range(6):
        m = masks_for(71, n, k)
        plain.set_actions(m)
        census.set_actions(m)
        plain.step(auto_reset=True)
        census.step(auto_reset=True, stats_mode=3)
        c = census.census()
        instructions = int(census.host(abi.VIEW_INSTRUCTIONS).astype(np.uint64).sum())
        _check_census(c, n, instructions, split=n > 8192)
        for kind in (abi.VIEW_RAM, abi.VIEW_REWARDS, abi.VIEW_DONES):
            a, b = plain.host(kind), census.host(kind)
            assert np.array_equal(a, b), f"step {k} view {kind}: {first_diff(a, b)}"
    for e in sorted({0, 1, 63, 64, n // 2, n - 1}):
        a, b = plain.save_state(e), census.save_state(e)
        assert np.array_equal(a, b), f"console {e}: {first_diff(a, b)}"
    plain.close()
    census.close()


def test_census_counts_auto_resets_and_timing_split():
    """16,384 consoles from snapshots with short episodes: the census of steps
    in which consoles end episodes, and the step and restore kernels timed
    apart (the restore kernel only runs on auto-reset steps)."""
    rom = synthrom.make_rom(2026).rom
    snaps = warm_snapshots(rom, [40, 75], seed=71)
    done_byte = synthrom.DONE_BYTE
    for i, s in enumerate(snaps):
        s[O.OFF["ram"] + done_byte] = 1 + i      # the ROM counts it down every 8th frame: episodes of 1-16 frames
    n = 16384
    levels = (np.arange(n) % 2).astype(np.uint8)
    say(f"[gpu] census with auto-resets and timing split: N={n}")
    b = _batch(rom, n)
    b.set_snapshots([bytes(s) for s in snaps], levels)
    b.set_timing(True)
    dones = 0
    for k in range(8):
        b.set_actions(masks_for(72, n, k))
        b.step(auto_reset=True, stats_mode=3 if k % 2 else 0)
        dones += int(b.host(abi.VIEW_DONES).sum())
        if k % 2:
            _check_census(b.census(), n, int(b.host(abi.VIEW_INSTRUCTIONS).astype(np.uint64).sum()), split=True)
    b.synchronize()
    step_ms, reset_ms, launches = b.timing_split()
    ms, launches1 = b.timing()
    assert dones > 0
    assert launches == launches1 == 8
    assert ms == step_ms and step_ms > 0.0 and 0.0 < reset_ms < step_ms, (step_ms, reset_ms, ms)

    quiet = _batch(rom, 64)
    quiet.set_timing(True)
    for k in range(3):
        quiet.set_actions(masks_for(73, 64, k))
        quiet.step(auto_reset=False)
    quiet.synchronize()
    s_ms, r_ms, q_launches = quiet.timing_split()
    assert q_launches == 3 and s_ms > 0.0 and r_ms == 0.0, (s_ms, r_ms, q_launches)
    b.close()
    quiet.close()
