"""Parity of the HIP batch (called through the C ABI) with the oracle and the
reference's golden per-frame hashes.

Bar: bit-exact canonical state (22,896 bytes per console: CPU registers and
cycle counter, PPU registers and frame position, pads, $4000-$4017, RAM, PRG
RAM, OAM, palette, nametables), identical instruction counts, identical
rewards (float32 built from integers, compared exactly) and done flags.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from nesle_amd import abi, synthrom
from oracle import oracle as O
from tests.helpers import OracleBatch, first_diff, masks_for, say, warm_snapshots

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _rom(seed: int) -> bytes:
    return synthrom.make_rom(seed).rom


@pytest.mark.parametrize("rom_seed", [1, 2, 3])
def test_single_env_matches_reference_golden(rom_seed):
    """Config 1: one console, frame-skip 1, 600 frames, seeded pad byte per frame;
    every recorded frame's section hashes equal the reference core's."""
    fx = json.loads((GOLDEN / f"console_rom{rom_seed}.json").read_text())
    rom = _rom(rom_seed)
    assert f"{O.fnv1a(rom):016x}" == fx["rom_fnv1a"]
    say(f"[gpu] golden rom{rom_seed}: N=1 fs=1 {fx['frames']} frames")
    b = abi.Batch(rom, 1, frameskip=1)
    recs = {r[0]: r for r in fx["records"]}
    cols = fx["columns"]
    checked = 0
    for k in range(fx["frames"]):
        b.set_actions(synthrom.action_masks(fx["action_seed"], 1, k))
        b.step(stats_mode=1)
        rec = recs.get(k + 1)
        if rec is None:
            continue
        state = b.save_state(0)
        got = O.section_hashes(state)
        assert int(b.host(abi.VIEW_INSTRUCTIONS)[0]) == rec[1], f"frame {k + 1} instruction count"
        for name in cols[2:]:
            assert f"{got[name]:016x}" == rec[cols.index(name)], f"frame {k + 1} section {name}"
        checked += 1
    assert checked == len(fx["records"])


def test_many_envs_match_oracle_frameskip4():
    """64 consoles, each on its own pad stream, frame-skip 4, 30 steps: full
    state, rewards, dones and instruction counts equal the oracle's per step."""
    rom = _rom(7)
    n, steps, seed = 64, 30, 77
    say(f"[gpu] many envs: N={n} fs=4 steps={steps}")
    b = abi.Batch(rom, n, frameskip=4)
    ob = OracleBatch(rom, list(range(n)))
    for k in range(steps):
        m = masks_for(seed, n, k)
        b.set_actions(m)
        b.step(stats_mode=1)
        ins, rew, don = ob.step(m, 4)
        np.testing.assert_array_equal(b.host(abi.VIEW_INSTRUCTIONS), ins, err_msg=f"step {k}")
        np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS), rew, err_msg=f"step {k}")
        np.testing.assert_array_equal(b.host(abi.VIEW_DONES), don, err_msg=f"step {k}")
        if k % 10 == 9 or k == steps - 1:
            for e, ref in enumerate(ob.states()):
                got = b.save_state(e)
                assert np.array_equal(got, ref), f"step {k} env {e}: {first_diff(got, ref)}"
    ram = b.host(abi.VIEW_RAM)
    for e, ref in enumerate(ob.states()):
        assert np.array_equal(ram[e], ref[O.OFF["ram"]:O.OFF["ram"] + 2048]), f"RAM view env {e}"


@pytest.mark.parametrize("num_envs,steps", [(4096, 4), (65536, 2)])
def test_full_size_sampled_envs(num_envs, steps):
    """At the benchmark sizes, sampled consoles (first, last, random) equal the
    oracle run on their own pad streams; duplicated pad streams give identical
    consoles (determinism across lanes, waves and XCDs)."""
    rom = _rom(11)
    seed = 1234
    rng = np.random.default_rng(num_envs)
    sample = sorted({0, 1, 63, 64, num_envs - 1, *rng.integers(0, num_envs, 6).tolist()})
    say(f"[gpu] full size: N={num_envs} fs=4 steps={steps} sample={sample}")
    b = abi.Batch(rom, num_envs, frameskip=4)
    ob = OracleBatch(rom, sample)
    for k in range(steps):
        m = masks_for(seed, num_envs, k)
        m[num_envs // 2] = m[3]  # twin of env 3
        b.set_actions(m)
        b.step(stats_mode=1)
        ins, rew, don = ob.step(m, 4)
        got_ins = b.host(abi.VIEW_INSTRUCTIONS)
        np.testing.assert_array_equal(got_ins[sample], ins)
        np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS)[sample], rew)
    for e, ref in zip(sample, ob.states()):
        got = b.save_state(e)
        assert np.array_equal(got, ref), f"env {e}: {first_diff(got, ref)}"
    assert np.array_equal(b.save_state(3), b.save_state(num_envs // 2))
    frames = b.host(abi.VIEW_FRAMES)
    assert (frames == 4).all()
    assert (b.host(abi.VIEW_BUDGET_HITS) == 0).all()


@pytest.mark.parametrize("num_envs", [1, 100, 12345, 30001, 50001])
def test_ragged_batch_sizes_sampled(num_envs):
    """Batch sizes that fill no whole wave or workgroup: 1 and 100 consoles
    (all RAM in LDS), 12,345 and 30,001 (16 and 32 consoles a wave, the
    split-layout kernel built for narrow waves) and 50,001 (64 a wave, the
    last wave holding 17).  Sampled consoles, the last one always among them,
    equal the oracle over 3 steps (instruction counts and rewards every step,
    state at the end)."""
    rom = _rom(13)
    rng = np.random.default_rng(num_envs)
    sample = sorted({0, num_envs - 1, *(rng.integers(0, num_envs, 6).tolist() if num_envs > 1 else [])})
    say(f"[gpu] ragged size: N={num_envs} fs=4 sample={sample}")
    b = abi.Batch(rom, num_envs, frameskip=4)
    ob = OracleBatch(rom, sample)
    for k in range(3):
        m = masks_for(4321, num_envs, k)
        b.set_actions(m)
        b.step(stats_mode=1)
        ins, rew, _ = ob.step(m, 4)
        np.testing.assert_array_equal(b.host(abi.VIEW_INSTRUCTIONS)[sample], ins, err_msg=f"step {k}")
        np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS)[sample], rew, err_msg=f"step {k}")
    for e, ref in zip(sample, ob.states()):
        got = b.save_state(e)
        assert np.array_equal(got, ref), f"env {e}: {first_diff(got, ref)}"
    assert (b.host(abi.VIEW_FRAMES) == 4).all()


def test_kernel_builds_agree_across_batch_sizes():
    """The production step kernel (no statistics, no frame budget) comes from
    three builds with different scheduler flags: all RAM in LDS (up to 8,192
    consoles), the split layout at 16 or 32 consoles per wave (16,384 and
    32,768) and at 64 (65,536).  The first 8,192 consoles of each batch, given
    the same pads, end every one of 4 steps with identical rewards and done
    flags, and the last with identical RAM (all 8,192) and canonical state (a
    sample).  The statistics counters, which only statistics steps write,
    read zero after these steps."""
    rom = _rom(13)
    sizes = (8192, 16384, 32768, 65536)
    n0 = sizes[0]
    masks = [masks_for(777, sizes[-1], k) for k in range(4)]
    sample = [0, 1, 63, 64, 4095, n0 - 1]
    ref = None
    for n in sizes:
        say(f"[gpu] kernel builds agree: N={n} fs=4 steps=4")
        b = abi.Batch(rom, n, frameskip=4, reward_kind=abi.REWARD_XDELTA, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI,
                      done_addr=synthrom.DONE_BYTE, clip=15, time_penalty=0.25)
        per_step = []
        for k in range(4):
            b.set_actions(masks[k][:n])
            b.step()
            per_step.append((b.host(abi.VIEW_REWARDS)[:n0].copy(), b.host(abi.VIEW_DONES)[:n0].copy()))
        # Steps without statistics leave the per-console counters as created: zero.
        assert not b.host(abi.VIEW_FRAMES).any() and not b.host(abi.VIEW_INSTRUCTIONS).any()
        got = (per_step, b.host(abi.VIEW_RAM)[:n0].copy(), [b.save_state(e) for e in sample])
        del b
        if ref is None:
            assert len({row.tobytes() for row in got[1][:256]}) > 1   # the pads made the consoles diverge
            ref = got
            continue
        for k, ((r0, d0), (r1, d1)) in enumerate(zip(ref[0], got[0])):
            np.testing.assert_array_equal(r1, r0, err_msg=f"N={n} step {k} rewards")
            np.testing.assert_array_equal(d1, d0, err_msg=f"N={n} step {k} dones")
        np.testing.assert_array_equal(got[1], ref[1], err_msg=f"N={n} RAM")
        for e, a, c in zip(sample, ref[2], got[2]):
            assert np.array_equal(c, a), f"N={n} env {e}: {first_diff(c, a)}"


def test_snapshot_autoreset_xdelta_reward():
    """Config 3 in miniature: 8 snapshots captured after seeded warm-up frames,
    done byte patched so episodes end within the run, x-delta reward with time
    penalty, auto-reset; rewards, dones and post-reset states equal the
    oracle restoring the same snapshot."""
    rom_info = synthrom.make_rom(5)
    rom = rom_info.rom
    warm = [100, 150, 200, 250, 300, 350, 400, 450]
    say("[gpu] snapshot bank: warm-up capture of 8 levels")
    snaps = warm_snapshots(rom, warm, seed=55)
    for i, s in enumerate(snaps):
        s[O.OFF["ram"] + synthrom.DONE_BYTE] = 1 + i  # done after 8*(1+i) frames at most
    blobs = [bytes(s) for s in snaps]
    n, steps = 64, 40
    levels = (np.arange(n) % 8).astype(np.uint8)
    reward = dict(kind=1, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI, done_addr=synthrom.DONE_BYTE, clip=15,
                  time_penalty=0.25)
    say(f"[gpu] snapshot auto-reset: N={n} fs=4 steps={steps}")
    b = abi.Batch(rom, n, frameskip=4, reward_kind=abi.REWARD_XDELTA, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI,
                  done_addr=synthrom.DONE_BYTE, clip=15, time_penalty=0.25)
    b.set_snapshots(blobs, levels)
    ob = OracleBatch(rom, list(range(n)), reward=reward)
    for e, c in enumerate(ob.cons):
        c.load(snaps[levels[e]])
    for e, ref in enumerate(ob.states()):
        assert np.array_equal(b.save_state(e), ref), f"initial env {e}"
    total_done = 0
    for k in range(steps):
        m = masks_for(99, n, k)
        b.set_actions(m)
        b.step(auto_reset=True)
        _, rew, don = ob.step(m, 4)
        np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS), rew, err_msg=f"step {k}")
        np.testing.assert_array_equal(b.host(abi.VIEW_DONES), don, err_msg=f"step {k}")
        for e in np.nonzero(don)[0]:
            ob.cons[e].load(snaps[levels[e]])
        total_done += int(don.sum())
        if k % 8 == 7:
            for e, ref in enumerate(ob.states()):
                got = b.save_state(e)
                assert np.array_equal(got, ref), f"step {k} env {e}: {first_diff(got, ref)}"
    assert total_done > n  # every env finished at least one episode
    assert (np.unique(b.host(abi.VIEW_REWARDS)) <= 15 - 0.25).all()


def test_benchmark_configuration_full_size_sampled():
    """The benchmark's configuration at full size: 65,536 consoles (RAM rows
    split between LDS and HBM), 8 snapshot levels spread at random, x-delta
    reward with time penalty and auto-reset.  Sampled consoles (edges of
    waves, workgroups and XCD ranges, random ones) have the rewards and dones
    of the oracle restoring the same snapshot after every step, and its state
    every third step; episodes end within the run."""
    rom = synthrom.make_rom(5).rom
    snaps = warm_snapshots(rom, [100, 150, 200, 250, 300, 350, 400, 450], seed=55)
    for i, s in enumerate(snaps):
        s[O.OFF["ram"] + synthrom.DONE_BYTE] = 1 + (i % 3)  # done after at most 3 frames x 8
    blobs = [bytes(s) for s in snaps]
    n, steps = 65536, 9
    rng = np.random.default_rng(2026)
    levels = rng.integers(0, 8, n).astype(np.uint8)
    sample = sorted({0, 1, 63, 64, 255, 256, 8191, 8192, 32768, n - 1, *rng.integers(0, n, 8).tolist()})
    reward = dict(kind=1, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI, done_addr=synthrom.DONE_BYTE, clip=15,
                  time_penalty=0.01)
    say(f"[gpu] benchmark configuration: N={n} fs=4 steps={steps} sample={sample}")
    b = abi.Batch(rom, n, frameskip=4, reward_kind=abi.REWARD_XDELTA, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI,
                  done_addr=synthrom.DONE_BYTE, clip=15, time_penalty=0.01)
    b.set_snapshots(blobs, levels)
    ob = OracleBatch(rom, sample, reward=reward)
    for e, c in zip(sample, ob.cons):
        c.load(snaps[levels[e]])
    ends = 0
    for k in range(steps):
        m = masks_for(4242, n, k)
        b.set_actions(m)
        b.step(auto_reset=True)
        _, rew, don = ob.step(m, 4)
        np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS)[sample], rew, err_msg=f"step {k} rewards")
        np.testing.assert_array_equal(b.host(abi.VIEW_DONES)[sample], don, err_msg=f"step {k} dones")
        for j in np.nonzero(don)[0]:
            ob.cons[j].load(snaps[levels[sample[j]]])
        ends += int(don.sum())
        if k % 3 == 2:
            for e, ref in zip(sample, ob.states()):
                got = b.save_state(e)
                assert np.array_equal(got, ref), f"step {k} env {e}: {first_diff(got, ref)}"
    assert ends >= len(sample)


def test_largest_batch_sampled():
    """The largest batch, NESLE_MAX_ENVS = 262,144 consoles: 1,024 workgroups
    of 256 consoles, four to a compute unit in turn, and RAM/PRG-RAM offsets up
    to 2.7e9.  Sampled consoles at workgroup-round and range edges equal the
    oracle (instruction counts and rewards every step, state and 84x84 gray
    frame at the end)."""
    rom = _rom(2026)
    n = abi.MAX_ENVS
    rng = np.random.default_rng(11)
    sample = sorted({0, 255, 256, 65535, 65536, 131071, 131072, 196607, 196608, n - 257, n - 256, n - 1,
                     *rng.integers(0, n, 8).tolist()})
    say(f"[gpu] largest batch: N={n} fs=4 sample={sample}")
    b = abi.Batch(rom, n, frameskip=4)
    ob = OracleBatch(rom, sample)
    for k in range(4):
        m = masks_for(99, n, k)
        b.set_actions(m)
        b.step(stats_mode=1)
        ins, rew, _ = ob.step(m, 4)
        np.testing.assert_array_equal(b.host(abi.VIEW_INSTRUCTIONS)[sample], ins, err_msg=f"step {k}")
        np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS)[sample], rew, err_msg=f"step {k}")
    for e, ref in zip(sample, ob.states()):
        got = b.save_state(e)
        assert np.array_equal(got, ref), f"env {e}: {first_diff(got, ref)}"
    # One render of the whole batch (262,144 workgroups, gray offsets up to
    # 1.8e9): the sampled consoles' 84x84 gray frames equal the oracle's.
    b.render(abi.FRAME_GRAY84)
    gray = b.host(abi.VIEW_GRAY84)
    for e, con in zip(sample, ob.cons):
        assert np.array_equal(gray[e], O.gray84(con.render(snapshot=True))), f"env {e}: gray84"
    b.close()


def test_benchmark_workload_long_run_full_size_sampled():
    """The benchmark workload over a longer run: 65,536 consoles on the
    benchmark ROM (seed 2026), 8 snapshot levels, a staggered done countdown
    poked into every console (episodes end throughout the run, as in the
    timed window of the benchmark), x-delta reward and auto-reset, 40 steps.
    64 sampled consoles (wave, workgroup and XCD-range edges, random ones)
    have the oracle's rewards and dones at every step and its state every
    eighth step; many episodes end and restart from snapshots meanwhile."""
    rom = synthrom.make_rom(2026).rom
    snaps = warm_snapshots(rom, [141, 270, 334, 486, 544, 650, 657, 706], seed=78)
    for i, s in enumerate(snaps):
        s[O.OFF["ram"] + synthrom.DONE_BYTE] = 2 + 2 * i   # episodes of 16-128 frames from a snapshot
    blobs = [bytes(s) for s in snaps]
    n, steps = 65536, 40
    rng = np.random.default_rng(79)
    levels = rng.integers(0, 8, n).astype(np.uint8)
    done_init = rng.integers(1, 13, n).astype(np.uint8)   # first episode ends within 24 steps
    edges = {0, 1, 63, 64, 255, 256, 1023, 1024, 8191, 8192, 16383, 16384, 32767, 32768, 65279, 65280, n - 1}
    sample = sorted(edges | set(rng.integers(0, n, 64 - len(edges)).tolist()))
    reward = dict(kind=1, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI, done_addr=synthrom.DONE_BYTE, clip=15,
                  time_penalty=0.01)
    say(f"[gpu] benchmark workload long run: N={n} fs=4 steps={steps} sample={len(sample)}")
    b = abi.Batch(rom, n, frameskip=4, reward_kind=abi.REWARD_XDELTA, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI,
                  done_addr=synthrom.DONE_BYTE, clip=15, time_penalty=0.01)
    b.set_snapshots(blobs, levels)
    b.poke_ram_envs(synthrom.DONE_BYTE, done_init)
    ob = OracleBatch(rom, sample, reward=reward)
    for e, c in zip(sample, ob.cons):
        c.load(snaps[levels[e]])
        c.write(synthrom.DONE_BYTE, int(done_init[e]))
    ends = 0
    for k in range(steps):
        m = masks_for(7070, n, k)
        b.set_actions(m)
        b.step(auto_reset=True)
        _, rew, don = ob.step(m, 4)
        np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS)[sample], rew, err_msg=f"step {k} rewards")
        np.testing.assert_array_equal(b.host(abi.VIEW_DONES)[sample], don, err_msg=f"step {k} dones")
        for j in np.nonzero(don)[0]:
            ob.cons[j].load(snaps[levels[sample[j]]])
        ends += int(don.sum())
        if k % 8 == 7:
            say(f"[gpu]   step {k}: {ends} sampled episode ends so far")
            for e, ref in zip(sample, ob.states()):
                got = b.save_state(e)
                assert np.array_equal(got, ref), f"step {k} env {e}: {first_diff(got, ref)}"
    assert ends >= len(sample) + 16


def test_benchmark_workload_soak_full_size_sampled():
    """A soak of the benchmark workload: 65,536 consoles, 240 steps (960
    frames, many episodes per console, each restarting from one of 8
    snapshots), x-delta reward and auto-reset; 16 sampled consoles have the
    oracle's rewards and dones at every step and its state every 40th step."""
    rom = synthrom.make_rom(2026).rom
    snaps = warm_snapshots(rom, [120, 233, 301, 415, 502, 611, 702, 777], seed=91)
    for i, s in enumerate(snaps):
        s[O.OFF["ram"] + synthrom.DONE_BYTE] = 3 + 3 * i   # episodes of 24-192 frames from a snapshot
    blobs = [bytes(s) for s in snaps]
    n, steps = 65536, 240
    rng = np.random.default_rng(92)
    levels = rng.integers(0, 8, n).astype(np.uint8)
    done_init = rng.integers(1, 25, n).astype(np.uint8)
    sample = sorted({0, 63, 64, 16383, 32768, n - 1} | set(rng.integers(0, n, 10).tolist()))
    reward = dict(kind=1, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI, done_addr=synthrom.DONE_BYTE, clip=15,
                  time_penalty=0.01)
    say(f"[gpu] benchmark workload soak: N={n} fs=4 steps={steps} sample={sample}")
    b = abi.Batch(rom, n, frameskip=4, reward_kind=abi.REWARD_XDELTA, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI,
                  done_addr=synthrom.DONE_BYTE, clip=15, time_penalty=0.01)
    b.set_snapshots(blobs, levels)
    b.poke_ram_envs(synthrom.DONE_BYTE, done_init)
    ob = OracleBatch(rom, sample, reward=reward)
    for e, c in zip(sample, ob.cons):
        c.load(snaps[levels[e]])
        c.write(synthrom.DONE_BYTE, int(done_init[e]))
    ends = 0
    for k in range(steps):
        m = masks_for(9191, n, k)
        b.set_actions(m)
        b.step(auto_reset=True)
        _, rew, don = ob.step(m, 4)
        np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS)[sample], rew, err_msg=f"step {k} rewards")
        np.testing.assert_array_equal(b.host(abi.VIEW_DONES)[sample], don, err_msg=f"step {k} dones")
        for j in np.nonzero(don)[0]:
            ob.cons[j].load(snaps[levels[sample[j]]])
        ends += int(don.sum())
        if k % 40 == 39:
            say(f"[gpu]   step {k}: {ends} sampled episode ends so far")
            for e, ref in zip(sample, ob.states()):
                got = b.save_state(e)
                assert np.array_equal(got, ref), f"step {k} env {e}: {first_diff(got, ref)}"
    assert ends >= 5 * len(sample)


def test_reset_envs_and_state_roundtrip():
    """Masked reset returns exactly the selected consoles to power-on; a saved
    state loaded into other consoles makes them identical; int64 device
    actions equal uint8 host actions."""
    import torch

    rom = _rom(3)
    n = 256
    say(f"[gpu] reset/state round trip: N={n}")
    b = abi.Batch(rom, n, frameskip=4)
    power_on = b.save_state(0)
    for k in range(3):
        b.set_actions(masks_for(5, n, k))
        b.step()
    mask = np.zeros(n, dtype=np.uint8)
    mask[::3] = 1
    before = [b.save_state(e) for e in (1, 2)]
    b.reset_envs(mask)
    for e in (0, 3, 255):
        assert np.array_equal(b.save_state(e), power_on)
    assert np.array_equal(b.save_state(1), before[0]) and np.array_equal(b.save_state(2), before[1])
    st = b.save_state(2)
    lm = np.zeros(n, dtype=np.uint8)
    lm[10:20] = 1
    b.load_state(st, lm)
    for e in range(10, 20):
        assert np.array_equal(b.save_state(e), st)
    # int64 device actions vs uint8 host actions on a twin batch.
    b2 = abi.Batch(rom, n, frameskip=4)
    b3 = abi.Batch(rom, n, frameskip=4)
    m = masks_for(8, n, 0)
    b2.set_actions(torch.from_numpy(m.astype(np.int64) | 0x300).cuda())
    b2.step()
    b3.set_actions(m)
    b3.step()
    np.testing.assert_array_equal(b2.host(abi.VIEW_RAM), b3.host(abi.VIEW_RAM))


def test_full_size_snapshot_reset_properties():
    """Size-independent properties at 65,536 consoles with 8 snapshot levels:
    two batches fed the same actions stay identical (RAM of every console);
    a snapshot captured from a console exports its state byte for byte; a
    masked reset puts every masked console's RAM (and, sampled, its whole
    state) exactly into its level's snapshot and leaves every other console's
    RAM untouched; the same reset again changes nothing."""
    rom = synthrom.make_rom(2026).rom
    snaps = warm_snapshots(rom, [120, 240, 360, 480, 600, 720, 840, 960], seed=21)
    blobs = [bytes(x) for x in snaps]
    n = 65536
    rng = np.random.default_rng(21)
    levels = rng.integers(0, 8, n).astype(np.uint8)
    say(f"[gpu] full-size snapshot/reset properties: N={n}")
    a = abi.Batch(rom, n, frameskip=4)
    b = abi.Batch(rom, n, frameskip=4)
    for x in (a, b):
        x.set_snapshots(blobs, levels)
    for k in range(6):
        m = masks_for(21, n, k)
        for x in (a, b):
            x.set_actions(m)
            x.step()
    before = a.host(abi.VIEW_RAM)
    np.testing.assert_array_equal(before, b.host(abi.VIEW_RAM))
    b.close()
    for e, slot in ((12345, 3), (n - 1, 5)):
        st = a.save_state(e)
        a.snapshot_capture(e, slot)
        assert np.array_equal(a.snapshot_export(slot), st), f"capture of env {e}"
    bank = [a.snapshot_export(lv) for lv in range(8)]
    mask = (rng.random(n) < 1 / 7).astype(np.uint8)
    a.reset_envs(mask)
    after = a.host(abi.VIEW_RAM)
    keep = mask == 0
    np.testing.assert_array_equal(after[keep], before[keep])
    ram = O.OFF["ram"]
    expect = np.stack([bk[ram:ram + 2048] for bk in bank])
    np.testing.assert_array_equal(after[~keep], expect[levels[~keep]])
    masked = np.nonzero(mask)[0]
    for e in masked[:: max(1, len(masked) // 16)][:16]:
        assert np.array_equal(a.save_state(int(e)), bank[levels[e]]), f"reset env {e}"
    a.reset_envs(mask)
    np.testing.assert_array_equal(a.host(abi.VIEW_RAM), after)


@pytest.mark.parametrize("n", [128, 16384])
def test_profile_counts_match_instructions(n):
    """step_profile's opcode histogram sums to the per-console instruction
    counts; only official opcodes appear (both LDS layouts)."""
    rom = _rom(4)
    say(f"[gpu] profile: N={n}")
    b = abi.Batch(rom, n, frameskip=4)
    b.set_actions(masks_for(1, n, 0))
    b.step(stats_mode=2)
    ops = b.host(abi.VIEW_OPCODES)
    pcs = b.host(abi.VIEW_PCS)
    ins = b.host(abi.VIEW_INSTRUCTIONS)
    assert ops.sum() == ins.sum() == pcs.sum()
    assert set(np.nonzero(ops)[0].tolist()) <= synthrom.OFFICIAL_OPCODES


def test_profile_step_clears_and_replays_in_a_graph():
    """A profiled step clears the opcode/PC histograms with a kernel (no
    memset), so they count only that step's instructions, eagerly and when
    the step is captured in a HIP graph: four replays, with eager work and
    host synchronisations between them, each equal to an eager twin batch
    (histograms, per-console instruction counts, canonical state)."""
    import torch

    rom = _rom(4)
    n = 128
    say(f"[gpu] profile step in a graph: N={n}")
    eager = abi.Batch(rom, n, frameskip=4)
    cap = abi.Batch(rom, n, frameskip=4)
    stream = torch.cuda.Stream()
    cap.set_stream(stream.cuda_stream)
    for b in (eager, cap):
        b.set_actions(masks_for(6, n, 0))
        b.step(stats_mode=2)   # first profiled step allocates the statistics
        b.synchronize()
    eager.set_actions(masks_for(6, n, 1))
    eager.step(stats_mode=2)
    ops, ins = eager.host(abi.VIEW_OPCODES), eager.host(abi.VIEW_INSTRUCTIONS)
    assert ops.sum() == ins.sum() == eager.host(abi.VIEW_PCS).sum()
    eager.set_actions(masks_for(6, n, 2))
    cap.set_actions(masks_for(6, n, 1))
    cap.step(stats_mode=2)
    cap.set_actions(masks_for(6, n, 2))
    cap.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        cap.step(stats_mode=2)
    for k in range(4):
        graph.replay()
        eager.step(stats_mode=2)
        torch.cuda.synchronize()
        cap.synchronize()
        for kind in (abi.VIEW_OPCODES, abi.VIEW_PCS, abi.VIEW_INSTRUCTIONS):
            np.testing.assert_array_equal(cap.host(kind), eager.host(kind), err_msg=f"replay {k} view {kind}")
        assert cap.host(abi.VIEW_OPCODES).sum() == cap.host(abi.VIEW_INSTRUCTIONS).sum()
        for e in (0, 63, n - 1):
            assert np.array_equal(cap.save_state(e), eager.save_state(e)), f"replay {k} env {e}"


@pytest.mark.parametrize("num_envs", [64, 16384])
def test_nrom128_cold_boot_nmi_loop_and_autoreset(num_envs):
    """A 16 KB PRG image (NROM-128) mirrored at $8000 and $C000 (the
    reference's read_nrom_prg, batch_bus.cuh:24-33; test_console.cpp:190-199):
    the console boots through the reset vector in the low copy, takes every
    frame's NMI there and runs its main loop and subroutines in the high
    copy.  Cold boot, then snapshot auto-reset with the x-delta rule, in both
    LDS layouts (64 consoles: all RAM in LDS; 16,384: split), sampled
    consoles against the oracle."""
    rom = synthrom.make_rom(5, prg_banks=1).rom
    assert abi.parse_ines(rom)["prg_rom_size"] == 16384
    n = num_envs
    rng = np.random.default_rng(n)
    sample = list(range(n)) if n <= 64 else sorted({0, 63, 64, 4095, n - 1, *rng.integers(0, n, 6).tolist()})
    say(f"[gpu] NROM-128 cold boot: N={n} fs=4 sample={len(sample)}")
    b = abi.Batch(rom, n, frameskip=4)
    ob = OracleBatch(rom, sample)
    for k in range(12):
        m = masks_for(31, n, k)
        b.set_actions(m)
        b.step(stats_mode=1)
        ins, rew, don = ob.step(m, 4)
        np.testing.assert_array_equal(b.host(abi.VIEW_INSTRUCTIONS)[sample], ins, err_msg=f"step {k}")
        np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS)[sample], rew, err_msg=f"step {k}")
    for e, ref in zip(sample, ob.states()):
        got = b.save_state(e)
        assert np.array_equal(got, ref), f"cold boot env {e}: {first_diff(got, ref)}"
    assert (b.host(abi.VIEW_FRAMES) == 4).all()

    say(f"[gpu] NROM-128 snapshot auto-reset: N={n}")
    snaps = warm_snapshots(rom, [60, 120, 180, 240], seed=8)
    for i, s in enumerate(snaps):
        s[O.OFF["ram"] + synthrom.DONE_BYTE] = 1 + i
    blobs = [bytes(s) for s in snaps]
    levels = rng.integers(0, 4, n).astype(np.uint8)
    reward = dict(kind=1, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI, done_addr=synthrom.DONE_BYTE, clip=15,
                  time_penalty=0.5)
    b = abi.Batch(rom, n, frameskip=4, reward_kind=abi.REWARD_XDELTA, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI,
                  done_addr=synthrom.DONE_BYTE, clip=15, time_penalty=0.5)
    b.set_snapshots(blobs, levels)
    ob = OracleBatch(rom, sample, reward=reward)
    for e, c in zip(sample, ob.cons):
        c.load(snaps[levels[e]])
    ends = 0
    for k in range(24):
        m = masks_for(32, n, k)
        b.set_actions(m)
        b.step(auto_reset=True)
        _, rew, don = ob.step(m, 4)
        np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS)[sample], rew, err_msg=f"step {k} rewards")
        np.testing.assert_array_equal(b.host(abi.VIEW_DONES)[sample], don, err_msg=f"step {k} dones")
        for j in np.nonzero(don)[0]:
            ob.cons[j].load(snaps[levels[sample[j]]])
        ends += int(don.sum())
        if k % 6 == 5:
            for e, ref in zip(sample, ob.states()):
                got = b.save_state(e)
                assert np.array_equal(got, ref), f"step {k} env {e}: {first_diff(got, ref)}"
    assert ends >= len(sample)


def test_poke_ram_envs_writes_one_byte_per_console():
    """nesle_poke_ram_envs: console e's RAM byte gets values[e], through the
    $0800 mirror too; nothing else changes and the reward baselines stay."""
    rom = _rom(3)
    n = 300
    say(f"[gpu] poke_ram_envs: N={n}")
    b = abi.Batch(rom, n, frameskip=4)
    b.set_actions(masks_for(2, n, 0))
    b.step()
    before = b.host(abi.VIEW_RAM).copy()
    vals = np.random.default_rng(1).integers(0, 256, n).astype(np.uint8)
    b.poke_ram_envs(0x0812, vals)
    after = b.host(abi.VIEW_RAM)
    assert np.array_equal(after[:, 0x12], vals)
    before[:, 0x12] = vals
    assert np.array_equal(after, before)
    with pytest.raises(ValueError):
        abi.lib()  # the library is loaded; a null values pointer is an argument error
        abi._check(abi.lib().nesle_poke_ram_envs(b.h, 0x12, None, 0))


def test_split_batch_with_consoles_at_different_frame_phases():
    """The split layout holds each console that reaches vblank until every
    running console of its wave has (the NMI handlers then run together).
    Consoles loaded from states saved in the middle of a frame reach vblank
    at very different points of a step than consoles at a frame boundary:
    16,384 consoles, a third of them (every third console, so each wave has
    both kinds) loaded with one of four mid-frame states, the rest from
    power-on, six steps at frame-skip 4 with the x-delta reward; every
    step's rewards, dones and instruction counts, and the final states of
    sampled consoles, equal oracle consoles given the same states."""
    rom = synthrom.make_rom(2026).rom
    reward = dict(kind=1, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI, done_addr=synthrom.DONE_BYTE, clip=15,
                  time_penalty=0.01)
    states = []
    for k, (frames, extra) in enumerate([(12, 1500), (20, 3700), (31, 5200), (45, 6900)]):
        o = O.Oracle(rom)
        for f in range(frames):
            o.step(int(masks_for(40 + k, 1, f)[0]), 1)
        for _ in range(extra):                     # into the middle of the next frame
            o.step_instruction()
        states.append(o.save())
    for st in states:
        dot = int(np.frombuffer(st[O.OFF["frame_dot"]:O.OFF["frame_dot"] + 4].tobytes(), np.uint32)[0])
        assert 1000 < dot < 88000, dot                 # not at a frame boundary
    n, steps = 16384, 6
    rng = np.random.default_rng(41)
    which = np.full(n, -1)
    which[::3] = rng.integers(0, len(states), which[::3].size)
    sample = sorted({0, 1, 2, 3, 63, 64, 8190, 8191, n - 1, *rng.integers(0, n, 9).tolist()})
    say(f"[gpu] split batch, mixed frame phases: N={n} steps={steps} sample={sample}")
    b = abi.Batch(rom, n, frameskip=4, reward_kind=abi.REWARD_XDELTA, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI,
                  done_addr=synthrom.DONE_BYTE, clip=15, time_penalty=0.01)
    for k, st in enumerate(states):
        b.load_state(st, (which == k).astype(np.uint8))
    ob = OracleBatch(rom, sample, reward=reward)
    for e, c in zip(sample, ob.cons):
        if which[e] >= 0:
            c.load(states[which[e]])
    for k in range(steps):
        m = masks_for(42, n, k)
        b.set_actions(m)
        b.step(stats_mode=1)
        ins, rew, don = ob.step(m, 4)
        got_ins = b.host(abi.VIEW_INSTRUCTIONS)[sample].astype(np.int64)
        got_rew, got_don = b.host(abi.VIEW_REWARDS)[sample], b.host(abi.VIEW_DONES)[sample]
        assert np.array_equal(got_ins, ins), (k, got_ins, ins)
        assert np.array_equal(got_rew, rew) and np.array_equal(got_don, don), (k, got_rew, rew, got_don, don)
    for e, st in zip(sample, ob.states()):
        got = b.save_state(e)
        assert np.array_equal(got, st), f"console {e}: {first_diff(got, st)}"
    b.close()
