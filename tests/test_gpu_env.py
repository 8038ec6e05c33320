"""The vector environment (nesle_amd.env) on the HIP batch: RAM-mode
trajectories equal oracle consoles under the SB3 auto-reset contract
(terminal observations, terminated/truncated, post-reset observations), the
reference's contract tests (tests/test_critical_fixes.py:59-196) on its
all-NOP ROM, snapshot levels (src/nesle/env.py:405-425 round robin and
explicit assignment, per-env resets keep the level) and frame observations."""

from __future__ import annotations

import gzip

import numpy as np
import pytest

from nesle_amd import actions as A
from nesle_amd import env as E
from nesle_amd import synthrom
from oracle import oracle as O
from tests.helpers import say, warm_snapshots

pytestmark = pytest.mark.gpu

RAM = O.OFF["ram"]


def nop_rom() -> bytes:
    """The contract tests' ROM: 32 KB of NOP, reset vector $8000, blank CHR."""
    prg = bytearray([0xEA] * 0x8000)
    prg[0x7FFC], prg[0x7FFD] = 0x00, 0x80
    return bytes(b"NES\x1a" + bytes([2, 1, 0, 0]) + bytes(8) + prg + bytes(0x2000))


def test_ram_trajectory_matches_oracle_with_auto_reset():
    rom = synthrom.make_rom(6).rom
    n, steps, limit = 8, 12, 3
    say(f"[gpu] vec env ram trajectory: N={n} steps={steps} max_episode_steps={limit}")
    env = E.NesleVecEnv("synthetic.nes", n, frameskip=4, action_space="complex", observation_mode="ram",
                        max_episode_steps=limit, rom_bytes=rom)
    cons = [O.Oracle(rom) for _ in range(n)]
    for c in cons:
        c.set_reward()
    obs = env.reset()
    assert obs.shape == (n, 2048) and obs.dtype == np.uint8
    for e in range(n):
        assert np.array_equal(obs[e], cons[e].save()[RAM:RAM + 2048])
    rng = np.random.default_rng(6)
    count = np.zeros(n, dtype=np.int64)
    table = np.asarray(A.COMPLEX_MOVEMENT_MASKS)
    for k in range(steps):
        act = rng.integers(0, 12, n)
        obs, rew, done, infos = env.step(act)
        count += 1
        for e in range(n):
            _, r, d = cons[e].step(int(table[act[e]]), 4)
            trunc = bool(count[e] >= limit)
            want_done = bool(d) or trunc
            assert rew[e] == np.float32(r), f"step {k} env {e} reward"
            assert bool(done[e]) == want_done, f"step {k} env {e} done"
            ram_now = cons[e].save()[RAM:RAM + 2048]
            if want_done:
                info = infos[e]
                assert np.array_equal(info["terminal_observation"], ram_now)
                assert info["truncated"] == trunc and info["terminated"] == (not trunc)
                cons[e] = O.Oracle(rom)
                cons[e].set_reward()
                count[e] = 0
                ram_now = cons[e].save()[RAM:RAM + 2048]
            assert np.array_equal(obs[e], ram_now), f"step {k} env {e} observation"
            assert infos[e]["backend"] == "cuda-console"


def test_auto_reset_contract_on_nop_rom():
    rom = nop_rom()
    say("[gpu] vec env contract: NOP ROM")
    env = E.NesleVecEnv("nop.nes", 2, max_episode_steps=2, rom_bytes=rom)
    reset_obs = env.reset()
    assert reset_obs.shape == (2, 240, 256, 3)
    env.step([1, 1])
    obs, _, dones, infos = env.step([1, 1])
    assert dones.all()
    for i in range(2):
        assert infos[i]["terminal_observation"].shape == (240, 256, 3)
        assert infos[i]["truncated"] and not infos[i]["terminated"]
    assert obs.shape == reset_obs.shape
    assert env.reset_infos[0]["backend"] == "cuda-console"
    np.testing.assert_array_equal(obs, env.render())

    ram_env = E.NesleVecEnv("nop.nes", 2, observation_mode="ram", max_episode_steps=2, rom_bytes=rom)
    ram_env.reset()
    ram_env.step([1, 1])
    _, _, dones, infos = ram_env.step([1, 1])
    assert dones.all() and infos[0]["terminal_observation"].shape == (2048,)

    rew_env = E.NesleVecEnv("nop.nes", 2, observation_mode="ram", max_episode_steps=2, rom_bytes=rom)
    rew_env.reset()
    rew_env.step_reward([1, 1])
    _, dones, infos = rew_env.step_reward([1, 1])
    assert dones.all() and all(infos[i]["truncated"] for i in range(2))
    assert infos[0]["terminal_observation"].shape == (2048,)
    _, dones, _ = rew_env.step_reward([1, 1])
    assert not dones.any()   # a fresh episode, not a stale step count

    start = E.NesleVecEnv("nop.nes", 2, action_space="simple_with_start", rom_bytes=rom)
    assert start.action_space.n == 8
    start.reset()
    obs, _, _, _ = start.step(np.array([0, 0]))
    assert obs.shape == (2, 240, 256, 3)

    single = E.NesleEnv("nop.nes", action_space="simple_with_start", rom_bytes=rom)
    o, info = single.reset(seed=42)
    assert o.shape == (240, 256, 3)
    o, r, term, trunc, info = single.step(0)
    assert isinstance(r, float) and isinstance(term, bool) and isinstance(trunc, bool)


def test_observation_cadence_marks_stale_frames():
    rom = synthrom.make_rom(6).rom
    say("[gpu] vec env cadence")
    env = E.NesleVecEnv("synthetic.nes", 4, observation_cadence=2, rom_bytes=rom)
    first = env.reset()
    obs, _, _, infos = env.step([1, 1, 1, 1])
    assert infos[0]["observations_stale"] and not infos[0]["observations_copied"]
    np.testing.assert_array_equal(obs, first)
    obs, _, _, infos = env.step([1, 1, 1, 1])
    assert infos[0]["observations_copied"] and not infos[0]["observations_stale"]
    np.testing.assert_array_equal(obs, env.render())


def test_snapshot_levels(tmp_path):
    rom = synthrom.make_rom(5).rom
    say("[gpu] vec env snapshot levels: capture 4 levels")
    snaps = warm_snapshots(rom, [40, 80, 120, 160], seed=9)
    paths = []
    for i, s in enumerate(snaps):
        p = tmp_path / f"level{i}.state"
        p.write_bytes(gzip.compress(bytes(s)) if i == 1 else bytes(s))
        paths.append(str(p))
    level_ram = [s[RAM:RAM + 2048] for s in snaps]

    env = E.make_vec("synthetic.nes", 8, observation_mode="ram", reset_state_paths=paths, rom_bytes=rom)
    assert env._cuda_batch.has_snapshot and env._cuda_batch.num_levels == 4
    obs = env.reset()
    for e in range(8):
        assert np.array_equal(obs[e], level_ram[e % 4]), f"env {e}"

    env = E.make_vec("synthetic.nes", 4, observation_mode="ram", reset_state_paths=paths,
                     env_to_level=[2, 2, 2, 2], rom_bytes=rom)
    obs = env.reset()
    assert all(np.array_equal(obs[e], level_ram[2]) for e in range(4))

    env = E.make_vec("synthetic.nes", 4, observation_mode="ram", action_space="raw", max_episode_steps=2,
                     reset_state_paths=paths, rom_bytes=rom)
    env.reset()
    for _ in range(3):
        obs, _, dones, _ = env.step(np.zeros(4, dtype=np.int64))
        if dones.all():
            break
    assert dones.all()
    for e in range(4):
        assert np.array_equal(obs[e], level_ram[e]), f"env {e} back at its own level"

    single = E.make_vec("synthetic.nes", 2, observation_mode="ram", reset_state_path=paths[0], rom_bytes=rom)
    assert single._cuda_batch.num_levels == 1
    obs = single.reset()
    assert np.array_equal(obs[0], level_ram[0]) and np.array_equal(obs[1], level_ram[0])


def test_partial_dones_return_reset_rows_and_step_rows(tmp_path):
    """Only some consoles end their episode in a step: their returned rows
    are the reset RAM (their own level's) and their infos hold the step's
    RAM as terminal observation; every other row is the step's RAM.  The
    ROM counts RAM[$10] up in a loop, so a step's RAM differs from a reset
    one; level 1 carries the SMB rule's "dead" player state (RAM[$0E] = 6),
    so exactly its consoles are done after every step."""
    from tests.kat_roms import nrom_bytes

    rom = nrom_bytes(2, code={0x8000: [0xE6, 0x10, 0x4C, 0x00, 0x80]}, reset=0x8000)
    base = O.Oracle(rom).save()
    blobs = []
    for level, state in enumerate((0x08, 0x06)):
        s = base.copy()
        s[RAM + 0x0E] = state
        s[RAM + 0x10] = 0x40 * level
        s[RAM + 0xB5] = 1
        blobs.append(s)
    paths = []
    for i, s in enumerate(blobs):
        p = tmp_path / f"lvl{i}.state"
        p.write_bytes(bytes(s))
        paths.append(str(p))
    levels = [0, 1, 0, 1, 1, 0]
    n = len(levels)
    say(f"[gpu] vec env partial dones: N={n}")
    env = E.NesleVecEnv("count.nes", n, observation_mode="ram", action_space="raw", reset_state_paths=paths,
                        env_to_level=levels, rom_bytes=rom)
    cons = [O.Oracle(rom) for _ in range(n)]
    obs = env.reset()
    for e in range(n):
        cons[e].set_reward()
        cons[e].load(blobs[levels[e]])
        assert np.array_equal(obs[e], blobs[levels[e]][RAM:RAM + 2048])
    for k in range(3):
        obs, rew, done, infos = env.step(np.zeros(n, dtype=np.int64))
        assert done.tolist() == [lv == 1 for lv in levels], f"step {k}"
        for e in range(n):
            _, r, d = cons[e].step(0, 4)
            stepped = cons[e].save()[RAM:RAM + 2048]
            assert rew[e] == np.float32(r) and bool(d) == bool(done[e])
            if done[e]:
                assert np.array_equal(infos[e]["terminal_observation"], stepped), f"step {k} env {e}"
                assert infos[e]["terminated"] and not infos[e]["truncated"]
                cons[e].load(blobs[levels[e]])
                assert np.array_equal(obs[e], blobs[levels[e]][RAM:RAM + 2048]), f"step {k} env {e} reset row"
            else:
                assert "terminal_observation" not in infos[e]
                assert np.array_equal(obs[e], stepped), f"step {k} env {e} step row"
                assert stepped[0x10] != blobs[levels[e]][RAM + 0x10]
