"""Host-side checks of the vector environment (no GPU): argument validation
happens before any device work, observation-mode names, spaces without
gymnasium, and reset-state file handling."""

from __future__ import annotations

import gzip

import numpy as np
import pytest

from nesle_amd import env as E


@pytest.mark.parametrize("kwargs", [dict(num_envs=0), dict(num_envs=2, frameskip=0),
                                    dict(num_envs=2, observation_cadence=0), dict(num_envs=2, render_mode="human"),
                                    dict(num_envs=2, backend="synthetic"), dict(num_envs=2, observation_mode="depth"),
                                    dict(num_envs=2, action_space="sideways"),
                                    dict(num_envs=2, reset_state_path="a", reset_state_paths=["b"])])
def test_bad_arguments_are_rejected_before_device_work(kwargs):
    with pytest.raises(ValueError):
        E.NesleVecEnv("missing.nes", **kwargs)


def test_env_to_level_checks(tmp_path):
    a, b = tmp_path / "a.state", tmp_path / "b.state"
    a.write_bytes(b"x")
    b.write_bytes(b"y")
    with pytest.raises(ValueError, match="requires more than one"):
        E.NesleVecEnv("missing.nes", 2, reset_state_path=str(a), env_to_level=[0, 0])
    with pytest.raises(ValueError, match="shape"):
        E.NesleVecEnv("missing.nes", 2, reset_state_paths=[str(a), str(b)], env_to_level=[0])
    with pytest.raises(ValueError, match=">= number"):
        E.NesleVecEnv("missing.nes", 2, reset_state_paths=[str(a), str(b)], env_to_level=[0, 2])


def test_observation_modes_and_spaces():
    assert E.observation_mode_of("RGB") == "rgb_array"
    assert E.observation_mode_of("frame") == "rgb_array"
    assert E.observation_mode_of("cpu-ram") == "ram"
    with pytest.raises(ValueError):
        E.observation_mode_of("depth")
    box, d = E._spaces((2048,), 12)
    assert d.n == 12 and d.contains(11) and not d.contains(12) and not d.contains("x")
    assert box.shape == (2048,) and box.contains(box.sample())


def test_level_map_round_robin_and_explicit():
    assert E.level_map(1, 4, None) is None and E.level_map(0, 4, None) is None
    assert E.level_map(3, 7, None).tolist() == [0, 1, 2, 0, 1, 2, 0]
    assert E.level_map(3, 3, [2, 2, 0]).tolist() == [2, 2, 0]
    with pytest.raises(ValueError):
        E.level_map(3, 2, [0, -1])


def test_episode_clock_limit_and_restart():
    c = E._EpisodeClock(3, 2)
    assert not c.tick().any()
    assert c.tick().all()
    c.restart(np.array([True, False, True]))
    assert c.tick().tolist() == [False, True, False]
    assert not E._EpisodeClock(2, 0).tick().any()


def test_gzip_reset_states_are_unpacked(tmp_path):
    raw = bytes(range(256)) * 4
    p = tmp_path / "level.state"
    p.write_bytes(gzip.compress(raw))
    assert E.read_state_file(p) == raw
    q = tmp_path / "plain.fcs"
    q.write_bytes(raw)
    assert E.read_state_file(q) == raw


def test_ram_rows_of_reset_consoles_without_torch(monkeypatch):
    """Without torch the observation reader takes the rows of reset consoles
    from a whole host copy of RAM (the reference env needs only numpy)."""
    import sys

    class FakeBatch:
        def __init__(self):
            self.ram_calls = 0

        def ram(self):
            self.ram_calls += 1
            return np.arange(4 * 2048, dtype=np.int64).reshape(4, 2048).astype(np.uint8) + 7

        def ram_device(self):  # pragma: no cover - must not be reached
            raise AssertionError("device view used without torch")

    monkeypatch.setitem(sys.modules, "torch", None)   # import torch -> ImportError
    batch = FakeBatch()
    obs_reader = E._Observer(batch, "ram", 1)
    obs = np.zeros((4, 2048), dtype=np.uint8)
    which = np.array([False, True, False, True])
    out = obs_reader.replace_rows(obs, which)
    full = batch.ram()
    assert np.array_equal(out[1], full[1]) and np.array_equal(out[3], full[3])
    assert not out[0].any() and not out[2].any()
