"""The trainer's shaped SMB reward without a GPU: its numpy float32
restatement (oracle/smart_reward.py) against one hand-worked case per term of
the reference's rule (src/nesle/native_ppo.py:120-316), and the trainer's
configuration surface for it (reward_mode="smart", the bonus/penalty
overrides, the progress bar flag)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle.smart_reward import SmartRewardModel

F = np.float32


def _ram(n: int = 1, x: int = 16) -> np.ndarray:
    ram = np.zeros((n, 2048), dtype=np.uint8)
    ram[:, 0x6D], ram[:, 0x86] = x >> 8, x & 0xFF
    ram[:, 0xB5] = 1          # on screen
    ram[:, 0x75A] = 2         # lives
    return ram


def _set_x(ram: np.ndarray, x: int) -> None:
    ram[:, 0x6D], ram[:, 0x86] = x >> 8, x & 0xFF


def _set_bcd(ram: np.ndarray, at: int, value: int, digits: int) -> None:
    for k in range(digits):
        ram[:, at + digits - 1 - k] = (value // 10 ** k) % 10


def _step(m: SmartRewardModel, ram, pad: int = 0, done: int = 0) -> float:
    return float(m.compute(ram, np.array([pad]), np.array([done]))[0])


TIME = F(-0.005)


def test_progress_backtrack_and_clamp():
    ram = _ram()
    m = SmartRewardModel(1)
    m.reset(ram)
    _set_x(ram, 16 + 10)
    assert _step(m, ram) == F(F(10) * F(0.18)) + TIME          # forward 10 px
    _set_x(ram, 16)
    assert _step(m, ram) == F(F(-10) * F(0.03)) + TIME         # back 10 px
    _set_x(ram, 16 + 40)
    assert _step(m, ram) == F(F(16) * F(0.18)) + TIME          # forward 40 px, clamped to 16


def test_first_step_of_an_episode_pays_every_checkpoint_below_x():
    """reset_where zeroes the checkpoint index whatever x is (native_ppo.py:
    178-193), so the first step pays floor(x / 128) checkpoints."""
    ram = _ram(x=500)
    m = SmartRewardModel(1)
    m.reset(ram)
    assert _step(m, ram) == F(F(3) * F(3.0)) + TIME
    assert _step(m, ram) == TIME


def test_checkpoint_every_128_pixels_of_the_furthest_x():
    ram = _ram(x=127)
    m = SmartRewardModel(1)
    m.reset(ram)
    _set_x(ram, 129)
    r = _step(m, ram)
    assert r == F(F(F(2) * F(0.18)) + F(3.0)) + TIME
    _set_x(ram, 100)                                           # back: no checkpoint lost or regained
    _step(m, ram)
    _set_x(ram, 130)
    assert _step(m, ram) == F(F(16) * F(0.18)) + TIME          # +30 px clamped; 130 < 2 * 128


def test_score_kills_and_coins_with_the_coin_wrap():
    ram = _ram()
    _set_bcd(ram, 0x7DE, 1000, 6)
    _set_bcd(ram, 0x7ED, 99, 2)
    m = SmartRewardModel(1)
    m.reset(ram)
    _set_bcd(ram, 0x7DE, 1100, 6)                              # +100 points, no coin: a kill
    r = _step(m, ram)
    assert r == F(F(F(0) + F(F(100) * F(0.04))) + F(8.0)) + TIME
    _set_bcd(ram, 0x7DE, 1300, 6)                              # +200 with one coin (99 -> 00): no kill
    _set_bcd(ram, 0x7ED, 0, 2)
    r = _step(m, ram)
    assert r == F(F(F(0) + F(F(200) * F(0.04))) + F(3.0)) + TIME


def test_finish_zone_and_flag_pay_once_per_episode():
    ram = _ram(x=3099)
    m = SmartRewardModel(1)
    m.reset(ram)
    assert _step(m, ram) == F(F(24) * F(3.0)) + TIME           # first step: 24 checkpoints below x
    _set_x(ram, 3100)
    assert _step(m, ram) == F(F(F(F(1) * F(0.18)) + F(0)) + F(100.0)) + TIME
    _set_x(ram, 3101)
    assert _step(m, ram) == F(F(1) * F(0.18)) + TIME           # no second finish bonus
    ram[:, 0x770] = 2                                          # flag by game mode, standing still
    assert _step(m, ram) == F(100.0) + TIME
    assert _step(m, ram) == TIME                               # once
    ram2 = _ram(x=3300)
    for done, want in ((1, F(100.0) + TIME), (0, TIME)):       # the flag zone pays only on a done step
        m2 = SmartRewardModel(1)
        m2.reset(ram2)
        assert _step(m2, ram2) == F(F(F(25) * F(3.0)) + F(100.0)) + TIME   # 25 checkpoints, the finish zone
        assert _step(m2, ram2, done=done) == want
    ram2[:, 0x0E] = 0x06                                       # dead at the flag zone: no flag, the penalty
    m3 = SmartRewardModel(1)
    m3.reset(ram2)
    _step(m3, ram2)
    assert _step(m3, ram2, done=1) == F(-75.0) + TIME


def test_flag_by_game_mode_exact():
    ram = _ram()
    m = SmartRewardModel(1)
    m.reset(ram)
    ram[:, 0x770] = 2
    assert _step(m, ram) == F(100.0) + TIME
    assert _step(m, ram) == TIME                               # once


def test_death_penalty_needs_done():
    ram = _ram()
    m = SmartRewardModel(1)
    m.reset(ram)
    ram[:, 0x0E] = 0x0B                                        # dying
    assert _step(m, ram, done=0) == TIME
    assert _step(m, ram, done=1) == F(-75.0) + TIME
    m2 = SmartRewardModel(1, death_penalty=10.0)               # the trainer's override
    m2.reset(ram)
    assert _step(m2, ram, done=1) == F(-10.0) + TIME


def test_stall_penalty_from_the_fortieth_step_without_progress():
    ram = _ram()
    m = SmartRewardModel(1)
    m.reset(ram)
    rs = [_step(m, ram) for _ in range(41)]
    assert all(r == TIME for r in rs[:39])
    assert rs[39] == F(-F(F(1) * F(0.02))) + TIME
    assert rs[40] == F(-F(F(2) * F(0.02))) + TIME
    for _ in range(30):
        r = _step(m, ram)
    assert r == F(-0.5) + TIME                                 # capped


def test_button_penalties():
    ram = _ram()
    m = SmartRewardModel(1)
    m.reset(ram)
    jr = F(0) - F(0.005)                                       # jump with Right
    rs = [_step(m, ram, pad=0x81) for _ in range(7)]
    assert all(r == jr + TIME for r in rs[:6])
    assert rs[6] == F(jr - F(F(1) * F(0.02))) + TIME           # 7th jump in a row: repeated
    want = F(F(F(F(0) - F(0.005)) - F(0.02)) - F(F(2) * F(0.02)))            # neutral jump, streak 8
    assert _step(m, ram, pad=0x01) == want + TIME
    m2 = SmartRewardModel(1)
    m2.reset(ram)
    assert _step(m2, ram, pad=0x01) == F(F(F(0) - F(0.005)) - F(0.02)) + TIME  # neutral jump, streak 1
    assert _step(m2, ram, pad=0xC0) == F(F(F(0) - F(0.01)) - F(0.25)) + TIME   # left + right
    assert _step(m2, ram, pad=0x08) == F(F(0) - F(0.25)) + TIME                # start
    assert _step(m2, ram, pad=0x04) == F(F(0) - F(0.25)) + TIME                # select


def test_masked_reset_starts_only_the_selected_episodes():
    ram = _ram(2, x=200)
    m = SmartRewardModel(2)
    m.reset(ram)
    _set_x(ram, 210)
    m.compute(ram, np.zeros(2), np.zeros(2))
    ram[1, 0x86] = 50
    m.reset(ram, np.array([False, True]))
    assert m.last_x[0] == 210 and m.last_x[1] == 50 and m.max_x[1] == 50 and m.max_x[0] == 210


def test_trainer_accepts_the_reference_smart_reward_configuration():
    from nesle_amd import native_ppo as P

    cfg = P.NativePPOConfig("rom.nes", reward_mode="smart", flag_bonus=50.0, finish_zone_bonus=20.0,
                            death_penalty=30.0, progress_bar=True)
    assert cfg.reward_mode == "smart" and cfg.flag_bonus == 50.0 and cfg.progress_bar
    params = P.smart_reward_params(cfg)
    assert params.flag_bonus == 50.0 and params.finish_zone_bonus == 20.0 and params.death_penalty == 30.0
    assert abs(params.progress_scale - 0.18) < 1e-7 and params.stall_window == 40
    with pytest.raises(ValueError, match="reward_mode"):
        P.train_native_ppo(P.NativePPOConfig("none.nes", num_envs=64, n_steps=128, reward_mode="shaped"))
    cfg2, _ = P.parse_args(["rom.nes", "--reward-mode", "smart", "--flag-bonus", "7", "--death-penalty", "9",
                            "--finish-zone-bonus", "3", "--progress-bar"])
    assert (cfg2.reward_mode, cfg2.flag_bonus, cfg2.death_penalty, cfg2.finish_zone_bonus, cfg2.progress_bar) == \
        ("smart", 7.0, 9.0, 3.0, True)
