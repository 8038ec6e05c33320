"""The trainer's shaped SMB reward on the GPU (nesle_smb_shaped_reward /
nesle_smb_shaped_reset through the C ABI, wrapped by
nesle_amd.native_ppo.SmartMarioReward) against its numpy float32 restatement
(oracle/smart_reward.py): rewards bit-identical and the tracking state equal
word for word after every step of random RAM walks with resets; and the
trainer running reward_mode="smart" eagerly and from a captured rollout
graph."""

from __future__ import annotations

import numpy as np
import pytest

from oracle.smart_reward import SmartRewardModel
from tests.helpers import say

pytestmark = pytest.mark.gpu


def _walk(rng: np.random.Generator, ram: np.ndarray) -> None:
    """One step of a random game: x moves -20..+20 (page carry, clamped), score
    and coins tick up now and then (coins wrap at 100), deaths, flags."""
    n = ram.shape[0]
    x = ram[:, 0x6D].astype(np.int64) * 256 + ram[:, 0x86] + rng.integers(-20, 21, n)
    x = np.clip(x, 0, 0xFFFF)
    ram[:, 0x6D], ram[:, 0x86] = x >> 8, x & 0xFF
    score = np.zeros(n, np.int64)
    for k in range(6):
        score = score * 10 + (ram[:, 0x7DE + k] & 15)
    score = (score + rng.choice([0, 0, 0, 50, 100, 200, 1000], n)) % 1_000_000
    for k in range(6):
        ram[:, 0x7DE + 5 - k] = (score // 10 ** k) % 10
    coins = (ram[:, 0x7ED] & 15) * 10 + (ram[:, 0x7EE] & 15)
    coins = (coins + (rng.random(n) < 0.1)) % 100
    ram[:, 0x7ED], ram[:, 0x7EE] = coins // 10, coins % 10
    ram[:, 0x0E] = np.where(rng.random(n) < 0.02, rng.choice([0x06, 0x0B], n), 0)
    ram[:, 0xB5] = np.where(rng.random(n) < 0.01, 2, 1)
    ram[:, 0x770] = np.where(rng.random(n) < 0.005, 2, 1)
    ram[:, 0x75A] = np.where(rng.random(n) < 0.005, 0xFF, 2)
    ram[:, 0x75F] = rng.integers(0, 8, n)


def test_shaped_reward_kernel_matches_its_restatement():
    import torch

    from nesle_amd import native_ppo as P

    n = 5000
    say(f"[gpu] shaped SMB reward kernel: N={n}")
    rng = np.random.default_rng(11)
    ram = rng.integers(0, 256, (n, 2048)).astype(np.uint8)
    ram[:, 0x7DE:0x7E4] &= 0x0F
    ram[:, 0x7ED:0x7EF] %= 10
    cfg = P.NativePPOConfig("rom.nes", reward_mode="smart", death_penalty=40.0)
    dev = P.SmartMarioReward(n, cfg)
    model = SmartRewardModel(n, death_penalty=40.0)
    ram_d = torch.from_numpy(ram).cuda()
    dev.reset(ram_d)
    model.reset(ram)
    for k in range(80):
        _walk(rng, ram)
        pads = rng.integers(0, 256, n).astype(np.uint8)
        pads[rng.random(n) < 0.5] &= 0x81          # runs of held jump+right build jump streaks
        done = (rng.random(n) < 0.05).astype(np.uint8)
        ram_d.copy_(torch.from_numpy(ram))
        got = dev.compute(ram_d, torch.from_numpy(pads).cuda(), torch.from_numpy(done).cuda()).cpu().numpy()
        want = model.compute(ram, pads, done)
        bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
        assert bad.size == 0, f"step {k}: {bad.size} rewards differ, e.g. console {bad[0]}: {got[bad[0]]!r} vs {want[bad[0]]!r}"
        np.testing.assert_array_equal(dev.state.cpu().numpy().view(np.uint32), model.state_words(),
                                      err_msg=f"step {k}: tracking state")
        if k % 7 == 3:                              # restart the done consoles, from their RAM
            mask = done.astype(bool)
            dev.reset_where(torch.from_numpy(done).cuda(), ram_d)
            model.reset(ram, mask)
    assert np.abs(want).max() > 50                  # bonuses and penalties were hit


def test_trainer_with_the_shaped_reward_eager_and_graph():
    from nesle_amd import native_ppo as P
    from nesle_amd import synthrom

    rom = synthrom.make_rom(2026).rom
    say("[gpu] trainer reward_mode=smart: N=512 n_steps=16, 2 updates")
    cfg = P.NativePPOConfig("synthetic.nes", num_envs=512, total_timesteps=512 * 16 * 2, n_steps=16,
                            batch_size=2048, update_epochs=1, reward_mode="smart", max_episode_steps=10,
                            save_checkpoints=False, seed=3, log_interval=1, progress_bar=True)
    seen = []
    stats = P.train_native_ppo(cfg, rom_bytes=rom,
                               on_rollout=lambda u, b: seen.append((b["graph"], b["rewards"].clone())))
    assert stats["updates"] == 2 and [g for g, _ in seen] == [False, True]
    for _, r in seen:
        assert bool(r.isfinite().all())
    # Every console ends an episode within 10 steps (the timeout) and restarts.
    assert stats["log"][-1]["episodes"] >= 512
