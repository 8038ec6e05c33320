"""The trainer's shaped Super Mario Bros. reward, restated in numpy float32.

TEST INFRASTRUCTURE ONLY: the checker of nesle_smb_shaped_reward /
nesle_smb_shaped_reset (tests/); the product never imports it.

Follows the reference trainer's TorchSmartMarioReward
(src/nesle/native_ppo.py:120-316): the same RAM addresses (:123-133), the same
constants (:135-157), the same terms in the same order of summation
(:259-271), each float32 operation rounded on its own as PyTorch's
element-wise kernels round it (a Python scalar operand becomes a float32
constant).  The tracking state is eleven arrays over the consoles.
"""

from __future__ import annotations

import numpy as np

F = np.float32
X_PAGE, X_SCREEN, Y_VIEWPORT, PLAYER_STATE = 0x006D, 0x0086, 0x00B5, 0x000E
LIVES, WORLD, STAGE, AREA, GAME_MODE = 0x075A, 0x075F, 0x075C, 0x0760, 0x0770
COINS, SCORE = 0x07ED, 0x07DE

DEFAULTS = dict(progress_scale=0.18, backtrack_scale=0.03, checkpoint_bonus=3.0, checkpoint_width=128.0,
                score_scale=0.04, coin_bonus=3.0, kill_bonus=8.0, finish_zone_x=3100.0, finish_zone_bonus=100.0,
                flag_zone_x=3300.0, flag_bonus=100.0, death_penalty=75.0, time_penalty=0.005, stall_penalty=0.02,
                stall_window=40, max_stall_penalty=0.5, jump_penalty=0.005, neutral_jump_penalty=0.02,
                repeated_jump_penalty=0.02, repeated_jump_window=6, max_repeated_jump_penalty=0.25,
                left_penalty=0.01, bad_button_penalty=0.25)


def _bcd(ram: np.ndarray, at: int, digits: int) -> np.ndarray:
    v = (ram[:, at] & 0x0F).astype(np.int32)
    for k in range(1, digits):
        v = v * 10 + (ram[:, at + k] & 0x0F).astype(np.int32)
    return v


class SmartRewardModel:
    def __init__(self, num_envs: int, **overrides) -> None:
        self.p = {**DEFAULTS, **overrides}
        n = num_envs
        self.last_x = np.zeros(n, F)
        self.max_x = np.zeros(n, F)
        self.checkpoint_index = np.zeros(n, np.int32)
        self.last_score = np.zeros(n, F)
        self.last_coins = np.zeros(n, np.int32)
        self.last_lives = np.zeros(n, np.int32)
        self.last_level = np.zeros(n, np.int32)
        self.stall_steps = np.zeros(n, np.int32)
        self.jump_streak = np.zeros(n, np.int32)
        self.finish_awarded = np.zeros(n, bool)
        self.flag_awarded = np.zeros(n, bool)

    @staticmethod
    def x_pos(ram: np.ndarray) -> np.ndarray:
        return ram[:, X_PAGE].astype(F) * F(256.0) + ram[:, X_SCREEN].astype(F)

    @staticmethod
    def level(ram: np.ndarray) -> np.ndarray:
        return ram[:, WORLD].astype(np.int32) * 65536 + ram[:, STAGE].astype(np.int32) * 256 + ram[:, AREA]

    def reset(self, ram: np.ndarray, mask: np.ndarray | None = None) -> None:
        """reset_where (native_ppo.py:174-207); mask None = all."""
        m = np.ones(ram.shape[0], bool) if mask is None else np.asarray(mask, bool)
        x = self.x_pos(ram)
        self.last_x[m] = x[m]
        self.max_x[m] = x[m]
        self.checkpoint_index[m] = 0
        self.last_score[m] = _bcd(ram, SCORE, 6).astype(F)[m]
        self.last_coins[m] = _bcd(ram, COINS, 2)[m]
        self.last_lives[m] = ram[m, LIVES]
        self.last_level[m] = self.level(ram)[m]
        self.stall_steps[m] = 0
        self.jump_streak[m] = 0
        self.finish_awarded[m] = False
        self.flag_awarded[m] = False

    def compute(self, ram: np.ndarray, masks: np.ndarray, done: np.ndarray) -> np.ndarray:
        """compute (native_ppo.py:209-278): the step's reward, float32 [n]."""
        p = self.p
        done = np.asarray(done, bool)
        x = self.x_pos(ram)
        dx = x - self.last_x
        forward = dx > 0
        progress = np.where(forward, np.minimum(dx, F(16.0)) * F(p["progress_scale"]),
                            np.maximum(dx, F(-16.0)) * F(p["backtrack_scale"]))
        self.stall_steps = np.where(forward, 0, self.stall_steps + 1).astype(np.int32)
        self.max_x = np.maximum(self.max_x, x)
        new_ci = np.floor(self.max_x / F(p["checkpoint_width"])).astype(np.int32)
        cd = np.maximum(new_ci - self.checkpoint_index, 0)
        checkpoint = cd.astype(F) * F(p["checkpoint_bonus"])
        self.checkpoint_index = np.maximum(self.checkpoint_index, new_ci)

        score = _bcd(ram, SCORE, 6).astype(F)
        score_delta = np.maximum(score - self.last_score, F(0.0))
        coins = _bcd(ram, COINS, 2)
        coin_delta = coins - self.last_coins
        coin_delta = np.where(coin_delta < 0, coin_delta + 100, coin_delta)
        coin_delta = np.maximum(coin_delta, 0)
        score_reward = score_delta * F(p["score_scale"])
        kill_score = score_delta - coin_delta.astype(F) * F(200.0)
        kill_reward = np.where(kill_score >= F(100.0), F(p["kill_bonus"]), F(0.0))
        coin_reward = coin_delta.astype(F) * F(p["coin_bonus"])

        finish_hit = ~self.finish_awarded & (self.max_x >= F(p["finish_zone_x"]))
        finish_reward = np.where(finish_hit, F(p["finish_zone_bonus"]), F(0.0))
        self.finish_awarded |= finish_hit
        st = ram[:, PLAYER_STATE]
        death = (st == 0x0B) | (st == 0x06) | (ram[:, Y_VIEWPORT] > 1) | (ram[:, LIVES] == 0xFF)
        flag_hit = ~self.flag_awarded & ((ram[:, GAME_MODE] == 2) | ((self.max_x >= F(p["flag_zone_x"])) & done & ~death))
        flag_reward = np.where(flag_hit, F(p["flag_bonus"]), F(0.0))
        self.flag_awarded |= flag_hit

        stall_over = np.maximum((self.stall_steps - p["stall_window"] + 1).astype(F), F(0.0))
        stall_reward = -np.minimum(stall_over * F(p["stall_penalty"]), F(p["max_stall_penalty"]))

        a = np.asarray(masks, dtype=np.int64)
        jump, right, left = (a & 0x01) != 0, (a & 0x80) != 0, (a & 0x40) != 0
        start, select = (a & 0x08) != 0, (a & 0x04) != 0
        self.jump_streak = np.where(jump, self.jump_streak + 1, 0).astype(np.int32)
        action = np.zeros(a.shape[0], F)
        action = action - jump.astype(F) * F(p["jump_penalty"])
        action = action - (jump & ~right).astype(F) * F(p["neutral_jump_penalty"])
        repeated = np.maximum((self.jump_streak - p["repeated_jump_window"]).astype(F), F(0.0))
        action = action - np.minimum(repeated * F(p["repeated_jump_penalty"]), F(p["max_repeated_jump_penalty"]))
        action = action - left.astype(F) * F(p["left_penalty"])
        action = action - (left & right).astype(F) * F(p["bad_button_penalty"])
        action = action - (start | select).astype(F) * F(p["bad_button_penalty"])

        death_reward = np.where(done & death, F(-p["death_penalty"]), F(0.0))
        time_reward = np.full(a.shape[0], F(-p["time_penalty"]), F)

        self.last_x = x
        self.last_score = score
        self.last_coins = coins
        self.last_lives = ram[:, LIVES].astype(np.int32)
        self.last_level = self.level(ram)
        total = progress + checkpoint
        for term in (score_reward, kill_reward, coin_reward, finish_reward, flag_reward, stall_reward, action,
                     death_reward, time_reward):
            total = total + term
        return total.astype(F)

    def state_words(self) -> np.ndarray:
        """The tracking state as the kernel stores it: [11][n] 32-bit words."""
        rows = [self.last_x.view(np.uint32), self.max_x.view(np.uint32), self.checkpoint_index,
                self.last_score.view(np.uint32), self.last_coins, self.last_lives, self.last_level,
                self.stall_steps, self.jump_streak, self.finish_awarded.astype(np.int32),
                self.flag_awarded.astype(np.int32)]
        return np.stack([np.asarray(r).view(np.uint32) if r.dtype != np.uint32 else r for r in rows])
