"""The ROM-less synthetic batch, restated in numpy.

TEST INFRASTRUCTURE ONLY: the checker of nesle_create_synthetic /
nesle_synthetic_step (tests/); the product never imports it.

Follows the reference's synthetic CudaBatch(num_envs, frameskip):

* power-on: RAM cleared, x page $006D = 1, x screen $0086 = 2, y viewport
  $00B5 = 1, lives $075A = 2, player state $000E = 0, BCD time $07F8-$07FA =
  4, 0, 0; baselines x = $0102, time = 400 (cpp/include/nesle/cuda/
  batch_step.cuh:244-260, cpp/bindings/cuda_module.cu:469-512); a full reset
  also clears rewards, dones and step counts;
* step() with actions (cuda_module.cu:319-354, 546-565): Right (bit 7) +1,
  +1 more with B (bit 1), Left (bit 6) -1, x clamped to 0..$FFFF; every
  max(1, 24 // frameskip)-th step of a console, counted from its first, takes
  one from the time (not below 0);
* then the SMB reward rule (kernels.cu:12-17 -> batch_step.cuh:61-106):
  dx zeroed outside [-5, 5], time increases ignored, -25 when dying or dead,
  done on flag, dying, dead or game over;
* step_device() runs the rule alone (cuda_module.cu:620-633).
"""

from __future__ import annotations

import numpy as np

X_PAGE, X_SCREEN, Y_VIEWPORT, LIVES, STATE, TIME = 0x6D, 0x86, 0xB5, 0x75A, 0x0E, 0x7F8
GAME_MODE, FLOAT_STATE, ENEMY_BASE = 0x770, 0x1D, 0x16


class SyntheticModel:
    def __init__(self, num_envs: int, frameskip: int) -> None:
        self.n, self.frameskip = num_envs, frameskip
        self.ram = np.zeros((num_envs, 2048), dtype=np.uint8)
        self.prev_x = np.zeros(num_envs, dtype=np.int64)
        self.prev_time = np.zeros(num_envs, dtype=np.int64)
        self.rewards = np.zeros(num_envs, dtype=np.float32)
        self.dones = np.zeros(num_envs, dtype=np.uint8)
        self.steps = np.zeros(num_envs, dtype=np.int64)
        self.reset()

    def _power_on(self, rows: np.ndarray) -> None:
        self.ram[rows] = 0
        self.ram[rows, X_PAGE] = 1
        self.ram[rows, X_SCREEN] = 2
        self.ram[rows, Y_VIEWPORT] = 1
        self.ram[rows, LIVES] = 2
        self.ram[rows, TIME] = 4
        self.prev_x[rows] = 0x102
        self.prev_time[rows] = 400

    def reset(self) -> None:
        everyone = np.arange(self.n)
        self._power_on(everyone)
        self.rewards[:] = 0
        self.dones[:] = 0
        self.steps[:] = 0

    def reset_envs(self, mask: np.ndarray) -> None:
        self._power_on(np.flatnonzero(mask))

    def x(self) -> np.ndarray:
        return self.ram[:, X_PAGE].astype(np.int64) * 256 + self.ram[:, X_SCREEN]

    def time(self) -> np.ndarray:
        d = self.ram[:, TIME:TIME + 3].astype(np.int64) & 0x0F
        return d[:, 0] * 100 + d[:, 1] * 10 + d[:, 2]

    def step(self, actions: np.ndarray | None, auto_reset: bool = False) -> tuple[np.ndarray, np.ndarray]:
        """One env-step; ``actions`` None is step_device() (the rule alone)."""
        if actions is not None:
            a = np.asarray(actions, dtype=np.int64)
            dx = np.where(a & 0x80, 1 + ((a & 0x02) != 0), 0) - ((a & 0x40) != 0)
            x = np.clip(self.x() + dx, 0, 0xFFFF)
            self.ram[:, X_PAGE] = x >> 8
            self.ram[:, X_SCREEN] = x & 0xFF
            cadence = max(1, 24 // max(1, self.frameskip))
            tick = self.steps % cadence == 0
            self.steps += 1
            t = np.where(tick, np.maximum(self.time() - 1, 0), self.time())
            self.ram[:, TIME] = np.where(tick, t // 100, self.ram[:, TIME])
            self.ram[:, TIME + 1] = np.where(tick, (t // 10) % 10, self.ram[:, TIME + 1])
            self.ram[:, TIME + 2] = np.where(tick, t % 10, self.ram[:, TIME + 2])
        x, t = self.x(), self.time()
        dx = x - self.prev_x
        dx = np.where((dx < -5) | (dx > 5), 0, dx)
        dt = np.minimum(t - self.prev_time, 0)
        st = self.ram[:, STATE]
        dying = (st == 0x0B) | (self.ram[:, Y_VIEWPORT] > 1)
        dead = st == 0x06
        over = self.ram[:, LIVES] == 0xFF
        enemies = self.ram[:, ENEMY_BASE:ENEMY_BASE + 5]
        stage_over = (((enemies == 0x2D) | (enemies == 0x31)).any(axis=1)) & (self.ram[:, FLOAT_STATE] == 3)
        flag = (self.ram[:, GAME_MODE] == 2) | stage_over
        self.rewards = (dx + dt + np.where(dying | dead, -25, 0)).astype(np.float32)
        self.dones = (flag | dying | dead | over).astype(np.uint8)
        self.prev_x, self.prev_time = x, t
        rewards, dones = self.rewards.copy(), self.dones.copy()
        if auto_reset:
            self._power_on(np.flatnonzero(dones))
        return rewards, dones
