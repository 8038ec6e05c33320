"""SB3-style vector environment and single Gymnasium-style environment over the
HIP batch: the drop-in for the reference's ``nesle.env`` CUDA backend
(src/nesle/env.py:365-818 ``NesleVecEnv``, 821-905 ``NesleEnv``,
src/nesle/__init__.py:58-61 ``make_vec``).

Semantics kept from the reference's CUDA branch (env.py:549-741):

* observations are the RAM (``observation_mode="ram"``, [N, 2048]) or RGB
  frames ([N, 240, 256, 3]) copied to host NumPy arrays; RGB frames can be
  copied every ``observation_cadence``-th step only (stale in between);
* rewards/dones come from the batch's in-kernel reward rule; with
  ``max_episode_steps`` an episode is also cut (``truncated``) after that
  many steps;
* SB3's auto-reset contract: a done env's info carries
  ``terminal_observation`` (the last observation of the episode),
  ``terminated`` and ``truncated``; the env is reset (snapshot level or
  power-on) and the returned observation is the first one of the new
  episode; ``reset_infos`` is refreshed;
* ``reset_state_path(s)`` load FCEUX FCS states (gzip-wrapped ``.state``
  files are unpacked) or canonical state blobs; several states are assigned
  round-robin unless ``env_to_level`` says otherwise.

Only the HIP backend exists here: the reference's CPU "synthetic" and
"native" backends are not provided (``backend`` must be "auto" or "cuda").
Per-env Python loops of the reference (action-mask mapping, terminal
observation copies) are NumPy operations.
"""

from __future__ import annotations

import gzip
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Iterable, Sequence

import numpy as np

from nesle_amd import actions as _actions

try:
    import gymnasium as gym
    from gymnasium import spaces
except ImportError:  # gymnasium is optional
    gym = None
    spaces = None

try:
    from stable_baselines3.common.vec_env import VecEnv as _SB3VecEnv
except ImportError:  # stable-baselines3 is optional
    _SB3VecEnv = None

CPU_RAM_BYTES = 2048
FRAME_SHAPE = (240, 256, 3)
RAM_SHAPE = (CPU_RAM_BYTES,)
FRAME_DTYPE = np.uint8
BACKEND_NAME = "cuda-console"


class DiscreteSpace:
    """Stand-in for gymnasium.spaces.Discrete when gymnasium is absent."""

    def __init__(self, n: int) -> None:
        self.n = int(n)
        self.shape = ()
        self.dtype = np.int64

    def sample(self) -> int:
        return int(np.random.default_rng().integers(self.n))

    def contains(self, value: Any) -> bool:
        try:
            item = int(value)
        except (TypeError, ValueError):
            return False
        return 0 <= item < self.n


class BoxSpace:
    """Stand-in for gymnasium.spaces.Box when gymnasium is absent."""

    def __init__(self, low: int, high: int, shape: tuple[int, ...], dtype: Any) -> None:
        self.low, self.high, self.shape, self.dtype = low, high, shape, np.dtype(dtype)

    def sample(self) -> np.ndarray:
        return np.random.default_rng().integers(self.low, self.high + 1, size=self.shape, dtype=self.dtype)

    def contains(self, value: Any) -> bool:
        a = np.asarray(value)
        return a.shape == self.shape and a.dtype == self.dtype


def _box(low: int, high: int, shape: tuple[int, ...], dtype: Any) -> Any:
    return spaces.Box(low, high, shape=shape, dtype=dtype) if spaces is not None else BoxSpace(low, high, shape, dtype)


def _discrete(n: int) -> Any:
    return spaces.Discrete(n) if spaces is not None else DiscreteSpace(n)


def _normalize_observation_mode(observation_mode: str) -> str:
    key = observation_mode.lower().replace("-", "_")
    if key in {"rgb", "rgb_array", "frame"}:
        return "rgb_array"
    if key in {"ram", "cpu_ram"}:
        return "ram"
    raise ValueError("observation_mode must be 'rgb_array' or 'ram'")


def _load_reset_state(path: str | Path) -> bytes:
    """A reset state file; gzip-wrapped Stable Retro / Gym Retro ``.state`` files are unpacked."""
    raw = Path(path).read_bytes()
    return gzip.decompress(raw) if raw[:2] == b"\x1f\x8b" else raw


def _resolve_reset_state_paths(reset_state_path, reset_state_paths) -> list[Path] | None:
    if reset_state_path is not None and reset_state_paths is not None:
        raise ValueError("Pass exactly one of reset_state_path or reset_state_paths, not both")
    if reset_state_paths is not None:
        if len(reset_state_paths) == 0:
            raise ValueError("reset_state_paths must contain at least one path")
        return [Path(p) for p in reset_state_paths]
    if reset_state_path is not None:
        return [Path(reset_state_path)]
    return None


@dataclass(frozen=True)
class BackendConfig:
    rom_path: str
    num_envs: int
    frameskip: int = 4
    action_space: str | Sequence[int] = "simple"
    device: str = "auto"
    backend: str = "auto"
    observation_mode: str = "rgb_array"
    observation_cadence: int = 1
    max_episode_steps: int = 0
    reset_state_path: str | None = None


_VecEnvBase = _SB3VecEnv if _SB3VecEnv is not None else object


class NesleVecEnv(_VecEnvBase):
    """N consoles behind SB3's VecEnv ``reset``/``step`` contract."""

    metadata = {"render_modes": ["rgb_array"], "render_fps": 60}

    def __init__(self, rom_path: str, num_envs: int, frameskip: int = 4,
                 action_space: str | Sequence[int] = "simple", device: str = "auto", backend: str = "auto",
                 render_mode: str | None = "rgb_array", observation_mode: str = "rgb_array",
                 seed: int | None = None, observation_cadence: int = 1, max_episode_steps: int = 0,
                 reset_state_path: str | Path | None = None,
                 reset_state_paths: Sequence[str | Path] | None = None,
                 env_to_level: Sequence[int] | np.ndarray | None = None, *, rom_bytes: bytes | None = None) -> None:
        if num_envs <= 0:
            raise ValueError("num_envs must be positive")
        if frameskip <= 0:
            raise ValueError("frameskip must be positive")
        if observation_cadence <= 0:
            raise ValueError("observation_cadence must be positive")
        if render_mode not in (None, "rgb_array"):
            raise ValueError("render_mode must be None or 'rgb_array'")
        if backend.lower() not in ("auto", "cuda"):
            raise ValueError(f"backend {backend!r} is not provided: this package runs the HIP console "
                             "(backend='cuda' or 'auto')")
        observation_mode = _normalize_observation_mode(observation_mode)
        masks = _actions.action_masks(action_space)
        snapshots: list[bytes] | None = None
        levels: np.ndarray | None = None
        paths = _resolve_reset_state_paths(reset_state_path, reset_state_paths)
        if paths is not None:
            snapshots = [_load_reset_state(p) for p in paths]
            if len(snapshots) > 1:
                if env_to_level is None:
                    levels = (np.arange(num_envs) % len(snapshots)).astype(np.uint8)
                else:
                    levels = np.asarray(env_to_level, dtype=np.uint8)
                    if levels.shape != (num_envs,):
                        raise ValueError(f"env_to_level shape must be ({num_envs},), got {levels.shape}")
                    if int(levels.max(initial=0)) >= len(snapshots):
                        raise ValueError("env_to_level contains index >= number of snapshots")
            elif env_to_level is not None:
                raise ValueError("env_to_level requires more than one snapshot")
        rom = rom_bytes if rom_bytes is not None else Path(rom_path).read_bytes()

        self.config = BackendConfig(rom_path=str(rom_path), num_envs=num_envs, frameskip=frameskip,
                                    action_space=action_space, device=device, backend=backend,
                                    observation_mode=observation_mode, observation_cadence=observation_cadence,
                                    max_episode_steps=max_episode_steps,
                                    reset_state_path=None if reset_state_path is None else str(reset_state_path))
        self.render_mode = render_mode
        self.observation_mode = observation_mode
        self.num_envs = num_envs
        self.frameskip = frameskip
        self.observation_cadence = observation_cadence
        self.action_masks = masks
        self._mask_table = np.asarray(masks, dtype=np.uint8)
        self.action_space = _discrete(len(masks))
        self.observation_space = _box(0, 255, RAM_SHAPE if observation_mode == "ram" else FRAME_SHAPE, np.uint8)
        if _SB3VecEnv is not None:
            _SB3VecEnv.__init__(self, num_envs, self.observation_space, self.action_space)
        self.reset_infos: list[dict[str, Any]] = [{} for _ in range(num_envs)]
        self.buf_infos: list[dict[str, Any]] = [{} for _ in range(num_envs)]
        self._pending_actions: np.ndarray | None = None
        self._seeds: list[int | None] = [None] * num_envs
        self._options: list[dict[str, Any]] = [{} for _ in range(num_envs)]
        self._closed = False
        self._cuda_observations: np.ndarray | None = None
        self._cuda_step_count = 0
        self._cuda_env_step_counts = np.zeros(num_envs, dtype=np.int64)
        self._cuda_batch = self._make_batch(rom, snapshots, levels)
        self._ram_device = None   # torch view of the batch's RAM observation (imported on first use)
        self._backends: list[Any] = []

    def _make_batch(self, rom: bytes, snapshots: list[bytes] | None, levels: np.ndarray | None):
        """env.py:334-362."""
        from nesle_amd import load_cuda_core

        core = load_cuda_core()
        if snapshots is None:
            return core.CudaBatch(self.num_envs, self.frameskip, rom)
        if len(snapshots) == 1:
            return core.CudaBatch(self.num_envs, self.frameskip, rom, snapshots[0])
        return core.CudaBatch(self.num_envs, self.frameskip, rom, snapshots, levels)

    def _infos(self, **extra) -> list[dict[str, Any]]:
        base = {"backend": BACKEND_NAME, "observation_mode": self.observation_mode, **extra}
        copy = base.copy
        return [copy() for _ in range(self.num_envs)]

    def _ram_rows(self, dones: np.ndarray) -> np.ndarray:
        """The current RAM of the ``dones`` consoles, copied to the host alone
        (a gather on the device through the DLPack view, instead of the whole
        [N, 2048] observation)."""
        try:
            import torch
        except ImportError:  # pragma: no cover - torch is part of the image
            return np.asarray(self._cuda_batch.ram(), dtype=np.uint8)[dones]
        if self._ram_device is None:
            self._ram_device = torch.from_dlpack(self._cuda_batch.ram_device())
        idx = torch.from_numpy(np.nonzero(dones)[0]).to(self._ram_device.device)
        return self._ram_device.index_select(0, idx).cpu().numpy()

    def _masks_for(self, actions: Iterable[int]) -> np.ndarray:
        a = np.asarray(actions, dtype=np.int64).ravel()
        if a.shape != (self.num_envs,):
            raise ValueError(f"expected actions with shape ({self.num_envs},), got {a.shape}")
        if (a < 0).any() or (a >= len(self.action_masks)).any():
            raise ValueError("action index out of range")
        return self._mask_table[a]

    # ---- SB3 VecEnv contract -------------------------------------------------
    def reset(self) -> np.ndarray:
        """env.py:478-507."""
        frame = np.asarray(self._cuda_batch.reset(), dtype=np.uint8)
        if self.observation_mode == "ram":
            observations = np.asarray(self._cuda_batch.ram(), dtype=np.uint8)
        else:
            observations = frame
        self._cuda_observations = frame
        self._cuda_step_count = 0
        self._cuda_env_step_counts[:] = 0
        infos = self._infos()
        for env in range(self.num_envs):
            if self._options[env]:
                infos[env]["reset_options"] = dict(self._options[env])
        self.reset_infos = infos
        self._seeds = [None] * self.num_envs
        self._options = [{} for _ in range(self.num_envs)]
        return observations

    def step_async(self, actions: Iterable[int]) -> None:
        a = np.asarray(actions, dtype=np.int64).ravel()
        if a.shape != (self.num_envs,):
            raise ValueError(f"expected actions with shape ({self.num_envs},), got {a.shape}")
        self._pending_actions = a

    def step_wait(self):
        if self._pending_actions is None:
            raise RuntimeError("step_async must be called before step_wait")
        return self.step(self._pending_actions)

    def _truncation(self, dones: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        max_steps = self.config.max_episode_steps
        if max_steps > 0:
            truncated = self._cuda_env_step_counts >= max_steps
            return dones | truncated, truncated
        return dones, np.zeros(self.num_envs, dtype=bool)

    def _finish_episodes(self, dones, truncated, terminal: np.ndarray, infos) -> None:
        """Record terminal observations, reset done envs on the device."""
        done_envs = np.nonzero(dones)[0]
        # One gathered copy per step; each info holds its console's row of it.
        last = terminal[done_envs]
        for i, env in enumerate(done_envs.tolist()):
            info = infos[env]
            info["terminal_observation"] = last[i]
            info["terminated"] = not bool(truncated[env])
            info["truncated"] = bool(truncated[env])
            self.reset_infos[env] = {"backend": BACKEND_NAME, "observation_mode": self.observation_mode}
        self._cuda_batch.reset_envs(dones.astype(np.uint8))
        self._cuda_env_step_counts[dones] = 0

    def step(self, actions: Iterable[int]):
        """env.py:549-675: (observations, rewards, dones, infos)."""
        masks = self._masks_for(actions)
        self._cuda_step_count += 1
        self._cuda_env_step_counts += 1
        if self.observation_mode == "ram":
            result = self._cuda_batch.step(masks, render_frame=False, copy_obs=False)
            observations = np.asarray(self._cuda_batch.ram(), dtype=np.uint8)
            copied, stale, rgb_copied = True, False, False
        else:
            copy = self.observation_cadence <= 1 or self._cuda_step_count % self.observation_cadence == 0
            result = self._cuda_batch.step(masks, render_frame=copy, copy_obs=copy)
            if copy:
                observations = np.asarray(result["obs"], dtype=np.uint8)
                self._cuda_observations = observations
            elif self._cuda_observations is not None:
                observations = self._cuda_observations
            else:
                observations = np.asarray(self._cuda_batch.render(), dtype=np.uint8)
                self._cuda_observations = observations
            copied, stale, rgb_copied = copy, not copy, copy
        rewards = np.asarray(result["rewards"], dtype=np.float32)
        dones, truncated = self._truncation(np.asarray(result["dones"], dtype=bool))
        infos = self._infos(observation_cadence=self.observation_cadence, observations_copied=copied,
                            observations_stale=stale, rgb_observations_copied=rgb_copied)
        if dones.any():
            # The returned observation of a done env is the first of its new episode.
            self._finish_episodes(dones, truncated, observations, infos)
            if self.observation_mode == "ram":
                observations[dones] = self._ram_rows(dones)
            else:
                fresh = np.asarray(self._cuda_batch.render(), dtype=np.uint8)
                self._cuda_observations = fresh
                observations = np.where(dones[:, None, None, None], fresh, observations)
        self._pending_actions = None
        self.buf_infos = infos
        return observations, rewards, dones, infos

    def step_reward(self, actions: Iterable[int]):
        """env.py:677-741: step without copying observations; (rewards, dones, infos)."""
        masks = self._masks_for(actions)
        self._cuda_env_step_counts += 1
        result = self._cuda_batch.step(masks, render_frame=False, copy_obs=False)
        rewards = np.asarray(result["rewards"], dtype=np.float32)
        dones, truncated = self._truncation(np.asarray(result["dones"], dtype=bool))
        infos = self._infos(observations_copied=False)
        if dones.any():
            terminal = (np.asarray(self._cuda_batch.ram(), dtype=np.uint8) if self.observation_mode == "ram"
                        else np.asarray(self._cuda_batch.render(), dtype=np.uint8))
            self._finish_episodes(dones, truncated, terminal, infos)
        self._pending_actions = None
        self.buf_infos = infos
        return rewards, dones, infos

    def render(self, mode: str | None = None) -> np.ndarray | None:
        mode = self.render_mode if mode is None else mode
        if mode is None:
            return None
        if mode != "rgb_array":
            raise ValueError("only rgb_array rendering is supported")
        return np.asarray(self._cuda_batch.render(), dtype=FRAME_DTYPE)

    def get_images(self) -> list[np.ndarray]:
        rendered = self.render()
        return [rendered[e].copy() for e in range(self.num_envs)] if rendered is not None else []

    def close(self) -> None:
        self._closed = True

    def seed(self, seed: int | None = None) -> list[int | None]:
        self._seeds = [None if seed is None else seed + env for env in range(self.num_envs)]
        return list(self._seeds)

    def set_options(self, options: dict[str, Any] | Sequence[dict[str, Any]] | None = None) -> None:
        if options is None:
            self._options = [{} for _ in range(self.num_envs)]
        elif isinstance(options, dict):
            self._options = [dict(options) for _ in range(self.num_envs)]
        elif len(options) != self.num_envs:
            raise ValueError(f"expected {self.num_envs} option dictionaries, got {len(options)}")
        else:
            self._options = [dict(o) for o in options]

    def get_attr(self, attr_name: str, indices=None) -> list[Any]:
        if attr_name == "render_mode":
            return [self.render_mode for _ in self._resolve_indices(indices)]
        if attr_name == "name":
            return [str(self._cuda_batch.name) for _ in self._resolve_indices(indices)]
        raise AttributeError(f"the HIP vector env has no per-env attribute {attr_name!r}")

    def set_attr(self, attr_name: str, value: Any, indices=None) -> None:
        raise AttributeError(f"the HIP vector env has no per-env attribute {attr_name!r}")

    def env_method(self, method_name: str, *method_args: Any, indices=None, **method_kwargs: Any) -> list[Any]:
        if method_name == "render":
            rendered = self.render()
            return [rendered[i].copy() for i in self._resolve_indices(indices)] if rendered is not None else []
        raise AttributeError(f"the HIP vector env has no per-env method {method_name!r}")

    def env_is_wrapped(self, wrapper_class: type[Any], indices=None) -> list[bool]:
        return [False for _ in self._resolve_indices(indices)]

    def _resolve_indices(self, indices) -> list[int]:
        if indices is None:
            return list(range(self.num_envs))
        if isinstance(indices, int):
            return [indices]
        return [int(i) for i in indices]


_EnvBase = gym.Env if gym is not None else object


class NesleEnv(_EnvBase):
    """One console behind the Gymnasium ``reset``/``step`` API (env.py:821-905)."""

    metadata = {"render_modes": ["rgb_array"], "render_fps": 60}

    def __init__(self, rom_path: str, frameskip: int = 4, action_space: str | Sequence[int] = "simple",
                 device: str = "auto", backend: str = "auto", render_mode: str | None = "rgb_array",
                 observation_mode: str = "rgb_array", observation_cadence: int = 1, max_episode_steps: int = 0,
                 reset_state_path: str | Path | None = None, reset_state_paths: Sequence[str | Path] | None = None,
                 env_to_level: Sequence[int] | np.ndarray | None = None, *, rom_bytes: bytes | None = None) -> None:
        if gym is not None:
            super().__init__()
        self.vector_env = NesleVecEnv(rom_path=rom_path, num_envs=1, frameskip=frameskip, action_space=action_space,
                                      device=device, backend=backend, render_mode=render_mode,
                                      observation_mode=observation_mode, observation_cadence=observation_cadence,
                                      max_episode_steps=max_episode_steps, reset_state_path=reset_state_path,
                                      reset_state_paths=reset_state_paths, env_to_level=env_to_level,
                                      rom_bytes=rom_bytes)
        self.render_mode = render_mode
        self.observation_space = self.vector_env.observation_space
        self.action_space = self.vector_env.action_space

    def reset(self, *, seed: int | None = None, options: dict[str, Any] | None = None):
        if gym is not None:
            super().reset(seed=seed)
        if seed is not None:
            self.vector_env.seed(seed)
        if options is not None:
            self.vector_env.set_options(options)
        observations = self.vector_env.reset()
        return observations[0], self.vector_env.reset_infos[0]

    def step(self, action: int):
        observations, rewards, dones, infos = self.vector_env.step([action])
        info = infos[0]
        return (observations[0], float(rewards[0]), bool(info.get("terminated", dones[0])),
                bool(info.get("truncated", False)), info)

    def render(self) -> np.ndarray | None:
        rendered = self.vector_env.render()
        return None if rendered is None else rendered[0]

    def close(self) -> None:
        self.vector_env.close()


def make_vec(*args, **kwargs) -> NesleVecEnv:
    """src/nesle/__init__.py:58-61."""
    return NesleVecEnv(*args, **kwargs)


def make(*args, **kwargs) -> NesleEnv:
    return NesleEnv(*args, **kwargs)
