"""Stable-Baselines3 / Gymnasium environments over the HIP console batch: the
drop-in for the CUDA backend of the reference's ``nesle.env``
(src/nesle/env.py: ``NesleVecEnv``, ``NesleEnv``; src/nesle/__init__.py
``make_vec``).

The contract, as the reference's tests state it
(tests/test_critical_fixes.py:59-196, tests/test_env_reset_state.py):

* ``reset()`` returns the observations of every console after a reset:
  RAM rows ``[N, 2048]`` (``observation_mode="ram"``) or RGB frames
  ``[N, 240, 256, 3]``, host NumPy arrays;
* ``step(actions)`` takes one action index per console (into the chosen
  action table) and returns ``(observations, rewards, dones, infos)``; a
  console whose episode ended (the batch's reward rule says done, or it ran
  ``max_episode_steps`` steps) is reset before ``step`` returns: its
  observation is the first of the new episode and its info holds
  ``terminal_observation`` (the last observation of the old one),
  ``terminated`` and ``truncated`` (a step-limit cut is a truncation even if
  the rule also said done); ``reset_infos`` is refreshed for it;
* RGB observations can be copied every ``observation_cadence``-th step
  only; in between the previous copy is returned and marked stale;
* ``step_reward(actions)`` is the same step without observation copies;
* several reset states are spread over the consoles round-robin unless
  ``env_to_level`` names each console's state; a console resets to its own.

Design here: the batch (``nesle_amd._cuda_core.CudaBatch``) does the
emulation and the resets on the device; this module keeps three small
host-side pieces — the action table lookup, an episode clock per console
(``_EpisodeClock``) and an observation reader (``_Observer``) that knows
which copy each mode needs — and builds the SB3 return values from whole
arrays (no per-console Python work except the info dicts SB3 requires).
Only the HIP backend exists (``backend`` "auto" or "cuda").
"""

from __future__ import annotations

import gzip
from pathlib import Path
from typing import Any, Iterable, Sequence

import numpy as np

from nesle_amd import actions as _actions

try:
    import gymnasium as gym
    from gymnasium import spaces as _gym_spaces
except ImportError:  # gymnasium is optional
    gym = None
    _gym_spaces = None

try:
    from stable_baselines3.common.vec_env import VecEnv as _SB3VecEnv
except ImportError:  # stable-baselines3 is optional
    _SB3VecEnv = None

CPU_RAM_BYTES = 2048
FRAME_SHAPE = (240, 256, 3)
BACKEND_NAME = "cuda-console"
GZIP_MAGIC = b"\x1f\x8b"

# Accepted spellings of the two observation modes (lower case, '-' as '_').
_MODE_ALIASES = {"rgb": "rgb_array", "rgb_array": "rgb_array", "frame": "rgb_array",
                 "ram": "ram", "cpu_ram": "ram"}


def observation_mode_of(name: str) -> str:
    """Canonical observation mode ("rgb_array" or "ram") for an accepted name."""
    mode = _MODE_ALIASES.get(str(name).lower().replace("-", "_"))
    if mode is None:
        raise ValueError("observation_mode must be 'rgb_array' or 'ram'")
    return mode


def read_state_file(path: str | Path) -> bytes:
    """Bytes of a reset-state file; Gym/Stable Retro ``.state`` files are
    gzip streams and come back unpacked."""
    data = Path(path).read_bytes()
    if data.startswith(GZIP_MAGIC):
        data = gzip.decompress(data)
    return data


def state_file_list(reset_state_path, reset_state_paths) -> list[Path]:
    """The reset-state files asked for (empty: power-on resets)."""
    given = [x for x in (reset_state_path, reset_state_paths) if x is not None]
    if len(given) == 2:
        raise ValueError("Pass exactly one of reset_state_path or reset_state_paths, not both")
    if reset_state_paths is not None and len(reset_state_paths) == 0:
        raise ValueError("reset_state_paths must contain at least one path")
    if reset_state_path is not None:
        return [Path(reset_state_path)]
    return [Path(p) for p in (reset_state_paths or ())]


def level_map(num_states: int, num_envs: int, env_to_level) -> np.ndarray | None:
    """Per-console reset state: explicit, or round-robin over the states;
    None when there is at most one state (every console shares it)."""
    if num_states <= 1:
        if env_to_level is not None:
            raise ValueError("env_to_level requires more than one snapshot")
        return None
    if env_to_level is None:
        return (np.arange(num_envs) % num_states).astype(np.uint8)
    levels = np.asarray(env_to_level)
    if levels.shape != (num_envs,):
        raise ValueError(f"env_to_level shape must be ({num_envs},), got {levels.shape}")
    if levels.size and (levels.min() < 0 or levels.max() >= num_states):
        raise ValueError("env_to_level contains index >= number of snapshots")
    return levels.astype(np.uint8)


class _Discrete:
    """Discrete(n) when gymnasium is not installed."""

    def __init__(self, n: int) -> None:
        self.n, self.shape, self.dtype = int(n), (), np.dtype(np.int64)

    def sample(self) -> int:
        return int(np.random.randint(self.n))

    def contains(self, x: Any) -> bool:
        return isinstance(x, (int, np.integer)) and 0 <= int(x) < self.n


class _Box:
    """Box(0, 255, shape, uint8) when gymnasium is not installed."""

    def __init__(self, shape: tuple[int, ...]) -> None:
        self.low, self.high, self.shape, self.dtype = 0, 255, tuple(shape), np.dtype(np.uint8)

    def sample(self) -> np.ndarray:
        return np.random.randint(0, 256, size=self.shape).astype(np.uint8)

    def contains(self, x: Any) -> bool:
        return isinstance(x, np.ndarray) and x.shape == self.shape and x.dtype == self.dtype


def _spaces(obs_shape: tuple[int, ...], n_actions: int) -> tuple[Any, Any]:
    if _gym_spaces is None:
        return _Box(obs_shape), _Discrete(n_actions)
    return _gym_spaces.Box(0, 255, shape=obs_shape, dtype=np.uint8), _gym_spaces.Discrete(n_actions)


class _EpisodeClock:
    """Steps since each console's episode began, and the optional limit."""

    def __init__(self, num_envs: int, limit: int) -> None:
        self.limit = int(limit)
        self.steps = np.zeros(num_envs, dtype=np.int64)

    def tick(self) -> np.ndarray:
        """Advance every console by one step; returns the consoles whose
        episode hit the limit."""
        self.steps += 1
        if self.limit <= 0:
            return np.zeros(self.steps.shape, dtype=bool)
        return self.steps >= self.limit

    def restart(self, which: np.ndarray | None = None) -> None:
        if which is None:
            self.steps.fill(0)
        else:
            self.steps[which] = 0


class _Observer:
    """Reads the observation a mode needs from the batch.

    RAM: the batch's RAM rows every step (after resets, only the reset rows
    are fetched again, gathered on the device).  RGB: the frame copy of the
    step on cadence steps, the previous copy otherwise."""

    def __init__(self, batch, mode: str, cadence: int) -> None:
        self.batch, self.mode, self.cadence = batch, mode, cadence
        self.frames: np.ndarray | None = None   # last RGB copy handed out
        self.steps = 0
        self._ram_dev = None

    def after_reset(self, frames: np.ndarray) -> np.ndarray:
        self.steps = 0
        self.frames = frames
        return self.batch.ram() if self.mode == "ram" else frames

    def step(self, masks: np.ndarray) -> tuple[dict, np.ndarray, dict]:
        """One batch step; returns (step result, observations, info flags)."""
        self.steps += 1
        if self.mode == "ram":
            result = self.batch.step(masks, render_frame=False, copy_obs=False)
            return result, self.batch.ram(), {"observations_copied": True, "observations_stale": False,
                                              "rgb_observations_copied": False}
        fresh = self.cadence <= 1 or self.steps % self.cadence == 0
        result = self.batch.step(masks, render_frame=fresh, copy_obs=fresh)
        if fresh:
            self.frames = result["obs"]
        elif self.frames is None:
            self.frames = self.batch.render()
        return result, self.frames, {"observations_copied": fresh, "observations_stale": not fresh,
                                     "rgb_observations_copied": fresh}

    def current(self) -> np.ndarray:
        """The observation of every console now (no cadence)."""
        return self.batch.ram() if self.mode == "ram" else self.batch.render()

    def replace_rows(self, obs: np.ndarray, which: np.ndarray) -> np.ndarray:
        """``obs`` with the rows of ``which`` replaced by the current state."""
        if self.mode == "ram":
            obs[which] = self._ram_gather(np.flatnonzero(which))
            return obs
        self.frames = self.batch.render()
        return np.where(which[:, None, None, None], self.frames, obs)

    def _ram_gather(self, rows: np.ndarray) -> np.ndarray:
        """RAM rows of ``rows`` now: gathered on the device through the DLPack
        view when torch is importable (only those rows cross PCIe), else from
        a whole host copy, as the reference re-reads ``ram()`` (torch is an
        optional dependency of the environment layer)."""
        try:
            import torch
        except ImportError:
            return self.batch.ram()[rows]
        if self._ram_dev is None:
            self._ram_dev = torch.from_dlpack(self.batch.ram_device())
        index = torch.as_tensor(rows, dtype=torch.long).to(self._ram_dev.device)
        return self._ram_dev.index_select(0, index).cpu().numpy()


_VecEnvBase = _SB3VecEnv if _SB3VecEnv is not None else object


class NesleVecEnv(_VecEnvBase):
    """``num_envs`` consoles behind SB3's ``VecEnv`` interface."""

    metadata = {"render_modes": ["rgb_array"], "render_fps": 60}

    def __init__(self, rom_path: str, num_envs: int, frameskip: int = 4,
                 action_space: str | Sequence[int] = "simple", device: str = "auto", backend: str = "auto",
                 render_mode: str | None = "rgb_array", observation_mode: str = "rgb_array",
                 seed: int | None = None, observation_cadence: int = 1, max_episode_steps: int = 0,
                 reset_state_path: str | Path | None = None,
                 reset_state_paths: Sequence[str | Path] | None = None,
                 env_to_level: Sequence[int] | np.ndarray | None = None, *, rom_bytes: bytes | None = None) -> None:
        # Every argument is checked before the ROM is read or the GPU touched.
        for name, value in (("num_envs", num_envs), ("frameskip", frameskip),
                            ("observation_cadence", observation_cadence)):
            if value <= 0:
                raise ValueError(f"{name} must be positive")
        if render_mode is not None and render_mode != "rgb_array":
            raise ValueError("render_mode must be None or 'rgb_array'")
        if str(backend).lower() not in ("auto", "cuda"):
            raise ValueError(f"backend {backend!r} is not provided: this package runs the HIP console "
                             "(backend='cuda' or 'auto')")
        mode = observation_mode_of(observation_mode)
        table = _actions.action_masks(action_space)
        files = state_file_list(reset_state_path, reset_state_paths)
        states = [read_state_file(p) for p in files]
        levels = level_map(len(states), num_envs, env_to_level)

        self.num_envs, self.frameskip = int(num_envs), int(frameskip)
        self.observation_mode, self.observation_cadence = mode, int(observation_cadence)
        self.max_episode_steps = int(max_episode_steps)
        self.render_mode = render_mode
        self.device, self.backend = device, backend
        self.action_masks = tuple(table)
        self._table = np.asarray(table, dtype=np.uint8)
        obs_shape = (CPU_RAM_BYTES,) if mode == "ram" else FRAME_SHAPE
        self.observation_space, self.action_space = _spaces(obs_shape, len(table))
        if _SB3VecEnv is not None:
            _SB3VecEnv.__init__(self, self.num_envs, self.observation_space, self.action_space)

        rom = rom_bytes if rom_bytes is not None else Path(rom_path).read_bytes()
        self._cuda_batch = self._open_batch(rom, states, levels)
        self._observer = _Observer(self._cuda_batch, mode, self.observation_cadence)
        self._clock = _EpisodeClock(self.num_envs, self.max_episode_steps)
        self._queued: np.ndarray | None = None
        self._seeds: list[int | None] = [None] * self.num_envs
        self._options: list[dict[str, Any]] = [{} for _ in range(self.num_envs)]
        self.reset_infos: list[dict[str, Any]] = [self._base_info() for _ in range(self.num_envs)]
        self.buf_infos: list[dict[str, Any]] = [{} for _ in range(self.num_envs)]
        self.closed = False

    def _open_batch(self, rom: bytes, states: list[bytes], levels: np.ndarray | None):
        """The batch: power-on resets, one shared reset state, or one state per
        console (the CudaBatch constructor forms of cuda_module.cu:389-467)."""
        from nesle_amd import load_cuda_core

        core = load_cuda_core()
        args: tuple = (self.num_envs, self.frameskip, rom)
        if len(states) == 1:
            args += (states[0],)
        elif states:
            args += (states, levels)
        return core.CudaBatch(*args)

    def _base_info(self) -> dict[str, Any]:
        return {"backend": BACKEND_NAME, "observation_mode": self.observation_mode}

    def _masks(self, actions: Iterable[int]) -> np.ndarray:
        index = np.asarray(actions, dtype=np.int64).reshape(-1)
        if index.shape != (self.num_envs,):
            raise ValueError(f"expected actions with shape ({self.num_envs},), got {index.shape}")
        if index.size and (index.min() < 0 or index.max() >= self._table.size):
            raise ValueError("action index out of range")
        return self._table[index]

    # ---- SB3 VecEnv ---------------------------------------------------------------
    def reset(self) -> np.ndarray:
        frames = self._cuda_batch.reset()
        obs = self._observer.after_reset(frames)
        self._clock.restart()
        infos = [self._base_info() for _ in range(self.num_envs)]
        for info, opts in zip(infos, self._options):
            if opts:
                info["reset_options"] = dict(opts)
        self.reset_infos = infos
        self._seeds = [None] * self.num_envs
        self._options = [{} for _ in range(self.num_envs)]
        return obs

    def step_async(self, actions: Iterable[int]) -> None:
        index = np.asarray(actions, dtype=np.int64).reshape(-1)
        if index.shape != (self.num_envs,):
            raise ValueError(f"expected actions with shape ({self.num_envs},), got {index.shape}")
        self._queued = index

    def step_wait(self):
        if self._queued is None:
            raise RuntimeError("step_async must be called before step_wait")
        return self.step(self._queued)

    def _end_episodes(self, rule_done: np.ndarray, cut: np.ndarray, last_obs: np.ndarray,
                      infos: list[dict[str, Any]]) -> np.ndarray:
        """Reset the consoles whose episode ended; fills their infos and
        reset_infos.  Returns the done mask."""
        done = rule_done | cut
        ended = np.flatnonzero(done)
        if ended.size == 0:
            return done
        terminal = last_obs[ended]          # one gathered copy; each info keeps its row
        for row, env in enumerate(ended.tolist()):
            infos[env]["terminal_observation"] = terminal[row]
            infos[env]["truncated"] = bool(cut[env])
            infos[env]["terminated"] = not cut[env]
            self.reset_infos[env] = self._base_info()
        self._cuda_batch.reset_envs(done.astype(np.uint8))
        self._clock.restart(done)
        return done

    def step(self, actions: Iterable[int]):
        masks = self._masks(actions)
        cut = self._clock.tick()
        result, obs, flags = self._observer.step(masks)
        rewards = np.asarray(result["rewards"], dtype=np.float32)
        info = {**self._base_info(), "observation_cadence": self.observation_cadence, **flags}
        infos = [info.copy() for _ in range(self.num_envs)]
        done = self._end_episodes(np.asarray(result["dones"], dtype=bool), cut, obs, infos)
        if done.any():
            # The returned observation of a reset console is its new episode's first.
            obs = self._observer.replace_rows(obs, done)
        self._queued = None
        self.buf_infos = infos
        return obs, rewards, done, infos

    def step_reward(self, actions: Iterable[int]):
        """A step that copies rewards and dones only: (rewards, dones, infos)
        (env.py:677-741); terminal observations are read only when an
        episode ends."""
        masks = self._masks(actions)
        cut = self._clock.tick()
        result = self._cuda_batch.step(masks, render_frame=False, copy_obs=False)
        rewards = np.asarray(result["rewards"], dtype=np.float32)
        rule_done = np.asarray(result["dones"], dtype=bool)
        infos = [{**self._base_info(), "observations_copied": False} for _ in range(self.num_envs)]
        last = self._observer.current() if (rule_done | cut).any() else None
        done = self._end_episodes(rule_done, cut, last, infos) if last is not None else rule_done | cut
        self._queued = None
        self.buf_infos = infos
        return rewards, done, infos

    def render(self, mode: str | None = None) -> np.ndarray | None:
        mode = mode or self.render_mode
        if mode is None:
            return None
        if mode != "rgb_array":
            raise ValueError("only rgb_array rendering is supported")
        return self._cuda_batch.render()

    def get_images(self) -> list[np.ndarray]:
        frames = self.render()
        return [] if frames is None else list(frames.copy())

    def close(self) -> None:
        self.closed = True

    def seed(self, seed: int | None = None) -> list[int | None]:
        self._seeds = [None] * self.num_envs if seed is None else list(range(seed, seed + self.num_envs))
        return list(self._seeds)

    def set_options(self, options: dict[str, Any] | Sequence[dict[str, Any]] | None = None) -> None:
        if options is None:
            options = [{}] * self.num_envs
        elif isinstance(options, dict):
            options = [options] * self.num_envs
        elif len(options) != self.num_envs:
            raise ValueError(f"expected {self.num_envs} option dictionaries, got {len(options)}")
        self._options = [dict(o) for o in options]

    def _indices(self, indices) -> list[int]:
        if indices is None:
            return list(range(self.num_envs))
        return [int(indices)] if isinstance(indices, (int, np.integer)) else [int(i) for i in indices]

    def get_attr(self, attr_name: str, indices=None) -> list[Any]:
        values = {"render_mode": self.render_mode, "name": str(self._cuda_batch.name)}
        if attr_name not in values:
            raise AttributeError(f"the HIP vector env has no per-env attribute {attr_name!r}")
        return [values[attr_name]] * len(self._indices(indices))

    def set_attr(self, attr_name: str, value: Any, indices=None) -> None:
        raise AttributeError(f"the HIP vector env has no per-env attribute {attr_name!r}")

    def env_method(self, method_name: str, *method_args: Any, indices=None, **method_kwargs: Any) -> list[Any]:
        if method_name != "render":
            raise AttributeError(f"the HIP vector env has no per-env method {method_name!r}")
        frames = self.render()
        return [] if frames is None else [frames[i].copy() for i in self._indices(indices)]

    def env_is_wrapped(self, wrapper_class: type[Any], indices=None) -> list[bool]:
        return [False] * len(self._indices(indices))


_EnvBase = gym.Env if gym is not None else object


class NesleEnv(_EnvBase):
    """One console behind Gymnasium's ``reset``/``step`` (five-tuple) API: a
    one-console ``NesleVecEnv`` underneath."""

    metadata = {"render_modes": ["rgb_array"], "render_fps": 60}

    def __init__(self, rom_path: str, frameskip: int = 4, action_space: str | Sequence[int] = "simple",
                 device: str = "auto", backend: str = "auto", render_mode: str | None = "rgb_array",
                 observation_mode: str = "rgb_array", observation_cadence: int = 1, max_episode_steps: int = 0,
                 reset_state_path: str | Path | None = None, reset_state_paths: Sequence[str | Path] | None = None,
                 env_to_level: Sequence[int] | np.ndarray | None = None, *, rom_bytes: bytes | None = None) -> None:
        if gym is not None:
            super().__init__()
        self.vector_env = NesleVecEnv(rom_path, 1, frameskip=frameskip, action_space=action_space, device=device,
                                      backend=backend, render_mode=render_mode, observation_mode=observation_mode,
                                      observation_cadence=observation_cadence, max_episode_steps=max_episode_steps,
                                      reset_state_path=reset_state_path, reset_state_paths=reset_state_paths,
                                      env_to_level=env_to_level, rom_bytes=rom_bytes)
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
        return self.vector_env.reset()[0], self.vector_env.reset_infos[0]

    def step(self, action: int):
        obs, rewards, dones, infos = self.vector_env.step([action])
        info = infos[0]
        truncated = bool(info.get("truncated", False))
        terminated = bool(info["terminated"]) if "terminated" in info else bool(dones[0])
        return obs[0], float(rewards[0]), terminated, truncated, info

    def render(self) -> np.ndarray | None:
        frames = self.vector_env.render()
        return None if frames is None else frames[0]

    def close(self) -> None:
        self.vector_env.close()


def make_vec(*args, **kwargs) -> NesleVecEnv:
    """The vector environment (src/nesle/__init__.py:58-61)."""
    return NesleVecEnv(*args, **kwargs)


def make(*args, **kwargs) -> NesleEnv:
    """The single-console environment."""
    return NesleEnv(*args, **kwargs)
