"""GPU-resident PPO on the MI355X console: the drop-in for the reference's
``nesle.native_ppo`` (src/nesle/native_ppo.py).

Same configuration (``NativePPOConfig``), model (2,048 RAM bytes / 255 -> 256
tanh -> 256 tanh -> action logits + value), GAE (``compute_gae``), clipped
PPO loss, Adam, checkpoint fields and log line as the reference trainer
(native_ppo.py:388-603).  The rollout keeps everything on the device and on
one stream:

* the batch runs on PyTorch's current stream (``CudaBatch.set_stream``), so
  policy kernels, the step kernel and the RAM transpose are ordered without
  host synchronisation;
* done consoles are restored by the step's auto-reset, a restore kernel on
  the same stream right after the step kernel (the reference calls
  ``reset_envs`` with a host mask after a ``done.any()`` host read every
  step, native_ppo.py:498-507); the RAM view after the step shows
  the post-reset state for them, exactly what the reference's
  ``reset_envs`` + ``ram_device`` sequence returns;
* episode-length timeouts (``max_episode_steps``) reset through a device
  mask; episode returns are summed on the device and read once per log line;
* the RAM, reward and done views are imported through DLPack once, before the
  loop (their device buffers never move).

``train_native_ppo`` returns the timing split the workload reports: wall time
of rollout and update phases and the step kernel's own time (HIP events on
the batch's stream), whose share of the wall time is the emulator share.
"""

from __future__ import annotations

import argparse
import ctypes
import math
import time
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Sequence

import numpy as np

from nesle_amd import actions as _actions


@dataclass
class NativePPOConfig:
    rom_path: str
    num_envs: int = 1024
    total_timesteps: int = 1_000_000
    n_steps: int = 128
    batch_size: int = 8192
    update_epochs: int = 4
    frameskip: int = 4
    action_space: str = "simple_with_start"
    reset_state_path: str | None = None
    reset_state_paths: tuple[str, ...] = ()
    max_episode_steps: int = 0
    learning_rate: float = 2.5e-4
    gamma: float = 0.99
    gae_lambda: float = 0.95
    clip_coef: float = 0.1
    ent_coef: float = 0.01
    vf_coef: float = 0.5
    max_grad_norm: float = 0.5
    hidden_size: int = 256
    # "minimal": the batch's in-kernel reward rule; "smart": the reference's
    # shaped SMB reward (SmartMarioReward, a HIP kernel over the step's RAM).
    reward_mode: str = "minimal"
    # Smart-reward overrides (None keeps the reward's defaults).
    flag_bonus: float | None = None
    finish_zone_bonus: float | None = None
    death_penalty: float | None = None
    seed: int = 1
    checkpoint_path: str = "nesle_native_ppo.pt"
    log_interval: int = 1
    progress_bar: bool = False
    # Additions: weight init ("orthogonal" as the reference trainer, or
    # "xavier"), the in-kernel reward rule (CudaBatch ``reward=`` spec; None =
    # the SMB rule), whether to write checkpoints, and whether rollouts after
    # the first replay a captured HIP graph.
    init: str = "orthogonal"
    reward: dict | None = None
    save_checkpoints: bool = True
    cuda_graph: bool = True
    env_to_level: tuple[int, ...] | None = field(default=None, repr=False)


def _require_torch():
    try:
        import torch
        import torch.nn as nn
        from torch.distributions.categorical import Categorical
    except ImportError as exc:  # pragma: no cover - torch is part of the image
        raise SystemExit("native PPO needs PyTorch (ROCm build)") from exc
    return torch, nn, Categorical


def _make_model(obs_dim: int, action_dim: int, hidden_size: int, init: str = "orthogonal", device=None):
    """The reference's RamActorCritic (native_ppo.py:76-101)."""
    torch, nn, _ = _require_torch()
    if init not in ("orthogonal", "xavier"):
        raise ValueError(f"unknown init {init!r}: 'orthogonal' or 'xavier'")

    def init_layer(layer, gain: float) -> None:
        if init == "orthogonal":
            nn.init.orthogonal_(layer.weight, gain)
        else:
            nn.init.xavier_uniform_(layer.weight, gain)
        nn.init.constant_(layer.bias, 0.0)

    class RamActorCritic(nn.Module):
        def __init__(self) -> None:
            super().__init__()
            self.net = nn.Sequential(nn.Linear(obs_dim, hidden_size), nn.Tanh(),
                                     nn.Linear(hidden_size, hidden_size), nn.Tanh())
            self.actor = nn.Linear(hidden_size, action_dim)
            self.critic = nn.Linear(hidden_size, 1)
            for layer in self.net:
                if isinstance(layer, nn.Linear):
                    init_layer(layer, math.sqrt(2.0))
            init_layer(self.actor, 0.01)
            init_layer(self.critic, 1.0)

        def forward(self, obs):
            x = obs.float().div_(255.0)
            features = self.net(x)
            return self.actor(features), self.critic(features).squeeze(-1)

    return RamActorCritic().to(device if device is not None else torch.device("cuda"))


def compute_gae(rewards, dones, values, next_done, next_value, gamma: float, gae_lambda: float):
    """Generalised advantage estimation over [T, N] tensors (native_ppo.py:609-624):
    ``dones[t]`` marks that the observation at t started a new episode."""
    torch, _, _ = _require_torch()
    T = rewards.shape[0]
    advantages = torch.empty_like(rewards)
    lastgaelam = torch.zeros_like(rewards[0])
    for t in range(T - 1, -1, -1):
        if t == T - 1:
            nonterminal, next_values = 1.0 - next_done, next_value
        else:
            nonterminal, next_values = 1.0 - dones[t + 1], values[t + 1]
        delta = rewards[t] + gamma * next_values * nonterminal - values[t]
        lastgaelam = delta + gamma * gae_lambda * nonterminal * lastgaelam
        advantages[t] = lastgaelam
    return advantages, advantages + values


def _explained_variance(values, returns) -> float:
    """1 - Var[returns - values] / Var[returns] (unbiased variances, one
    device reduction for both); NaN when the returns are constant."""
    torch, _, _ = _require_torch()
    with torch.no_grad():
        var_ret, var_err = torch.stack((returns, returns - values)).var(dim=1).tolist()
    return float("nan") if var_ret == 0.0 else 1.0 - var_err / var_ret


# ---- shaped reward ---------------------------------------------------------

def smart_reward_params(config: NativePPOConfig):
    """The shaped reward's constants (the reference's TorchSmartMarioReward
    values, native_ppo.py:135-157) with the config's overrides
    (native_ppo.py:424-432)."""
    from nesle_amd import abi

    params = abi.ShapedParams()
    abi.lib().nesle_smb_shaped_defaults(ctypes.byref(params))
    for name in ("flag_bonus", "finish_zone_bonus", "death_penalty"):
        value = getattr(config, name)
        if value is not None:
            setattr(params, name, float(value))
    return params


class SmartMarioReward:
    """The reference trainer's shaped Super Mario Bros. reward
    (TorchSmartMarioReward, native_ppo.py:120-316) as one HIP kernel per call
    (``nesle_smb_shaped_reward``, include/nesle_ppo.h): progress, checkpoints,
    score, kills, coins, finish zone, flag, stalling, button, death and time
    terms, bit-identical to the reference's float32 tensor arithmetic.  The
    tracking state is an [11, N] int32 device tensor; every call is enqueued
    on the current stream, allocates nothing and reads nothing back, so a
    rollout graph can hold it."""

    def __init__(self, num_envs: int, config: NativePPOConfig | None = None, device=None) -> None:
        torch, _, _ = _require_torch()
        from nesle_amd import abi

        self.n = int(num_envs)
        self.params = smart_reward_params(config or NativePPOConfig(""))
        dev = device if device is not None else torch.device("cuda")
        self.state = torch.zeros((abi.SHAPED_STATE_WORDS, self.n), dtype=torch.int32, device=dev)
        self.out = torch.zeros(self.n, dtype=torch.float32, device=dev)
        self._lib = abi.lib()
        self._check = abi._check

    def _checked(self, t, dtype, what: str):
        torch, _, _ = _require_torch()
        if not t.is_cuda or t.dtype != dtype or not t.is_contiguous() or t.shape[0] != self.n:
            raise ValueError(f"SmartMarioReward: {what} must be a contiguous {dtype} GPU tensor with "
                             f"{self.n} rows, got {tuple(t.shape)} {t.dtype} on {t.device}")
        return t

    def reset(self, ram) -> None:
        self.reset_where(None, ram)

    def reset_where(self, mask, ram) -> None:
        """Start episodes of the consoles in ``mask`` (bool/uint8 [N]; None =
        all) from ``ram`` ([N, 2048] uint8)."""
        torch, _, _ = _require_torch()
        self._checked(ram, torch.uint8, "ram")
        m = None
        if mask is not None:
            m = self._checked(mask.to(torch.uint8) if mask.dtype != torch.uint8 else mask, torch.uint8, "mask")
            self._mask_keep = m    # keep the converted mask alive until the kernel is enqueued
        stream = torch.cuda.current_stream().cuda_stream
        self._check(self._lib.nesle_smb_shaped_reset(ram.data_ptr(), None if m is None else m.data_ptr(), self.n,
                                                     self.state.data_ptr(), stream))

    def compute(self, ram, action_masks, done):
        """Reward of the step that produced ``ram`` (before any reset) from
        the step's pad masks and done flags; updates the tracking state.
        Returns a float32 [N] tensor that the next call overwrites."""
        torch, _, _ = _require_torch()
        self._checked(ram, torch.uint8, "ram")
        pads = self._checked(action_masks, torch.uint8, "action_masks")
        d = done.to(torch.uint8) if done.dtype != torch.uint8 else done
        self._checked(d, torch.uint8, "done")
        self._done_keep = d
        stream = torch.cuda.current_stream().cuda_stream
        self._check(self._lib.nesle_smb_shaped_reward(ram.data_ptr(), pads.data_ptr(), d.data_ptr(), self.n,
                                                      ctypes.byref(self.params), self.state.data_ptr(),
                                                      self.out.data_ptr(), stream))
        return self.out


# ---- checkpoints -----------------------------------------------------------
# A checkpoint keeps the reference trainer's top-level keys (native_ppo.py:
# 319-368: model, optimizer, config, global_step, torch_rng_state,
# cuda_rng_state, numpy_rng_state), so tools that read those names keep
# working, but every value is a tensor, number, string or list: numpy's RNG
# state is [name, key tensor, pos, has_gauss, cached], so that
# torch.load(weights_only=True) reads the file back without running pickled
# code.  Loading also accepts the layout that kept the RNG states under one
# "rng" entry (format "nesle_amd.native_ppo/1").

CHECKPOINT_FORMAT = "nesle_amd.native_ppo/2"
_RNG_DICT_FORMAT = "nesle_amd.native_ppo/1"


def _numpy_rng_list(torch) -> list:
    name, keys, pos, has_gauss, cached = np.random.get_state()
    return [str(name), torch.from_numpy(np.asarray(keys, dtype=np.int64)), int(pos), int(has_gauss), float(cached)]


def _set_numpy_rng(name, keys, pos, has_gauss, cached) -> None:
    keys = keys.cpu().numpy() if hasattr(keys, "cpu") else np.asarray(keys)
    np.random.set_state((str(name), keys.astype(np.uint32), int(pos), int(has_gauss), float(cached)))


def _save_checkpoint(path: str, model, optimizer, config: NativePPOConfig, global_step: int) -> None:
    torch, _, _ = _require_torch()
    plain = {}
    for key, value in asdict(config).items():
        plain[key] = list(value) if isinstance(value, tuple) else value
    ckpt = {"model": model.state_dict(), "optimizer": optimizer.state_dict(), "config": plain,
            "global_step": int(global_step), "torch_rng_state": torch.get_rng_state(),
            "numpy_rng_state": _numpy_rng_list(torch), "format": CHECKPOINT_FORMAT}
    if torch.cuda.is_available():
        ckpt["cuda_rng_state"] = torch.cuda.get_rng_state()
    target = Path(path)
    target.resolve().parent.mkdir(parents=True, exist_ok=True)
    torch.save(ckpt, target)


def _load_checkpoint(path: str | None, model, optimizer) -> int:
    """Restore model, optimizer and RNGs from ``path``; returns the env-step
    count it was saved at (0 when there is no such file)."""
    if not path or not Path(path).is_file():
        return 0
    torch, _, _ = _require_torch()
    where = torch.device("cuda") if torch.cuda.is_available() else torch.device("cpu")
    ckpt = torch.load(path, map_location=where, weights_only=True)
    if not all(k in ckpt for k in ("model", "optimizer", "global_step")):
        raise ValueError(f"{path} is not a PPO checkpoint (needs model, optimizer and global_step)")
    model.load_state_dict(ckpt["model"])
    optimizer.load_state_dict(ckpt["optimizer"])
    if ckpt.get("format") == _RNG_DICT_FORMAT:
        rng = ckpt["rng"]
        torch_state, cuda_state = rng["torch"], rng.get("cuda")
        mt = ("MT19937", rng["numpy_key"], rng["numpy_pos"], rng["numpy_has_gauss"], rng["numpy_gauss"])
    else:
        torch_state, cuda_state = ckpt.get("torch_rng_state"), ckpt.get("cuda_rng_state")
        mt = ckpt.get("numpy_rng_state")
    if torch_state is not None:
        torch.set_rng_state(torch_state.cpu())
    if cuda_state is not None and torch.cuda.is_available():
        torch.cuda.set_rng_state(cuda_state.cpu())
    if mt is not None:
        _set_numpy_rng(*mt)
    return int(ckpt["global_step"])


# ---- environment -------------------------------------------------------------

def make_batch(config: NativePPOConfig, rom_bytes: bytes | None = None,
               snapshot_bytes: Sequence[bytes] | None = None):
    """The HIP batch for a config: ROM from ``rom_path`` (or ``rom_bytes``), the
    snapshot bank from ``reset_state_path(s)`` (or ``snapshot_bytes``; FCEUX FCS
    or canonical blobs), levels round-robin unless ``env_to_level`` is given
    (src/nesle/env.py:405-425), no frames (the policy reads RAM)."""
    from nesle_amd import load_cuda_core

    core = load_cuda_core()
    rom = rom_bytes if rom_bytes is not None else Path(config.rom_path).read_bytes()
    if snapshot_bytes is None:
        if config.reset_state_path and config.reset_state_paths:
            raise ValueError("pass either reset_state_path or reset_state_paths, not both")
        paths = list(config.reset_state_paths) or ([config.reset_state_path] if config.reset_state_path else [])
        snapshot_bytes = [Path(p).read_bytes() for p in paths]
    kw = {"frames": False}
    if config.reward is not None:
        kw["reward"] = dict(config.reward)
    n = config.num_envs
    if not snapshot_bytes:
        return core.CudaBatch(n, config.frameskip, rom, **kw)
    if len(snapshot_bytes) == 1 and config.env_to_level is None:
        return core.CudaBatch(n, config.frameskip, rom, bytes(snapshot_bytes[0]), **kw)
    levels = (np.asarray(config.env_to_level, dtype=np.uint8) if config.env_to_level is not None
              else (np.arange(n) % len(snapshot_bytes)).astype(np.uint8))
    return core.CudaBatch(n, config.frameskip, rom, [bytes(s) for s in snapshot_bytes], levels, **kw)


# ---- training ------------------------------------------------------------------

def _capture_rollout(torch, batch, rollout_step, T: int, model, ram):
    """Capture T rollout steps into one HIP graph.  The batch's kernels are
    enqueued on the capture stream (its stream is switched for the capture
    and switched back), the policy is warmed up on that stream first, and the
    captured work holds no memset or host synchronisation: sampling noise is
    drawn before each replay and the episode statistics are per-console sums."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side), torch.no_grad():
        for _ in range(2):
            model(ram)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    batch.set_stream(side.cuda_stream)
    try:
        with torch.cuda.graph(graph, stream=side):
            for t in range(T):
                rollout_step(t)
    finally:
        torch.cuda.synchronize()
        batch.set_stream(torch.cuda.current_stream().cuda_stream)
    return graph


def _configure_adam(torch, optimizer) -> None:
    """The trainer's Adam runs fused (one kernel per step) with its step
    counters on the device (``capturable``, which the captured minibatch step
    needs).  A checkpoint restores the flags it was saved with, so they are
    set again after loading and the counters moved to match."""
    for group in optimizer.param_groups:
        group["capturable"] = True
        group["fused"] = True
        group["foreach"] = None
        for p in group["params"]:
            state = optimizer.state.get(p)
            if state and "step" in state:
                state["step"] = state["step"].to(dtype=torch.float32, device=p.device)


_PPO_HEAD = None


def ppo_head_loss(logits, value, actions, old_logprob, advantages, returns, clip_coef: float, ent_coef: float,
                  vf_coef: float, accum=None):
    """(loss, clip fraction) of one minibatch by the HIP loss head
    (``nesle_ppo_head``, include/nesle_ppo.h): the reference's loss lines
    (native_ppo.py:546-566) in three kernels, with d loss / d logits and
    d loss / d value computed in the same pass and returned by the autograd
    backward.  Every tensor must live on the GPU (contiguous float32, int64
    actions); ``accum`` (two floats on the GPU) receives loss and clip
    fraction added to it."""
    global _PPO_HEAD
    torch, _, _ = _require_torch()
    if _PPO_HEAD is None:
        _PPO_HEAD = _make_ppo_head(torch)
    return _PPO_HEAD.apply(logits, value, actions, old_logprob, advantages, returns, float(clip_coef),
                           float(ent_coef), float(vf_coef), accum)


def _make_ppo_head(torch):
    from nesle_amd import abi

    L = abi.lib()

    def need(t, name, dtype, shape):
        if not (t.is_cuda and t.dtype == dtype and tuple(t.shape) == shape and t.is_contiguous()):
            raise ValueError(f"ppo_head_loss: {name} must be a contiguous {dtype} GPU tensor of shape {shape}, "
                             f"got {tuple(t.shape)} {t.dtype} on {t.device}")

    class PPOHead(torch.autograd.Function):
        @staticmethod
        def forward(ctx, logits, value, actions, old_logprob, advantages, returns, clip_coef, ent_coef, vf_coef,
                    accum):
            if logits.dim() != 2:
                raise ValueError("ppo_head_loss: logits must be [batch, actions]")
            n, a = logits.shape
            need(logits, "logits", torch.float32, (n, a))
            need(value, "value", torch.float32, (n,))
            need(actions, "actions", torch.int64, (n,))
            for t, name in ((old_logprob, "old_logprob"), (advantages, "advantages"), (returns, "returns")):
                need(t, name, torch.float32, (n,))
            if accum is not None:
                need(accum, "accum", torch.float32, (2,))
            dev = logits.device
            if any(t.device != dev for t in (value, actions, old_logprob, advantages, returns)):
                raise ValueError("ppo_head_loss: all tensors must be on one device")
            dlogits = torch.empty_like(logits)
            dvalue = torch.empty_like(value)
            scratch = torch.empty(int(L.nesle_ppo_head_scratch_floats(n)), dtype=torch.float32, device=dev)
            loss = torch.empty((), dtype=torch.float32, device=dev)
            clipfrac = torch.empty((), dtype=torch.float32, device=dev)
            with torch.cuda.device(dev):
                stream = torch.cuda.current_stream(dev).cuda_stream
                abi._check(L.nesle_ppo_head(
                    logits.data_ptr(), value.data_ptr(), actions.data_ptr(), old_logprob.data_ptr(),
                    advantages.data_ptr(), returns.data_ptr(), n, a, clip_coef, ent_coef, vf_coef,
                    dlogits.data_ptr(), dvalue.data_ptr(), scratch.data_ptr(), loss.data_ptr(), clipfrac.data_ptr(),
                    accum.data_ptr() if accum is not None else None, stream))
            ctx.grads = (dlogits, dvalue)
            ctx.mark_non_differentiable(clipfrac)
            return loss, clipfrac

        @staticmethod
        def backward(ctx, g_loss, g_clipfrac):
            dlogits, dvalue = ctx.grads
            return dlogits * g_loss, dvalue * g_loss, None, None, None, None, None, None, None, None

    return PPOHead


class MinibatchUpdate:
    """Clipped-PPO minibatch steps over the rollout buffers
    (native_ppo.py:540-575): forward, the loss head (``ppo_head_loss``),
    backward, gradient-norm clipping and Adam, with the loss and clip fraction
    summed on the device.

    ``run(idx)`` takes one minibatch of sample indices.  After ``capture()``
    a full minibatch replays one HIP graph of the whole step instead (about
    40 launches): ``idx`` is copied into the graph's index buffer and the
    graph gathers the minibatch from ``sources``, whose device buffers must
    stay in place.  The captured work holds no host synchronisation (the
    loss head runs no memset and reads nothing back, clipping is a
    device-side scale, Adam is fused and ``capturable``)."""

    def __init__(self, torch, model, optimizer, config: NativePPOConfig, sources: dict):
        self.torch = torch
        self.model, self.optimizer, self.config = model, optimizer, config
        self.sources = sources          # obs, actions, logprobs, advantages, returns: [count, ...]
        dev = sources["obs"].device
        self.sums = torch.zeros(2, dtype=torch.float32, device=dev)    # loss, clip fraction
        self.minibatches = 0
        self.idx = torch.zeros(config.batch_size, dtype=torch.long, device=dev)
        self.graph = None

    def _loss(self, idx, accum=None):
        cfg, src = self.config, self.sources
        logits, newvalue = self.model(src["obs"][idx])
        return ppo_head_loss(logits, newvalue, src["actions"][idx], src["logprobs"][idx], src["advantages"][idx],
                             src["returns"][idx], cfg.clip_coef, cfg.ent_coef, cfg.vf_coef, accum)

    def _step(self, idx) -> None:
        loss, _ = self._loss(idx, self.sums)
        self.optimizer.zero_grad(set_to_none=True)
        loss.backward()
        self.torch.nn.utils.clip_grad_norm_(self.model.parameters(), self.config.max_grad_norm)
        self.optimizer.step()

    def run(self, idx) -> None:
        if self.graph is not None and idx.shape[0] == self.idx.shape[0]:
            self.idx.copy_(idx)
            self.graph.replay()
        else:
            self._step(idx)
        self.minibatches += 1

    def capture(self) -> None:
        """Capture one full-minibatch step.  Forward and backward are warmed
        up on the capture stream first (library handles and workspaces for
        that stream; the warm-up's gradients are dropped, no parameter
        changes), and the gradients are released so the captured backward
        writes them afresh on every replay."""
        torch = self.torch
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                loss, _ = self._loss(self.idx)
                loss.backward()
                self.optimizer.zero_grad(set_to_none=True)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            self._step(self.idx)
        torch.cuda.synchronize()
        self.graph = graph

    def reset_sums(self) -> None:
        self.sums.zero_()
        self.minibatches = 0

    def means(self) -> tuple[float, float]:
        """(mean loss, mean clip fraction) over the minibatches since ``reset_sums``."""
        loss, clipfrac = (self.sums / max(self.minibatches, 1)).tolist()
        return loss, clipfrac


def train_native_ppo(config: NativePPOConfig, resume_from: str | None = None, *, rom_bytes: bytes | None = None,
                     snapshot_bytes: Sequence[bytes] | None = None, batch=None, record=None,
                     on_rollout=None) -> dict:
    """Train; returns {"global_step", "updates", "rollout_s", "update_s",
    "emulator_s", "wall_s", "log", "per_update", "graph_updates", "model"}
    (emulator_s: step-kernel plus auto-reset restore-kernel time per rollout
    step from HIP events on the batch's stream during the eager first
    rollout, times the steps).
    ``record(step, masks, rewards, dones)`` receives each step's device tensors
    and keeps every rollout eager; ``on_rollout(update, buffers)`` receives
    the rollout buffers after each rollout (tests)."""
    rollout_timesteps = config.num_envs * config.n_steps
    if rollout_timesteps < config.batch_size:
        raise ValueError(
            f"rollout produces {rollout_timesteps} samples per update (num_envs={config.num_envs} * "
            f"n_steps={config.n_steps}) but batch_size={config.batch_size} is larger")
    if config.reward_mode not in ("minimal", "smart"):
        raise ValueError(f"unknown reward_mode {config.reward_mode!r} (expected 'minimal' or 'smart')")
    torch, _, _ = _require_torch()
    if not torch.cuda.is_available():
        raise SystemExit("native PPO needs a GPU")
    torch.manual_seed(config.seed)
    np.random.seed(config.seed)

    masks = _actions.action_masks(config.action_space)
    if batch is None:
        batch = make_batch(config, rom_bytes, snapshot_bytes)
    if batch.num_envs != config.num_envs or batch.frameskip != config.frameskip:
        raise ValueError("batch shape does not match the config")
    stream = torch.cuda.current_stream()
    batch.set_stream(stream.cuda_stream)
    batch.reset_device()

    dev = torch.device("cuda")
    obs_dim, action_dim, n = 2048, len(masks), config.num_envs
    model = _make_model(obs_dim, action_dim, config.hidden_size, config.init, dev)
    # Fused Adam with its step counters on the device in both modes (the
    # captured minibatch step needs them), so eager and graph training compute
    # the same numbers.
    optimizer = torch.optim.Adam(model.parameters(), lr=config.learning_rate, eps=1e-5, capturable=True, fused=True)
    global_step = _load_checkpoint(resume_from, model, optimizer)
    _configure_adam(torch, optimizer)
    resume_step = global_step
    mask_table = torch.tensor(masks, dtype=torch.uint8, device=dev)

    from torch.utils.dlpack import from_dlpack

    ram = from_dlpack(batch.ram_device())          # [N, 2048] uint8, refreshed by every step
    rewards_view = from_dlpack(batch.rewards_device())
    dones_view = from_dlpack(batch.last_done_device())
    # The shaped reward reads the step's RAM before any reset, so with it the
    # step runs without auto-reset and done consoles are reset afterwards
    # through a device mask (the reference's order, native_ppo.py:486-509,
    # without its host reads).
    rewarder = None
    if config.reward_mode == "smart":
        rewarder = SmartMarioReward(config.num_envs, config, dev)
        rewarder.reset(ram)

    T = config.n_steps
    obs_buf = torch.empty((T, n, obs_dim), dtype=torch.uint8, device=dev)
    actions_buf = torch.empty((T, n), dtype=torch.long, device=dev)
    logprobs_buf = torch.empty((T, n), dtype=torch.float32, device=dev)
    rewards_buf = torch.empty((T, n), dtype=torch.float32, device=dev)
    dones_buf = torch.empty((T, n), dtype=torch.float32, device=dev)
    values_buf = torch.empty((T, n), dtype=torch.float32, device=dev)
    episode_returns = torch.zeros(n, dtype=torch.float32, device=dev)
    episode_lengths = torch.zeros(n, dtype=torch.float32, device=dev)
    # Finished episodes per console (count, return sum, length sum), summed at log time.
    fin_count = torch.zeros(n, dtype=torch.float32, device=dev)
    fin_return = torch.zeros(n, dtype=torch.float64, device=dev)
    fin_length = torch.zeros(n, dtype=torch.float64, device=dev)
    next_done = torch.zeros(n, dtype=torch.float32, device=dev)
    adv_buf = torch.empty((T, n), dtype=torch.float32, device=dev)
    ret_buf = torch.empty((T, n), dtype=torch.float32, device=dev)
    noise = torch.empty((T, n, action_dim), dtype=torch.float32, device=dev)
    rows = torch.arange(n, device=dev)

    def rollout_step(t: int) -> None:
        """One rollout step, entirely on the device: policy, sampling, the
        console step and episode bookkeeping (captured into a graph as is)."""
        obs_buf[t].copy_(ram)
        dones_buf[t].copy_(next_done)
        with torch.no_grad():
            logits, value = model(ram)
            # Categorical sample by Gumbel-max over uniforms drawn before the
            # rollout (same distribution as Categorical.sample).
            action = (logits - torch.log(-torch.log(noise[t]))).argmax(dim=-1)
            logprobs_buf[t].copy_(torch.log_softmax(logits, dim=-1)[rows, action])
        actions_buf[t].copy_(action)
        values_buf[t].copy_(value)
        pad = mask_table[action]
        batch.step_device(pad, auto_reset=rewarder is None, synchronize=False)
        done = dones_view.bool()
        episode_lengths.add_(1.0)
        if rewarder is None:
            reward = rewards_view
            if config.max_episode_steps > 0:
                timeout = (episode_lengths >= float(config.max_episode_steps)) & ~done
                batch.reset_envs_device(timeout.to(torch.uint8))   # consoles not in the mask are untouched
                done = done | timeout
        else:
            reward = rewarder.compute(ram, pad, done)
            if config.max_episode_steps > 0:
                done = done | (episode_lengths >= float(config.max_episode_steps))
            reset_mask = done.to(torch.uint8)
            batch.reset_envs_device(reset_mask)
            rewarder.reset_where(reset_mask, ram)              # from the post-reset RAM
        rewards_buf[t].copy_(reward)
        next_done.copy_(done.float())
        episode_returns.add_(reward)
        fin_count.add_(next_done)
        fin_return.add_(episode_returns * next_done)
        fin_length.add_(episode_lengths * next_done)
        keep = 1.0 - next_done
        episode_returns.mul_(keep)
        episode_lengths.mul_(keep)

    updater = MinibatchUpdate(torch, model, optimizer, config, {
        "obs": obs_buf.reshape((-1, obs_dim)), "actions": actions_buf.reshape(-1),
        "logprobs": logprobs_buf.reshape(-1), "advantages": adv_buf.reshape(-1), "returns": ret_buf.reshape(-1)})
    update_graph_ok = config.cuda_graph and rollout_timesteps % config.batch_size == 0

    remaining = max(0, config.total_timesteps - global_step)
    num_updates = math.ceil(remaining / rollout_timesteps)
    stats = {"global_step": global_step, "updates": 0, "rollout_s": 0.0, "update_s": 0.0, "emulator_s": 0.0,
             "wall_s": 0.0, "log": [], "per_update": [], "graph_updates": 0}
    graph = None
    step_ms = None   # step + restore kernel time per rollout step, from the eager first rollout
    progress = _progress_bar(config.progress_bar, global_step + num_updates * rollout_timesteps, global_step)
    t_start = time.perf_counter()
    for update in range(1, num_updates + 1):
        # The first rollout runs eagerly (HIP-event timing of the step kernel,
        # library warm-up); with cuda_graph the later ones replay a graph of
        # all T steps captured once, and so do the minibatch steps.
        use_graph = config.cuda_graph and update > 1 and record is None
        if use_graph and graph is None:
            graph = _capture_rollout(torch, batch, rollout_step, T, model, ram)
        if use_graph and update_graph_ok and updater.graph is None:
            updater.capture()
        noise.uniform_(1e-20, 1.0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        if use_graph:
            graph.replay()
        else:
            batch.set_timing(True)
            for t in range(T):
                rollout_step(t)
                if record is not None:
                    record(t, mask_table[actions_buf[t]], rewards_buf[t], next_done.bool())
        global_step += rollout_timesteps
        if progress is not None:
            progress.update(rollout_timesteps)   # per rollout: a graph replay runs all its steps at once
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        if not use_graph:
            kernel_ms, reset_ms, launches = batch.kernel_timing_split()
            batch.set_timing(False)
            step_ms = (kernel_ms + reset_ms) / max(launches, 1)   # step kernel + auto-reset restore
        else:
            stats["graph_updates"] += 1
        if on_rollout is not None:
            on_rollout(update, {"actions": actions_buf, "rewards": rewards_buf, "dones": dones_buf,
                                "values": values_buf, "logprobs": logprobs_buf, "graph": use_graph})

        with torch.no_grad():
            _, next_value = model(ram)
            advantages, returns = compute_gae(rewards_buf, dones_buf, values_buf, next_done, next_value,
                                              config.gamma, config.gae_lambda)
            adv_buf.copy_(advantages)
            ret_buf.copy_(returns)
        # Minibatch updates: the first update runs eagerly; with cuda_graph
        # and minibatches that tile the rollout, the later ones replay the
        # captured graph of one minibatch step per minibatch.
        count = rollout_timesteps
        updater.reset_sums()
        for _ in range(config.update_epochs):
            perm = torch.randperm(count, device=dev)
            for start in range(0, count, config.batch_size):
                updater.run(perm[start:start + config.batch_size])
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        stats["rollout_s"] += t1 - t0
        stats["update_s"] += t2 - t1
        stats["updates"] = update
        emu = step_ms * T / 1000.0
        stats["per_update"].append({"rollout_s": t1 - t0, "update_s": t2 - t1, "emulator_s": emu,
                                    "graph": use_graph, "update_graph": updater.graph is not None})
        stats["emulator_s"] += emu

        if update % max(1, config.log_interval) == 0 or update == num_updates:
            # Episodes finished since the previous log line (the reference
            # averages the last 100, read back every step).
            fin = [float(fin_count.sum()), float(fin_return.sum()), float(fin_length.sum())]
            for acc in (fin_count, fin_return, fin_length):
                acc.zero_()
            mean_loss, mean_clipfrac = updater.means()
            elapsed = max(1e-6, time.perf_counter() - t_start)
            line = {
                "update": update, "step": global_step, "fps": int((global_step - resume_step) / elapsed),
                "loss": mean_loss, "clipfrac": mean_clipfrac,
                "explained_var": _explained_variance(values_buf.reshape(-1), ret_buf.reshape(-1)),
                "episodes": int(fin[0]),
                "ep_return_mean": fin[1] / fin[0] if fin[0] else float("nan"),
                "ep_len_mean": fin[2] / fin[0] if fin[0] else float("nan"),
            }
            stats["log"].append(line)
            print(f"update={update}/{num_updates} step={global_step} fps={line['fps']} loss={line['loss']:.4f} "
                  f"clipfrac={line['clipfrac']:.3f} explained_var={line['explained_var']:.3f} "
                  f"episodes={line['episodes']} ep_return={line['ep_return_mean']:.2f} "
                  f"ep_len={line['ep_len_mean']:.1f}", flush=True)
            if config.save_checkpoints:
                _save_checkpoint(config.checkpoint_path, model, optimizer, config, global_step)
    torch.cuda.synchronize()
    if progress is not None:
        progress.close()
    stats["wall_s"] = time.perf_counter() - t_start
    stats["global_step"] = global_step
    if config.save_checkpoints and num_updates > 0:
        _save_checkpoint(config.checkpoint_path, model, optimizer, config, global_step)
    stats["model"] = model
    return stats


def _progress_bar(enabled: bool, total: int, initial: int):
    """A tqdm bar over env-steps when asked for and tqdm is importable (the
    reference's --progress-bar, native_ppo.py:606-613); else None."""
    if not enabled:
        return None
    try:
        from tqdm.auto import tqdm
    except ImportError:
        print("progress bar requested but tqdm is not importable; the update log lines remain")
        return None
    return tqdm(total=total, initial=min(initial, total), desc="native PPO", unit="env-steps")


def parse_args(argv: Sequence[str] | None = None) -> tuple[NativePPOConfig, str | None]:
    p = argparse.ArgumentParser(description="Train with the GPU-resident PPO path on the MI355X console.")
    p.add_argument("rom_path")
    p.add_argument("--num-envs", type=int, default=1024)
    p.add_argument("--total-timesteps", type=int, default=1_000_000)
    p.add_argument("--n-steps", type=int, default=128)
    p.add_argument("--batch-size", type=int, default=8192)
    p.add_argument("--update-epochs", type=int, default=4)
    p.add_argument("--frameskip", type=int, default=4)
    p.add_argument("--action-space", default="simple_with_start",
                   choices=["right_only", "simple", "simple_with_start", "complex", "mario", "raw"])
    p.add_argument("--reset-state-path", default=None)
    p.add_argument("--reset-state-paths", nargs="+", default=())
    p.add_argument("--max-episode-steps", type=int, default=0)
    p.add_argument("--learning-rate", type=float, default=2.5e-4)
    p.add_argument("--gamma", type=float, default=0.99)
    p.add_argument("--gae-lambda", type=float, default=0.95)
    p.add_argument("--clip-coef", type=float, default=0.1)
    p.add_argument("--ent-coef", type=float, default=0.01)
    p.add_argument("--vf-coef", type=float, default=0.5)
    p.add_argument("--max-grad-norm", type=float, default=0.5)
    p.add_argument("--hidden-size", type=int, default=256)
    p.add_argument("--reward-mode", default="minimal", choices=["minimal", "smart"])
    p.add_argument("--flag-bonus", type=float, default=None, help="override SmartMarioReward's flag bonus (smart mode)")
    p.add_argument("--finish-zone-bonus", type=float, default=None,
                   help="override SmartMarioReward's finish-zone bonus (smart mode)")
    p.add_argument("--death-penalty", type=float, default=None,
                   help="override SmartMarioReward's death penalty (smart mode)")
    p.add_argument("--init", default="orthogonal", choices=["orthogonal", "xavier"])
    p.add_argument("--seed", type=int, default=1)
    p.add_argument("--checkpoint-path", default="nesle_native_ppo.pt")
    p.add_argument("--resume-from", default=None)
    p.add_argument("--log-interval", type=int, default=1)
    p.add_argument("--progress-bar", action="store_true")
    a = p.parse_args(argv)
    if a.reset_state_path and a.reset_state_paths:
        raise SystemExit("Pass either --reset-state-path or --reset-state-paths, not both.")
    cfg = NativePPOConfig(
        rom_path=a.rom_path, num_envs=a.num_envs, total_timesteps=a.total_timesteps, n_steps=a.n_steps,
        batch_size=a.batch_size, update_epochs=a.update_epochs, frameskip=a.frameskip, action_space=a.action_space,
        reset_state_path=a.reset_state_path, reset_state_paths=tuple(a.reset_state_paths),
        max_episode_steps=a.max_episode_steps, learning_rate=a.learning_rate, gamma=a.gamma,
        gae_lambda=a.gae_lambda, clip_coef=a.clip_coef, ent_coef=a.ent_coef, vf_coef=a.vf_coef,
        max_grad_norm=a.max_grad_norm, hidden_size=a.hidden_size, reward_mode=a.reward_mode,
        flag_bonus=a.flag_bonus, finish_zone_bonus=a.finish_zone_bonus, death_penalty=a.death_penalty,
        init=a.init, seed=a.seed, checkpoint_path=a.checkpoint_path, log_interval=a.log_interval,
        progress_bar=a.progress_bar)
    return cfg, a.resume_from


def main() -> None:
    cfg, resume = parse_args()
    train_native_ppo(cfg, resume_from=resume)


if __name__ == "__main__":
    main()
