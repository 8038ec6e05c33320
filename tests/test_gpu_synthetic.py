"""The ROM-less synthetic batch on the GPU (nesle_create_synthetic /
nesle_synthetic_step through the C ABI, and the drop-in's two-argument
CudaBatch) against its numpy restatement (oracle/synthetic.py): RAM bytes,
rewards and dones after every step, with and without the pad applied
(step() / step_device()), masked resets, auto-reset, a full reset, and the
refusals of a batch without a console."""

from __future__ import annotations

import numpy as np
import pytest

from nesle_amd import abi, synthrom
from oracle.synthetic import SyntheticModel
from tests.helpers import say

pytestmark = pytest.mark.gpu

ROWS = [0x0E, 0x1D, 0x6D, 0x86, 0xB5, 0x75A, 0x770, 0x7F8, 0x7F9, 0x7FA]


def _compare(b: abi.Batch, m: SyntheticModel, tag: str) -> None:
    ram = b.host(abi.VIEW_RAM)
    np.testing.assert_array_equal(ram, m.ram, err_msg=f"{tag}: RAM")
    np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS), m.rewards, err_msg=f"{tag}: rewards")
    np.testing.assert_array_equal(b.host(abi.VIEW_DONES), m.dones, err_msg=f"{tag}: dones")


@pytest.mark.parametrize("num_envs,frameskip", [(1000, 4), (20000, 1)])
def test_synthetic_batch_matches_its_model(num_envs, frameskip):
    say(f"[gpu] synthetic batch: N={num_envs} fs={frameskip}")
    b = abi.Batch(None, num_envs, frameskip=frameskip)
    m = SyntheticModel(num_envs, frameskip)
    _compare(b, m, "power-on")
    rng = np.random.default_rng(num_envs)
    for k in range(60):
        acts = synthrom.action_masks(900 + frameskip, num_envs, k)
        b.set_actions(acts)
        if k % 10 == 9:            # step_device(): the rule alone
            b.synthetic_step(apply_actions=False)
            m.step(None)
        else:
            b.step()               # nesle_step on a synthetic batch: the pad applied
            m.step(acts)
        if k == 20:                # some consoles die: done, -25, then auto-reset next step
            pick = rng.random(num_envs) < 0.1
            st = m.ram[:, 0x0E].copy()
            st[pick] = 0x06
            b.poke_ram_envs(0x0E, st)
            m.ram[:, 0x0E] = st
        if k == 21:
            b.set_actions(acts)
            b.synthetic_step(apply_actions=True, auto_reset=True)
            r, d = m.step(acts, auto_reset=True)
            assert d.sum() > 0
        if k == 40:
            mask = (rng.random(num_envs) < 0.3).astype(np.uint8)
            b.reset_envs(mask)
            m.reset_envs(mask)
        _compare(b, m, f"step {k}")
    b.reset()
    m.reset()
    _compare(b, m, "full reset")


def test_synthetic_batch_refuses_console_work():
    say("[gpu] synthetic batch refusals: N=16")
    b = abi.Batch(None, 16, frameskip=4)
    b.set_actions(np.zeros(16, dtype=np.uint8))
    with pytest.raises(RuntimeError):
        b.step(stats_mode=1)
    with pytest.raises(ValueError):
        b.snapshot_capture(0, 0)
    with pytest.raises(ValueError):
        b.load_state(np.zeros(abi.STATE_BYTES, dtype=np.uint8))
    console = abi.Batch(synthrom.make_rom(1).rom, 16, frameskip=4)
    with pytest.raises(ValueError):
        console.synthetic_step()
    b.render(abi.FRAME_PALETTE)
    assert not b.host(abi.VIEW_FRAME_PALETTE).any()      # a blank frame: backdrop colour 0


def test_two_argument_cuda_batch_is_the_synthetic_batch():
    """CudaBatch(num_envs, frameskip): name "cuda", step() moves x by the pad,
    step_device() only scores, step_stats is refused (cuda_module.cu:368-379,
    546-565, 620-633, 667-670)."""
    import torch

    from nesle_amd import load_cuda_core

    core = load_cuda_core()
    n = 256
    say(f"[gpu] two-argument CudaBatch: N={n}")
    b = core.CudaBatch(n, 4)
    assert b.name == "cuda"
    m = SyntheticModel(n, 4)
    frames = b.reset()
    assert frames.shape == (n, 240, 256, 3)
    acts = synthrom.action_masks(5, n, 0)
    out = b.step(acts, render_frame=False, copy_obs=False)
    r, d = m.step(acts)
    np.testing.assert_array_equal(out["rewards"], r)
    np.testing.assert_array_equal(b.ram(), m.ram)
    dev = b.step_device(torch.from_numpy(acts).cuda(), auto_reset=True, synchronize=True)
    r, d = m.step(None, auto_reset=True)
    np.testing.assert_array_equal(torch.from_dlpack(dev["rewards"]).cpu().numpy(), r)
    np.testing.assert_array_equal(b.ram(), m.ram)
    with pytest.raises(RuntimeError):
        b.step_stats(acts)
