"""The drop-in binding's own contract (nesle_amd._cuda_core, the reference's
nesle._cuda_core surface), restated from the reference's device-path tests on
the synthetic ROM (the reference's ROM is not in this image):

* a DLPack tensor keeps its batch alive after the batch object is gone
  (tests/test_env_reset_state.py:119-153);
* frames_device() after render_device() equals the host render()
  (tests/test_device_frames.py:34-68);
* render() after throughput steps is fresh, and equals the step(render_frame)
  path (tests/test_render_freshness.py);
* the step()/step_device()/reset() return contracts and the view protocols
  (cpp/bindings/cuda_module.cu:114-183, 469-666).
"""

from __future__ import annotations

import gc

import numpy as np
import pytest

from nesle_amd import synthrom
from oracle import oracle as O
from tests.helpers import say, warm_snapshots

pytestmark = pytest.mark.gpu

RIGHT = 0x80


def _core():
    from nesle_amd import load_cuda_core

    return load_cuda_core()


def _rom() -> bytes:
    return synthrom.make_rom(3).rom


def test_device_view_outlives_batch_reference():
    """A RAM tensor taken through DLPack stays readable after ``del batch``
    and a collection: the capsule holds the batch (the reference binding's
    keep_alive regression).  Its content is the snapshot's RAM."""
    import torch

    rom = _rom()
    snap = bytes(warm_snapshots(rom, [50], seed=4)[0])
    core = _core()
    say("[gpu] shim: view outlives batch")
    batch = core.CudaBatch(2, 4, rom, snap)
    batch.reset()
    ram = torch.utils.dlpack.from_dlpack(batch.ram_device())
    out = batch.step_device(torch.zeros(2, dtype=torch.uint8, device="cuda"), auto_reset=False)
    rewards = torch.utils.dlpack.from_dlpack(out["rewards"])
    view = batch.ram_device()
    del batch, out
    gc.collect()
    copied = ram.detach().clone().cpu()
    assert copied.shape == (2, 2048)
    assert rewards.cpu().shape == (2,)
    # The plain view (no DLPack) also keeps its batch: its protocol still works.
    assert view.__cuda_array_interface__["shape"] == (2, 2048)
    again = torch.utils.dlpack.from_dlpack(view).cpu()
    assert np.array_equal(again.numpy(), copied.numpy())
    del ram, rewards, view, again
    gc.collect()
    torch.cuda.synchronize()


def test_frames_device_matches_host_render():
    """20 throughput steps with the Right button, then the host frames and the
    device frames of one render agree byte for byte."""
    import torch

    core = _core()
    say("[gpu] shim: frames_device vs render")
    batch = core.CudaBatch(2, 4, _rom())
    batch.reset()
    right = np.array([RIGHT, 0x00], dtype=np.uint8)
    for _ in range(20):
        batch.step(right, render_frame=False, copy_obs=False)
    host = batch.render().copy()
    batch.render_device()
    dev = torch.utils.dlpack.from_dlpack(batch.frames_device())
    assert tuple(dev.shape) == (2, 240, 256, 3)
    assert dev.dtype == torch.uint8 and dev.device.type == "cuda"
    np.testing.assert_array_equal(dev.cpu().numpy(), host)
    assert int((dev != 0).sum().item()) > 1000
    del dev
    gc.collect()
    torch.cuda.synchronize()


def test_render_is_fresh_after_throughput_steps():
    """render() after step(render_frame=False, copy_obs=False) draws the
    current state (the reference's render-freeze regression), and matches
    what the step(render_frame=True) path returns."""
    core = _core()
    rom = _rom()
    snap = bytes(warm_snapshots(rom, [30], seed=6)[0])
    say("[gpu] shim: render freshness")
    batch = core.CudaBatch(1, 4, rom, snap)
    first = batch.reset()[0].copy()
    right = np.array([RIGHT], dtype=np.uint8)
    for _ in range(30):
        batch.step(right, render_frame=False, copy_obs=False)
    after = batch.render()[0].copy()
    assert int(np.sum(first != after)) > 100

    a = core.CudaBatch(1, 4, rom)
    a.reset()
    b = core.CudaBatch(1, 4, rom)
    b.reset()
    for _ in range(20):
        a.step(right, render_frame=False, copy_obs=False)
        out = b.step(right, render_frame=True, copy_obs=True)
    frame_a = a.render()[0].copy()
    assert np.array_equal(frame_a, out["obs"][0])
    assert np.array_equal(frame_a, b.render()[0])


def test_step_and_reset_return_contracts():
    """step(): ``obs`` (RGB frames, or RAM on a batch without frames) only
    with copy_obs, float32 rewards and uint8 dones of shape (N,); reset():
    host RGB frames; step_device(): rewards/dones/ram views with
    __cuda_array_interface__ v3 and DLPack device (kDLROCM, id); the views
    equal the host copies; bad shapes raise ValueError."""
    import torch

    core = _core()
    rom = _rom()
    n = 3
    say("[gpu] shim: return contracts")
    batch = core.CudaBatch(n, 4, rom)
    frames = batch.reset()
    assert frames.shape == (n, 240, 256, 3) and frames.dtype == np.uint8
    m = synthrom.action_masks(1, n, 0)
    out = batch.step(m, render_frame=True, copy_obs=True)
    assert set(out) == {"obs", "rewards", "dones"}
    assert out["obs"].shape == (n, 240, 256, 3) and out["obs"].dtype == np.uint8
    assert out["rewards"].shape == (n,) and out["rewards"].dtype == np.float32
    assert out["dones"].shape == (n,) and out["dones"].dtype == np.uint8
    out = batch.step(m, render_frame=False, copy_obs=False)
    assert set(out) == {"rewards", "dones"}

    ram_only = core.CudaBatch(n, 4, rom, frames=False)
    out = ram_only.step(m, render_frame=False, copy_obs=True)
    assert out["obs"].shape == (n, 2048)
    assert np.array_equal(out["obs"], ram_only.ram())

    dev = batch.step_device(torch.from_numpy(m).cuda(), auto_reset=True, synchronize=True)
    assert set(dev) == {"rewards", "dones", "ram"}
    for key, shape, typestr in (("rewards", (n,), "<f4"), ("dones", (n,), "|u1"), ("ram", (n, 2048), "|u1")):
        iface = dev[key].__cuda_array_interface__
        assert iface["version"] == 3 and iface["shape"] == shape and iface["typestr"] == typestr
        assert iface["data"][1] is False and iface["data"][0] == dev[key].ptr
        assert dev[key].__dlpack_device__() == (10, torch.cuda.current_device())
    ram = torch.utils.dlpack.from_dlpack(dev["ram"]).cpu().numpy()
    assert np.array_equal(ram, batch.ram())
    rew = torch.utils.dlpack.from_dlpack(dev["rewards"]).cpu().numpy()
    assert rew.dtype == np.float32 and rew.shape == (n,)
    assert batch.name == "cuda-console" and not batch.has_snapshot and batch.num_levels == 0
    with pytest.raises(ValueError):
        batch.step(np.zeros(n + 1, dtype=np.uint8))
    with pytest.raises(ValueError):
        batch.step_device(torch.zeros(n, dtype=torch.int32, device="cuda"))
    with pytest.raises(ValueError):
        batch.step_device(torch.zeros(n, dtype=torch.uint8))   # host tensor
    with pytest.raises(ValueError):
        core.CudaBatch(0, 4, rom)


def test_ram_device_matches_oracle_after_steps():
    """The RAM view after steps is the console RAM the oracle computes."""
    import torch

    core = _core()
    rom = _rom()
    n = 4
    say("[gpu] shim: RAM view vs oracle")
    batch = core.CudaBatch(n, 4, rom)
    oracles = [O.Oracle(rom) for _ in range(n)]
    for k in range(5):
        m = synthrom.action_masks(2, n, k)
        batch.step_device(torch.from_numpy(m).cuda(), auto_reset=False, synchronize=False)
        for e, o in enumerate(oracles):
            o.step(int(m[e]), 4)
    ram = torch.utils.dlpack.from_dlpack(batch.ram_device()).cpu().numpy()
    for e, o in enumerate(oracles):
        assert np.array_equal(ram[e], o.save()[O.OFF["ram"]:O.OFF["ram"] + 2048])
