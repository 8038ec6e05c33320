"""Shared helpers for the parity tests: run the oracle on the same inputs as
the HIP batch and compare canonical state blobs."""

from __future__ import annotations

import sys

import numpy as np

from nesle_amd import abi, synthrom
from oracle import oracle as O


def say(msg: str) -> None:
    """Name the case before a GPU step (flushed, so a fault still shows it)."""
    print(msg, flush=True)
    sys.stdout.flush()


def first_diff(a: np.ndarray, b: np.ndarray) -> str:
    idx = np.nonzero(np.asarray(a) != np.asarray(b))[0]
    if idx.size == 0:
        return "identical"
    names = sorted(O.OFF.items(), key=lambda kv: kv[1])
    def where(i: int) -> str:
        name = "?"
        for n, off in names:
            if off <= i:
                name = f"{n}+{i - off}"
        return name
    return "; ".join(f"{where(int(i))}: gpu={int(a[i])} ref={int(b[i])}" for i in idx[:8]) + \
        f" ({idx.size} bytes differ)"


class OracleBatch:
    """N independent oracle consoles stepped like a HIP batch."""

    def __init__(self, rom: bytes, envs: list[int], reward: dict | None = None) -> None:
        self.envs = list(envs)
        self.cons = [O.Oracle(rom) for _ in self.envs]
        self.reward = reward
        for c in self.cons:
            if reward is not None:
                c.set_reward(**reward)
            else:
                c.set_reward()

    def step(self, masks: np.ndarray, frameskip: int):
        """masks: full-batch mask array; returns (instructions, rewards, dones)."""
        ins, rew, don = [], [], []
        for e, c in zip(self.envs, self.cons):
            n, r, d = c.step(int(masks[e]), frameskip)
            ins.append(n)
            rew.append(r)
            don.append(d)
        return np.array(ins), np.array(rew, dtype=np.float32), np.array(don, dtype=np.uint8)

    def states(self) -> list[np.ndarray]:
        return [c.save() for c in self.cons]


def masks_for(seed: int, num_envs: int, step: int) -> np.ndarray:
    return synthrom.action_masks(seed, num_envs, step)


def warm_snapshots(rom: bytes, warm_frames: list[int], seed: int) -> list[np.ndarray]:
    """Capture one snapshot per entry after that many frame-skip-1 frames."""
    n = len(warm_frames)
    b = abi.Batch(rom, n, frameskip=1)
    for f in range(max(warm_frames) + 1):
        for slot, wf in enumerate(warm_frames):
            if wf == f:
                b.snapshot_capture(slot, slot)
        if f == max(warm_frames):
            break
        b.set_actions(masks_for(seed, n, f))
        b.step()
    assert b.num_levels == n
    return [b.snapshot_export(s) for s in range(n)]


_HIP = None


def device_rows(b: abi.Batch, kind: int, rows, row_shape: tuple[int, ...]) -> dict[int, np.ndarray]:
    """Selected rows of a device view, each copied alone (hipMemcpy of the HIP
    runtime the batch runs on) -- for full-size batches whose whole view would
    be gigabytes on the host."""
    import ctypes

    global _HIP
    if _HIP is None:
        abi.lib()                                    # torch first: one HIP runtime in the process
        _HIP = ctypes.CDLL("libamdhip64.so.7")
        _HIP.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _HIP.hipMemcpy.restype = ctypes.c_int
    b.synchronize()
    v = b.view(kind)
    row_bytes = int(np.prod(row_shape))
    out = {}
    for r in rows:
        buf = np.empty(row_shape, dtype=np.uint8)
        rc = _HIP.hipMemcpy(buf.ctypes.data, v.data + int(r) * row_bytes, row_bytes, 2)   # device to host
        assert rc == 0, f"hipMemcpy failed ({rc})"
        out[int(r)] = buf
    return out
