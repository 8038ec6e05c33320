"""The ROM-less synthetic batch without a GPU: its numpy restatement
(oracle/synthetic.py) against hand-worked cases of the reference's rules
(cpp/bindings/cuda_module.cu:319-354, batch_step.cuh:61-106, 244-260), and
argument checks of nesle_create_synthetic that precede any device work."""

from __future__ import annotations

import ctypes

import numpy as np

from nesle_amd import abi
from oracle.synthetic import SyntheticModel


def test_power_on_state():
    m = SyntheticModel(3, 4)
    assert (m.x() == 0x102).all() and (m.time() == 400).all()
    assert (m.ram[:, 0xB5] == 1).all() and (m.ram[:, 0x75A] == 2).all()
    assert int(m.ram.astype(np.int64).sum()) == 3 * (1 + 2 + 1 + 2 + 4)


def test_pad_moves_x_and_time_ticks_every_24_over_frameskip_steps():
    m = SyntheticModel(4, 4)                        # cadence 6 steps
    right, right_b, left, none = 0x80, 0x82, 0x40, 0x00
    acts = np.array([right, right_b, left, none])
    r, d = m.step(acts)
    # First step: x moves, the time ticks (step 0 is a multiple of the cadence).
    np.testing.assert_array_equal(m.x(), [0x103, 0x104, 0x101, 0x102])
    assert (m.time() == 399).all()
    np.testing.assert_array_equal(r, [1 - 1, 2 - 1, -1 - 1, 0 - 1])
    assert not d.any()
    for _ in range(5):                              # steps 1-5: no tick
        r, _ = m.step(acts)
    assert (m.time() == 399).all()
    np.testing.assert_array_equal(r, [1, 2, -1, 0])
    r, _ = m.step(acts)                             # step 6 ticks again
    assert (m.time() == 398).all()
    np.testing.assert_array_equal(r, [0, 1, -2, -1])
    m1 = SyntheticModel(1, 1)                       # frame-skip 1: cadence 24; 30: cadence 1
    for _ in range(24):
        m1.step(np.array([0]))
    assert m1.time()[0] == 399
    m30 = SyntheticModel(1, 30)
    for _ in range(3):
        m30.step(np.array([0]))
    assert m30.time()[0] == 397


def test_clamps_and_the_reward_rule():
    m = SyntheticModel(2, 4)
    m.ram[0, 0x6D], m.ram[0, 0x86] = 0, 0           # x = 0: Left cannot go below
    m.ram[1, 0x6D], m.ram[1, 0x86] = 0xFF, 0xFF     # x = $FFFF: Right cannot go above
    m.prev_x[:] = m.x()
    m.ram[:, 0x7F8:0x7FB] = 0                       # time 0: stays 0
    m.prev_time[:] = 0
    r, _ = m.step(np.array([0x40, 0x82]))
    np.testing.assert_array_equal(m.x(), [0, 0xFFFF])
    assert (m.time() == 0).all() and (r == 0).all()
    m.ram[0, 0x86] = 9                              # a jump of 9: dx zeroed by the rule
    m.ram[1, 0x0E] = 0x0B                           # dying: -25 and done
    r, d = m.step(None)                             # step_device(): the rule alone, nothing moves
    np.testing.assert_array_equal(r, [0, -25])
    np.testing.assert_array_equal(d, [0, 1])
    assert m.x()[0] == 9


def test_auto_reset_powers_on_done_consoles_and_keeps_their_step_values():
    m = SyntheticModel(3, 4)
    m.ram[1, 0x75A] = 0xFF                          # game over
    m.ram[2, 0x770] = 2                             # flag
    r, d = m.step(np.array([0x80, 0x80, 0x80]), auto_reset=True)
    np.testing.assert_array_equal(d, [0, 1, 1])
    np.testing.assert_array_equal(m.x(), [0x103, 0x102, 0x102])
    assert (m.time()[1:] == 400).all() and m.time()[0] == 399
    np.testing.assert_array_equal(m.dones, d)


def test_create_synthetic_rejects_bad_sizes_before_device_work():
    L = abi.lib()
    for n, fs in ((0, 4), (abi.MAX_ENVS + 1, 4), (8, 0)):
        cfg = abi.Config()
        L.nesle_config_init(ctypes.byref(cfg))
        cfg.num_envs, cfg.frameskip = n, fs
        h = ctypes.c_void_p()
        assert L.nesle_create_synthetic(ctypes.byref(cfg), ctypes.byref(h)) == abi.EINVAL
        assert not h.value
    assert L.nesle_synthetic_step(None, 1, 0) == abi.EINVAL
