"""Known answers for the two reward/done rules, on the oracle (CPU) and on the
HIP batch (GPU), so that a mistake shared by the oracle's rule and the
kernel's (a wrap sign, a clip bound, a death constant) fails here.

Every case is a pair of RAM images: the one the reward baselines are seeded
from (a state load seeds them, as the reference's warm reset does,
batch_step.cuh:174-242) and the one the rule then reads.  The console runs an
idle ROM (``JMP $8000`` forever, NMI off), so a step leaves RAM as written and
applies the rule once to the second image.

* SMB rule (batch_step.cuh:61-106): the reference's own known answers,
  tests/cpp/test_cuda_batch.cpp:82-87 (2.0; -1.0; -24.0 with done) and
  tests/cpp/test_core.cpp:117-122 (x 258 -> 261, time 400 -> 399: total 2),
  then one case per clause of the rule, worked by hand from its definition.
* x-delta rule of the benchmark (clip(int16(x - x_prev), -c, c) - penalty;
  done when RAM[done_addr] == 0): closed-form answers at the 16-bit wrap, at
  the clip bounds on both sides, the float32 rounding of ``dx - penalty``,
  and the done byte.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from tests.kat_roms import nrom_bytes

IDLE_ROM = nrom_bytes(2, code={0x8000: [0x4C, 0x00, 0x80]}, reset=0x8000)

# SMB RAM map (cpp/include/nesle/smb.hpp:12-26).
PLAYER_STATE, FLOAT_STATE, ENEMY_BASE, X_PAGE, X_SCREEN, Y_VIEWPORT = 0x0E, 0x1D, 0x16, 0x6D, 0x86, 0xB5
LIVES, GAME_MODE, TIME = 0x75A, 0x770, 0x7F8


def smb_ram(x: int, time: int, player_state: int = 8, y_viewport: int = 1,
            extra: dict[int, int] | None = None) -> dict[int, int]:
    """RAM bytes the SMB rule reads, in the reference test's seeding
    (test_cuda_batch.cpp:21-35): 16-bit x split over page/screen, BCD time."""
    ram = {X_PAGE: x >> 8, X_SCREEN: x & 0xFF, Y_VIEWPORT: y_viewport, PLAYER_STATE: player_state, LIVES: 2,
           TIME: time // 100, TIME + 1: (time // 10) % 10, TIME + 2: time % 10}
    ram.update(extra or {})
    return ram


SMB = {"kind": 0}
SMB_CASES = [
    # (name, seeded-from RAM, current RAM, reward, done)
    ("ref_cuda_batch_env0", smb_ram(40, 400), smb_ram(43, 399), 2.0, 0),
    ("ref_cuda_batch_env1", smb_ram(80, 399), smb_ram(90, 398), -1.0, 0),
    ("ref_cuda_batch_env2", smb_ram(48, 400), smb_ram(50, 399, player_state=0x0B), -24.0, 1),
    ("ref_core_x258_to_261", smb_ram(258, 400, player_state=0), smb_ram(261, 399, player_state=0), 2.0, 0),
    ("dx_plus5_kept", smb_ram(100, 300), smb_ram(105, 300), 5.0, 0),
    ("dx_plus6_zeroed", smb_ram(100, 300), smb_ram(106, 300), 0.0, 0),
    ("dx_minus5_kept", smb_ram(100, 300), smb_ram(95, 300), -5.0, 0),
    ("dx_minus6_zeroed", smb_ram(100, 300), smb_ram(94, 300), 0.0, 0),
    ("x_page_carry", smb_ram(0x1FE, 300), smb_ram(0x201, 300), 3.0, 0),
    ("time_up_ignored", smb_ram(100, 300), smb_ram(101, 305), 1.0, 0),
    ("time_down_by_12", smb_ram(100, 312), smb_ram(100, 300), -12.0, 0),
    ("bcd_high_nibbles_ignored", smb_ram(100, 300),
     smb_ram(100, 300, extra={TIME: 0xF3, TIME + 1: 0xA0, TIME + 2: 0x50}), 0.0, 0),
    ("dead_state_6", smb_ram(100, 300), smb_ram(101, 300, player_state=0x06), -24.0, 1),
    ("falling_viewport_2", smb_ram(100, 300), smb_ram(100, 299, y_viewport=2), -26.0, 1),
    ("viewport_0_alive", smb_ram(100, 300), smb_ram(100, 300, y_viewport=0), 0.0, 0),
    ("game_over_lives_ff", smb_ram(100, 300), smb_ram(102, 300, extra={LIVES: 0xFF}), 2.0, 1),
    ("flag_game_mode_2", smb_ram(100, 300), smb_ram(104, 300, extra={GAME_MODE: 2}), 4.0, 1),
    ("game_mode_1_not_done", smb_ram(100, 300), smb_ram(104, 300, extra={GAME_MODE: 1}), 4.0, 0),
    ("stage_over_enemy_31_floating", smb_ram(100, 300),
     smb_ram(100, 300, extra={ENEMY_BASE + 4: 0x31, FLOAT_STATE: 3}), 0.0, 1),
    ("stage_over_enemy_2d_floating", smb_ram(100, 300),
     smb_ram(100, 300, extra={ENEMY_BASE: 0x2D, FLOAT_STATE: 3}), 0.0, 1),
    ("enemy_2d_not_floating", smb_ram(100, 300), smb_ram(100, 300, extra={ENEMY_BASE: 0x2D, FLOAT_STATE: 2}), 0.0, 0),
    ("enemy_slot_5_out_of_range", smb_ram(100, 300),
     smb_ram(100, 300, extra={ENEMY_BASE + 5: 0x31, FLOAT_STATE: 3}), 0.0, 0),
]

X_LO, X_HI, DONE_AT, PENALTY = 0x12, 0x13, 0x14, 0.01
XD = {"kind": 1, "x_lo": X_LO, "x_hi": X_HI, "done_addr": DONE_AT, "clip": 15, "time_penalty": PENALTY}


def x_ram(x: int, done_byte: int = 7) -> dict[int, int]:
    return {X_LO: x & 0xFF, X_HI: (x >> 8) & 0xFF, DONE_AT: done_byte}


def f32_minus(dx: int, penalty: float = PENALTY) -> float:
    """dx - penalty rounded once in float32 (the rule's arithmetic type)."""
    return float(np.float32(dx) - np.float32(penalty))


XDELTA_CASES = [
    ("wrap_ffff_to_0001", x_ram(0xFFFF), x_ram(0x0001), f32_minus(2), 0),
    ("wrap_0001_to_ffff", x_ram(0x0001), x_ram(0xFFFF), f32_minus(-2), 0),
    ("plus15_kept", x_ram(1000), x_ram(1015), f32_minus(15), 0),
    ("plus16_clipped", x_ram(1000), x_ram(1016), f32_minus(15), 0),
    ("minus15_kept", x_ram(1000), x_ram(985), f32_minus(-15), 0),
    ("minus16_clipped", x_ram(1000), x_ram(984), f32_minus(-15), 0),
    ("half_range_minus_clipped", x_ram(0x0000), x_ram(0x8000), f32_minus(-15), 0),
    ("half_range_plus_clipped", x_ram(0x0000), x_ram(0x7FFF), f32_minus(15), 0),
    ("high_byte_step", x_ram(0x01FF), x_ram(0x0200), f32_minus(1), 0),
    ("no_move_is_minus_penalty", x_ram(0x1234), x_ram(0x1234), f32_minus(0), 0),
    ("done_byte_zero", x_ram(50), x_ram(53, done_byte=0), f32_minus(3), 1),
    ("done_byte_one", x_ram(50), x_ram(53, done_byte=1), f32_minus(3), 0),
    ("done_byte_ff", x_ram(50), x_ram(53, done_byte=0xFF), f32_minus(3), 0),
]


def _base_state() -> np.ndarray:
    return O.Oracle(IDLE_ROM).save()


def _seeded(ram: dict[int, int]) -> np.ndarray:
    s = _base_state()
    for a, v in ram.items():
        s[O.OFF["ram"] + a] = v
    return s


def test_cases_are_hand_worked_not_trivial():
    """The closed-form x-delta answers differ from the unclipped, unwrapped
    and penalty-free answers, so each case can fail a plausible slip."""
    assert f32_minus(3) != 3.0 and f32_minus(3) != float(np.float64(3) - 0.01)
    assert {c[3] for c in XDELTA_CASES} >= {f32_minus(15), f32_minus(-15), f32_minus(2), f32_minus(-2)}


ALL_CASES = [(SMB, *c) for c in SMB_CASES] + [(XD, *c) for c in XDELTA_CASES]


def _still_dying(ram: dict[int, int]) -> bool:
    return ram.get(PLAYER_STATE) in (0x0B, 0x06) or ram.get(Y_VIEWPORT, 1) > 1


@pytest.mark.parametrize("spec,name,before,after,reward,done", ALL_CASES, ids=[c[1] for c in ALL_CASES])
def test_oracle_reward_known_answers(spec, name, before, after, reward, done):
    o = O.Oracle(IDLE_ROM)
    o.set_reward(**spec)
    o.load(_seeded(before))            # seeds the baselines from `before`
    for a, v in after.items():
        o.write(a, v)                  # RAM writes through the bus, no side effects
    _, r, d = o.step(0, 1)
    assert (r, d) == (reward, done), name
    # The rule moved its baselines to `after`: the same RAM again gives no
    # progress (x-delta: exactly -penalty).
    _, r2, _ = o.step(0, 1)
    assert r2 == (f32_minus(0) if spec is XD else (-25.0 if _still_dying(after) else 0.0))


def test_oracle_baseline_reseeded_by_load():
    """After a load the first reward is measured from the loaded RAM: with x
    unchanged it is exactly -penalty, whatever x was before the load."""
    o = O.Oracle(IDLE_ROM)
    o.set_reward(**XD)
    o.load(_seeded(x_ram(100)))
    o.write(X_LO, 110)
    assert o.step(0, 1)[1] == f32_minus(10)
    o.load(_seeded(x_ram(0x4000)))
    assert o.step(0, 1)[1] == f32_minus(0)


def _gpu_reward(spec: dict, before: dict[int, int], after: dict[int, int]) -> tuple[float, int, float]:
    from nesle_amd import abi

    kw = {"reward_kind": spec["kind"]}
    if spec["kind"] == 1:
        kw.update(x_lo=spec["x_lo"], x_hi=spec["x_hi"], done_addr=spec["done_addr"], clip=spec["clip"],
                  time_penalty=spec["time_penalty"])
    b = abi.Batch(IDLE_ROM, 1, frameskip=1, **kw)
    b.load_state(_seeded(before))
    for a, v in after.items():
        b.poke_ram(a, v)
    b.set_actions(np.zeros(1, dtype=np.uint8))
    b.step()
    r, d = float(b.host(abi.VIEW_REWARDS)[0]), int(b.host(abi.VIEW_DONES)[0])
    b.step()
    r2 = float(b.host(abi.VIEW_REWARDS)[0])
    b.close()
    return r, d, r2


@pytest.mark.gpu
def test_gpu_reward_known_answers():
    """The same cases through the C ABI: state load seeds the baselines,
    nesle_poke_ram writes the second image, one step applies the rule."""
    from tests.helpers import say

    for spec, name, before, after, reward, done in ALL_CASES:
        say(f"reward case {name}")
        r, d, r2 = _gpu_reward(spec, before, after)
        assert (r, d) == (reward, done), name
        assert r2 == (f32_minus(0) if spec is XD else (-25.0 if _still_dying(after) else 0.0)), name
