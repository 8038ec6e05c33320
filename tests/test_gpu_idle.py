"""The step kernel's idle-loop fast-forward (kernels.cu:66-76: a `JMP *`
repeats until the next PPU timing event) against the oracle, which steps
every jump: an NMI-driven program (SMB's shape) whose handler reads the pad
and does button-dependent work, so consoles idle for different spans each
frame.  Full state, instruction counts (skipped jumps counted) and rewards
are bit-exact at frame-skip 1 and 4 and with the per-frame instruction
budget cutting frames inside the idle loop."""

from __future__ import annotations

import numpy as np
import pytest

from nesle_amd import abi
from oracle import oracle as O
from tests.helpers import first_diff, masks_for, say
from tests.kat_roms import nrom_bytes

pytestmark = pytest.mark.gpu

RESET = [0x78, 0xD8, 0xA2, 0xFF, 0x9A,          # SEI; CLD; LDX #$FF; TXS
         0xA9, 0x80, 0x8D, 0x00, 0x20,          # LDA #$80; STA $2000 (NMI on)
         0xA9, 0x1E, 0x8D, 0x01, 0x20,          # LDA #$1E; STA $2001
         0x4C, 0x0F, 0x80]                      # $800F: JMP $800F
NMI = [0x48, 0x8A, 0x48, 0x98, 0x48,            # save A, X, Y
       0xA9, 0x01, 0x8D, 0x16, 0x40, 0xA9, 0x00, 0x8D, 0x16, 0x40,   # strobe pad 1
       0xA2, 0x08,                              # LDX #8
       0xAD, 0x16, 0x40, 0x4A, 0x26, 0x10, 0xCA, 0xD0, 0xF7,        # read 8 bits into $10
       0xE6, 0x11,                              # INC $11 (frames)
       0xA5, 0x10, 0x18, 0x65, 0x12, 0x85, 0x12,                    # $12 += buttons
       0xA4, 0x10, 0xF0, 0x0B,                  # LDY $10; BEQ done
       0xB9, 0x00, 0x03, 0x69, 0x01, 0x99, 0x00, 0x03, 0x88, 0xD0, 0xF5,   # buttons x RMW of $0300,Y
       0xA9, 0x02, 0x8D, 0x14, 0x40,            # done: OAM DMA from $0200
       0xAD, 0x02, 0x20,                        # LDA $2002
       0x68, 0xA8, 0x68, 0xAA, 0x68, 0x40]      # restore, RTI


def idle_rom() -> bytes:
    return nrom_bytes(2, code={0x8000: RESET, 0x9000: NMI}, reset=0x8000, nmi=0x9000, irq=0x8000)


@pytest.mark.parametrize("n,frameskip,budget", [(64, 1, 200000), (64, 4, 200000), (64, 2, 3000),
                                                 (16384, 4, 200000), (16384, 2, 3000)])
def test_idle_loop_fast_forward_matches_oracle(n, frameskip, budget):
    """64 consoles (all RAM in LDS, every console checked) and 16,384
    (RAM split between LDS and HBM, sampled consoles)."""
    rom = idle_rom()
    steps = 12
    rng = np.random.default_rng(n)
    envs = list(range(n)) if n <= 64 else sorted({0, 63, 64, 255, 256, n - 1, *rng.integers(0, n, 26).tolist()})
    say(f"[gpu] idle loop: N={n} fs={frameskip} budget={budget} steps={steps} checked={len(envs)}")
    b = abi.Batch(rom, n, frameskip=frameskip, max_instructions_per_frame=budget)
    cons = [O.Oracle(rom) for _ in envs]
    for c in cons:
        c.set_reward()
    for k in range(steps):
        m = masks_for(4242, n, k)
        b.set_actions(m)
        b.step(stats_mode=1)
        want = [c.step(int(m[e]), frameskip, budget) for e, c in zip(envs, cons)]
        np.testing.assert_array_equal(b.host(abi.VIEW_INSTRUCTIONS)[envs], [w[0] for w in want], err_msg=f"step {k}")
        np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS)[envs], np.array([w[1] for w in want], np.float32))
        if k % 4 == 3:
            for e, c in zip(envs, cons):
                got, ref = b.save_state(e), c.save()
                assert np.array_equal(got, ref), f"step {k} env {e}: {first_diff(got, ref)}"
    ins = b.host(abi.VIEW_INSTRUCTIONS)[envs]
    assert ins.min() != ins.max()   # consoles idled for different spans
