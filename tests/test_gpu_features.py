"""Step-kernel paths the synthetic benchmark ROM never takes, against the
oracle: PRG RAM reads and writes, code executing from RAM (fetched through
the bus), `JMP ($xxFF)` with the 6502 page-wrap, a stack driven 192 bytes
deep (below the LDS-resident $0180-$01FF when RAM is split), OAM DMA from
RAM, PRG RAM, PRG ROM and PPU register pages (`$2000-$20FF`: reads with
their side effects), and illegal opcodes that stop a console.  Both LDS
layouts run: all RAM in LDS (64 consoles) and split RAM (16,384 consoles,
sampled)."""

from __future__ import annotations

import numpy as np
import pytest

from nesle_amd import abi
from nesle_amd.synthrom import _Asm
from oracle import oracle as O
from tests.helpers import first_diff, masks_for, say

pytestmark = pytest.mark.gpu


def feature_rom() -> bytes:
    a = _Asm()
    a.org(0x8000)
    a.op("SEI"); a.op("CLD"); a.op("LDX", "imm", 0xFF); a.op("TXS")
    a.op("LDX", "imm", 6)                       # copy the RAM routine to $0300
    cp = a.label()
    a.op("LDA", "absx", 0x8100); a.op("STA", "absx", 0x0300); a.op("DEX"); a.op("BPL", "rel", cp)
    a.op("LDA", "imm", 0x00); a.op("STA", "abs", 0x0400)   # vector $0400 -> $8200
    a.op("LDA", "imm", 0x82); a.op("STA", "abs", 0x0401)
    a.op("LDA", "imm", 0x80); a.op("STA", "abs", 0x2000)   # NMI on
    a.op("LDA", "imm", 0x1E); a.op("STA", "abs", 0x2001)
    a.op("JMP", "ind", 0x0400)
    a.org(0x8100)                               # RAM routine: $12 = buttons ^ $5A
    a.byte(0xA5, 0x10, 0x49, 0x5A, 0x85, 0x12, 0x60)
    a.org(0x8200)
    a.label("MAIN")
    a.op("INC", "zp", 0x20); a.op("LDX", "zp", 0x20)
    a.op("TXA"); a.op("STA", "absx", 0x6000)              # PRG RAM write
    a.op("LDA", "absx", 0x7F00); a.op("STA", "zp", 0x21)  # PRG RAM read
    a.op("LDA", "absx", 0x6000); a.op("CLC"); a.op("ADC", "zp", 0x21); a.op("STA", "absx", 0x6100)
    a.op("JSR", "abs", 0x0300)                            # code in RAM
    a.op("LDA", "zp", 0x10); a.op("AND", "imm", 0x01); a.op("BEQ", "rel", "nodeep")
    a.op("LDX", "imm", 0xC0)
    push = a.label()
    a.op("PHA"); a.op("DEX"); a.op("BNE", "rel", push)
    a.op("LDX", "imm", 0xC0)
    pull = a.label()
    a.op("PLA"); a.op("DEX"); a.op("BNE", "rel", pull)
    a.label("nodeep")
    a.op("LDA", "zp", 0x10); a.op("AND", "imm", 0x02); a.op("BEQ", "rel", "nowrap")
    a.op("LDA", "imm", "back"); a.op("STA", "abs", 0x04FF)   # JMP ($04FF) takes its high byte
    a.op("LDA", "imm", 0x82); a.op("STA", "abs", 0x0400)     # from $0400, not $0500
    a.op("LDA", "imm", 0x00); a.op("STA", "abs", 0x0500)
    a.op("JMP", "ind", 0x04FF)
    a.byte(0x02)                                # reached only without the page wrap
    a.label("back")
    a.label("nowrap")
    a.op("LDA", "zp", 0x10); a.op("AND", "imm", 0xF0); a.op("CMP", "imm", 0xF0); a.op("BNE", "rel", "noill")
    a.byte(0x02)                                # illegal: the console stops
    a.label("noill")
    a.op("JMP", "abs", "MAIN")
    a.org(0x9000)                               # NMI: read pad 1, OAM DMA from a rotating page
    a.op("PHA"); a.op("TXA"); a.op("PHA")
    a.op("LDA", "imm", 1); a.op("STA", "abs", 0x4016); a.op("LDA", "imm", 0); a.op("STA", "abs", 0x4016)
    a.op("LDX", "imm", 8)
    rd = a.label()
    a.op("LDA", "abs", 0x4016); a.op("LSR", "acc"); a.op("ROL", "zp", 0x10); a.op("DEX"); a.op("BNE", "rel", rd)
    a.op("INC", "zp", 0x11)
    a.op("LDA", "zp", 0x11); a.op("AND", "imm", 3); a.op("TAX"); a.op("LDA", "absx", 0x9100)
    a.op("STA", "abs", 0x4014)
    a.op("PLA"); a.op("TAX"); a.op("PLA"); a.op("RTI")
    a.org(0x9100)
    a.byte(0x02, 0x60, 0x80, 0x20)              # DMA pages: RAM, PRG RAM, PRG ROM, PPU registers
    a.resolve()
    prg = bytearray(a.prg)
    for at, v in ((0xFFFA, 0x9000), (0xFFFC, 0x8000), (0xFFFE, 0x8000)):
        prg[at - 0x8000] = v & 0xFF
        prg[at - 0x8000 + 1] = v >> 8
    chr_rom = bytes((i * 37 + 11) & 0xFF for i in range(0x2000))
    return bytes(b"NES\x1a" + bytes([2, 1, 0x01, 0]) + bytes(8)) + bytes(prg) + chr_rom


@pytest.mark.parametrize("num_envs", [64, 16384])
def test_rare_paths_match_oracle(num_envs):
    rom = feature_rom()
    steps = 12
    sample = list(range(64)) if num_envs == 64 else sorted({0, 1, 63, 64, 4095, 8191, 12000, num_envs - 1,
                                                             *np.random.default_rng(7).integers(0, num_envs, 8)})
    say(f"[gpu] rare paths: N={num_envs} fs=4 steps={steps} sample={len(sample)}")
    b = abi.Batch(rom, num_envs, frameskip=4)
    cons = {e: O.Oracle(rom) for e in sample}
    for c in cons.values():
        c.set_reward()
    stopped: dict[int, int] = {}
    deep = wrapped = 0
    for k in range(steps):
        m = masks_for(909, num_envs, k)
        b.set_actions(m)
        b.step(stats_mode=1)
        ins, rew, don = b.host(abi.VIEW_INSTRUCTIONS), b.host(abi.VIEW_REWARDS), b.host(abi.VIEW_DONES)
        for e, c in cons.items():
            if e in stopped:
                assert don[e] == 1 and rew[e] == 0.0, f"stopped env {e}"
                continue
            try:
                n, r, d = c.step(int(m[e]), 4)
            except RuntimeError:
                stopped[e] = k
                assert don[e] == 1 and rew[e] == 0.0, f"env {e} stopped at step {k}"
                continue
            assert ins[e] == n and rew[e] == np.float32(r) and don[e] == d, f"step {k} env {e}"
            deep += int(m[e] & 1)
            wrapped += int((m[e] >> 1) & 1)
        if k % 4 == 3 or k == steps - 1:
            for e, c in cons.items():
                got, ref = b.save_state(e), c.save()
                if e in stopped:
                    # The oracle's PC has moved past the illegal opcode; the
                    # stopped console's pad latch still takes each step's
                    # buttons.  Everything else is frozen.
                    got, ref = got.copy(), ref.copy()
                    for name, size in (("pc", 2), ("c1_buttons", 1), ("c1_shift", 1), ("c1_count", 1)):
                        got[O.OFF[name]:O.OFF[name] + size] = ref[O.OFF[name]:O.OFF[name] + size]
                    assert got[O.OFF["fault"]] & 1
                assert np.array_equal(got, ref), f"step {k} env {e}: {first_diff(got, ref)}"
    assert stopped and len(stopped) < len(sample) and deep and wrapped


def oam_rom() -> bytes:
    """OAMADDR and OAMDATA traffic in every order: `$2003` writes, `$2004`
    reads before and after `$2004` writes, and an OAM DMA every frame from a
    page that cycles through HBM-row RAM ($05), LDS-resident RAM ($00), PRG
    RAM ($61) and the PPU registers ($20, read through the bus with their side
    effects), each followed by a `$2004` read.  Every value read lands in RAM."""
    a = _Asm()
    a.org(0x8000)
    a.op("SEI"); a.op("CLD"); a.op("LDX", "imm", 0xFF); a.op("TXS")
    a.op("LDA", "imm", 0x80); a.op("STA", "abs", 0x2000)   # NMI on
    a.op("LDA", "imm", 0x1E); a.op("STA", "abs", 0x2001)
    a.label("MAIN")
    a.op("INC", "zp", 0x20); a.op("LDX", "zp", 0x20)
    a.op("TXA"); a.op("STA", "absx", 0x0500); a.op("STA", "absx", 0x6100)   # DMA source pages
    a.op("LDA", "zp", 0x10); a.op("EOR", "zp", 0x20); a.op("STA", "abs", 0x2003)
    a.op("LDA", "abs", 0x2004); a.op("STA", "absx", 0x0300)                # OAM[OAMADDR]
    a.op("TXA"); a.op("EOR", "imm", 0xA5); a.op("STA", "abs", 0x2004)       # write, OAMADDR + 1
    a.op("LDA", "abs", 0x2004); a.op("STA", "absx", 0x0400)                # the next byte
    a.op("LDA", "zp", 0x10); a.op("AND", "imm", 0x03); a.op("BNE", "rel", "MAIN")
    a.op("LDA", "abs", 0x2004); a.op("STA", "absx", 0x0700)
    a.op("JMP", "abs", "MAIN")
    a.org(0x9000)                               # NMI: read pad 1, DMA from the next page, read OAMDATA
    a.op("PHA"); a.op("TXA"); a.op("PHA")
    a.op("LDA", "imm", 1); a.op("STA", "abs", 0x4016); a.op("LDA", "imm", 0); a.op("STA", "abs", 0x4016)
    a.op("LDX", "imm", 8)
    rd = a.label()
    a.op("LDA", "abs", 0x4016); a.op("LSR", "acc"); a.op("ROL", "zp", 0x10); a.op("DEX"); a.op("BNE", "rel", rd)
    a.op("INC", "zp", 0x11)
    a.op("LDA", "zp", 0x11); a.op("AND", "imm", 3); a.op("TAX"); a.op("LDA", "absx", 0x9100)
    a.op("STA", "abs", 0x4014)
    a.op("LDX", "zp", 0x11); a.op("LDA", "abs", 0x2004); a.op("STA", "absx", 0x0600)
    a.op("PLA"); a.op("TAX"); a.op("PLA"); a.op("RTI")
    a.org(0x9100)
    a.byte(0x05, 0x00, 0x61, 0x20)
    a.resolve()
    prg = bytearray(a.prg)
    for at, v in ((0xFFFA, 0x9000), (0xFFFC, 0x8000), (0xFFFE, 0x8000)):
        prg[at - 0x8000] = v & 0xFF
        prg[at - 0x8000 + 1] = v >> 8
    chr_rom = bytes((i * 53 + 7) & 0xFF for i in range(0x2000))
    return bytes(b"NES\x1a" + bytes([2, 1, 0x01, 0]) + bytes(8)) + bytes(prg) + chr_rom


@pytest.mark.parametrize("num_envs", [64, 16384])
def test_oam_data_reads_match_oracle(num_envs):
    """The step kernel keeps the OAM byte at OAMADDR in a register, refreshed
    by `$2003`/`$2004` writes, by OAM DMA (whole-wave, lane-parallel and
    through-the-bus copies) and when a launch loads its state; every `$2004`
    read of this ROM is stored in RAM, and RAM, OAM and OAMADDR are compared
    with the oracle after every step."""
    rom = oam_rom()
    steps = 10
    sample = list(range(64)) if num_envs == 64 else sorted({0, 1, 31, 63, 64, 4095, 8191, 12000, num_envs - 1,
                                                             *np.random.default_rng(11).integers(0, num_envs, 8)})
    say(f"[gpu] OAM data reads: N={num_envs} fs=4 steps={steps} sample={len(sample)}")
    b = abi.Batch(rom, num_envs, frameskip=4)
    cons = {e: O.Oracle(rom) for e in sample}
    for c in cons.values():
        c.set_reward()
    for k in range(steps):
        m = masks_for(911, num_envs, k)
        b.set_actions(m)
        b.step(stats_mode=1)
        ins = b.host(abi.VIEW_INSTRUCTIONS)
        for e, c in cons.items():
            n, _, _ = c.step(int(m[e]), 4)
            assert ins[e] == n, f"step {k} env {e}"
            got, ref = b.save_state(e), c.save()
            assert np.array_equal(got, ref), f"step {k} env {e}: {first_diff(got, ref)}"


def stack_wrap_rom() -> bytes:
    """The stack pointer at both ends of page 1: JSR/RTS, PHA/PLA, PHP/PLP and
    the NMI's pushes with SP at $00-$07 (pushes wrap from $0100 to $01FF) and
    pulls with SP at $FE/$FF (pulls wrap from $01FF to $0100), so the
    six-byte stack window the step kernel reads wraps around the page."""
    a = _Asm()
    a.org(0x8000)
    a.op("SEI"); a.op("CLD"); a.op("LDX", "imm", 0xFF); a.op("TXS")
    a.op("LDA", "imm", 0x80); a.op("STA", "abs", 0x2000)   # NMI on
    a.label("MAIN")
    a.op("INC", "zp", 0x20); a.op("LDA", "zp", 0x20); a.op("AND", "imm", 0x07); a.op("TAX"); a.op("TXS")
    a.op("JSR", "abs", "SUB")
    a.op("LDA", "zp", 0x10); a.op("PHA"); a.op("PHP"); a.op("EOR", "imm", 0xFF); a.op("PLP"); a.op("PLA")
    a.op("STA", "zp", 0x22)
    a.op("TSX"); a.op("STX", "zp", 0x23)
    a.op("LDX", "imm", 0xFE); a.op("TXS"); a.op("PLA"); a.op("STA", "zp", 0x24); a.op("PLA"); a.op("STA", "zp", 0x25)
    a.op("LDA", "zp", 0x20); a.op("PHA"); a.op("PHA"); a.op("TSX"); a.op("STX", "zp", 0x26)
    a.op("LDX", "imm", 0xFF); a.op("TXS")
    a.op("JMP", "abs", "MAIN")
    a.label("SUB")
    a.op("LDA", "zp", 0x10); a.op("EOR", "imm", 0x5A); a.op("STA", "zp", 0x21); a.op("PHA"); a.op("PLA"); a.op("RTS")
    a.org(0x9000)                               # NMI: read pad 1 into $10 (pushes wherever SP is)
    a.op("PHA"); a.op("TXA"); a.op("PHA")
    a.op("LDA", "imm", 1); a.op("STA", "abs", 0x4016); a.op("LDA", "imm", 0); a.op("STA", "abs", 0x4016)
    a.op("LDX", "imm", 8)
    rd = a.label()
    a.op("LDA", "abs", 0x4016); a.op("LSR", "acc"); a.op("ROL", "zp", 0x10); a.op("DEX"); a.op("BNE", "rel", rd)
    a.op("INC", "zp", 0x11)
    a.op("PLA"); a.op("TAX"); a.op("PLA"); a.op("RTI")
    a.resolve()
    prg = bytearray(a.prg)
    for at, v in ((0xFFFA, 0x9000), (0xFFFC, 0x8000), (0xFFFE, 0x8000)):
        prg[at - 0x8000] = v & 0xFF
        prg[at - 0x8000 + 1] = v >> 8
    chr_rom = bytes((i * 29 + 3) & 0xFF for i in range(0x2000))
    return bytes(b"NES\x1a" + bytes([2, 1, 0x01, 0]) + bytes(8)) + bytes(prg) + chr_rom


@pytest.mark.parametrize("num_envs", [64, 16384])
def test_stack_wrap_matches_oracle(num_envs):
    """Stack accesses that wrap around page 1 (the step kernel's stack window
    then goes through its rare path in both LDS layouts), compared with the
    oracle after every step: instruction counts and whole console states."""
    rom = stack_wrap_rom()
    steps = 8
    sample = list(range(64)) if num_envs == 64 else sorted({0, 1, 31, 63, 64, 4095, 8191, 12000, num_envs - 1,
                                                             *np.random.default_rng(13).integers(0, num_envs, 8)})
    say(f"[gpu] stack wrap: N={num_envs} fs=4 steps={steps} sample={len(sample)}")
    b = abi.Batch(rom, num_envs, frameskip=4)
    cons = {e: O.Oracle(rom) for e in sample}
    for c in cons.values():
        c.set_reward()
    for k in range(steps):
        m = masks_for(913, num_envs, k)
        b.set_actions(m)
        b.step(stats_mode=1)
        ins = b.host(abi.VIEW_INSTRUCTIONS)
        for e, c in cons.items():
            n, _, _ = c.step(int(m[e]), 4)
            assert ins[e] == n, f"step {k} env {e}"
            got, ref = b.save_state(e), c.save()
            assert np.array_equal(got, ref), f"step {k} env {e}: {first_diff(got, ref)}"


def io_corner_rom() -> bytes:
    """I/O register paths the benchmark ROM never takes: pad 2 reads, `$4015`
    written and read, palette writes and reads through `$2006/$2007`
    (including the `$3F10` mirror and the buffer fill a palette read does),
    `$2007` with the 32-byte increment, `$2002` reads between `$2005` writes
    (the write toggle), reads of `$4016` with the strobe held high, and NMI
    switched off and on again during vblank (an immediate NMI).  Every value
    read is stored in RAM."""
    a = _Asm()
    a.org(0x8000)
    a.op("SEI"); a.op("CLD"); a.op("LDX", "imm", 0xFF); a.op("TXS")
    a.op("LDA", "imm", 0x80); a.op("STA", "abs", 0x2000)
    a.label("MAIN")
    a.op("INC", "zp", 0x20); a.op("LDA", "zp", 0x20); a.op("AND", "imm", 0x0F); a.op("TAX")
    a.op("LDA", "abs", 0x4017); a.op("STA", "absx", 0x0300); a.op("LDA", "abs", 0x4017); a.op("STA", "absx", 0x0310)
    a.op("LDA", "zp", 0x20); a.op("STA", "abs", 0x4015); a.op("LDA", "abs", 0x4015); a.op("STA", "absx", 0x0320)
    a.op("LDA", "imm", 0x3F); a.op("STA", "abs", 0x2006); a.op("LDA", "imm", 0x10); a.op("STA", "abs", 0x2006)
    a.op("LDA", "zp", 0x20); a.op("STA", "abs", 0x2007)                        # $3F10 -> $3F00
    a.op("LDA", "imm", 0x3F); a.op("STA", "abs", 0x2006); a.op("LDA", "imm", 0x00); a.op("STA", "abs", 0x2006)
    a.op("LDA", "abs", 0x2007); a.op("STA", "absx", 0x0330)                     # palette read, buffer fill
    a.op("LDA", "abs", 0x2007); a.op("STA", "absx", 0x0340)
    a.op("LDA", "imm", 0x84); a.op("STA", "abs", 0x2000)                        # +32 per $2007 access
    a.op("LDA", "imm", 0x20); a.op("STA", "abs", 0x2006); a.op("STX", "abs", 0x2006)
    a.op("LDA", "zp", 0x10); a.op("STA", "abs", 0x2007); a.op("EOR", "imm", 0xFF); a.op("STA", "abs", 0x2007)
    a.op("LDA", "imm", 0x20); a.op("STA", "abs", 0x2006); a.op("STX", "abs", 0x2006)
    a.op("LDA", "abs", 0x2007); a.op("LDA", "abs", 0x2007); a.op("STA", "absx", 0x0350)
    a.op("LDA", "abs", 0x2007); a.op("STA", "absx", 0x0360)
    a.op("LDA", "imm", 0x80); a.op("STA", "abs", 0x2000)
    a.op("LDA", "zp", 0x20); a.op("STA", "abs", 0x2005); a.op("LDA", "abs", 0x2002); a.op("STA", "absx", 0x0370)
    a.op("LDA", "zp", 0x10); a.op("STA", "abs", 0x2005); a.op("STA", "abs", 0x2005)
    a.op("LDA", "imm", 1); a.op("STA", "abs", 0x4016)                          # strobe held high
    a.op("LDA", "abs", 0x4016); a.op("STA", "absx", 0x0380); a.op("LDA", "abs", 0x4016); a.op("STA", "absx", 0x0390)
    a.op("LDA", "imm", 0); a.op("STA", "abs", 0x4016)
    a.op("LDA", "abs", 0x4016); a.op("STA", "absx", 0x03A0)
    a.op("LDA", "imm", 0x00); a.op("STA", "abs", 0x2000)                       # NMI off, then on again:
    a.op("LDA", "zp", 0x20); a.op("AND", "imm", 0x03); a.op("BEQ", "rel", "skip")
    a.op("LDA", "imm", 0x80); a.op("STA", "abs", 0x2000)                       # in vblank -> NMI at once
    a.label("skip")
    a.op("LDA", "imm", 0x80); a.op("STA", "abs", 0x2000)
    a.op("JMP", "abs", "MAIN")
    a.org(0x9000)                               # NMI: read pad 1 into $10, count, read PPUSTATUS
    a.op("PHA"); a.op("TXA"); a.op("PHA")
    a.op("LDA", "imm", 1); a.op("STA", "abs", 0x4016); a.op("LDA", "imm", 0); a.op("STA", "abs", 0x4016)
    a.op("LDX", "imm", 8)
    rd = a.label()
    a.op("LDA", "abs", 0x4016); a.op("LSR", "acc"); a.op("ROL", "zp", 0x10); a.op("DEX"); a.op("BNE", "rel", rd)
    a.op("INC", "zp", 0x11); a.op("LDX", "zp", 0x11); a.op("LDA", "abs", 0x2002); a.op("STA", "absx", 0x0400)
    a.op("PLA"); a.op("TAX"); a.op("PLA"); a.op("RTI")
    a.resolve()
    prg = bytearray(a.prg)
    for at, v in ((0xFFFA, 0x9000), (0xFFFC, 0x8000), (0xFFFE, 0x8000)):
        prg[at - 0x8000] = v & 0xFF
        prg[at - 0x8000 + 1] = v >> 8
    chr_rom = bytes((i * 41 + 5) & 0xFF for i in range(0x2000))
    return bytes(b"NES\x1a" + bytes([2, 1, 0x01, 0]) + bytes(8)) + bytes(prg) + chr_rom


@pytest.mark.parametrize("num_envs", [64, 16384])
def test_io_corner_cases_match_oracle(num_envs):
    """The I/O register paths of `io_corner_rom`, compared with the oracle
    after every step: instruction counts and whole console states (RAM with
    every value read, PPU registers, palette, nametables, pads)."""
    rom = io_corner_rom()
    steps = 8
    sample = list(range(64)) if num_envs == 64 else sorted({0, 1, 31, 63, 64, 4095, 8191, 12000, num_envs - 1,
                                                             *np.random.default_rng(17).integers(0, num_envs, 8)})
    say(f"[gpu] I/O corner cases: N={num_envs} fs=4 steps={steps} sample={len(sample)}")
    b = abi.Batch(rom, num_envs, frameskip=4)
    cons = {e: O.Oracle(rom) for e in sample}
    for c in cons.values():
        c.set_reward()
    for k in range(steps):
        m = masks_for(917, num_envs, k)
        b.set_actions(m)
        b.step(stats_mode=1)
        ins = b.host(abi.VIEW_INSTRUCTIONS)
        for e, c in cons.items():
            n, _, _ = c.step(int(m[e]), 4)
            assert ins[e] == n, f"step {k} env {e}"
            got, ref = b.save_state(e), c.save()
            assert np.array_equal(got, ref), f"step {k} env {e}: {first_diff(got, ref)}"


def address_wrap_rom() -> bytes:
    """Effective addresses that wrap: a `(zp),Y` pointer at $FF/$00, `(zp,X)`
    pointers whose zero-page address wraps past $FF, `abs,X` and `abs,Y` past
    $FFFF into RAM (loads and stores), and `zp,X` past $FF, with pad-dependent
    index values; every value loaded is stored in RAM."""
    a = _Asm()
    a.org(0x8000)
    a.op("SEI"); a.op("CLD"); a.op("LDX", "imm", 0xFF); a.op("TXS")
    a.op("LDA", "imm", 0x80); a.op("STA", "abs", 0x2000)
    a.label("MAIN")
    a.op("INC", "zp", 0x20)
    a.op("LDA", "zp", 0x20); a.op("STA", "zp", 0xFF); a.op("LDA", "imm", 0x03); a.op("STA", "zp", 0x00)  # ($FF) -> $03xx
    a.op("LDY", "zp", 0x10); a.op("LDA", "indy", 0xFF); a.op("STA", "zp", 0x30)
    a.op("LDA", "zp", 0x20); a.op("STA", "indy", 0xFF)
    a.op("LDX", "imm", 0x01); a.op("LDA", "indx", 0xFE); a.op("STA", "zp", 0x31)   # ($FE,X) -> pointer at $FF/$00
    a.op("LDX", "zp", 0x10); a.op("LDA", "indx", 0xF0); a.op("STA", "zp", 0x32)   # ($F0+X) wraps for X >= $10
    a.op("LDA", "absx", 0xFFF0); a.op("STA", "zp", 0x33)                           # $FFF0+X past $FFFF
    a.op("LDA", "zp", 0x20); a.op("STA", "absx", 0xFFF0)                           # store into RAM $00xx
    a.op("LDY", "zp", 0x20); a.op("LDA", "absy", 0xFF80); a.op("STA", "zp", 0x34)
    a.op("LDA", "zpx", 0xC0); a.op("STA", "zp", 0x35)                              # $C0+X wraps in page 0
    a.op("LDA", "zp", 0x11); a.op("STA", "zpx", 0xE0)
    a.op("JMP", "abs", "MAIN")
    a.org(0x9000)
    a.op("PHA"); a.op("TXA"); a.op("PHA")
    a.op("LDA", "imm", 1); a.op("STA", "abs", 0x4016); a.op("LDA", "imm", 0); a.op("STA", "abs", 0x4016)
    a.op("LDX", "imm", 8)
    rd = a.label()
    a.op("LDA", "abs", 0x4016); a.op("LSR", "acc"); a.op("ROL", "zp", 0x10); a.op("DEX"); a.op("BNE", "rel", rd)
    a.op("INC", "zp", 0x11)
    a.op("PLA"); a.op("TAX"); a.op("PLA"); a.op("RTI")
    a.resolve()
    prg = bytearray(a.prg)
    for at, v in ((0xFFFA, 0x9000), (0xFFFC, 0x8000), (0xFFFE, 0x8000)):
        prg[at - 0x8000] = v & 0xFF
        prg[at - 0x8000 + 1] = v >> 8
    chr_rom = bytes((i * 23 + 9) & 0xFF for i in range(0x2000))
    return bytes(b"NES\x1a" + bytes([2, 1, 0x01, 0]) + bytes(8)) + bytes(prg) + chr_rom


@pytest.mark.parametrize("num_envs", [64, 16384])
def test_address_wrap_matches_oracle(num_envs):
    """Wrapping effective addresses of `address_wrap_rom`, compared with the
    oracle after every step: instruction counts and whole console states."""
    rom = address_wrap_rom()
    steps = 6
    sample = list(range(64)) if num_envs == 64 else sorted({0, 1, 31, 63, 64, 4095, 8191, 12000, num_envs - 1,
                                                             *np.random.default_rng(19).integers(0, num_envs, 8)})
    say(f"[gpu] address wrap: N={num_envs} fs=4 steps={steps} sample={len(sample)}")
    b = abi.Batch(rom, num_envs, frameskip=4)
    cons = {e: O.Oracle(rom) for e in sample}
    for c in cons.values():
        c.set_reward()
    for k in range(steps):
        m = masks_for(919, num_envs, k)
        b.set_actions(m)
        b.step(stats_mode=1)
        ins = b.host(abi.VIEW_INSTRUCTIONS)
        for e, c in cons.items():
            n, _, _ = c.step(int(m[e]), 4)
            assert ins[e] == n, f"step {k} env {e}"
            got, ref = b.save_state(e), c.save()
            assert np.array_equal(got, ref), f"step {k} env {e}: {first_diff(got, ref)}"
