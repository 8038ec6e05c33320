"""The oracle (oracle/nes_oracle.cpp) pinned on the CPU, before it judges the
HIP kernel:

* against the reference core's golden per-frame hashes (tests/golden/);
* against the reference's own ``nesle::Console`` compiled from its sources
  (oracle/_ref), frame by frame and instruction by instruction on random
  machine states, where that library has been built;
* against the known answers the reference's C++ tests assert
  (tests/cpp/test_cpu.cpp, test_cpu_runner.cpp, test_console.cpp,
  test_cuda_bus.cpp), restated on the oracle's bus;
* against arithmetic that fixes the results independently of the oracle's
  code (ADC/SBC/CMP over every operand, PPU event dots in closed form).
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from nesle_amd import synthrom
from oracle import oracle as O
from tests.kat_roms import nrom_bytes, state_with

GOLDEN = Path(__file__).resolve().parent / "golden"

needs_ref = pytest.mark.skipif(not O.ref_available(),
                               reason="oracle/_ref not built (needs the reference sources: make -C oracle ref)")


# ---- golden fixtures written from the reference core --------------------------------

@pytest.mark.parametrize("rom_seed", [1, 2, 3])
def test_oracle_matches_golden_hashes(rom_seed):
    fx = json.loads((GOLDEN / f"console_rom{rom_seed}.json").read_text())
    rom = synthrom.make_rom(rom_seed).rom
    assert f"{O.fnv1a(rom):016x}" == fx["rom_fnv1a"], "synthetic ROM generator drifted"
    o = O.Oracle(rom)
    recs = {r[0]: r for r in fx["records"]}
    cols = fx["columns"]
    for k in range(fx["frames"]):
        n, _, _ = o.step(int(synthrom.action_masks(fx["action_seed"], 1, k)[0]), 1)
        rec = recs.get(k + 1)
        if rec is None:
            continue
        assert n == rec[1], f"frame {k + 1}: instructions"
        h = O.section_hashes(o.save())
        for name in cols[2:]:
            assert f"{h[name]:016x}" == rec[cols.index(name)], f"frame {k + 1}: section {name}"


# ---- the reference core itself -------------------------------------------------------

@needs_ref
@pytest.mark.parametrize("rom_seed,prg_banks", [(5, 2), (11, 2), (2026, 2), (5, 1), (2026, 1)])
def test_oracle_matches_reference_core_frameskip4(rom_seed, prg_banks):
    """40 frame-skip-4 steps, full state after each; the 1-bank cases run the
    16 KB (NROM-128) image mirrored at $8000 and $C000 (rom.cpp:65-121,
    batch_bus.cuh:24-33), with vectors into the low copy."""
    rom = synthrom.make_rom(rom_seed, prg_banks).rom
    o, r = O.Oracle(rom), O.RefConsole(rom)
    for k in range(40):
        m = int(synthrom.action_masks(rom_seed, 1, k)[0])
        assert o.step(m, 4)[0] == r.step(m, 4), f"step {k}: instruction count"
        a, b = o.save(), r.save()
        assert np.array_equal(a, b), f"step {k}: first differing byte {int(np.nonzero(a != b)[0][0])}"


def _random_state(rng: np.random.Generator, base: np.ndarray, opcode: int) -> np.ndarray:
    """A random machine about to execute `opcode` from RAM or PRG ROM."""
    s = base.copy()
    s[O.OFF["ram"]:O.OFF["ram"] + 2048] = rng.integers(0, 256, 2048, dtype=np.uint8)
    s[O.OFF["prg_ram"]:O.OFF["prg_ram"] + 8192] = rng.integers(0, 256, 8192, dtype=np.uint8)
    for name in ("a", "x", "y", "sp", "p"):
        s[O.OFF[name]] = rng.integers(0, 256)
    # Code in RAM ($0000-$07FF, mirrored) so every opcode/operand combination is reachable.
    pc = int(rng.integers(0, 0x800)) | (int(rng.integers(0, 4)) << 11)
    s[O.OFF["pc"]], s[O.OFF["pc"] + 1] = pc & 0xFF, pc >> 8
    ram = O.OFF["ram"]
    s[ram + (pc & 0x7FF)] = opcode
    cyc = int(rng.integers(0, 1 << 40))
    s[O.OFF["cycles"]:O.OFF["cycles"] + 8] = np.frombuffer(cyc.to_bytes(8, "little"), dtype=np.uint8)
    fd = int(rng.integers(0, 341 * 262))
    s[O.OFF["frame_dot"]:O.OFF["frame_dot"] + 4] = np.frombuffer(fd.to_bytes(4, "little"), dtype=np.uint8)
    s[O.OFF["ctrl"]] = rng.integers(0, 256)
    s[O.OFF["mask"]] = rng.integers(0, 256)
    s[O.OFF["status"]] = rng.integers(0, 256) & 0xE0
    s[O.OFF["nmi_pending"]] = int(rng.integers(0, 8) == 0)
    for name in ("oam_addr", "open_bus", "read_buffer", "c1_buttons", "c1_shift"):
        s[O.OFF[name]] = rng.integers(0, 256)
    s[O.OFF["v"]], s[O.OFF["v"] + 1] = rng.integers(0, 256), rng.integers(0, 0x40)
    s[O.OFF["t"]], s[O.OFF["t"] + 1] = rng.integers(0, 256), rng.integers(0, 0x80)
    s[O.OFF["fine_x"]] = rng.integers(0, 8)
    s[O.OFF["w"]] = rng.integers(0, 2)
    s[O.OFF["c1_count"]] = rng.integers(0, 10)
    s[O.OFF["c2_count"]] = rng.integers(0, 10)
    s[O.OFF["strobe"]] = int(rng.integers(0, 4) == 0)
    s[O.OFF["oam"]:O.OFF["oam"] + 256] = rng.integers(0, 256, 256, dtype=np.uint8)
    s[O.OFF["palette"]:O.OFF["palette"] + 32] = rng.integers(0, 64, 32, dtype=np.uint8)
    s[O.OFF["nametable"]:O.OFF["nametable"] + 2048] = rng.integers(0, 256, 2048, dtype=np.uint8)
    return s


@needs_ref
def test_every_official_opcode_matches_reference_on_random_states():
    """Each official opcode, 24 random machines (registers, RAM, PRG RAM, PPU
    and pad state, NMI pending or not): one console instruction leaves the
    oracle and the reference core in identical full states with equal cycle
    counts.  Pointers land anywhere in the 64 KB map, so PPU registers, pads,
    $4014 DMA, PRG RAM and PRG ROM are all reached."""
    rom = synthrom.make_rom(3).rom
    o, r = O.Oracle(rom), O.RefConsole(rom)
    base = o.save()
    rng = np.random.default_rng(2024)
    for opcode in sorted(synthrom.OFFICIAL_OPCODES):
        for trial in range(24):
            s = _random_state(rng, base, opcode)
            o.load(s)
            r.load(s)
            co, fo = o.step_instruction()
            cr, fr = r.step_instruction()
            a, b = o.save(), r.save()
            where = np.nonzero(a != b)[0]
            assert (co, fo) == (cr, fr) and where.size == 0, (
                f"opcode {opcode:02X} trial {trial}: cycles {co}/{cr} frames {fo}/{fr} "
                f"first diff {where[:4].tolist()}")


@needs_ref
def test_illegal_opcodes_fault_like_reference():
    rom = synthrom.make_rom(3).rom
    o, r = O.Oracle(rom), O.RefConsole(rom)
    base = o.save()
    rng = np.random.default_rng(5)
    for opcode in sorted(set(range(256)) - synthrom.OFFICIAL_OPCODES):
        s = _random_state(rng, base, opcode)
        s[O.OFF["nmi_pending"]] = 0
        o.load(s)
        r.load(s)
        with pytest.raises(RuntimeError):
            o.step_instruction()
        with pytest.raises(RuntimeError):
            r.step_instruction()


# ---- known answers from the reference's C++ tests -----------------------------------

def _cpu_at(rom: bytes, pc: int, p: int = 0x20, cycles: int = 0) -> O.Oracle:
    o = O.Oracle(rom)
    o.load(state_with(o.save(), pc=pc, p=p, cycles=cycles, sp=0xFD))
    return o


def test_kat_lda_tax_inx_sta_cycles():
    """tests/cpp/test_cpu.cpp:36-57."""
    rom = nrom_bytes(2, code={0x8000: [0xA9, 0x41, 0xAA, 0xE8, 0x8D, 0x00, 0x02]})
    o = _cpu_at(rom, 0x8000)
    assert [o.step_instruction()[0] for _ in range(4)] == [2, 2, 2, 4]
    s = o.save()
    assert O.field(s, "a") == 0x41 and O.field(s, "x") == 0x42
    assert o.read(0x0200) == 0x41
    assert O.field(s, "cycles", 8) == 10


def test_kat_jsr_rts():
    """tests/cpp/test_cpu.cpp:59-80."""
    rom = nrom_bytes(2, code={0x8000: [0x20, 0x00, 0x90, 0x85, 0x10], 0x9000: [0xA9, 0x77, 0x60]})
    o = _cpu_at(rom, 0x8000)
    o.step_instruction()
    s = o.save()
    assert O.field(s, "pc", 2) == 0x9000 and O.field(s, "sp") == 0xFB
    o.step_instruction()
    o.step_instruction()
    assert O.field(o.save(), "pc", 2) == 0x8003
    o.step_instruction()
    assert o.read(0x0010) == 0x77


def test_kat_branch_taken_page_cross():
    """tests/cpp/test_cpu.cpp:82-90: BNE +1 at $80FD costs 4 cycles, lands on $8100."""
    rom = nrom_bytes(2, code={0x80FD: [0xD0, 0x01]})
    o = _cpu_at(rom, 0x80FD)
    assert o.step_instruction()[0] == 4
    assert O.field(o.save(), "pc", 2) == 0x8100


def test_kat_sbc():
    """tests/cpp/test_cpu.cpp:92-104."""
    rom = nrom_bytes(2, code={0x8000: [0x38, 0xA9, 0x10, 0xE9, 0x01]})
    o = _cpu_at(rom, 0x8000)
    for _ in range(3):
        o.step_instruction()
    s = o.save()
    assert O.field(s, "a") == 0x0F and O.field(s, "p") & 1


def test_kat_2a03_ignores_decimal_mode():
    """tests/cpp/test_cpu_runner.cpp:91-103: SED; CLC; LDA #$45; ADC #$55 gives
    the binary sum $9A with carry clear on the Ricoh 2A03."""
    rom = nrom_bytes(2, code={0x8000: [0xF8, 0x18, 0xA9, 0x45, 0x69, 0x55]})
    o = _cpu_at(rom, 0x8000)
    for _ in range(4):
        o.step_instruction()
    s = o.save()
    assert O.field(s, "a") == 0x9A and not (O.field(s, "p") & 1)


def test_kat_illegal_opcode_faults():
    """tests/cpp/test_cpu_runner.cpp:64-74: opcode $02 is a CPU exception."""
    rom = nrom_bytes(2, code={0x8000: [0x02]})
    o = _cpu_at(rom, 0x8000)
    with pytest.raises(RuntimeError):
        o.step_instruction()
    assert O.field(o.save(), "fault") == 1


def test_kat_nrom_mirroring():
    """tests/cpp/test_cpu.cpp:106-123 and test_console.cpp:190-199."""
    o = O.Oracle(nrom_bytes(1))
    o.write(0x0001, 0xAB)
    assert o.read(0x0801) == o.read(0x1001) == o.read(0x1801) == 0xAB
    o.write(0x2000, 0x80)
    assert o.read(0x2008) == 0x80          # open bus holds the last register write
    assert o.read(0x8000) == o.read(0xC000)
    o2 = O.Oracle(nrom_bytes(2))
    assert (o2.read(0x8000), o2.read(0xC000), o2.read(0xC001)) == (0x00, 0x80, 0x81)
    o2.write(0x8000, 0xEE)
    assert o2.read(0x8000) == 0x00


def test_kat_status_read_side_effects():
    """tests/cpp/test_console.cpp:100-113."""
    o = O.Oracle(nrom_bytes(2))
    o.write(0x2008, 0x80)
    assert O.field(o.save(), "ctrl") == 0x80
    o.ppu_run(241 * 341 + 1)                 # enter vblank with NMI enabled
    assert O.field(o.save(), "nmi_pending") == 1
    o.write(0x2005, 0x23)
    assert O.field(o.save(), "w") == 1
    assert o.read(0x2002) & 0x80
    s = o.save()
    assert O.field(s, "status") & 0x80 == 0 and O.field(s, "nmi_pending") == 0 and O.field(s, "w") == 0


def test_kat_nmi_on_enable_during_vblank():
    """tests/cpp/test_console.cpp:115-121."""
    o = O.Oracle(nrom_bytes(2))
    o.ppu_run(241 * 341 + 1)
    assert O.field(o.save(), "nmi_pending") == 0
    o.write(0x2000, 0x80)
    assert O.field(o.save(), "nmi_pending") == 1


def test_kat_ppu_data_port():
    """tests/cpp/test_console.cpp:123-137: $2006/$2007 and increment 32."""
    o = O.Oracle(nrom_bytes(2))
    for a, v in ((0x2006, 0x21), (0x2006, 0x00), (0x2007, 0x99)):
        o.write(a, v)
    assert o.ppu_peek(0x2100) == 0x99 and O.field(o.save(), "v", 2) == 0x2101
    for a, v in ((0x2000, 0x04), (0x2006, 0x22), (0x2006, 0x00), (0x2007, 0x55)):
        o.write(a, v)
    assert o.ppu_peek(0x2200) == 0x55 and O.field(o.save(), "v", 2) == 0x2220


def test_kat_chr_rom_is_read_only():
    """tests/cpp/test_console.cpp:139-147."""
    o = O.Oracle(nrom_bytes(2, chr_pokes={0x0010: 0x44, 0x1FFF: 0x55}))
    assert o.ppu_peek(0x0010) == 0x44 and o.ppu_peek(0x1FFF) == 0x55
    for a, v in ((0x2006, 0x00), (0x2006, 0x10), (0x2007, 0x99)):
        o.write(a, v)
    assert o.ppu_peek(0x0010) == 0x44


def test_kat_vertical_mirroring_and_palette_alias():
    """tests/cpp/test_console.cpp:149-163."""
    o = O.Oracle(nrom_bytes(2, flags6=0x01))
    for a, v in ((0x2006, 0x20), (0x2006, 0x00), (0x2007, 0x12)):
        o.write(a, v)
    assert o.ppu_peek(0x2000) == o.ppu_peek(0x2800) == o.ppu_peek(0x3000) == 0x12
    for a, v in ((0x2006, 0x3F), (0x2006, 0x10), (0x2007, 0x2A)):
        o.write(a, v)
    assert o.ppu_peek(0x3F00) == o.ppu_peek(0x3F10) == 0x2A


def test_kat_oam_dma_wraps_from_oamaddr():
    """tests/cpp/test_console.cpp:165-176."""
    o = O.Oracle(nrom_bytes(2))
    o.write(0x2003, 0xFE)
    for i in range(256):
        o.write(0x0200 + i, i)
    o.write(0x4014, 0x02)
    s = o.save()
    oam = s[O.OFF["oam"]:O.OFF["oam"] + 256]
    assert (oam[0xFE], oam[0xFF], oam[0x00]) == (0x00, 0x01, 0x02)
    assert O.field(s, "oam_addr") == 0xFE


def test_kat_controller_serial_bits():
    """tests/cpp/test_console.cpp:178-188: A|Right reads 1,0,0,0,0,0,0,1 then 1s."""
    o = O.Oracle(nrom_bytes(2))
    o.step(0x01 | 0x80, 0)                   # set the pad, run no frame
    o.write(0x4016, 1)
    assert o.read(0x4016) & 1 == 1
    o.write(0x4016, 0)
    assert [o.read(0x4016) & 1 for _ in range(10)] == [1, 0, 0, 0, 0, 0, 0, 1, 1, 1]


def test_kat_controller_matches_standard_pad():
    """tests/cpp/test_cuda_bus.cpp:150-163 (A|Start|Right): strobe-high read,
    then the serial sequence; reads carry open-bus bit 6."""
    o = O.Oracle(nrom_bytes(2))
    o.step(0x01 | 0x08 | 0x80, 0)
    o.write(0x4016, 1)
    assert o.read(0x4016) == 0x41
    o.write(0x4016, 0)
    assert [o.read(0x4016) for _ in range(10)] == [0x41, 0x40, 0x40, 0x41, 0x40, 0x40, 0x40, 0x41, 0x41, 0x41]


def test_kat_status_open_bus_low_bits():
    """tests/cpp/test_cuda_bus.cpp:122-131: status $A0 with open bus $44 reads $A4."""
    o = O.Oracle(nrom_bytes(2))
    o.write(0x2000, 0x80)
    o.write(0x2001, 0x1E)
    o.write(0x2003, 0x44)
    s = o.save()
    s[O.OFF["status"]] = 0xA0
    o.load(s)
    assert o.read(0x2002) == 0xA4


def test_kat_scroll_and_address_latches():
    """tests/cpp/test_cuda_bus.cpp:134-148."""
    o = O.Oracle(nrom_bytes(2))
    o.write(0x2005, 0x23)
    o.write(0x2005, 0x45)
    s = o.save()
    assert (O.field(s, "scroll_x"), O.field(s, "scroll_y"), O.field(s, "fine_x"), O.field(s, "w")) == (0x23, 0x45, 3, 0)
    for a, v in ((0x2006, 0x20), (0x2006, 0x00), (0x2007, 0x34)):
        o.write(a, v)
    s = o.save()
    assert s[O.OFF["nametable"]] == 0x34 and O.field(s, "v", 2) == 0x2001
    for a, v in ((0x2006, 0x3F), (0x2006, 0x10), (0x2007, 0x21)):
        o.write(a, v)
    assert o.save()[O.OFF["palette"]] == 0x21


def test_kat_program_runs_to_trap():
    """tests/cpp/test_console.cpp:201-209: LDA #$42; STA $02; JMP * within 10 instructions."""
    rom = nrom_bytes(2, code={0x8000: [0xA9, 0x42, 0x85, 0x02, 0x4C, 0x04, 0x80]}, reset=0x8000)
    o = O.Oracle(rom)
    assert O.field(o.save(), "pc", 2) == 0x8000
    for _ in range(3):
        o.step_instruction()
    assert O.field(o.save(), "pc", 2) == 0x8004 and o.read(0x0002) == 0x42


def test_kat_ppu_frame_timing():
    """tests/cpp/test_console.cpp:211-233: vblank at scanline 241 dot 1; one
    frame is 341 x 262 dots."""
    o = O.Oracle(nrom_bytes(2))
    assert o.ppu_run(241 * 341 + 1) == 0
    s = o.save()
    assert O.field(s, "status") & 0x80 and O.field(s, "frame_dot", 4) == 241 * 341 + 1
    assert o.ppu_run((262 - 241) * 341 - 1) == 1
    s = o.save()
    assert O.field(s, "frame", 8) == 1 and O.field(s, "frame_dot", 4) == 0 and O.field(s, "status") & 0x80 == 0


def test_kat_sprite0_coarse_hit():
    """tests/cpp/test_console.cpp:235-248."""
    o = O.Oracle(nrom_bytes(2))
    o.write(0x2001, 0x18)
    assert o.ppu_run(30 * 341 + 1) == 0
    assert O.field(o.save(), "status") & 0x40
    assert o.ppu_run((261 - 30) * 341) == 0
    assert O.field(o.save(), "status") & 0x40 == 0


def test_kat_nmi_rom_frame():
    """tests/cpp/test_console.cpp:317-325: the NMI handler runs once per frame."""
    rom = nrom_bytes(2, code={0x8000: [0xA9, 0x80, 0x8D, 0x00, 0x20, 0x4C, 0x05, 0x80],
                              0x9000: [0xE6, 0x00, 0x40]}, reset=0x8000, nmi=0x9000)
    o = O.Oracle(rom)
    n, _, _ = o.step(0, 1, 20000)
    s = o.save()
    assert n > 0 and o.read(0x0000) == 1
    assert O.field(s, "nmi_pending") == 0 and O.field(s, "status") & 0x80 == 0
    assert O.field(s, "frame", 8) == 1


def test_kat_dma_stall_517_cycles():
    """tests/cpp/test_console.cpp:327-345."""
    rom = nrom_bytes(2, code={0x8000: [0xA9, 0x02, 0x8D, 0x14, 0x40, 0x4C, 0x05, 0x80]}, reset=0x8000)
    o = O.Oracle(rom)
    for i in range(256):
        o.write(0x0200 + i, 0xFF - i)
    assert o.step_instruction()[0] == 2
    before = O.field(o.save(), "frame_dot", 4)
    assert o.step_instruction()[0] == 517
    s = o.save()
    assert O.field(s, "frame_dot", 4) - before == 1551
    assert (s[O.OFF["oam"]], s[O.OFF["oam"] + 1]) == (0xFF, 0xFE)


# ---- arithmetic fixed independently of the oracle's code --------------------------

def test_adc_sbc_cmp_exhaustive_against_signed_arithmetic():
    """ADC/SBC/CMP immediate over a grid of (A, operand, carry) plus random
    triples: result, C, Z, N and V equal what integer arithmetic gives (V =
    the signed sum leaves [-128, 127]; SBC borrows when carry is clear).  A
    dropped carry term, a flipped sign or a wrong overflow rule fails here."""
    o = O.Oracle(nrom_bytes(2))
    base = o.save()
    rng = np.random.default_rng(1)
    cases = [(a, m, c) for a in range(0, 256, 3) for m in range(0, 256, 5) for c in (0, 1)]
    cases += [tuple(int(v) for v in t) for t in rng.integers(0, 256, (2000, 3)) % [256, 256, 2]]

    def signed(v: int) -> int:
        return v - 256 if v >= 128 else v

    for a, m, c in cases:
        for kind, opcode in (("adc", 0x69), ("sbc", 0xE9), ("cmp", 0xC9)):
            s = state_with(base, pc=0x0300, p=0x20 | c, a=a)
            s[O.OFF["ram"] + 0x300] = opcode       # execute from RAM: any operand
            s[O.OFF["ram"] + 0x301] = m
            o.load(s)
            o.step_instruction()
            r = o.save()
            ra, rp = O.field(r, "a"), O.field(r, "p")
            assert rp & 0x20, "unused flag reads as 1"
            if kind == "cmp":
                res = (a - m) & 0xFF
                assert ra == a and (rp & 1) == int(a >= m), (kind, a, m, c)
                assert bool(rp & 2) == (res == 0) and bool(rp & 0x80) == bool(res & 0x80), (kind, a, m, c)
                continue
            if kind == "adc":
                total, sres = a + m + c, signed(a) + signed(m) + c
            else:
                total, sres = a + (255 - m) + c, signed(a) - signed(m) - (1 - c)
            exp = total & 0xFF
            assert ra == exp and (rp & 1) == int(total > 255), (kind, a, m, c)
            assert bool(rp & 0x40) == (not -128 <= sres <= 127), (kind, a, m, c)
            assert bool(rp & 2) == (exp == 0) and bool(rp & 0x80) == bool(exp & 0x80), (kind, a, m, c)


def test_ppu_event_dots_closed_form():
    """Frame = 341 x 262 = 89,342 dots; sprite-0 flag at 30*341+1, vblank at
    241*341+1, cleared at 261*341+1 (ppu.hpp:19-25): stepping the PPU dot by
    dot in chunks lands every transition exactly there."""
    o = O.Oracle(nrom_bytes(2))
    o.write(0x2001, 0x18)
    o.write(0x2000, 0x80)
    seen = {}
    prev = O.field(o.save(), "status")
    for dot in range(1, 89342 + 1):
        o.ppu_run(1)
        s = o.save()
        st = O.field(s, "status")
        if st != prev:
            seen.setdefault(st, dot)
        prev = st
    assert seen.get(0x40) == 30 * 341 + 1
    assert seen.get(0xC0) == 241 * 341 + 1
    assert seen.get(0x00) == 261 * 341 + 1
    assert O.field(o.save(), "frame", 8) == 1 and O.field(o.save(), "frame_dot", 4) == 0


# ---- FCS snapshots (tests/test_fcs_parser.py:32-83 known answers) -----------------

def test_fcs_known_answers_via_oracle_blob_layout():
    """The canonical blob that nesle_parse_fcs builds from the reference's
    bundled W1-1 state carries the known register values; checked through the
    C ABI's host-only parser (no GPU call)."""
    import gzip

    from nesle_amd import abi

    raw = gzip.decompress((GOLDEN / "smb_level1_1.state").read_bytes())
    s = abi.parse_fcs(raw)
    assert O.field(s, "pc", 2) == 0x8057
    assert (O.field(s, "a"), O.field(s, "x"), O.field(s, "y"), O.field(s, "sp"), O.field(s, "p")) == \
        (0x90, 0x00, 0x01, 0xFF, 0xA5)
    assert (O.field(s, "ctrl"), O.field(s, "mask"), O.field(s, "status")) == (0x90, 0x1E, 0x40)
    assert O.field(s, "v", 2) == 0x0800 and O.field(s, "t", 2) == 0
    assert (O.field(s, "fine_x"), O.field(s, "w"), O.field(s, "read_buffer"), O.field(s, "open_bus")) == \
        (0, 0, 0xFF, 0x90)
    ram = s[O.OFF["ram"]:O.OFF["ram"] + 2048]
    assert ram[0x770] == 1 and ram[0x75F] == 0 and ram[0x75C] == 0
    assert int(ram[0x7F8]) * 100 + int(ram[0x7F9]) * 10 + int(ram[0x7FA]) > 0
    assert s[O.OFF["palette"]] == 0x22
    # Warm-reset mapping (batch_step.cuh:174-242): frame position, NMI, pads,
    # DMA and scroll start at zero.
    assert O.field(s, "frame_dot", 4) == 0 and O.field(s, "frame", 8) == 0 and O.field(s, "nmi_pending") == 0
    with pytest.raises(RuntimeError):
        abi.parse_fcs(raw[:32])
    with pytest.raises(RuntimeError):
        abi.parse_fcs(b"XXXX" + raw[4:])
