"""Seeded synthetic mapper-0 (NROM) ROMs and controller streams.

The workload every parity test and benchmark of this package runs on.  A ROM is
a pure function of its seed:

* 32 KB PRG ($8000-$FFFF) holding a RESET routine, a branch-heavy main loop of
  uniformly drawn official 6502 opcodes with valid operands (counted loops,
  data-dependent forward branches, subroutine calls, balanced stack pairs,
  indexed and indirect loads/stores to RAM $0000-$07FF), an NMI handler that
  runs every frame and an IRQ/BRK handler.
* 8 KB CHR of seeded random 2bpp tiles, vertical mirroring.

The NMI handler saves A/X/Y, starts OAM DMA from page $02 ($4014), strobes and
reads controller 1 into ``BUTTONS``, moves a 16-bit x position (right/B add,
left subtracts), counts frames, decrements the done byte every 8th frame while
it is non-zero, writes $2006/$2007 (nametable tiles), reads $2007 once, writes
$2005 scroll, $2000 and $2001, then returns with RTI.

Every load hits RAM, PRG ROM or $2002/$2004/$2007/$4016, every store or
read-modify-write hits RAM, $2000-$2007, $4014 or $4016, and $2001 is written
only by the NMI handler.  Those are the inputs on which the reference's CPU core
(cpp/include/nesle/console.hpp) and its batched device core
(cpp/include/nesle/cuda/batch_bus.cuh) agree, so the ROM pins both at once.

Controller streams use a counter-based splitmix64 so that host, device and CPU
baseline draw identical masks without any transfer:
``mask(seed, env, step) = splitmix64(seed ^ (env << 32) ^ step) & 0xFF``.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

MASK64 = (1 << 64) - 1

# Fixed RAM map of the synthetic ROM (the reward/done spec points here).
PTR_BASE = 0x00        # 8 little-endian pointers into $0300-$0700
FRAME_COUNTER = 0x10
BUTTONS = 0x11
X_LO = 0x12
X_HI = 0x13
DONE_BYTE = 0x14
LOOP_COUNTERS = 0x16   # one byte per loop nesting level (2 levels)
NMI_TEMP = 0x1A
SCRATCH_ZP_LO = 0x20   # random stores/RMW in zero page land in [$20, $FF]
OAM_PAGE = 0x02

NMI_ADDR = 0xF800
IRQ_ADDR = 0xFF00
DATA_ADDR = 0xF000
CODE_END = 0xEF00


def splitmix64(x: int) -> int:
    """One splitmix64 output for the 64-bit counter ``x``."""
    z = (x + 0x9E3779B97F4A7C15) & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def splitmix64_np(x: np.ndarray) -> np.ndarray:
    """Vectorised splitmix64 over a uint64 array (wrapping arithmetic)."""
    x = x.astype(np.uint64, copy=False)
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def action_masks(seed: int, num_envs: int, step: int, env_offset: int = 0) -> np.ndarray:
    """Controller masks (uint8, shape (num_envs,)) for one step of every env."""
    env = np.arange(env_offset, env_offset + num_envs, dtype=np.uint64)
    ctr = np.uint64(seed & MASK64) ^ (env << np.uint64(32)) ^ np.uint64(step & MASK64)
    return (splitmix64_np(ctr) & np.uint64(0xFF)).astype(np.uint8)


def action_table(seed: int, num_envs: int, num_steps: int) -> np.ndarray:
    """Masks for ``num_steps`` steps, shape (num_steps, num_envs), uint8."""
    out = np.empty((num_steps, num_envs), dtype=np.uint8)
    for k in range(num_steps):
        out[k] = action_masks(seed, num_envs, k)
    return out


class _Rng:
    """Deterministic stream built on splitmix64 (independent of numpy's RNGs)."""

    def __init__(self, seed: int) -> None:
        self.state = seed & MASK64

    def next(self) -> int:
        self.state = (self.state + 1) & MASK64
        return splitmix64(self.state ^ 0x5DEECE66D)

    def below(self, n: int) -> int:
        return self.next() % n

    def range(self, lo: int, hi: int) -> int:
        """Uniform integer in [lo, hi]."""
        return lo + self.below(hi - lo + 1)

    def chance(self, num: int, den: int) -> bool:
        return self.below(den) < num

    def choice(self, seq):
        return seq[self.below(len(seq))]


# Official 6502 opcodes by (mnemonic, mode).  Modes: imp acc imm zp zpx zpy abs
# absx absy indx indy ind rel.
_OPCODES: dict[tuple[str, str], int] = {}


def _def(mn: str, pairs: list[tuple[str, int]]) -> None:
    for mode, op in pairs:
        _OPCODES[(mn, mode)] = op


_def("ORA", [("imm", 0x09), ("zp", 0x05), ("zpx", 0x15), ("abs", 0x0D), ("absx", 0x1D), ("absy", 0x19), ("indx", 0x01), ("indy", 0x11)])
_def("AND", [("imm", 0x29), ("zp", 0x25), ("zpx", 0x35), ("abs", 0x2D), ("absx", 0x3D), ("absy", 0x39), ("indx", 0x21), ("indy", 0x31)])
_def("EOR", [("imm", 0x49), ("zp", 0x45), ("zpx", 0x55), ("abs", 0x4D), ("absx", 0x5D), ("absy", 0x59), ("indx", 0x41), ("indy", 0x51)])
_def("ADC", [("imm", 0x69), ("zp", 0x65), ("zpx", 0x75), ("abs", 0x6D), ("absx", 0x7D), ("absy", 0x79), ("indx", 0x61), ("indy", 0x71)])
_def("SBC", [("imm", 0xE9), ("zp", 0xE5), ("zpx", 0xF5), ("abs", 0xED), ("absx", 0xFD), ("absy", 0xF9), ("indx", 0xE1), ("indy", 0xF1)])
_def("CMP", [("imm", 0xC9), ("zp", 0xC5), ("zpx", 0xD5), ("abs", 0xCD), ("absx", 0xDD), ("absy", 0xD9), ("indx", 0xC1), ("indy", 0xD1)])
_def("LDA", [("imm", 0xA9), ("zp", 0xA5), ("zpx", 0xB5), ("abs", 0xAD), ("absx", 0xBD), ("absy", 0xB9), ("indx", 0xA1), ("indy", 0xB1)])
_def("STA", [("zp", 0x85), ("zpx", 0x95), ("abs", 0x8D), ("absx", 0x9D), ("absy", 0x99), ("indx", 0x81), ("indy", 0x91)])
_def("LDX", [("imm", 0xA2), ("zp", 0xA6), ("zpy", 0xB6), ("abs", 0xAE), ("absy", 0xBE)])
_def("LDY", [("imm", 0xA0), ("zp", 0xA4), ("zpx", 0xB4), ("abs", 0xAC), ("absx", 0xBC)])
_def("STX", [("zp", 0x86), ("zpy", 0x96), ("abs", 0x8E)])
_def("STY", [("zp", 0x84), ("zpx", 0x94), ("abs", 0x8C)])
_def("CPX", [("imm", 0xE0), ("zp", 0xE4), ("abs", 0xEC)])
_def("CPY", [("imm", 0xC0), ("zp", 0xC4), ("abs", 0xCC)])
_def("BIT", [("zp", 0x24), ("abs", 0x2C)])
_def("INC", [("zp", 0xE6), ("zpx", 0xF6), ("abs", 0xEE), ("absx", 0xFE)])
_def("DEC", [("zp", 0xC6), ("zpx", 0xD6), ("abs", 0xCE), ("absx", 0xDE)])
_def("ASL", [("acc", 0x0A), ("zp", 0x06), ("zpx", 0x16), ("abs", 0x0E), ("absx", 0x1E)])
_def("LSR", [("acc", 0x4A), ("zp", 0x46), ("zpx", 0x56), ("abs", 0x4E), ("absx", 0x5E)])
_def("ROL", [("acc", 0x2A), ("zp", 0x26), ("zpx", 0x36), ("abs", 0x2E), ("absx", 0x3E)])
_def("ROR", [("acc", 0x6A), ("zp", 0x66), ("zpx", 0x76), ("abs", 0x6E), ("absx", 0x7E)])
_def("JMP", [("abs", 0x4C), ("ind", 0x6C)])
_def("JSR", [("abs", 0x20)])
for _mn, _op in [("BPL", 0x10), ("BMI", 0x30), ("BVC", 0x50), ("BVS", 0x70),
                 ("BCC", 0x90), ("BCS", 0xB0), ("BNE", 0xD0), ("BEQ", 0xF0)]:
    _OPCODES[(_mn, "rel")] = _op
for _mn, _op in [("BRK", 0x00), ("PHP", 0x08), ("CLC", 0x18), ("PLP", 0x28), ("SEC", 0x38),
                 ("RTI", 0x40), ("PHA", 0x48), ("CLI", 0x58), ("RTS", 0x60), ("PLA", 0x68),
                 ("SEI", 0x78), ("DEY", 0x88), ("TXA", 0x8A), ("TYA", 0x98), ("TXS", 0x9A),
                 ("TAY", 0xA8), ("TAX", 0xAA), ("CLV", 0xB8), ("TSX", 0xBA), ("INY", 0xC8),
                 ("DEX", 0xCA), ("CLD", 0xD8), ("INX", 0xE8), ("NOP", 0xEA), ("SED", 0xF8)]:
    _OPCODES[(_mn, "imp")] = _op

# Every official opcode byte (151 of them).
OFFICIAL_OPCODES: frozenset[int] = frozenset(_OPCODES.values())

_STORES = {"STA", "STX", "STY"}
_RMW = {"INC", "DEC", "ASL", "LSR", "ROL", "ROR"}
_CONTROL = {"JMP", "JSR", "RTS", "RTI", "BRK", "PHA", "PHP", "PLA", "PLP", "TXS"}

# The uniformly drawn "data" opcodes of the main loop: every official opcode
# that is not control flow, stack or TXS.
DATA_OPCODES: list[tuple[str, str, int]] = sorted(
    (mn, mode, op) for (mn, mode), op in _OPCODES.items()
    if mode != "rel" and mn not in _CONTROL
)
_MODE_LEN = {"imp": 1, "acc": 1, "imm": 2, "zp": 2, "zpx": 2, "zpy": 2, "abs": 3,
             "absx": 3, "absy": 3, "indx": 2, "indy": 2, "ind": 3, "rel": 2}


class _Asm:
    """Tiny 6502 assembler over the 32 KB PRG image ($8000-$FFFF)."""

    def __init__(self) -> None:
        self.prg = bytearray(0x8000)
        self.pc = 0x8000
        self.fixups: list[tuple[int, str, str]] = []   # (offset, label, kind)
        self.labels: dict[str, int] = {}
        self._anon = 0

    def org(self, addr: int) -> None:
        self.pc = addr

    def label(self, name: str | None = None) -> str:
        if name is None:
            self._anon += 1
            name = f"_L{self._anon}"
        self.labels[name] = self.pc
        return name

    def new_label(self) -> str:
        self._anon += 1
        return f"_L{self._anon}"

    def byte(self, *values: int) -> None:
        for v in values:
            self.prg[self.pc - 0x8000] = v & 0xFF
            self.pc += 1

    def op(self, mn: str, mode: str = "imp", arg: int | str | None = None) -> None:
        code = _OPCODES[(mn, mode)]
        self.byte(code)
        n = _MODE_LEN[mode] - 1
        if n == 0:
            return
        if isinstance(arg, str):
            kind = "rel" if mode == "rel" else ("abs" if n == 2 else "zp")
            self.fixups.append((self.pc - 0x8000, arg, kind))
            self.byte(*([0] * n))
            return
        assert arg is not None
        if n == 1:
            self.byte(arg & 0xFF)
        else:
            self.byte(arg & 0xFF, (arg >> 8) & 0xFF)

    def resolve(self) -> None:
        for off, name, kind in self.fixups:
            target = self.labels[name]
            if kind == "abs":
                self.prg[off] = target & 0xFF
                self.prg[off + 1] = (target >> 8) & 0xFF
            elif kind == "rel":
                disp = target - (0x8000 + off + 1)
                if not -128 <= disp <= 127:
                    raise ValueError(f"branch to {name} out of range ({disp})")
                self.prg[off] = disp & 0xFF
            else:
                self.prg[off] = target & 0xFF


@dataclass
class SynthRom:
    seed: int
    rom: bytes                     # full iNES image
    prg: bytes
    chr: bytes
    done_init: int
    nmi_addr: int = NMI_ADDR
    labels: dict[str, int] = field(default_factory=dict)


class _Gen:
    def __init__(self, seed: int) -> None:
        self.r = _Rng(seed)
        self.a = _Asm()
        self.subs: list[str] = []

    # -- operand choices ---------------------------------------------------
    def _read_abs(self) -> int:
        if self.r.chance(2, 3):
            return self.r.range(0x0000, 0x07FF)
        return self.r.range(0x8000, 0xFFFF)

    def _read_abs_indexed(self) -> int:
        if self.r.chance(2, 3):
            return self.r.range(0x0000, 0x0700)
        return self.r.range(0x8000, 0xFEFF)

    def emit_data_op(self) -> None:
        """One uniformly drawn data opcode with operands that stay in bounds."""
        mn, mode, _ = self.r.choice(DATA_OPCODES)
        writes = mn in _STORES or (mn in _RMW and mode != "acc")
        a, r = self.a, self.r
        if mode in ("imp", "acc"):
            a.op(mn, mode)
        elif mode == "imm":
            a.op(mn, mode, r.below(256))
        elif mode == "zp":
            a.op(mn, mode, r.range(SCRATCH_ZP_LO, 0xFF) if writes else r.below(256))
        elif mode in ("zpx", "zpy"):
            if writes:
                # Pin the index so the wrapped zero-page address stays in scratch.
                k = r.range(0, 0x3F)
                a.op("LDX" if mode == "zpx" else "LDY", "imm", k)
                a.op(mn, mode, r.range(SCRATCH_ZP_LO, 0xFF - k))
            else:
                a.op(mn, mode, r.below(256))
        elif mode == "abs":
            a.op(mn, mode, r.range(0x0200, 0x07FF) if writes else self._read_abs())
        elif mode in ("absx", "absy"):
            a.op(mn, mode, r.range(0x0200, 0x0700) if writes else self._read_abs_indexed())
        elif mode == "indx":
            k = r.range(0, 7) * 2
            slot = r.range(0, 7) * 2
            a.op("LDX", "imm", k)
            a.op(mn, mode, (PTR_BASE + slot - k) & 0xFF)
        elif mode == "indy":
            a.op(mn, mode, PTR_BASE + r.range(0, 7) * 2)
        else:
            raise AssertionError(mode)

    # -- structured blocks ---------------------------------------------------
    def emit_block(self, depth: int, budget: int, sub_index: int | None) -> None:
        a, r = self.a, self.r
        n = r.range(max(2, budget // 2), budget)
        i = 0
        while i < n:
            k = r.below(100)
            if k < 62:
                self.emit_data_op()
            elif k < 74:
                # Data-dependent forward branch over a balanced sub-block.
                br = r.choice(["BPL", "BMI", "BVC", "BVS", "BCC", "BCS", "BNE", "BEQ"])
                skip = a.new_label()
                a.op(br, "rel", skip)
                self.emit_small(depth + 1)
                a.label(skip)
            elif k < 79 and depth < 2:
                # Counted loop: the counter byte is never a random store target.
                ctr = LOOP_COUNTERS + depth
                a.op("LDA", "imm", r.range(2, 5))
                a.op("STA", "zp", ctr)
                top = a.label()
                self.emit_small(depth + 1)
                a.op("DEC", "zp", ctr)
                a.op("BNE", "rel", top)
            elif k < 83:
                # Controller-dependent branch: makes envs diverge.
                skip = a.new_label()
                a.op("LDA", "zp", BUTTONS)
                a.op("AND", "imm", 1 << r.below(8))
                a.op(r.choice(["BEQ", "BNE"]), "rel", skip)
                self.emit_small(depth + 1)
                a.label(skip)
            elif k < 87:
                callee = self._pick_sub(sub_index)
                if callee is not None:
                    a.op("JSR", "abs", callee)
            elif k < 90:
                a.op("PHA")
                self.emit_small(depth + 1)
                a.op("PLA")
            elif k < 92:
                a.op("PHP")
                self.emit_small(depth + 1)
                a.op("PLP")
            elif k < 95:
                # PPU status / OAM data reads (side effects on $2002).
                src = r.choice([0x2002, 0x2002, 0x2004])
                a.op(r.choice(["LDA", "BIT"]) if src == 0x2002 else "LDA", "abs", src)
            elif k < 96:
                a.op("LDA", "abs", 0x4016)
            elif k < 97:
                a.op("BRK")
                a.byte(r.below(256))
            else:
                # JMP over a short dead sub-block (also exercises JMP abs).
                skip = a.new_label()
                a.op("JMP", "abs", skip)
                for _ in range(r.range(1, 3)):
                    self.emit_data_op()
                a.label(skip)
            i += 1

    def emit_small(self, depth: int) -> None:
        """A balanced sub-block short enough for an 8-bit branch displacement.

        Depth 1 holds at most 5 items of at most 23 bytes each; depth 2 and
        deeper holds 1-3 plain data ops (at most 5 bytes each).
        """
        if depth >= 2:
            for _ in range(self.r.range(1, 3)):
                self.emit_data_op()
            return
        self.emit_block(depth, 5, None)

    def _pick_sub(self, sub_index: int | None) -> str | None:
        """Main loop calls any subroutine, subroutines 0-7 call leaves 8-15."""
        if sub_index is None:
            return self.subs[self.r.below(len(self.subs))]
        if sub_index < 8:
            return self.subs[self.r.range(8, len(self.subs) - 1)]
        return None

    # -- whole ROM ---------------------------------------------------------
    def build(self, seed: int, prg_banks: int = 2, split: bool = False) -> SynthRom:
        """``prg_banks`` 2: 32 KB PRG at $8000-$FFFF.  1: a 16 KB image (NROM-128),
        mirrored at $8000 and $C000: the program is assembled at $C000-$FFFF
        (RESET/main loop $C000-$CFFF, subroutines $D000-$EEFF) and the
        vectors point into the $8000 mirror, so the console starts, takes
        NMIs and BRKs in the low copy and jumps or returns into the high one.

        ``split``: the status-bar variant.  Sprite 0 sits at a seeded row near
        the top of the screen, the NMI handler sets the status bar's scroll
        (0, 0), and every pass of the main loop first waits for the sprite-0
        flag of PPUSTATUS to clear (pre-render line) and set again (line 30),
        burns a seeded, frame-dependent delay and then writes the play
        field's scroll to $2005 (x from the x position, a seeded y), all
        without IRQs; a shorter block of random work follows.  Frames then
        start with the status-bar scroll and end with the play-field one."""
        a, r = self.a, self.r
        small = prg_banks == 1
        code_lo = 0xC000 if small else 0x8000
        main_stop = 0xCC00 if small else 0xB800   # the main loop's last block starts below this
        if split:
            main_stop = code_lo + 0x1000
        subs_at = 0xD000 if small else 0xC000
        done_init = r.range(25, 250)     # done fires after 8*done_init frames
        pointers = [r.range(0x0300, 0x0700) for _ in range(8)]
        ctrl = 0x90 | r.below(4)         # NMI on, BG table $1000, seeded nametable
        mask = r.choice([0x1E, 0x18, 0x1A, 0x1C])

        # Subroutines first (placed high, called from the main loop).
        n_subs = 16
        self.subs = [a.new_label() for _ in range(n_subs)]
        a.org(subs_at)
        for i in range(n_subs - 1, -1, -1):
            a.label(self.subs[i])
            self.emit_block(1, 24, i)
            a.op("RTS")
        sub_end = a.pc
        if sub_end > CODE_END:
            raise ValueError("subroutines overflow the code area")

        # RESET routine.
        a.org(code_lo)
        a.label("RESET")
        a.op("SEI"); a.op("CLD")
        a.op("LDX", "imm", 0xFF); a.op("TXS")
        for i, p in enumerate(pointers):
            a.op("LDA", "imm", p & 0xFF); a.op("STA", "zp", PTR_BASE + 2 * i)
            a.op("LDA", "imm", p >> 8); a.op("STA", "zp", PTR_BASE + 2 * i + 1)
        a.op("LDA", "imm", 0x00); a.op("STA", "zp", X_LO)
        a.op("LDA", "imm", 0x01); a.op("STA", "zp", X_HI)
        a.op("LDA", "imm", done_init); a.op("STA", "zp", DONE_BYTE)
        # Palette: 32 bytes from the data table.
        a.op("LDA", "abs", 0x2002)
        a.op("LDA", "imm", 0x3F); a.op("STA", "abs", 0x2006)
        a.op("LDA", "imm", 0x00); a.op("STA", "abs", 0x2006)
        a.op("LDX", "imm", 0x00)
        pal = a.label()
        a.op("LDA", "absx", DATA_ADDR); a.op("STA", "abs", 0x2007)
        a.op("INX"); a.op("CPX", "imm", 0x20); a.op("BNE", "rel", pal)
        # Nametable 0: 256 tiles + attributes, nametable 1: 256 tiles.
        for hi, lo, src in ((0x20, 0x00, DATA_ADDR + 0x100), (0x23, 0xC0, DATA_ADDR + 0x200),
                            (0x24, 0x00, DATA_ADDR + 0x300)):
            a.op("LDA", "imm", hi); a.op("STA", "abs", 0x2006)
            a.op("LDA", "imm", lo); a.op("STA", "abs", 0x2006)
            a.op("LDX", "imm", 0x00)
            lp = a.label()
            a.op("LDA", "absx", src); a.op("STA", "abs", 0x2007)
            a.op("INX")
            if hi == 0x23:
                a.op("CPX", "imm", 0x40)
            a.op("BNE", "rel", lp)
        # OAM source page from the data table.
        a.op("LDX", "imm", 0x00)
        lp = a.label()
        a.op("LDA", "absx", DATA_ADDR + 0x400); a.op("STA", "absx", OAM_PAGE << 8)
        a.op("INX"); a.op("BNE", "rel", lp)
        a.op("LDA", "imm", ctrl); a.op("STA", "abs", 0x2000)
        a.op("JMP", "abs", "MAIN")

        # Main loop fills the rest of the low code area.
        a.label("MAIN")
        if split:
            # Sprite-0 timed scroll split: PPUSTATUS bit 6 clears at the
            # pre-render line and sets at line 30 (BIT copies it into V).
            w0 = a.label()
            a.op("BIT", "abs", 0x2002); a.op("BVS", "rel", w0)
            w1 = a.label()
            a.op("BIT", "abs", 0x2002); a.op("BVC", "rel", w1)
            a.op("LDA", "zp", FRAME_COUNTER); a.op("AND", "imm", 0x1F)
            a.op("CLC"); a.op("ADC", "imm", r.range(1, 64)); a.op("TAY")
            dl = a.label()
            a.op("DEY"); a.op("BNE", "rel", dl)
            a.op("LDA", "zp", X_LO); a.op("STA", "abs", 0x2005)
            a.op("LDA", "imm", r.range(0, 239)); a.op("STA", "abs", 0x2005)
        while a.pc < main_stop:
            self.emit_block(0, 12, None)
        a.op("JMP", "abs", "MAIN")
        if a.pc > subs_at:
            raise ValueError("main loop overflows into subroutines")

        # Data tables at $F000: palette, nametables, attributes, sprites, noise.
        data = bytearray(r.below(256) for _ in range(0x800))
        if split:
            data[0x400] = r.range(16, 40)   # sprite 0's top row - 1: the split lands at rows 25-49
        pal_bytes = bytes(b & 0x3F for b in data[:0x20])
        a.org(DATA_ADDR)
        a.byte(*pal_bytes)
        a.byte(*data[0x20:0x800])

        # NMI handler.
        a.org(NMI_ADDR)
        a.label("NMI")
        a.op("PHA"); a.op("TXA"); a.op("PHA"); a.op("TYA"); a.op("PHA")
        a.op("LDA", "imm", OAM_PAGE); a.op("STA", "abs", 0x4014)
        a.op("LDA", "imm", 0x01); a.op("STA", "abs", 0x4016)
        a.op("LDA", "imm", 0x00); a.op("STA", "abs", 0x4016)
        a.op("LDX", "imm", 0x08)
        rd = a.label()
        a.op("LDA", "abs", 0x4016); a.op("LSR", "acc"); a.op("ROR", "zp", BUTTONS)
        a.op("DEX"); a.op("BNE", "rel", rd)
        # x position: Right +1 (+1 more with B), Left -1.
        noright = a.new_label(); r1 = a.new_label(); noleft = a.new_label(); l1 = a.new_label()
        a.op("LDA", "zp", BUTTONS); a.op("BPL", "rel", noright)
        a.op("INC", "zp", X_LO); a.op("BNE", "rel", r1); a.op("INC", "zp", X_HI)
        a.label(r1)
        a.op("LDA", "zp", BUTTONS); a.op("AND", "imm", 0x02); a.op("BEQ", "rel", noright)
        a.op("INC", "zp", X_LO); a.op("BNE", "rel", noright); a.op("INC", "zp", X_HI)
        a.label(noright)
        a.op("LDA", "zp", BUTTONS); a.op("AND", "imm", 0x40); a.op("BEQ", "rel", noleft)
        a.op("LDA", "zp", X_LO); a.op("BNE", "rel", l1); a.op("DEC", "zp", X_HI)
        a.label(l1)
        a.op("DEC", "zp", X_LO)
        a.label(noleft)
        # Frame counter and done countdown (every 8th frame while non-zero).
        nodone = a.new_label()
        a.op("INC", "zp", FRAME_COUNTER)
        a.op("LDA", "zp", FRAME_COUNTER); a.op("AND", "imm", 0x07); a.op("BNE", "rel", nodone)
        a.op("LDA", "zp", DONE_BYTE); a.op("BEQ", "rel", nodone); a.op("DEC", "zp", DONE_BYTE)
        a.label(nodone)
        # Nametable writes at a frame-dependent address, one buffered read.
        a.op("LDA", "abs", 0x2002)
        a.op("LDA", "zp", FRAME_COUNTER); a.op("AND", "imm", 0x03); a.op("ORA", "imm", 0x20)
        a.op("STA", "abs", 0x2006)
        a.op("LDA", "zp", FRAME_COUNTER); a.op("ASL", "acc"); a.op("ASL", "acc"); a.op("ASL", "acc")
        a.op("STA", "abs", 0x2006)
        for src in (BUTTONS, X_LO, X_HI, DONE_BYTE):
            a.op("LDA", "zp", src); a.op("STA", "abs", 0x2007)
        a.op("LDA", "abs", 0x2007); a.op("STA", "zp", NMI_TEMP)
        # Scroll, control and mask.
        a.op("LDA", "abs", 0x2002)
        if split:   # the status bar's scroll: the frame starts with it
            a.op("LDA", "imm", 0x00); a.op("STA", "abs", 0x2005)
        else:
            a.op("LDA", "zp", X_LO); a.op("STA", "abs", 0x2005)
        a.op("LDA", "imm", 0x00); a.op("STA", "abs", 0x2005)
        a.op("LDA", "imm", ctrl); a.op("STA", "abs", 0x2000)
        a.op("LDA", "imm", mask); a.op("STA", "abs", 0x2001)
        a.op("PLA"); a.op("TAY"); a.op("PLA"); a.op("TAX"); a.op("PLA")
        a.op("RTI")

        a.org(IRQ_ADDR)
        a.label("IRQ")
        a.op("RTI")

        mirror = 0x4000 if small else 0
        a.org(0xFFFA)
        a.byte(NMI_ADDR & 0xFF, (NMI_ADDR - mirror) >> 8)
        a.byte(0x00, (code_lo - mirror) >> 8)
        a.byte(IRQ_ADDR & 0xFF, (IRQ_ADDR - mirror) >> 8)
        a.resolve()

        chr_bytes = bytes(r.below(256) for _ in range(0x2000))
        header = bytes([0x4E, 0x45, 0x53, 0x1A, prg_banks, 1, 0x01, 0x00, 0, 0, 0, 0, 0, 0, 0, 0])
        prg = bytes(a.prg[0x4000:]) if small else bytes(a.prg)
        return SynthRom(seed=seed, rom=header + prg + chr_bytes, prg=prg, chr=chr_bytes,
                        done_init=done_init, labels=dict(a.labels))


def make_rom(seed: int, prg_banks: int = 2, split: bool = False) -> SynthRom:
    """The synthetic NROM image for ``seed`` (deterministic); ``prg_banks`` 1
    gives the 16 KB (NROM-128) variant; ``split`` the status-bar variant
    (sprite-0 timed mid-frame $2005 writes, see _Gen.build)."""
    if prg_banks not in (1, 2):
        raise ValueError("prg_banks must be 1 or 2")
    return _Gen(seed).build(seed, prg_banks, split)
