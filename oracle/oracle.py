"""ctypes access to the parity oracle and to the reference-core harness.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or as the timed CPU baseline.  The
product path (nesle_amd) never imports this module.

* ``Oracle`` wraps oracle/_bin/libnes_oracle.so, the clean-room C++
  restatement of the reference CPU core (oracle/nes_oracle.cpp).
* ``RefConsole`` wraps oracle/_ref/libnesle_ref.so, the reference's own
  ``nesle::Console`` compiled from its sources by ``make -C oracle ref``.

Both expose the same canonical 22,896-byte state blob (layout in
oracle/nes_oracle.cpp) so that states can be compared byte for byte.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "_bin" / "libnes_oracle.so"
REF_SO = HERE / "_ref" / "libnesle_ref.so"
STATE_BYTES = 22896

# Offsets into the canonical state blob.
OFF = {
    "pc": 4, "a": 6, "x": 7, "y": 8, "sp": 9, "p": 10, "nmi_pending": 11, "cycles": 12,
    "frame": 20, "frame_dot": 28, "ctrl": 32, "mask": 33, "status": 34, "oam_addr": 35,
    "open_bus": 36, "read_buffer": 37, "v": 38, "t": 40, "fine_x": 42, "w": 43,
    "scroll_x": 44, "scroll_y": 45, "c1_buttons": 46, "c1_shift": 47, "c1_count": 48,
    "strobe": 49, "c2_count": 50, "fault": 51, "pending_dma": 52, "apu_io": 56, "ram": 80,
    "prg_ram": 2128, "oam": 10320, "palette": 10576, "nametable": 10608, "chr_ram": 14704,
}
SECTIONS = {
    # name: byte ranges of the state blob hashed (concatenated) per frame by
    # the golden fixtures.
    "cpu": [(4, 16)],                      # pc, a, x, y, sp, p, nmi_pending, cycles
    "ppu": [(20, 36), (56, 24)],           # PPU scalars, pads, fault, DMA, $4000-$4017
    "ram": [(80, 2048)],
    "mem": [(2128, 8192), (10320, 256), (10576, 32), (10608, 4096), (14704, 8192)],
}

_U8P = ctypes.POINTER(ctypes.c_uint8)

# Presentation state as Oracle.presentation / RefConsole.presentation lay it out.
PRESENT_BYTES = 2352
PRESENT_OFF = {"fields": 0, "latch": 7, "oam": 16, "palette": 272, "nametable": 304}


def build(ref: bool = False) -> None:
    """Compile the oracle (and, if asked, the reference harness) with make."""
    cmd = ["make", "-s", "-C", str(HERE), "all"]
    if ref:
        cmd.append("ref")
    subprocess.run(cmd, check=True)


def fnv1a(data: bytes | np.ndarray) -> int:
    h = 0xCBF29CE484222325
    for b in bytes(data):
        h ^= b
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def fnv1a_np(data: np.ndarray) -> int:
    """FNV-1a 64 of a uint8 array (vectorised over rows is not possible; loop in C)."""
    return _oracle_lib().oracle_fnv1a(data.ctypes.data_as(_U8P), data.nbytes)


def section_hashes(state: bytes | np.ndarray) -> dict[str, int]:
    buf = np.frombuffer(bytes(state), dtype=np.uint8)
    return {k: fnv1a_np(np.concatenate([buf[o:o + n] for o, n in ranges]))
            for k, ranges in SECTIONS.items()}


def field(state: bytes | np.ndarray, name: str, size: int = 1) -> int:
    o = OFF[name]
    return int.from_bytes(bytes(state[o:o + size]), "little")


_LIB = None
_REF = None


def _oracle_lib():
    global _LIB
    if _LIB is None:
        if not ORACLE_SO.exists():
            build()
        lib = ctypes.CDLL(str(ORACLE_SO))
        lib.oracle_create.restype = ctypes.c_void_p
        lib.oracle_create.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
        lib.oracle_destroy.argtypes = [ctypes.c_void_p]
        lib.oracle_last_error.restype = ctypes.c_char_p
        lib.oracle_step.restype = ctypes.c_int64
        lib.oracle_step.argtypes = [ctypes.c_void_p, ctypes.c_uint8, ctypes.c_uint32, ctypes.c_uint64,
                                    ctypes.POINTER(ctypes.c_float), _U8P]
        lib.oracle_set_reward.argtypes = [ctypes.c_void_p] + [ctypes.c_uint32] * 5 + [ctypes.c_float]
        lib.oracle_step_instruction.restype = ctypes.c_int64
        lib.oracle_step_instruction.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32)]
        lib.oracle_bus_read.restype = ctypes.c_uint32
        lib.oracle_bus_read.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        lib.oracle_bus_write.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32]
        lib.oracle_ppu_peek.restype = ctypes.c_uint32
        lib.oracle_ppu_peek.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        lib.oracle_ppu_run.restype = ctypes.c_uint32
        lib.oracle_ppu_run.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        lib.oracle_save.argtypes = [ctypes.c_void_p, _U8P]
        lib.oracle_load.argtypes = [ctypes.c_void_p, _U8P]
        lib.oracle_fnv1a.restype = ctypes.c_uint64
        lib.oracle_fnv1a.argtypes = [_U8P, ctypes.c_size_t]
        lib.oracle_splitmix64.restype = ctypes.c_uint64
        lib.oracle_splitmix64.argtypes = [ctypes.c_uint64]
        lib.oracle_render.argtypes = [ctypes.c_void_p, ctypes.c_uint32, _U8P]
        lib.oracle_seed_presentation.argtypes = [ctypes.c_void_p]
        lib.oracle_set_presentation.argtypes = [ctypes.c_void_p, _U8P]
        lib.oracle_present_get.argtypes = [ctypes.c_void_p, _U8P]
        lib.oracle_palette_rgb.argtypes = [_U8P]
        lib.oracle_gray84.argtypes = [_U8P, _U8P]
        lib.oracle_run_batch.restype = ctypes.c_double
        lib.oracle_run_batch.argtypes = [ctypes.c_char_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_uint32,
                                         ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint32,
                                         ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]
        lib.oracle_run_levels.restype = ctypes.c_double
        lib.oracle_run_levels.argtypes = [ctypes.c_char_p, ctypes.c_size_t, _U8P, ctypes.c_uint32, _U8P, _U8P,
                                          ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                          ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32,
                                          ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                                          ctypes.POINTER(ctypes.c_uint64)]
        _LIB = lib
    return _LIB


def ref_available() -> bool:
    return REF_SO.exists()


def _ref_lib():
    global _REF
    if _REF is None:
        lib = ctypes.CDLL(str(REF_SO))
        lib.ref_create.restype = ctypes.c_void_p
        lib.ref_create.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
        lib.ref_destroy.argtypes = [ctypes.c_void_p]
        lib.ref_last_error.restype = ctypes.c_char_p
        lib.ref_step.restype = ctypes.c_int64
        lib.ref_step.argtypes = [ctypes.c_void_p, ctypes.c_uint8, ctypes.c_uint32, ctypes.c_uint64]
        lib.ref_save.argtypes = [ctypes.c_void_p, _U8P]
        lib.ref_load.argtypes = [ctypes.c_void_p, _U8P]
        lib.ref_step_instruction.restype = ctypes.c_int64
        lib.ref_step_instruction.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32)]
        lib.ref_render_rgb.argtypes = [ctypes.c_void_p, _U8P]
        lib.ref_present_seed.argtypes = [ctypes.c_void_p]
        lib.ref_present_step.restype = ctypes.c_int64
        lib.ref_present_step.argtypes = [ctypes.c_void_p, ctypes.c_uint8, ctypes.c_uint32, ctypes.c_uint64]
        lib.ref_present_get.argtypes = [ctypes.c_void_p, _U8P]
        lib.ref_batch_render.argtypes = [_U8P, ctypes.c_uint32, ctypes.c_uint32, _U8P, _U8P, _U8P, _U8P,
                                         ctypes.c_uint32, _U8P]
        lib.ref_run_batch.restype = ctypes.c_double
        lib.ref_run_batch.argtypes = _oracle_lib().oracle_run_batch.argtypes
        lib.ref_run_levels.restype = ctypes.c_double
        lib.ref_run_levels.argtypes = _oracle_lib().oracle_run_levels.argtypes
        _REF = lib
    return _REF


class Oracle:
    """One console of the clean-room CPU core."""

    def __init__(self, rom: bytes) -> None:
        self.lib = _oracle_lib()
        self.h = self.lib.oracle_create(rom, len(rom))
        if not self.h:
            raise ValueError(self.lib.oracle_last_error().decode())

    def __del__(self) -> None:
        if getattr(self, "h", None):
            self.lib.oracle_destroy(self.h)
            self.h = None

    def set_reward(self, kind: int = 0, x_lo: int = 0x86, x_hi: int = 0x6D, done_addr: int = 0x14,
                   clip: int = 15, time_penalty: float = 0.0) -> None:
        self.lib.oracle_set_reward(self.h, kind, x_lo, x_hi, done_addr, clip, time_penalty)

    def step(self, buttons: int, frameskip: int = 1, max_instructions: int = 200000):
        """One env-step; returns (instructions, reward, done)."""
        r = ctypes.c_float()
        d = ctypes.c_uint8()
        n = self.lib.oracle_step(self.h, buttons & 0xFF, frameskip, max_instructions,
                                 ctypes.byref(r), ctypes.byref(d))
        if n < 0:
            raise RuntimeError(self.lib.oracle_last_error().decode())
        return n, r.value, d.value

    def step_instruction(self) -> tuple[int, int]:
        """One console instruction; returns (CPU cycles incl. NMI/DMA, frames completed)."""
        f = ctypes.c_uint32()
        c = self.lib.oracle_step_instruction(self.h, ctypes.byref(f))
        if c < 0:
            raise RuntimeError(self.lib.oracle_last_error().decode())
        return c, f.value

    def read(self, addr: int) -> int:
        return self.lib.oracle_bus_read(self.h, addr)

    def write(self, addr: int, value: int) -> None:
        self.lib.oracle_bus_write(self.h, addr, value)

    def ppu_peek(self, addr: int) -> int:
        return self.lib.oracle_ppu_peek(self.h, addr)

    def ppu_run(self, dots: int) -> int:
        return self.lib.oracle_ppu_run(self.h, dots)

    def save(self) -> np.ndarray:
        out = np.empty(STATE_BYTES, dtype=np.uint8)
        self.lib.oracle_save(self.h, out.ctypes.data_as(_U8P))
        return out

    def load(self, state: np.ndarray) -> None:
        st = np.ascontiguousarray(state, dtype=np.uint8)
        assert st.size == STATE_BYTES
        self.lib.oracle_load(self.h, st.ctypes.data_as(_U8P))

    def render(self, snapshot: bool = True, cpu_rules: bool = False) -> np.ndarray:
        """Palette values (240, 256): the batched core's frame from the
        presentation snapshot, or from live state; `cpu_rules` follows the
        reference CPU core's renderer instead (live state)."""
        out = np.empty((240, 256), dtype=np.uint8)
        self.lib.oracle_render(self.h, (1 if snapshot else 0) | (2 if cpu_rules else 0), out.ctypes.data_as(_U8P))
        return out

    def seed_presentation(self) -> None:
        self.lib.oracle_seed_presentation(self.h)

    def presentation(self) -> np.ndarray:
        """The presentation state (PRESENT_BYTES): frame-start x, y, ctrl,
        frame-end x, y, ctrl, mask, the pre-render latch x, y, ctrl, then OAM,
        palette and the first 2,048 bytes of nametable RAM (PRESENT_OFF)."""
        out = np.empty(PRESENT_BYTES, dtype=np.uint8)
        self.lib.oracle_present_get(self.h, out.ctypes.data_as(_U8P))
        return out

    def set_presentation(self, sx_start: int, sy_start: int, ctrl_start: int, sx_end: int, sy_end: int,
                         ctrl_end: int, mask: int) -> None:
        f = np.array([sx_start, sy_start, ctrl_start, sx_end, sy_end, ctrl_end, mask], dtype=np.uint8)
        self.lib.oracle_set_presentation(self.h, f.ctypes.data_as(_U8P))


class RefConsole:
    """One console of the reference's own CPU core (oracle/_ref)."""

    def __init__(self, rom: bytes) -> None:
        self.lib = _ref_lib()
        self.h = self.lib.ref_create(rom, len(rom))
        if not self.h:
            raise ValueError(self.lib.ref_last_error().decode())

    def __del__(self) -> None:
        if getattr(self, "h", None):
            self.lib.ref_destroy(self.h)
            self.h = None

    def step(self, buttons: int, frameskip: int = 1, max_instructions: int = 200000) -> int:
        n = self.lib.ref_step(self.h, buttons & 0xFF, frameskip, max_instructions)
        if n < 0:
            raise RuntimeError(self.lib.ref_last_error().decode())
        return n

    def step_instruction(self) -> tuple[int, int]:
        f = ctypes.c_uint32()
        c = self.lib.ref_step_instruction(self.h, ctypes.byref(f))
        if c < 0:
            raise RuntimeError(self.lib.ref_last_error().decode())
        return c, f.value

    def save(self) -> np.ndarray:
        out = np.empty(STATE_BYTES, dtype=np.uint8)
        self.lib.ref_save(self.h, out.ctypes.data_as(_U8P))
        return out

    def load(self, state: np.ndarray) -> None:
        st = np.ascontiguousarray(state, dtype=np.uint8)
        assert st.size == STATE_BYTES
        self.lib.ref_load(self.h, st.ctypes.data_as(_U8P))

    def render_rgb(self) -> np.ndarray:
        """The reference CPU core's frame (240, 256, 3) (ppu.hpp:213-230)."""
        out = np.empty((240, 256, 3), dtype=np.uint8)
        self.lib.ref_render_rgb(self.h, out.ctypes.data_as(_U8P))
        return out

    def present_seed(self) -> None:
        """Seed the batched core's presentation state from live state."""
        self.lib.ref_present_seed(self.h)

    def present_step(self, buttons: int, frameskip: int = 1, max_instructions: int = 200000) -> int:
        """One env-step in which every instruction's dots also advance the
        batched core's PPU timing (batch_ppu_step_env_hot); returns
        instructions."""
        n = self.lib.ref_present_step(self.h, buttons & 0xFF, frameskip, max_instructions)
        if n < 0:
            raise RuntimeError(self.lib.ref_last_error().decode())
        return n

    def presentation(self) -> np.ndarray:
        """The batched core's presentation state, laid out as Oracle.presentation."""
        out = np.empty(PRESENT_BYTES, dtype=np.uint8)
        self.lib.ref_present_get(self.h, out.ctypes.data_as(_U8P))
        return out


def ref_batch_render(chr_rom: bytes, arrangement: int, fields, oam: np.ndarray, nametable: np.ndarray,
                     palette: np.ndarray, snapshot: bool = True, per_pixel: bool = False) -> np.ndarray:
    """The reference batched core's RGB frame (240, 256, 3) of one console
    given directly (oracle/_ref, batch_render.cuh): `fields` = frame-start
    x, y, ctrl, frame-end x, y, ctrl, mask; nametable of 4,096 bytes; CHR RAM
    when `chr_rom` is empty.  `snapshot` False: live state (frame-end values,
    no split); `per_pixel`: the per-pixel renderer of its device kernel."""
    chr_arr = np.frombuffer(bytes(chr_rom) or b"\0", dtype=np.uint8).copy()
    f = np.ascontiguousarray(fields, dtype=np.uint8)
    o = np.ascontiguousarray(oam, dtype=np.uint8)
    n = np.ascontiguousarray(nametable, dtype=np.uint8)
    p = np.ascontiguousarray(palette, dtype=np.uint8)
    assert f.size == 7 and o.size == 256 and n.size == 4096 and p.size == 32
    out = np.empty((240, 256, 3), dtype=np.uint8)
    _ref_lib().ref_batch_render(chr_arr.ctypes.data_as(_U8P), len(chr_rom), arrangement, f.ctypes.data_as(_U8P),
                                o.ctypes.data_as(_U8P), n.ctypes.data_as(_U8P), p.ctypes.data_as(_U8P),
                                (1 if snapshot else 0) | (2 if per_pixel else 0), out.ctypes.data_as(_U8P))
    return out


def palette_rgb() -> np.ndarray:
    """The 64-entry NES palette (64, 3) of the batched core's renderer."""
    out = np.empty((64, 3), dtype=np.uint8)
    _oracle_lib().oracle_palette_rgb(out.ctypes.data_as(_U8P))
    return out


def gray84(frame: np.ndarray) -> np.ndarray:
    """Palette values (240, 256) -> the 84x84 gray observation (restated)."""
    f = np.ascontiguousarray(frame, dtype=np.uint8)
    assert f.shape == (240, 256)
    out = np.empty((84, 84), dtype=np.uint8)
    _oracle_lib().oracle_gray84(f.ctypes.data_as(_U8P), out.ctypes.data_as(_U8P))
    return out


def run_batch(rom: bytes, num_envs: int, steps: int, frameskip: int, seed: int, threads: int,
              kind: str = "port") -> tuple[float, int, int]:
    """Multi-threaded CPU run; returns (seconds, ram checksum, instructions)."""
    lib = _oracle_lib() if kind == "port" else _ref_lib()
    fn = lib.oracle_run_batch if kind == "port" else lib.ref_run_batch
    cs = ctypes.c_uint64()
    ins = ctypes.c_uint64()
    secs = fn(rom, len(rom), num_envs, steps, frameskip, seed & 0xFFFFFFFFFFFFFFFF, threads,
              ctypes.byref(cs), ctypes.byref(ins))
    if secs < 0:
        raise RuntimeError("CPU batch run failed")
    return secs, cs.value, ins.value


def run_levels(rom: bytes, blobs: list[bytes], levels: np.ndarray, done_init: np.ndarray, done_addr: int,
               steps: int, frameskip: int, seed: int, step0: int, threads: int,
               kind: str = "port") -> tuple[float, int, int, int]:
    """Multi-threaded CPU run of the snapshot workload (one console per entry
    of ``levels``, auto-reset from its blob when RAM[done_addr] reaches 0);
    returns (seconds, ram checksum, instructions, resets)."""
    fn = _oracle_lib().oracle_run_levels if kind == "port" else _ref_lib().ref_run_levels
    bank = np.frombuffer(b"".join(bytes(b) for b in blobs), dtype=np.uint8).copy()
    assert bank.size == len(blobs) * STATE_BYTES
    lv = np.ascontiguousarray(levels, dtype=np.uint8)
    di = np.ascontiguousarray(done_init, dtype=np.uint8)
    assert lv.shape == di.shape
    cs, ins, rs = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    secs = fn(rom, len(rom), bank.ctypes.data_as(_U8P), len(blobs), lv.ctypes.data_as(_U8P),
              di.ctypes.data_as(_U8P), done_addr, lv.size, steps, frameskip, seed & 0xFFFFFFFFFFFFFFFF,
              step0, threads, ctypes.byref(cs), ctypes.byref(ins), ctypes.byref(rs))
    if secs < 0:
        raise RuntimeError("CPU snapshot run failed")
    return secs, cs.value, ins.value, rs.value


def cpu_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1
