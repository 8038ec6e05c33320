"""Tiny iNES images and state edits for the known-answer tests.

``nrom_bytes`` builds the same NROM image the reference's C++ tests build
(tests/cpp/test_console.cpp:13-23): PRG byte ``i`` of bank ``b`` is
``(b << 7) | (i & 0x7F)``, 8 KB of zero CHR, then pokes programs, vectors and
CHR bytes into it.
"""

from __future__ import annotations

import numpy as np

from oracle import oracle as O


def nrom_bytes(prg_banks: int, flags6: int = 0, code: dict[int, list[int]] | None = None,
               reset: int | None = None, nmi: int | None = None, irq: int | None = None,
               chr_pokes: dict[int, int] | None = None) -> bytes:
    header = bytearray(b"NES\x1a") + bytes([prg_banks, 1, flags6, 0]) + bytes(8)
    size = prg_banks * 16384
    prg = bytearray(((i // 16384) << 7) | (i & 0x7F) for i in range(size))
    mask = size - 1
    for addr, data in (code or {}).items():
        for k, v in enumerate(data):
            prg[(addr + k - 0x8000) & mask] = v
    for vec, at in ((nmi, 0xFFFA), (reset, 0xFFFC), (irq, 0xFFFE)):
        if vec is not None:
            prg[(at - 0x8000) & mask] = vec & 0xFF
            prg[(at + 1 - 0x8000) & mask] = vec >> 8
    chr_rom = bytearray(8192)
    for addr, v in (chr_pokes or {}).items():
        chr_rom[addr] = v
    return bytes(header + prg + chr_rom)


def state_with(base: np.ndarray, **fields: int) -> np.ndarray:
    """Copy of a canonical state blob with named fields replaced."""
    s = np.array(base, dtype=np.uint8, copy=True)
    width = {"pc": 2, "cycles": 8, "frame": 8, "frame_dot": 4, "v": 2, "t": 2, "pending_dma": 4}
    for name, value in fields.items():
        n = width.get(name, 1)
        o = O.OFF[name]
        s[o:o + n] = np.frombuffer(int(value).to_bytes(n, "little"), dtype=np.uint8)
    return s
