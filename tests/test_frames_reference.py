"""The oracle's batched frame rules, pinned against the reference's own batched
core (no GPU).

oracle/_ref compiles the reference's batched PPU timing and renderer headers
(cpp/include/nesle/cuda/batch_ppu.cuh, batch_render.cuh) as host C++, the
way its own host tests do (tests/cpp/test_cuda_render.cpp), next to its CPU
core.  Checked here:

* presentation capture: the reference CPU core stepped instruction by
  instruction, each instruction's PPU dots also fed to
  batch_ppu_step_env_hot (batch_ppu.cuh:183-269), gives the same frame-start
  latch and vblank snapshot (scroll/ctrl at both ends of the frame, mask,
  OAM, palette, nametables) as the oracle after every env-step -- on the
  status-bar ROM, whose frames start and end with different scrolls, on the
  plain workload ROM and on an NROM-128 ROM, at frame-skip 1 and 4, and after
  a state load;
* rendering: the oracle's batched-rule frame equals the reference renderer's
  frame (render_batch_rgb_frame_env, and the per-pixel form its device kernel
  runs) on random presentation records with distinct frame-start and
  frame-end views, splits above, inside and below the screen, 8x16 sprites,
  sprites behind the background in the status-bar rows, palette values 0,
  grayscale, left-column clipping, every nametable arrangement and CHR RAM;
  and in live mode (no snapshot);
* both together: the frame drawn from the reference's own captured record
  equals the oracle's frame after the same steps.
"""

from __future__ import annotations

import numpy as np
import pytest

from nesle_amd import synthrom
from oracle import oracle as O

pytestmark = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref (reference cores) not built here")

P = O.PRESENT_OFF


def _rom(seed: int = 1, chr_bytes: bytes | None = None, arrangement: int = 0) -> bytes:
    """A workload ROM with its CHR replaced (b"" = CHR RAM) and the given
    nametable arrangement (0 vertical, 1 horizontal, 2 four-screen)."""
    rom = bytearray(synthrom.make_rom(seed).rom)
    flags6 = {0: 0x01, 1: 0x00, 2: 0x08}[arrangement]
    rom[6] = flags6
    prg = bytes(rom[16:16 + 32768])
    if chr_bytes is None:
        chr_bytes = bytes(rom[16 + 32768:])
    rom[5] = len(chr_bytes) // 8192
    return bytes(rom[:16]) + prg + chr_bytes


def _lockstep(rom: bytes, steps: int, frameskip: int, seed: int, load_at: int | None = None) -> int:
    """Oracle and reference stepped together; presentation states compared
    after every env-step.  Returns how many steps had distinct frame-start
    and frame-end scroll/ctrl."""
    con, ref = O.Oracle(rom), O.RefConsole(rom)
    ref.present_seed()
    distinct = 0
    for k in range(steps):
        if k == load_at:   # a mid-run state from a third console, loaded into both
            other = O.Oracle(rom)
            for j in range(37):
                other.step(int(synthrom.action_masks(seed + 1, 1, j)[0]), 1)
            st = other.save()
            con.load(st)
            con.seed_presentation()
            ref.load(st)
            ref.present_seed()
        m = int(synthrom.action_masks(seed, 1, k)[0])
        n_con, _, _ = con.step(m, frameskip)
        n_ref = ref.present_step(m, frameskip)
        assert n_con == n_ref, f"step {k}: instructions"
        got, want = con.presentation(), ref.presentation()
        np.testing.assert_array_equal(got, want, err_msg=f"step {k}: presentation state")
        distinct += tuple(got[0:3]) != tuple(got[3:6])
    return distinct


def test_presentation_state_matches_the_reference_batched_ppu_on_the_status_bar_rom():
    rom = synthrom.make_rom(2026, split=True).rom
    distinct = _lockstep(rom, 90, 1, 31)
    assert distinct >= 80      # nearly every frame starts and ends with different scrolls
    assert _lockstep(rom, 25, 4, 32, load_at=12) >= 20


@pytest.mark.parametrize("rom_seed,banks", [(1, 2), (3, 1)])
def test_presentation_state_matches_the_reference_batched_ppu(rom_seed, banks):
    rom = synthrom.make_rom(rom_seed, prg_banks=banks).rom
    _lockstep(rom, 60, 1, 40 + rom_seed)
    _lockstep(rom, 15, 4, 50 + rom_seed, load_at=7)


def _record(rng: np.random.Generator, case: int) -> dict:
    """A random presentation record; `case` steers the split row and sprite
    size so every kind is covered."""
    fields = rng.integers(0, 256, 7).astype(np.uint8)
    fields[6] = rng.choice([0x1E, 0x18, 0x1A, 0x1C, 0x1F, 0x0E, 0x16, 0x0A, 0x10])   # mask
    tall = case % 3 == 1
    for i in (2, 5):   # ctrl: sprite size from the case, the rest random
        fields[i] = (int(fields[i]) & ~0x20) | (0x20 if tall else 0)
    oam = rng.integers(0, 256, 256).astype(np.uint8)
    kind = case % 4
    if kind == 0:
        oam[0] = rng.integers(8, 60)          # split near the top (status bar)
    elif kind == 1:
        oam[0] = rng.integers(60, 200)        # split mid-screen
    elif kind == 2:   # split exactly at row 240 (frame-start view everywhere) or at 239
        oam[0] = (223 if tall else 231) - (case // 4) % 2
    # Sprites that reach into the status-bar rows, some behind the background.
    for s in range(1, 9):
        oam[4 * s] = rng.integers(0, 40)
        oam[4 * s + 2] = (int(oam[4 * s + 2]) & ~0x20) | (0x20 if s % 2 else 0)
    palette = rng.integers(0, 64, 32).astype(np.uint8)
    palette[rng.random(32) < 0.25] = 0        # palette value 0: transparent background in these rules
    nametable = rng.integers(0, 256, 4096).astype(np.uint8)
    return {"fields": fields, "oam": oam, "palette": palette, "nametable": nametable}


def _oracle_frame(rom: bytes, rec: dict, snapshot: bool = True) -> np.ndarray:
    con = O.Oracle(rom)
    st = con.save()
    st[O.OFF["oam"]:O.OFF["oam"] + 256] = rec["oam"]
    st[O.OFF["palette"]:O.OFF["palette"] + 32] = rec["palette"]
    st[O.OFF["nametable"]:O.OFF["nametable"] + 4096] = rec["nametable"]
    # CHR RAM (carts without CHR ROM) holds tiles the batched rules must not see.
    st[O.OFF["chr_ram"]:O.OFF["chr_ram"] + 8192] = rec["nametable"].repeat(2) ^ 0x5A
    f = rec["fields"]
    st[O.OFF["ctrl"]], st[O.OFF["mask"]] = f[5], f[6]
    st[O.OFF["scroll_x"]], st[O.OFF["scroll_y"]] = f[3], f[4]
    con.load(st)
    con.seed_presentation()
    con.set_presentation(*(int(v) for v in f))
    return O.palette_rgb()[con.render(snapshot=snapshot)]


@pytest.mark.parametrize("arrangement", [0, 1, 2])
def test_batched_frames_match_the_reference_renderer_on_random_records(arrangement):
    rng = np.random.default_rng(100 + arrangement)
    chr_rom = rng.integers(0, 256, 8192).astype(np.uint8).tobytes()
    rom = _rom(1, chr_rom, arrangement)
    for case in range(12):
        rec = _record(rng, case)
        want = O.ref_batch_render(chr_rom, arrangement, rec["fields"], rec["oam"], rec["nametable"], rec["palette"])
        got = _oracle_frame(rom, rec)
        np.testing.assert_array_equal(got, want, err_msg=f"case {case}")
        if case % 4 == 0:   # the per-pixel form the reference's device kernel runs agrees too
            np.testing.assert_array_equal(
                O.ref_batch_render(chr_rom, arrangement, rec["fields"], rec["oam"], rec["nametable"],
                                   rec["palette"], per_pixel=True), want, err_msg=f"case {case} per pixel")


def test_batched_frames_match_the_reference_renderer_with_chr_ram_and_in_live_mode():
    rng = np.random.default_rng(7)
    rom = _rom(2, b"", 0)
    for case in range(4):
        rec = _record(rng, case)
        want = O.ref_batch_render(b"", 0, rec["fields"], rec["oam"], rec["nametable"], rec["palette"])
        np.testing.assert_array_equal(_oracle_frame(rom, rec), want, err_msg=f"CHR RAM case {case}")
    chr_rom = rng.integers(0, 256, 8192).astype(np.uint8).tobytes()
    rom = _rom(2, chr_rom, 1)
    for case in range(4):
        rec = _record(rng, case)
        want = O.ref_batch_render(chr_rom, 1, rec["fields"], rec["oam"], rec["nametable"], rec["palette"],
                                  snapshot=False)
        np.testing.assert_array_equal(_oracle_frame(rom, rec, snapshot=False), want, err_msg=f"live case {case}")


def test_frames_from_the_reference_capture_equal_the_oracle_frames():
    """The status-bar ROM stepped by both cores: the reference renderer drawing
    the reference's own captured record gives the oracle's frame."""
    sr = synthrom.make_rom(2026, split=True)
    chr_rom = sr.rom[16 + 32768:]
    con, ref = O.Oracle(sr.rom), O.RefConsole(sr.rom)
    ref.present_seed()
    for k in range(40):
        m = int(synthrom.action_masks(61, 1, k)[0])
        con.step(m, 1)
        ref.present_step(m, 1)
        if k % 5 != 4:
            continue
        pr = ref.presentation()
        nt = np.zeros(4096, dtype=np.uint8)
        nt[:2048] = pr[P["nametable"]:P["nametable"] + 2048]
        want = O.ref_batch_render(chr_rom, 0, pr[0:7], pr[P["oam"]:P["oam"] + 256], nt,
                                  pr[P["palette"]:P["palette"] + 32])
        np.testing.assert_array_equal(O.palette_rgb()[con.render(snapshot=True)], want, err_msg=f"frame {k + 1}")
        assert tuple(pr[0:3]) != tuple(pr[3:6])
