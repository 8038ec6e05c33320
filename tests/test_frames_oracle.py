"""The frame path's oracle, pinned (no GPU).

* Renderer, CPU-core rules: the oracle's frame of live state under the
  reference CPU core's rules equals the reference core's own RGB frames
  (golden hashes from tests/golden/make_frame_golden.py, plus a live
  comparison with oracle/_ref where it is built).
* Renderer, batched rules: where the two rule sets cannot differ (snapshot
  seeded from live state, no HUD split, no background palette value 0, CHR
  ROM) the batched frame equals the CPU-rules frame; each rule where they do
  differ is checked against its closed form.
* Gray observation: equals numpy luma + Pillow BILINEAR, the reference
  training wrapper's preprocessing (wrappers.py:209-215), on the golden
  frames, on every palette colour and on random frames.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from nesle_amd import synthrom
from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def _pil_gray84(rgb: np.ndarray) -> np.ndarray:
    from PIL import Image

    gray = np.dot(rgb[..., :3].astype(np.float32), [0.299, 0.587, 0.114])
    img = Image.fromarray(gray.astype(np.uint8)).resize((84, 84), Image.BILINEAR)
    return np.array(img, dtype=np.uint8)


def _h(a: np.ndarray) -> str:
    return f"{O.fnv1a_np(np.ascontiguousarray(a)):016x}"


def _rgb(pal: np.ndarray) -> np.ndarray:
    return O.palette_rgb()[pal]


@pytest.mark.parametrize("rom_seed", [1, 2, 3])
def test_cpu_rules_frames_match_reference_golden(rom_seed):
    fx = json.loads((GOLDEN / f"frames_rom{rom_seed}.json").read_text())
    rom = synthrom.make_rom(rom_seed).rom
    assert _h(np.frombuffer(rom, dtype=np.uint8)) == fx["rom_fnv1a"]
    con = O.Oracle(rom)
    want = {r[0]: r for r in fx["records"]}
    for k in range(max(want)):
        con.step(int(synthrom.action_masks(fx["action_seed"], 1, k)[0]), 1)
        rec = want.get(k + 1)
        if rec is None:
            continue
        rgb = _rgb(con.render(snapshot=False, cpu_rules=True))
        assert _h(rgb) == rec[1], f"frame {k + 1} RGB"
        assert _h(O.gray84(con.render(snapshot=False, cpu_rules=True))) == rec[2], f"frame {k + 1} gray84"


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref (reference CPU core) not built here")
def test_cpu_rules_frames_match_reference_core_live():
    rom = synthrom.make_rom(5).rom
    con, ref = O.Oracle(rom), O.RefConsole(rom)
    for k in range(120):
        m = int(synthrom.action_masks(55, 1, k)[0])
        con.step(m, 1)
        ref.step(m, 1)
        if k % 7 == 0:
            np.testing.assert_array_equal(_rgb(con.render(snapshot=False, cpu_rules=True)), ref.render_rgb(),
                                          err_msg=f"frame {k + 1}")


def _warm(rom_seed: int, frames: int) -> O.Oracle:
    con = O.Oracle(synthrom.make_rom(rom_seed).rom)
    for k in range(frames):
        con.step(int(synthrom.action_masks(9, 1, k)[0]), 1)
    return con


def _edit(con: O.Oracle, **fields) -> None:
    """Overwrite blob fields (name -> value or (offset, bytes)) and reload."""
    st = con.save()
    for name, val in fields.items():
        if isinstance(val, tuple):
            st[val[0]:val[0] + len(val[1])] = np.frombuffer(bytes(val[1]), dtype=np.uint8)
        else:
            st[O.OFF[name]] = val
    con.load(st)
    con.seed_presentation()


@pytest.mark.parametrize("rom_seed,frames", [(1, 30), (2, 61), (3, 90)])
def test_batched_rules_equal_cpu_rules_where_they_cannot_differ(rom_seed, frames):
    con = _warm(rom_seed, frames)
    st = con.save()
    rng = np.random.default_rng(rom_seed)
    pal = st[O.OFF["palette"]:O.OFF["palette"] + 32].copy()
    pal[pal == 0] = rng.integers(1, 64, int((pal == 0).sum()))   # no palette value 0
    oam = st[O.OFF["oam"]:O.OFF["oam"] + 256].copy()
    oam[0] = 0xF0                                                  # sprite 0 below the screen: no split
    for mask in (0x1E, 0x18, 0x1A, 0x1C, 0x08, 0x10, 0x0E):
        _edit(con, mask=mask, palette=(O.OFF["palette"], pal), oam=(O.OFF["oam"], oam))
        np.testing.assert_array_equal(con.render(snapshot=True), con.render(snapshot=False, cpu_rules=True),
                                      err_msg=f"mask {mask:#x}")


def test_background_palette_value_zero_is_transparent():
    con = _warm(2, 40)
    st = con.save()
    pal = np.zeros(32, dtype=np.uint8)
    pal[0] = 0x21
    _edit(con, mask=0x0A, palette=(O.OFF["palette"], pal))   # background only, left column shown
    batched = con.render(snapshot=True)
    cpu = con.render(snapshot=False, cpu_rules=True)
    assert (batched == 0x21).all()                 # every pixel is the backdrop
    assert (cpu == 0).any() and set(np.unique(cpu)) <= {0x00, 0x21}
    del st


def test_chr_ram_reads_zero_in_batched_frames():
    rom = bytearray(synthrom.make_rom(4).rom)
    rom[5] = 0                                      # no CHR ROM: the cart has CHR RAM
    rom = bytes(rom[:16 + 32768])
    con = O.Oracle(rom)
    for k in range(20):
        con.step(int(synthrom.action_masks(3, 1, k)[0]), 1)
    con.seed_presentation()
    frame = con.render(snapshot=True)
    st = con.save()
    backdrop = st[O.OFF["palette"]] & (0x30 if st[O.OFF["mask"]] & 1 else 0x3F)
    assert (frame == backdrop).all()


def test_grayscale_mask_keeps_the_high_bits():
    con = _warm(3, 25)
    st = con.save()
    # Every palette value keeps a high bit, so no pixel turns transparent
    # under grayscale and the frames differ only by the mask 0x30.
    pal = st[O.OFF["palette"]:O.OFF["palette"] + 32] | 0x10
    _edit(con, mask=0x1F, palette=(O.OFF["palette"], pal))
    g = con.render(snapshot=True)
    _edit(con, mask=0x1E, palette=(O.OFF["palette"], pal))
    c = con.render(snapshot=True)
    np.testing.assert_array_equal(g, c & 0x30)
    assert not np.array_equal(g, c)


def test_hud_split_uses_frame_start_scroll_above_sprite0():
    con = _warm(1, 50)
    st = con.save()
    oam = st[O.OFF["oam"]:O.OFF["oam"] + 256].copy()
    oam[0] = 99                                     # split row = 99 + 1 + 8 = 108
    ctrl = int(st[O.OFF["ctrl"]]) & ~0x20
    _edit(con, ctrl=ctrl, mask=0x0A, oam=(O.OFF["oam"], oam))   # background only
    con.set_presentation(0, 0, ctrl, 100, 0, ctrl, 0x0A)
    split = con.render(snapshot=True)
    con.set_presentation(0, 0, ctrl, 0, 0, ctrl, 0x0A)
    hud = con.render(snapshot=True)
    con.set_presentation(100, 0, ctrl, 100, 0, ctrl, 0x0A)
    play = con.render(snapshot=True)
    np.testing.assert_array_equal(split[:108], hud[:108])
    np.testing.assert_array_equal(split[108:], play[108:])
    assert not np.array_equal(hud, play)
    oam[0] = 231                                    # split >= 240: frame-start values everywhere
    _edit(con, ctrl=ctrl, mask=0x0A, oam=(O.OFF["oam"], oam))
    con.set_presentation(0, 0, ctrl, 100, 0, ctrl, 0x0A)
    np.testing.assert_array_equal(con.render(snapshot=True), hud)


def test_snapshot_is_frozen_at_vblank_with_scroll_latched_at_pre_render():
    """Step one instruction at a time: the frame drawn after the frame ends
    equals a frame built directly from the state right after the instruction
    that crossed vblank, with the frame-start scroll/ctrl read at the
    pre-render line before it (batch_ppu.cuh:219-261)."""
    from oracle.oracle import Oracle

    con = _warm(3, 12)
    rom = synthrom.make_rom(3).rom
    off_dot, off_sx, off_sy, off_ctrl, off_mask = (O.OFF[k] for k in ("frame_dot", "scroll_x", "scroll_y",
                                                                     "ctrl", "mask"))
    dot = lambda st: int.from_bytes(bytes(st[off_dot:off_dot + 4]), "little")  # noqa: E731
    vblank, pre = 241 * 341 + 1, 261 * 341 + 1
    st = con.save()
    lat = at_vblank = None
    frames = 0
    while frames < 2:
        d0 = dot(st)
        _, f = con.step_instruction()
        frames += f
        st = con.save()
        d1 = dot(st) + (89342 if f else 0)
        for ev in (vblank, pre, vblank + 89342, pre + 89342):
            if d0 < ev <= d1:
                if ev % 89342 == pre:
                    lat = (int(st[off_sx]), int(st[off_sy]), int(st[off_ctrl]))
                elif ev % 89342 == vblank and lat is not None:
                    at_vblank = (st.copy(), lat)
    assert at_vblank is not None
    got = con.render(snapshot=True)
    sv, (sx0, sy0, c0) = at_vblank
    ref = Oracle(rom)
    ref.load(sv)
    ref.seed_presentation()
    ref.set_presentation(sx0, sy0, c0, int(sv[off_sx]), int(sv[off_sy]), int(sv[off_ctrl]), int(sv[off_mask]))
    np.testing.assert_array_equal(got, ref.render(snapshot=True))


def test_gray84_matches_pillow_on_every_colour_and_random_frames():
    rgb = O.palette_rgb()
    for c in range(64):
        frame = np.full((240, 256), c, dtype=np.uint8)
        np.testing.assert_array_equal(O.gray84(frame), _pil_gray84(rgb[frame]), err_msg=f"colour {c}")
    rng = np.random.default_rng(84)
    for t in range(6):
        if t < 3:
            frame = rng.integers(0, 64, (240, 256), dtype=np.uint8)
        else:   # blocky frames (tiles of one colour), closer to real screens
            frame = np.kron(rng.integers(0, 64, (30, 32), dtype=np.uint8), np.ones((8, 8), dtype=np.uint8))
        np.testing.assert_array_equal(O.gray84(frame), _pil_gray84(rgb[frame]), err_msg=f"frame {t}")
