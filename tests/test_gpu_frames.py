"""Frames of the HIP batch (called through the C ABI) equal the oracle's.

Bar: bit-exact palette-value frames (240 x 256), RGB frames and 84x84 gray
observations against the oracle's batched-rule renderer of the same console
(its presentation snapshot), after power-on, resets, state loads and steps
at several frame-skips, the instruction-budget path, both nametable
mirrorings, four-screen carts and CHR RAM.
"""

from __future__ import annotations

import numpy as np
import pytest

from nesle_amd import abi, synthrom
from oracle import oracle as O
from tests.helpers import masks_for, say

pytestmark = pytest.mark.gpu

ALL = abi.FRAME_RGB | abi.FRAME_PALETTE | abi.FRAME_GRAY84


def _rom(seed: int, *, mirroring: str = "vertical", chr_ram: bool = False) -> bytes:
    rom = bytearray(synthrom.make_rom(seed).rom)
    if mirroring == "horizontal":
        rom[6] &= ~0x01 & 0xFF
    elif mirroring == "four_screen":
        rom[6] |= 0x08
    if chr_ram:
        rom[5] = 0
        rom = rom[:16 + 32768]
    return bytes(rom)


def _check(b: abi.Batch, oracles: dict[int, O.Oracle], tag: str, outputs: int = ALL) -> None:
    b.render(outputs)
    pal = b.host(abi.VIEW_FRAME_PALETTE) if outputs & abi.FRAME_PALETTE else None
    rgb = b.host(abi.VIEW_FRAME_RGB) if outputs & abi.FRAME_RGB else None
    gray = b.host(abi.VIEW_GRAY84) if outputs & abi.FRAME_GRAY84 else None
    lut = O.palette_rgb()
    for e, con in oracles.items():
        want = con.render(snapshot=True)
        if pal is not None:
            bad = int((pal[e] != want).sum())
            assert bad == 0, f"{tag} env {e}: {bad} palette values differ"
        if rgb is not None:
            assert np.array_equal(rgb[e], lut[want]), f"{tag} env {e}: RGB frame"
        if gray is not None:
            assert np.array_equal(gray[e], O.gray84(want)), f"{tag} env {e}: gray84"


def _step_all(b: abi.Batch, oracles: dict[int, O.Oracle], seed: int, k: int, frameskip: int,
              max_instructions: int = 200000) -> None:
    m = masks_for(seed, b.n, k)
    b.set_actions(m)
    b.step()
    for e, con in oracles.items():
        con.step(int(m[e]), frameskip, max_instructions)


def test_frames_at_power_on_and_after_reset():
    rom = _rom(7)
    n = 8
    say(f"[gpu] frames power-on/reset: N={n}")
    b = abi.Batch(rom, n, frameskip=4)
    _check(b, {e: O.Oracle(rom) for e in range(n)}, "power-on")
    oracles = {e: O.Oracle(rom) for e in range(n)}
    for k in range(3):
        _step_all(b, oracles, 5, k, 4)
    _check(b, oracles, "after 3 steps")
    b.reset()
    _check(b, {e: O.Oracle(rom) for e in range(n)}, "after reset")


@pytest.mark.parametrize("rom_seed,frameskip,steps", [(7, 4, 16), (3, 1, 24), (9, 3, 10)])
def test_frames_track_oracle_over_steps(rom_seed, frameskip, steps):
    rom = _rom(rom_seed)
    n = 64
    say(f"[gpu] frames over steps: rom{rom_seed} N={n} fs={frameskip} steps={steps}")
    b = abi.Batch(rom, n, frameskip=frameskip)
    oracles = {e: O.Oracle(rom) for e in range(n)}
    for k in range(steps):
        _step_all(b, oracles, 100 + rom_seed, k, frameskip)
        if k % 4 == 3 or k == steps - 1:
            _check(b, oracles, f"step {k}")


def test_frames_with_instruction_budget():
    """A budget below one frame's instructions ends frames early; every
    vblank crossed then reaches the snapshot."""
    rom = _rom(11)
    n, budget = 16, 4000
    say(f"[gpu] frames budget: N={n} fs=2 budget={budget}")
    b = abi.Batch(rom, n, frameskip=2, max_instructions_per_frame=budget)
    oracles = {e: O.Oracle(rom) for e in range(n)}
    for k in range(12):
        _step_all(b, oracles, 31, k, 2, budget)
        if k % 3 == 2:
            _check(b, oracles, f"step {k}")


@pytest.mark.parametrize("variant", ["horizontal", "four_screen", "chr_ram"])
def test_frames_mirroring_and_chr_ram(variant):
    rom = _rom(5, mirroring=variant if variant != "chr_ram" else "vertical", chr_ram=variant == "chr_ram")
    n = 16
    say(f"[gpu] frames {variant}: N={n} fs=4")
    b = abi.Batch(rom, n, frameskip=4)
    oracles = {e: O.Oracle(rom) for e in range(n)}
    for k in range(6):
        _step_all(b, oracles, 77, k, 4)
    _check(b, oracles, variant)


def test_frames_of_random_ppu_states():
    """Random video memory, OAM, scroll, ctrl (8x16 sprites, both pattern
    tables) and mask (grayscale, left-column clipping), loaded per console:
    the device renderer equals the oracle's on every console."""
    rom = _rom(2)
    n = 64
    say(f"[gpu] frames random PPU states: N={n}")
    b = abi.Batch(rom, n, frameskip=1)
    base = O.Oracle(rom)
    for k in range(20):
        base.step(int(masks_for(4, 1, k)[0]), 1)
    st0 = base.save()
    rng = np.random.default_rng(2024)
    oracles = {}
    for e in range(n):
        st = st0.copy()
        st[O.OFF["oam"]:O.OFF["oam"] + 256] = rng.integers(0, 256, 256, dtype=np.uint8)
        st[O.OFF["oam"]] = rng.choice([rng.integers(0, 256), 0xF0, 20, 120])   # split above, inside, none
        st[O.OFF["palette"]:O.OFF["palette"] + 32] = rng.integers(0, 64, 32, dtype=np.uint8)
        st[O.OFF["nametable"]:O.OFF["nametable"] + 2048] = rng.integers(0, 256, 2048, dtype=np.uint8)
        st[O.OFF["ctrl"]] = rng.integers(0, 256)
        st[O.OFF["mask"]] = rng.integers(0, 256)
        st[O.OFF["scroll_x"]] = rng.integers(0, 256)
        st[O.OFF["scroll_y"]] = rng.integers(0, 240)
        mask = np.zeros(n, dtype=np.uint8)
        mask[e] = 1
        b.load_state(st, mask)
        con = O.Oracle(rom)
        con.load(st)
        con.seed_presentation()
        oracles[e] = con
    _check(b, oracles, "random state")


def _crafted_oam(rng: np.random.Generator, kind: int) -> np.ndarray:
    """OAM (64 sprites) of one layout: 0 stacks of same-position sprites with
    mixed priority/flip/palette, 1 sprites on the left and right screen edges
    and the top/bottom rows, 2 a column of 8x16-style vertical neighbours, 3
    uniform random."""
    oam = rng.integers(0, 256, 256, dtype=np.uint8).reshape(64, 4)
    if kind == 0:
        for g in range(8):
            y, x = rng.integers(0, 232), rng.integers(0, 256)
            oam[8 * g:8 * g + 8, 0] = y + rng.integers(0, 3, 8)
            oam[8 * g:8 * g + 8, 3] = x + rng.integers(0, 3, 8)
    elif kind == 1:
        oam[:, 3] = rng.choice(np.r_[0:9, 247:256], 64)
        oam[:, 0] = rng.choice(np.r_[0:8, 224:240, 239:256], 64)
    elif kind == 2:
        x = rng.integers(0, 256)
        oam[:, 3] = x + rng.integers(-4, 5, 64)
        oam[:, 0] = np.arange(64) * 4 + rng.integers(0, 4, 64)
    return oam.reshape(-1)


def test_frames_of_crafted_sprite_layouts():
    """Sprite layouts that stress the lowest-index-wins rule and the window
    edges (stacks of overlapping sprites with mixed priority, flips and
    palettes; sprites on the left and right edges with and without left-column
    clipping; the top and bottom rows; 8x8 and 8x16), over every fine-x
    scroll and y scrolls past 239, with palettes holding zero values (a
    transparent background colour): the device renderer equals the oracle's
    on every console."""
    rom = _rom(5)
    n = 256
    say(f"[gpu] frames crafted sprite layouts: N={n}")
    b = abi.Batch(rom, n, frameskip=1)
    base = O.Oracle(rom)
    for k in range(12):
        base.step(int(masks_for(6, 1, k)[0]), 1)
    st0 = base.save()
    rng = np.random.default_rng(77)
    states = []
    for e in range(n):
        st = st0.copy()
        st[O.OFF["oam"]:O.OFF["oam"] + 256] = _crafted_oam(rng, e % 4)
        pal = rng.integers(0, 64, 32, dtype=np.uint8)
        pal[rng.integers(0, 32, 6)] = 0
        st[O.OFF["palette"]:O.OFF["palette"] + 32] = pal
        st[O.OFF["nametable"]:O.OFF["nametable"] + 2048] = rng.integers(0, 256, 2048, dtype=np.uint8)
        st[O.OFF["ctrl"]] = (rng.integers(0, 256) & ~0x20) | (0x20 if e % 8 >= 4 else 0)
        st[O.OFF["mask"]] = 0x18 | (rng.integers(0, 256) & 0x07) if e % 16 else rng.integers(0, 256)
        st[O.OFF["scroll_x"]] = e % 8 + 8 * rng.integers(0, 32)
        st[O.OFF["scroll_y"]] = rng.integers(0, 256)
        states.append(st)
    # One load per console (masked), then one render of the whole batch.
    oracles = {}
    for e, st in enumerate(states):
        mask = np.zeros(n, dtype=np.uint8)
        mask[e] = 1
        b.load_state(st, mask)
        con = O.Oracle(rom)
        con.load(st)
        con.seed_presentation()
        oracles[e] = con
    _check(b, oracles, "crafted sprites")


@pytest.mark.parametrize("num_envs", [4096])
def test_frames_full_size_sampled(num_envs):
    rom = _rom(11)
    rng = np.random.default_rng(num_envs)
    sample = sorted({0, 1, 63, 64, num_envs - 1, *rng.integers(0, num_envs, 6).tolist()})
    say(f"[gpu] frames full size: N={num_envs} fs=4 sample={sample}")
    b = abi.Batch(rom, num_envs, frameskip=4)
    oracles = {e: O.Oracle(rom) for e in sample}
    for k in range(3):
        m = masks_for(1234, num_envs, k)
        m[num_envs // 2] = m[3]
        b.set_actions(m)
        b.step()
        for e, con in oracles.items():
            con.step(int(m[e]), 4)
    _check(b, oracles, "full size", abi.FRAME_PALETTE | abi.FRAME_GRAY84)
    pal = b.host(abi.VIEW_FRAME_PALETTE)
    assert np.array_equal(pal[3], pal[num_envs // 2])


def test_frames_off_batch_refuses_render():
    rom = _rom(7)
    say("[gpu] frames off: N=4")
    b = abi.Batch(rom, 4, frameskip=4, frames=False)
    b.set_actions(np.zeros(4, dtype=np.uint8))
    b.step()
    with pytest.raises(ValueError):
        b.render(abi.FRAME_RGB)
    with pytest.raises(ValueError):
        b.view(abi.VIEW_FRAME_RGB)
    with pytest.raises(ValueError):
        abi.Batch(rom, 4, frameskip=4).render(0)


def test_pixel_workload_full_size_sampled():
    """The pixel-observation workload at its full size: 16,384 consoles,
    frame-skip 4, an 84x84 gray frame of every console rendered after every
    step; sampled consoles (wave, workgroup and range edges, random ones)
    equal the oracle's batched-renderer frame turned gray, at every step."""
    num_envs = 16384
    rom = _rom(2026)
    rng = np.random.default_rng(7)
    sample = sorted({0, 1, 63, 64, 255, 256, 8191, 8192, num_envs - 1, *rng.integers(0, num_envs, 6).tolist()})
    say(f"[gpu] pixel workload: N={num_envs} fs=4 sample={sample}")
    b = abi.Batch(rom, num_envs, frameskip=4)
    oracles = {e: O.Oracle(rom) for e in sample}
    for k in range(3):
        _step_all(b, oracles, 0x5EED, k, 4)
        _check(b, oracles, f"step {k}", abi.FRAME_GRAY84)
