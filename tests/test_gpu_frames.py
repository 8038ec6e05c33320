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
from tests.helpers import OracleBatch, device_rows, masks_for, say, warm_snapshots

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


def _record_matches(rec: np.ndarray, pres: np.ndarray, tag: str) -> None:
    """A device presentation record (16-byte header, then palette, OAM and
    nametable RAM) against the oracle's presentation state."""
    P = O.PRESENT_OFF
    np.testing.assert_array_equal(rec[0:7], pres[0:7], err_msg=f"{tag}: scroll/ctrl/mask")
    np.testing.assert_array_equal(rec[16:48], pres[P["palette"]:P["palette"] + 32], err_msg=f"{tag}: palette")
    np.testing.assert_array_equal(rec[48:304], pres[P["oam"]:P["oam"] + 256], err_msg=f"{tag}: OAM")
    np.testing.assert_array_equal(rec[304:304 + 2048], pres[P["nametable"]:P["nametable"] + 2048],
                                  err_msg=f"{tag}: nametables")


def test_status_bar_rom_pixel_workload_full_size_with_auto_resets():
    """The pixel workload on the status-bar ROM (sprite-0 timed mid-frame
    $2005 writes, IRQ-free): 16,384 consoles, frame-skip 4, 4 snapshot levels
    with short episodes, x-delta reward and auto-reset.  After every step,
    sampled consoles' presentation records equal the oracle's (frames that
    start with the status-bar scroll and end with the play-field scroll),
    and so do their palette-value frames and 84x84 gray frames -- including
    the frames of consoles restarted from a snapshot, whose first frame-start
    scroll is the one latched before the reset."""
    rom = synthrom.make_rom(2026, split=True).rom
    snaps = warm_snapshots(rom, [33, 57, 90, 121], seed=303)
    for i, s in enumerate(snaps):
        s[O.OFF["ram"] + synthrom.DONE_BYTE] = 2 + i      # episodes of 9-32 frames from a snapshot
    blobs = [bytes(s) for s in snaps]
    n, steps = 16384, 16
    rng = np.random.default_rng(305)
    levels = rng.integers(0, 4, n).astype(np.uint8)
    sample = sorted({0, 1, 63, 64, 255, 256, 8191, 8192, n - 1, *rng.integers(0, n, 7).tolist()})
    reward = dict(kind=1, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI, done_addr=synthrom.DONE_BYTE, clip=15,
                  time_penalty=0.01)
    say(f"[gpu] status-bar pixel workload: N={n} fs=4 steps={steps} sample={sample}")
    b = abi.Batch(rom, n, frameskip=4, reward_kind=abi.REWARD_XDELTA, x_lo=synthrom.X_LO, x_hi=synthrom.X_HI,
                  done_addr=synthrom.DONE_BYTE, clip=15, time_penalty=0.01)
    b.set_snapshots(blobs, levels)
    ob = OracleBatch(rom, sample, reward=reward)
    for e, c in zip(sample, ob.cons):
        c.load(snaps[levels[e]])
        c.seed_presentation()          # a full reset seeds the presentation records from live state
    distinct = after_reset = ends = 0
    restarted: set[int] = set()
    for k in range(steps):
        m = masks_for(404, n, k)
        b.set_actions(m)
        b.step(auto_reset=True)
        _, rew, don = ob.step(m, 4)
        np.testing.assert_array_equal(b.host(abi.VIEW_REWARDS)[sample], rew, err_msg=f"step {k} rewards")
        np.testing.assert_array_equal(b.host(abi.VIEW_DONES)[sample], don, err_msg=f"step {k} dones")
        b.render(abi.FRAME_PALETTE | abi.FRAME_GRAY84)
        recs = device_rows(b, abi.VIEW_PRESENT, sample, (b.view(abi.VIEW_PRESENT).shape[1],))
        pals = device_rows(b, abi.VIEW_FRAME_PALETTE, sample, (240, 256))
        grays = device_rows(b, abi.VIEW_GRAY84, sample, (84, 84))
        for j, e in enumerate(sample):
            con = ob.cons[j]
            _record_matches(recs[e], con.presentation(), f"step {k} env {e}")
            want = con.render(snapshot=True)
            bad = int((pals[e] != want).sum())
            assert bad == 0, f"step {k} env {e}: {bad} palette values differ"
            assert np.array_equal(grays[e], O.gray84(want)), f"step {k} env {e}: gray84"
            distinct += tuple(recs[e][0:3]) != tuple(recs[e][3:6])
            after_reset += j in restarted
        restarted = set(np.nonzero(don)[0].tolist())
        for j in restarted:
            ob.cons[j].load(snaps[levels[sample[j]]])
        ends += len(restarted)
    say(f"[gpu]   {distinct} split frames, {ends} episode ends, {after_reset} frames right after a restart")
    assert distinct >= steps * len(sample) // 2
    assert ends >= len(sample) and after_reset >= len(sample) // 2


def _h(a: np.ndarray) -> str:
    return f"{O.fnv1a_np(np.ascontiguousarray(a)):016x}"


@pytest.mark.parametrize("rom_seed", [1, 2, 3])
def test_live_frames_match_the_reference_core_golden(rom_seed):
    """One console over 600 frames (frame-skip 1, the single-env workload):
    frames drawn from live state by the CPU core's rules (NESLE_FRAME_LIVE)
    hash exactly as the reference nesle::Console's own RGB frames and their
    84x84 gray observations (tests/golden/frames_rom{1,2,3}.json)."""
    import json
    from pathlib import Path

    fx = json.loads((Path(__file__).resolve().parent / "golden" / f"frames_rom{rom_seed}.json").read_text())
    rom = synthrom.make_rom(rom_seed).rom
    assert _h(np.frombuffer(rom, dtype=np.uint8)) == fx["rom_fnv1a"]
    want = {r[0]: r for r in fx["records"]}
    say(f"[gpu] live frames vs reference golden: rom{rom_seed} N=1 frames={max(want)}")
    b = abi.Batch(rom, 1, frameskip=1)
    checked = 0
    for k in range(max(want)):
        b.set_actions(masks_for(fx["action_seed"], 1, k))
        b.step()
        rec = want.get(k + 1)
        if rec is None:
            continue
        b.render(abi.FRAME_RGB | abi.FRAME_GRAY84 | abi.FRAME_LIVE)
        assert _h(b.host(abi.VIEW_FRAME_RGB)[0]) == rec[1], f"frame {k + 1}: RGB"
        assert _h(b.host(abi.VIEW_GRAY84)[0]) == rec[2], f"frame {k + 1}: gray84"
        checked += 1
    assert checked == len(want)


def test_live_frames_of_random_states_with_chr_ram():
    """Live-state frames by the CPU core's rules on 64 consoles of a CHR RAM
    cart, each loaded with its own random video memory, registers and CHR RAM
    tiles: equal the oracle's CPU-rule frame of the same state (background
    palette value 0 opaque, CHR RAM read, one scroll), and leave the
    presentation snapshot as it was."""
    rom = _rom(5, chr_ram=True)
    n = 64
    say(f"[gpu] live frames, random states, CHR RAM: N={n}")
    b = abi.Batch(rom, n, frameskip=1)
    base = O.Oracle(rom)
    for k in range(15):
        base.step(int(masks_for(8, 1, k)[0]), 1)
    st0 = base.save()
    rng = np.random.default_rng(4242)
    oracles = {}
    for e in range(n):
        st = st0.copy()
        st[O.OFF["oam"]:O.OFF["oam"] + 256] = rng.integers(0, 256, 256, dtype=np.uint8)
        pal = rng.integers(0, 64, 32, dtype=np.uint8)
        pal[rng.integers(0, 32, 8)] = 0
        st[O.OFF["palette"]:O.OFF["palette"] + 32] = pal
        st[O.OFF["nametable"]:O.OFF["nametable"] + 2048] = rng.integers(0, 256, 2048, dtype=np.uint8)
        st[O.OFF["chr_ram"]:O.OFF["chr_ram"] + 8192] = rng.integers(0, 256, 8192, dtype=np.uint8)
        st[O.OFF["ctrl"]] = rng.integers(0, 256)
        st[O.OFF["mask"]] = 0x18 | rng.integers(0, 256) if e % 4 else rng.integers(0, 256)
        st[O.OFF["scroll_x"]] = rng.integers(0, 256)
        st[O.OFF["scroll_y"]] = rng.integers(0, 256)
        mask = np.zeros(n, dtype=np.uint8)
        mask[e] = 1
        b.load_state(st, mask)
        con = O.Oracle(rom)
        con.load(st)
        con.seed_presentation()
        oracles[e] = con
    before = b.host(abi.VIEW_PRESENT)
    b.render(abi.FRAME_PALETTE | abi.FRAME_RGB | abi.FRAME_GRAY84 | abi.FRAME_LIVE)
    pal, rgb, gray = b.host(abi.VIEW_FRAME_PALETTE), b.host(abi.VIEW_FRAME_RGB), b.host(abi.VIEW_GRAY84)
    lut = O.palette_rgb()
    for e, con in oracles.items():
        want = con.render(snapshot=False, cpu_rules=True)
        bad = int((pal[e] != want).sum())
        assert bad == 0, f"env {e}: {bad} palette values differ"
        assert np.array_equal(rgb[e], lut[want]) and np.array_equal(gray[e], O.gray84(want)), f"env {e}"
    assert np.array_equal(b.host(abi.VIEW_PRESENT), before)
    # The batched rules still draw the snapshot, with CHR RAM read as 0.
    _check(b, oracles, "snapshot after a live render")
