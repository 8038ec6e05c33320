"""Write the golden frame fixtures from the reference's own CPU core.

Run in a container where /root/reference exists:

    make -C oracle ref && python tests/golden/make_frame_golden.py

The reference ``nesle::Console`` (oracle/_ref/libnesle_ref.so, compiled from the
reference sources by oracle/Makefile) runs the single-env workload of
``console_rom{1,2,3}.json`` (frame-skip 1, controller byte for frame ``k`` =
``splitmix64(action_seed ^ k) & 0xFF``).  At the listed frames its RGB frame
(``PPU::render_rgb_frame``, ppu.hpp:213-230) is FNV-1a hashed, and so is the
84x84 gray observation of that frame computed the way the reference's training
wrapper does it (project/mario-rl-ram/src/mario_rl/wrappers.py:209-215: numpy
luma, uint8 truncation, Pillow BILINEAR resize).  Only hashes are stored.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from nesle_amd import synthrom  # noqa: E402
from oracle import oracle as O  # noqa: E402

CASES = [(1, 1001), (2, 1002), (3, 1003)]
FRAMES = [1, 2, 3, 10, 50, 100, 200, 400, 600]


def gray84_pil(rgb: np.ndarray) -> np.ndarray:
    from PIL import Image

    gray = np.dot(rgb[..., :3].astype(np.float32), [0.299, 0.587, 0.114])
    img = Image.fromarray(gray.astype(np.uint8)).resize((84, 84), Image.BILINEAR)
    return np.array(img, dtype=np.uint8)


def main() -> None:
    if not O.ref_available():
        O.build(ref=True)
    out_dir = Path(__file__).resolve().parent
    for rom_seed, action_seed in CASES:
        rom = synthrom.make_rom(rom_seed).rom
        con = O.RefConsole(rom)
        records = []
        for k in range(max(FRAMES)):
            con.step(int(synthrom.action_masks(action_seed, 1, k)[0]), frameskip=1)
            if k + 1 in FRAMES:
                rgb = con.render_rgb()
                records.append([k + 1, f"{O.fnv1a(rgb):016x}", f"{O.fnv1a(gray84_pil(rgb)):016x}"])
        doc = {
            "source": "reference nesle::Console render_rgb_frame via oracle/_ref; gray84 per wrappers.py:209-215",
            "rom_seed": rom_seed,
            "rom_fnv1a": f"{O.fnv1a(rom):016x}",
            "action_seed": action_seed,
            "frameskip": 1,
            "columns": ["frame", "rgb_fnv1a", "gray84_fnv1a"],
            "records": records,
        }
        path = out_dir / f"frames_rom{rom_seed}.json"
        path.write_text(json.dumps(doc, indent=1) + "\n")
        print(f"wrote {path.name}: {len(records)} frames")


if __name__ == "__main__":
    main()
