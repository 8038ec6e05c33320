"""Compiled resources of the kernels, read from the gfx950 assembly hipcc
writes for them (no GPU needed): the render kernel's LDS stays within the 25
allocation units of 1,280 bytes that let 5 workgroups share a compute unit
(one unit more leaves room for 4 and the launch runs about 14 % slower),
and no kernel spills to scratch memory."""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from nesle_amd import build

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
pytestmark = pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")


def _kernels(source: Path, tmp_path: Path) -> dict[str, dict[str, int]]:
    out = tmp_path / (source.stem + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "--offload-device-only", "-S", *build.source_flags(source), "-o", str(out),
           str(source)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    meta = out.read_text().split("amdhsa.kernels:", 1)[1]
    kernels = {}
    for block in meta.split("  - .")[1:]:
        name = re.search(r"\.name:\s+(\S+)", block)
        if name is None:
            continue
        fields = {k: int(v) for k, v in re.findall(r"\.(group_segment_fixed_size|private_segment_fixed_size):\s+(\d+)",
                                                     block)}
        kernels[name.group(1)] = fields
    return kernels


def test_render_kernel_lds_fits_five_workgroups(tmp_path):
    kernels = _kernels(build.CSRC / "nes_render.hip", tmp_path)
    render = [v for k, v in kernels.items() if "render_kernel" in k]
    assert len(render) == 1
    assert render[0]["group_segment_fixed_size"] <= 25 * 1280
    assert render[0]["private_segment_fixed_size"] == 0


@pytest.mark.parametrize("source,full", [("nes_step.hip", 0), ("nes_step_full.hip", 1), ("nes_step_narrow.hip", 0)])
def test_step_kernels_use_no_scratch(tmp_path, source, full):
    """Every step kernel but the census build (stats mode 3, a measurement
    variant whose counters may spill) keeps its state in registers and LDS.
    The split-layout instances come from nes_step.hip (64 consoles per wave)
    and nes_step_narrow.hip (16 or 32), the all-RAM-in-LDS ones from
    nes_step_full.hip, each built with the flags the package build gives it."""
    kernels = _kernels(build.CSRC / source, tmp_path)
    steps = {k: v for k, v in kernels.items() if "step_kernel" in k and "step_kernelILi3E" not in k}
    assert len(steps) == 4
    assert all(re.search(r"step_kernelILi\dELb(\d)E", k).group(1) == str(full) for k in steps), sorted(steps)
    assert all(v["private_segment_fixed_size"] == 0 for v in steps.values()), steps
