"""HIP build of the package's native code for gfx950 (MI355X).

Replaces the reference's nvcc build script (scripts/build_cuda_extension.py):

* ``libnesle_hip.so``  -- kernels + C ABI (include/nesle_hip.h), built by hipcc
  for ``--offload-arch=gfx950``;
* ``_cuda_core_native*.so`` -- the pybind11 drop-in for nesle._cuda_core
  (re-exported by nesle_amd/_cuda_core.py), host-only C++ linked against
  libnesle_hip.so (rpath $ORIGIN).

Both land in-tree next to this file.  ``python -m nesle_amd.build`` rebuilds.
Environment: ``HIPCC`` (default: hipcc on PATH or /opt/rocm/bin/hipcc),
``NESLE_HIP_ARCH`` (default gfx950), ``CXX`` (default g++).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig
import tempfile
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libnesle_hip.so"
HIP_SOURCES = [CSRC / "nes_step.hip", CSRC / "nes_step_full.hip", CSRC / "nes_step_narrow.hip", CSRC / "nes_kernels.hip",
               CSRC / "nes_render.hip", CSRC / "nes_host.hip", CSRC / "ppo_head.hip", CSRC / "smb_shaped.hip"]
SHIM_SOURCE = CSRC / "cuda_core_module.cpp"

HIP_FLAGS = [
    # -O2: the step kernel runs about 1 % faster than at -O3 (65,536 consoles,
    # same-box A/B), the renderer and the PPO head no slower.
    "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
    # Keep the compiler from forming packed fp32 VALU ops.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Flags of one source on top of HIP_FLAGS.  The step kernel's instances come
# from three translation units, each with the scheduler setting measured
# fastest for it: all RAM in LDS (nes_step_full.hip, up to 8,192 consoles)
# LLVM's iterative ILP scheduler, 2-3 % faster; the split layout at 16 or 32
# consoles per wave (nes_step_narrow.hip) the machine scheduler off, 2-3 %
# faster; at 64 per wave (nes_step.hip, 65,536 consoles) the default strategy,
# as both of the others run 0.6-2.5 % slower there.  Where the machine
# scheduler runs, its macro-op fusion (keeping fusible instruction pairs
# adjacent) is off: 2.3 % faster at 65,536 consoles, 1 % with all RAM in LDS.
_NO_FUSION = ["-mllvm", "-misched-fusion=false"]
SOURCE_FLAGS = {
    CSRC / "nes_step.hip": _NO_FUSION,
    CSRC / "nes_step_full.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp", *_NO_FUSION],
    CSRC / "nes_step_narrow.hip": ["-mllvm", "-enable-misched=false"],
}


def source_flags(source: Path) -> list[str]:
    """Device-compile flags of one HIP source (no -shared / -fPIC)."""
    return [f for f in HIP_FLAGS if f not in ("-shared", "-fPIC")] + SOURCE_FLAGS.get(source, [])


def _hipcc() -> str:
    env = os.environ.get("HIPCC")
    if env:
        return env
    found = shutil.which("hipcc")
    return found or "/opt/rocm/bin/hipcc"


def shim_path() -> Path:
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    return PKG / f"_cuda_core_native{suffix}"


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd[:3])} ...")


def build_hip(arch: str | None = None) -> Path:
    """Compile every HIP source to an object (in parallel, each with its own
    flags), then link them into LIB."""
    arch = arch or os.environ.get("NESLE_HIP_ARCH", "gfx950")
    tmp = LIB.with_suffix(".so.tmp")
    with tempfile.TemporaryDirectory(prefix="nesle_hip_") as work:
        objs = [Path(work) / (src.stem + ".o") for src in HIP_SOURCES]
        cmds = [[_hipcc(), f"--offload-arch={arch}", "-fPIC", *source_flags(src), "-c", str(src), "-o", str(obj)]
                for src, obj in zip(HIP_SOURCES, objs)]
        workers = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
        with concurrent.futures.ThreadPoolExecutor(workers) as pool:
            list(pool.map(_run, cmds))
        _run([_hipcc(), f"--offload-arch={arch}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    tmp.replace(LIB)
    return LIB


def build_shim() -> Path:
    import pybind11

    out = shim_path()
    tmp = out.with_name(out.name + ".tmp")
    include = [f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}"]
    cxx = os.environ.get("CXX", "g++")
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden", *include,
          str(SHIM_SOURCE), "-o", str(tmp), f"-L{PKG}", "-lnesle_hip", "-Wl,-rpath,$ORIGIN"])
    tmp.replace(out)
    return out


def build_all() -> None:
    build_hip()
    build_shim()


if __name__ == "__main__":
    build_all()
    print(f"built {LIB.name} and {shim_path().name}")
