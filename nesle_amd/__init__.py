"""nesle_amd -- MI355X-native batched NROM (mapper 0) emulator.

* ``nesle_amd._cuda_core``  drop-in for the reference's ``nesle._cuda_core``
  (``CudaBatch``, ``CudaDeviceArrayView``, ``parse_fcs_state``), built by
  ``python -m nesle_amd.build`` over libnesle_hip.so;
* ``nesle_amd.abi``         ctypes binding of the C ABI (include/nesle_hip.h);
* ``nesle_amd.synthrom``    seeded synthetic NROM ROMs and controller streams;
* ``nesle_amd.env``         SB3/Gymnasium vector and single environments
  (``make_vec``, ``NesleVecEnv``, ``NesleEnv``), drop-in for ``nesle.env``;
* ``nesle_amd.native_ppo``  GPU-resident PPO, drop-in for ``nesle.native_ppo``;
* ``nesle_amd.actions``     controller masks and action sets.

The native pieces are imported on first use, so importing the package never
touches a GPU; using them without the built libraries raises ImportError.
"""

from __future__ import annotations

__version__ = "0.1.0"

from . import abi, synthrom  # noqa: F401
from .actions import (  # noqa: F401  (the reference package exports these at its root)
    COMPLEX_MOVEMENT,
    COMPLEX_MOVEMENT_MASKS,
    MARIO_MOVEMENT,
    MARIO_MOVEMENT_MASKS,
    RIGHT_ONLY,
    RIGHT_ONLY_MASKS,
    SIMPLE_MOVEMENT,
    SIMPLE_MOVEMENT_MASKS,
    SIMPLE_MOVEMENT_WITH_START,
    SIMPLE_MOVEMENT_WITH_START_MASKS,
    Button,
    encode_action,
)

__all__ = ["__version__", "load_cuda_core", "make", "make_vec", "synthrom", "abi", "Button", "encode_action",
           "COMPLEX_MOVEMENT", "COMPLEX_MOVEMENT_MASKS", "MARIO_MOVEMENT", "MARIO_MOVEMENT_MASKS", "RIGHT_ONLY",
           "RIGHT_ONLY_MASKS", "SIMPLE_MOVEMENT", "SIMPLE_MOVEMENT_MASKS", "SIMPLE_MOVEMENT_WITH_START",
           "SIMPLE_MOVEMENT_WITH_START_MASKS"]


def load_cuda_core():
    """The drop-in module; raises ImportError when it has not been built."""
    from . import _cuda_core  # type: ignore[attr-defined]

    return _cuda_core


def make(*args, **kwargs):
    """``NesleEnv(*args, **kwargs)`` (the reference's ``nesle.make``)."""
    from .env import NesleEnv

    return NesleEnv(*args, **kwargs)


def make_vec(*args, **kwargs):
    """``NesleVecEnv(*args, **kwargs)`` (the reference's ``nesle.make_vec``)."""
    from .env import NesleVecEnv

    return NesleVecEnv(*args, **kwargs)
