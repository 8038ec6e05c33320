"""nesle_amd._cuda_core -- drop-in for the reference's ``nesle._cuda_core``.

Re-exports the pybind11 module built from nesle_amd/csrc/cuda_core_module.cpp
(``CudaBatch``, ``CudaDeviceArrayView``, ``parse_fcs_state``,
``parse_ines_metadata``) after binding the process to PyTorch's HIP runtime
(see ``nesle_amd.abi.bind_runtime``).  Raises ImportError when the native
module has not been built.
"""

from .abi import bind_runtime

bind_runtime()

from ._cuda_core_native import *  # noqa: E402,F401,F403
from ._cuda_core_native import DLPACK_DEVICE_TYPE, STATE_BYTES  # noqa: E402,F401
