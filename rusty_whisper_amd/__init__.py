"""rusty_whisper_amd -- MI355X (gfx950) implementation of rusty_whisper's
quantized linear-layer matmul (src/quant.rs `matmul_t_q` / `linear_w`).

Layers:
  librw_rocm.so   HIP kernels + the C ABI of include/rw_rocm.h
  _abi            ctypes binding of that ABI (status codes -> RwError)
  quant           the reference's QTensor / Weight / matmul_t_q / linear_w API,
                  via the C++ mirror in host/ (pybind11 module _rw_quant)
"""


def _one_hip_runtime() -> None:
    """PyTorch-ROCm wheels carry their own libamdhip64.so.  A process that
    loads librw_rocm.so (linked against /opt/rocm's libamdhip64.so.7) before
    torch ends up with two HIP runtimes, and torch then sees no GPU.  When
    torch is installed it is imported first, so the dynamic linker hands its
    runtime (same SONAME) to librw_rocm.so and the process holds one."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


_one_hip_runtime()

from ._abi import (  # noqa: E402,F401
    DTYPES, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, QK, DeviceWeight, RwError, block_bytes, check, device_count,
    init, lib, quantize_acts, workspace_size,
)

__version__ = "0.1.0"
