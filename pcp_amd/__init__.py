"""pcp_amd — MI355X (gfx950) GRPO loss head behind PCP's worker-backend interface.

Hand-written HIP kernels in libpcp_grpo.so (C ABI: include/pcp_grpo.h); this
package binds them with ctypes. torch supplies device memory and streams only.
"""
from ._lib import (DType, Backend, LossMode, PcpError, IGNORE_INDEX, LIB_PATH, lib)  # noqa: F401

__version__ = "0.1.0"
