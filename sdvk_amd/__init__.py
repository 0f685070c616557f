"""sdvk_amd -- MI355X-native Q8_0 GEMM and fused attention behind a C-ABI.

The kernels are hand-written HIP for gfx950 in sdvk_amd/csrc, built into
sdvk_amd/libmi_sdvk.so (include/mi_sdvk.h). This package holds the Python
side: the ctypes binding (_lib), HIP runtime plumbing (hip) and the mirror of
the reference operator surface (ops).
"""
from .ops import *  # noqa: F401,F403
from .ops import __all__ as _ops_all

__all__ = list(_ops_all)
__version__ = "0.1.0"
