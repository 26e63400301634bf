"""vai_amd -- MI355X-native (gfx950) kernels for vAi's matmul hot path.

The product is libvai_amd.so (include/vai_amd.h, plus the C++ engine under
vai_amd/engine). This package builds it and binds it with ctypes.
"""
from . import _capi  # noqa: F401
