"""lumenrl_amd: MI355X-native (gfx950 HIP) weight quantization for Lumen-RL weight sync.

Host code is Python on PyTorch-ROCm; the kernels live in liblrq.so (C ABI in
include/lrq.h), loaded through ``lumenrl_amd._lib``.
"""

from lumenrl_amd import quantization
from lumenrl_amd._lib import LIB_PATH, LrqError, version

__all__ = ["LIB_PATH", "LrqError", "quantization", "version"]
