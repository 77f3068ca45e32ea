"""``qwen35_fused.kernels`` -> ``ppu_amd.kernels`` (same module object)."""
import sys

from ppu_amd import kernels as _k

sys.modules[__name__] = _k
