"""``qwen35_fused.integration`` -> ``ppu_amd.integration`` (same module object)."""
import sys

from ppu_amd import integration as _m

sys.modules[__name__] = _m
