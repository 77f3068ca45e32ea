"""``qwen35_fused.graph`` -> ``ppu_amd.graph`` (same module object)."""
import sys

from ppu_amd import graph as _m

sys.modules[__name__] = _m
