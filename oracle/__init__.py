"""CPU oracle for the Qwen3.5 decode hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference operator
module (PingGuoLiZiJvZi/ppu qwen35_fused/kernels.py and integration.py) with
the same bf16 rounding points, tie rules and fp32 formulations. It exists to
check the MI355X kernels: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or
as the timed CPU baseline. The product package ``ppu_amd`` never imports it and
has no CPU fallback.

Modules:
  ops    — per-operator restatements (torch CPU, fp32 with explicit bf16 rounds)
  a8w8   — integer A8W8 path in numpy (int8 quantisers, exact int32 products)
  model  — the decoder data flow of the patched text forward (integration.py)
  synth  — seeded synthetic inputs and the 2B-shaped configuration

Pinning (what checks each function against something other than itself) is
listed in each module's header. Functions without such a check are marked
"parity unpinned" there.
"""
