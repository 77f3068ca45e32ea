"""Host-side checks of bench.py (no GPU): the one-GPU contract of the
command line and the CPU leg's per-config table."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_bench_refuses_more_than_one_gpu():
    """``--gpus N`` with N > 1 exits with status 2 and says why (every box
    here has one GPU; the sharding is design only), before touching a GPU."""
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], cwd=ROOT,
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 2
    assert "one GPU" in res.stderr or "1 GPU" in res.stderr or "--gpus 1" in res.stderr


def test_cpu_kernel_table_on_host():
    """The CPU leg times configs 1-4 through the oracle ops on the host: every
    config of the GPU table has a positive time and a byte rate."""
    sys.path.insert(0, str(ROOT))
    import torch

    import bench

    torch.set_num_threads(min(8, torch.get_num_threads()))
    out = bench.cpu_kernel_table()
    names = {"cfg1_resnorm_gemv_6144x2048", "cfg3_gqa_decode_L512", "cfg3_gqa_decode_L8192",
             "cfg4_delta_decode_chain_per_token"}
    names |= {f"cfg2_a8w8_{s}_m{m}" for s in ("12288x2048", "2048x6144") for m in (1, 4, 16)}
    assert names <= set(out)
    for rec in out.values():
        assert rec["us"] > 0 and rec["GB/s"] > 0
