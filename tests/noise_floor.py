"""Measures the CPU oracle's own noise floor on the 2B shape (not a test).

Runs the oracle decoder twice on the same random-init 2B-shaped weights, a
1024-token prompt and 16 teacher-forced tokens: once as written and once with
every RMSNorm variance summed in fp64 (then rounded to fp32), a change of at
most one fp32 ulp per variance. The relative L2 change of the final hidden
state per step is the floor the GPU-vs-oracle bounds in test_gpu_model.py are
set from. Needs about 25 GB of host memory for a8w8 (fp64 integer weights).

    python tests/noise_floor.py bf16|a8w8 [steps]
"""

from __future__ import annotations

import os
import sys
import time

import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

from oracle import ops  # noqa: E402
from oracle.model import OracleDecoder  # noqa: E402
from ppu_amd import synth  # noqa: E402


def main(mode: str, steps: int = 64) -> None:
    t0 = time.time()
    cfg = synth.config_2b()
    model = synth.build_model(cfg, device="cpu", seed=1234)
    state = {k: v.detach() for k, v in model.state_dict().items()}
    del model
    dec = OracleDecoder(state, cfg, a8w8=mode == "a8w8")
    ids = torch.randint(0, cfg.vocab_size, (1, 1024), generator=torch.Generator().manual_seed(7))
    forced = torch.randint(0, cfg.vocab_size, (steps - 1,),
                           generator=torch.Generator().manual_seed(8)).tolist()

    def run():
        cache = dec.new_cache(1024 + steps + 8)
        hs = [dec.forward(ids, cache)[:, -1]]
        for t in forced:
            hs.append(dec.forward(torch.tensor([[t]]), cache)[:, -1])
        return hs

    h1 = run()
    print(f"run 1 done at {time.time() - t0:.0f} s", flush=True)
    orig = ops.rms_norm

    def rms64(x, weight, eps=1e-6):
        x32 = ops._f(x)
        var = (x32.double() * x32.double()).sum(-1, keepdim=True).float() / x.shape[-1]
        return ops._bf(x32 * ops._rsqrt(var + eps) * (1.0 + ops._f(weight)))

    try:
        ops.rms_norm = rms64
        h2 = run()
    finally:
        ops.rms_norm = orig
    errs = [float((a.double() - b.double()).norm() / b.double().norm()) for a, b in zip(h1, h2)]
    print(mode, "per step", " ".join(f"{e:.3f}" for e in errs))
    srt = sorted(errs)
    print(f"{mode} {len(errs)} steps: mean {sum(errs) / len(errs):.4f} "
          f"p90 {srt[int(0.9 * (len(srt) - 1))]:.4f} max {srt[-1]:.4f}")


if __name__ == "__main__":
    torch.set_num_threads(os.cpu_count() or 1)
    main(sys.argv[1] if len(sys.argv) > 1 else "bf16", int(sys.argv[2]) if len(sys.argv) > 2 else 64)
