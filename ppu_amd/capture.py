"""Graph-capture set-up shared by the library's captured paths.

Every ``torch.cuda.graph`` capture registers the capture device's default
random-number generator with the graph, and the generator's capture-time
state tensors are created at its first registration. If that first capture
runs under ``torch.inference_mode`` (as the decode, prefill and vision-tower
captures do when the caller generates under inference mode), those tensors
are inference tensors, and every later capture outside inference mode in the
same process fails in ``capture_begin`` ("Inplace update to inference tensor
outside InferenceMode is not allowed"). ``prime_capture_state`` makes the
first registration happen outside inference mode, with one tiny capture that
is kept alive for the process, so captures work afterwards in either mode.
"""

from __future__ import annotations

import torch

_PRIMED: dict[int, tuple] = {}


def prime_capture_state(device: torch.device | int | str | None = None) -> None:
    """Once per device: capture one small fill outside inference mode and keep
    the graph, so the generator's capture state holds ordinary tensors. If a
    capture under inference mode already made them inference tensors (a
    capture outside the library), this priming capture fails the same way;
    that state cannot be repaired here, and the caller's own capture then runs
    in whatever mode the caller is in."""
    dev = torch.device(device) if device is not None else torch.device("cuda")
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx in _PRIMED:
        return
    with torch.inference_mode(False), torch.cuda.device(idx):
        buf = torch.zeros(1, device=torch.device("cuda", idx))
        graph = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(graph):
                buf.add_(1)
        except RuntimeError:
            _PRIMED[idx] = ()
            return
    _PRIMED[idx] = (graph, buf)
