"""q35_lm_head_top1_noalloc (the entry point that allocates nothing) against
q35_lm_head_top1, called through the C ABI.

The process's first no-alloc call is made under graph capture and the
graph's replays give the eager entry point's token and advance. Then two
calls in a row, the second with a smaller vocabulary, on the persistent
K = 2048 path and on the generic path (K = 256, which needs (V + 3) / 4
scratch slots): the token index equals the workspace entry point's bit for
bit, the ``advance`` tensor is incremented the same way, and a generic-path
vocabulary beyond the scratch array is rejected on the host.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _call_both(lib, stream, W, h):
    from ppu_amd import _lib

    V, K = W.shape
    slots = lib.q35_lm_head_top1_workspace(V, K)
    ws = torch.empty(slots, device=W.device, dtype=torch.int64)
    out_ws = torch.full((1, 1), -1, device=W.device, dtype=torch.int64)
    out_na = torch.full((1, 1), -1, device=W.device, dtype=torch.int64)
    adv_ws = torch.tensor([[7]], device=W.device, dtype=torch.int64)
    adv_na = adv_ws.clone()
    _lib.check(lib.q35_lm_head_top1(W.data_ptr(), h.data_ptr(), V, K, ws.data_ptr(), slots,
                                    out_ws.data_ptr(), None, adv_ws.data_ptr(), 1, stream),
               "q35_lm_head_top1")
    _lib.check(lib.q35_lm_head_top1_noalloc(W.data_ptr(), h.data_ptr(), V, K, out_na.data_ptr(),
                                            adv_na.data_ptr(), 1, stream),
               "q35_lm_head_top1_noalloc")
    torch.cuda.synchronize()
    return int(out_ws), int(out_na), int(adv_ws), int(adv_na)


def test_noalloc_top1_under_graph_capture(gpu):
    """First in this file, so the first no-alloc call of a run that starts
    here happens inside torch.cuda.graph capture; three replays, with eager
    work between them, each give the workspace entry point's token and
    advance the position the same way."""
    from ppu_amd import _lib

    lib = _lib.load()
    g = torch.Generator().manual_seed(20260819)
    V, K = 248320, 2048
    W = (torch.randn(V, K, generator=g) * 0.02).to(torch.bfloat16).to(gpu)
    h = torch.randn(1, K, generator=g).to(torch.bfloat16).to(gpu)
    out = torch.full((1, 1), -1, device=gpu, dtype=torch.int64)
    adv = torch.tensor([[100]], device=gpu, dtype=torch.int64)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.check(lib.q35_lm_head_top1_noalloc(W.data_ptr(), h.data_ptr(), V, K, out.data_ptr(),
                                                adv.data_ptr(), 1,
                                                torch.cuda.current_stream().cuda_stream),
                   "q35_lm_head_top1_noalloc")
    stream = torch.cuda.current_stream().cuda_stream
    for rep in range(3):
        out.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        ws_tok, _, _, _ = _call_both(lib, stream, W, h)  # eager work between the replays
        assert int(out) == ws_tok
        assert int(adv) == 101 + rep


@pytest.mark.parametrize("K", [2048, 256])
def test_noalloc_top1_matches_workspace_entry(gpu, K):
    from oracle import ops as ref
    from ppu_amd import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(20260819 + K)
    for V in (248320 if K == 2048 else 200003, 4099):  # second call smaller
        W = (torch.randn(V, K, generator=g) * 0.02).to(torch.bfloat16)
        h = torch.randn(1, K, generator=g).to(torch.bfloat16)
        # plant a tie at the maximum: the lower index must win on both paths
        best = int(ref.lm_head_argmax(h, W))
        dup = min(V - 1, best + 17)
        W[dup] = W[best]
        expect = min(best, dup)
        ws_tok, na_tok, ws_adv, na_adv = _call_both(lib, stream, W.to(gpu), h.to(gpu))
        assert ws_tok == na_tok == expect == int(ref.lm_head_argmax(h, W))
        assert ws_adv == na_adv == 8


def test_noalloc_top1_rejects_beyond_scratch(gpu):
    from ppu_amd import _lib

    lib = _lib.load()
    V, K = 262_142 + 3, 256  # (V + 3) / 4 > 65,536 slots on the generic path
    W = torch.zeros(V, K, device=gpu, dtype=torch.bfloat16)
    h = torch.zeros(1, K, device=gpu, dtype=torch.bfloat16)
    out = torch.full((1, 1), -1, device=gpu, dtype=torch.int64)
    rc = lib.q35_lm_head_top1_noalloc(W.data_ptr(), h.data_ptr(), V, K, out.data_ptr(), None, 0,
                                      torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 1 and int(out) == -1  # hipErrorInvalidValue, nothing launched
