"""Decode tokens/s and TTFT of the synthetic Qwen3.5-2B-shaped decoder on one MI355X.

Workload (Benchmark config 5): the 24-layer 2B-shaped decoder with seeded
random-init bf16 weights (synthetic; no checkpoint), batch 1, a 1024-token
prompt of uniform-random token ids, then greedy decode. A "step" is one
greedy decode token: one replay of the captured decode graph (24 layers +
lm_head top-1 + token feedback) followed by the host read of the token, as
the reference's decode loop does (evaluation_wrapper.py:412-419).

Printed (one JSON line on stdout):
  value        decode tokens/s over the K timed steps (inputs resident in HBM)
  ttft_ms      prefill (1024 tokens) + first token, timed as the reference
               does (evaluation_wrapper.py:342-365), median of warm runs
  roofline     the decode kernel with the largest share of the step: the
               residual add + RMSNorm + SwiGLU GEMV [12288, 2048] (24 per
               token), timed with HIP events on its stream over the model's
               own 24 layer weights (1.2 GB, rotated in one graph);
               traffic = its HBM bytes per launch from the committed
               rocprofv3 --pmc summary profiles/decode_step_traffic_pmc.txt
               (``bench.py --counter-probe`` runs); roofline_detail adds a
               plain streaming read of the same byte count rotated the same
               way (the launch-size ceiling), and the lm_head GEMV + top-1
  step_roofline  the whole decode step: HBM bytes one token needs (packed
               weights, lm_head, recurrent/conv state read + write, K/V read
               at the mean context of the timed steps) / ms_per_step
  kernels     per-kernel achieved HBM GB/s of the Benchmark configs 1-4
               (rotating >= 640 MB of distinct buffers so the 256 MB MALL does
               not serve the weights), in-graph time per launch
  variants     the same decode and TTFT measurement for the other linear
               variant of config 5 (A8W8 when the headline runs bf16), on the
               same seeded weights
  cpu_baseline the CPU oracle decoder (the reference's PyTorch CPU path,
               restated) on the config-5 prompt: the full 1024-token prefill
               then 16 greedy decode steps, same process, host cores; beside
               it Transformers' own eager forward (what the reference runs for
               CPU tensors) on the same weights and threads
  inputs_sha256  SHA-256 of the prompt and of the generated weights, with
               whether they equal the committed tests/golden/digests.json
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0
PROMPT_LEN = 1024
NEW_TOKENS = 64


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def graph_time_us(fn, calls: int, reps: int) -> float:
    """Average time per call of ``fn(i)`` captured ``calls`` times in one graph."""
    import torch

    for i in range(2):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(calls):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * calls)


def pmc_traffic(name: str, kernel: str | None = None):
    """HBM bytes per launch read from a committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE passes scaled by a copy kernel of known size):
    the ``traffic_bytes_per_launch`` line, or with ``kernel`` the summary row
    whose first field starts with that kernel name; None when absent."""
    try:
        for line in (ROOT / "profiles" / name).read_text().splitlines():
            if kernel is None and line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
            if kernel is not None and line.startswith(kernel + " |"):
                return int(line.split("|")[3])
    except (OSError, ValueError, IndexError):
        pass
    return None


def lm_head_roofline(model) -> dict:
    import torch

    from ppu_amd import kernels as K

    w = model.lm_head.weight
    v, k = w.shape
    h = torch.randn(1, k, device=w.device, dtype=torch.bfloat16)
    us = graph_time_us(lambda i: K.lm_head_argmax(h, w), calls=10, reps=10)
    slots = (v + 3) // 4
    algo = v * k * 2 + k * 2 + 8  # weights + hidden + index
    achieved = algo / us / 1e3
    # the device's achievable read rate: the same weight bytes read once by
    # the plain streaming-read probe (same loads, no arithmetic)
    read_us = graph_time_us(lambda i: K.stream_read(w), calls=10, reps=10)
    read_gbs = v * k * 2 / read_us / 1e3
    log(f"lm_head top-1: {us:.1f} us, {achieved:.0f} GB/s; plain read of the same bytes "
        f"{read_us:.1f} us, {read_gbs:.0f} GB/s ({100 * achieved / read_gbs:.1f}% of it)")
    from ppu_amd.integration import lm_head_screen

    screened = None
    screen = lm_head_screen(model)
    if screen is not None:
        hs = [torch.randn(1, k, device=w.device, dtype=torch.bfloat16) for _ in range(10)]
        s_us = graph_time_us(lambda i: K.lm_head_argmax(hs[i], w, screen=screen), calls=10, reps=10)
        same, cands = True, []
        for x in hs:
            tok, n = K.lm_head_argmax(x, w, screen=screen, return_candidates=True)
            same = same and int(tok) == int(K.lm_head_argmax(x, w))
            cands.append(int(n))
        # bf16 rows the rescore reads beyond the int8 screen; the screen stops
        # paying off near V/2 of them (int8 copy + rows = the plain bf16 bytes)
        screened = {"us_per_call": round(s_us, 2), "same_index_as_full": same,
                    "int8_bytes": v * k + 8 * v,
                    "candidate_rows": {"max": max(cands), "mean": round(sum(cands) / len(cands), 1),
                                       "frac_of_vocab": round(max(cands) / v, 6),
                                       "hidden": "N(0,1) bf16, 10 draws"},
                    "speedup_vs_full": round(us / s_us, 3)}
        log(f"screened lm_head top-1: {s_us:.1f} us ({us / s_us:.2f}x), same index: {same}, "
            f"candidate rows max {max(cands)} of {v}")
    return {"kernel": "lm_head GEMV + top-1 [248320,2048] bf16", "bound": "hbm",
            "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": pmc_traffic("lm_head_top1_traffic_pmc.txt"),
            "us_per_launch": round(us, 2), "algorithmic_bytes": algo,
            "workspace_bytes": slots * 8,
            "read_ceiling": {"GB/s": round(read_gbs, 1), "us": round(read_us, 2),
                             "frac_of_peak": round(read_gbs / PEAK_HBM_GBS, 4),
                             "lm_head_frac_of_ceiling": round(achieved / read_gbs, 4)},
            "screened": screened}


def swiglu_roofline(model, variant: str) -> dict:
    """The residual add + RMSNorm + SwiGLU GEMV ``[2*6144, 2048]`` of the
    decode step (the kernel with the largest share of it: 24 launches per
    token), launched over the model's own 24 layer weights in one graph, and a
    plain streaming read of the same bytes rotated the same way."""
    import torch

    from ppu_amd import kernels as K
    from ppu_amd.integration import text_stack

    layers = text_stack(model).layers
    dev = layers[0].mlp.q35_gate_up.w.device
    g = torch.Generator(device=dev).manual_seed(20260819)
    r = torch.randn(1, 1, 2048, device=dev, generator=g).to(torch.bfloat16)
    u = torch.randn(1, 1, 2048, device=dev, generator=g).to(torch.bfloat16)
    ops = [(l.mlp.q35_gate_up.w, l.mlp.q35_gate_up.s, l.post_attention_layernorm) for l in layers]
    n = len(ops)

    def launch(i):
        w, sc, ln = ops[i % n]
        return K.residual_norm_linear(r, u, ln.weight, ln.eps, w, swiglu=True, weight_scale=sc)

    us = graph_time_us(launch, calls=n, reps=10)
    w0, s0, _ = ops[0]
    n_rows, k = w0.shape
    wbytes = w0.numel() * w0.element_size() + (0 if s0 is None else s0.numel() * 4)
    algo = wbytes + 3 * k * 2 + k * 2 + (n_rows // 2) * 2  # W (+scales), r, u, norm w, r', y
    achieved = algo / us / 1e3
    read_us = graph_time_us(lambda i: K.stream_read(ops[i % n][0]), calls=n, reps=10)
    read_gbs = w0.numel() * w0.element_size() / read_us / 1e3
    kname = f"gemv_fused<4, {4 if variant == 'a8w8' else 2}, {2 if variant == 'a8w8' else 4}, 2, 1, " \
            f"{'true' if variant == 'a8w8' else 'false'}>"
    log(f"SwiGLU GEMV [{n_rows},{k}] ({variant}): {us:.2f} us, {achieved:.0f} GB/s "
        f"({100 * achieved / PEAK_HBM_GBS:.1f}% of 8 TB/s); plain read of the same bytes "
        f"{read_us:.2f} us ({100 * read_us / us:.1f}% of the GEMV time)")
    return {"kernel": f"residual add + RMSNorm + SwiGLU GEMV [{n_rows},{k}] {variant} ({kname})",
            "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": pmc_traffic("decode_step_traffic_pmc.txt", kname) if variant == "bf16" else None,
            "us_per_launch": round(us, 3), "algorithmic_bytes": algo, "launches_per_token": n,
            "same_size_read": {"us": round(read_us, 3), "GB/s": round(read_gbs, 1),
                               "gemv_frac_of_read_rate": round(achieved / read_gbs, 4)}}


def profile_frac(roof: dict) -> dict:
    """The roofline fraction of the dominant kernel from its average duration
    in the committed decode-step profile (profiles/decode_step_2b.txt, the
    in-step kernel under rocprofv3), beside the bench's own graph-timed one."""
    import re

    name = re.search(r"\((gemv_fused<[^>]*>)\)", roof["kernel"])
    try:
        text = (ROOT / "profiles" / "decode_step_2b.txt").read_text()
    except OSError:
        return {}
    if not name:
        return {}
    m = re.search(re.escape(name.group(1)) + r" g\d+\s+n=\s*\d+ total\s+[\d.]+ us\s+avg\s+([\d.]+) us", text)
    if not m:
        return {}
    us = float(m.group(1))
    ach = roof["algorithmic_bytes"] / us / 1e3
    return {"frac_bench": roof["frac"], "us_bench": roof["us_per_launch"],
            "frac_profile": round(ach / roof["peak"], 4), "us_profile": us,
            "profile": "profiles/decode_step_2b.txt (first decode-step table)"}


def step_bytes(model, context: float) -> int:
    """HBM bytes one decode token needs: every packed weight (and int8 scale)
    once, the lm_head (tied embedding) once (with the screened top-1
    installed: its int8 copy, per-row scale and bound factor and the per-row
    upper bounds written and read back, in place of the bf16 weight; the
    recomputed rows are not counted), the small per-layer parameters
    the decode kernels read (norm weights, conv taps, ``A_log``, ``dt_bias``),
    the embedding row, the recurrent and conv states read and written, and
    the K/V cache read over ``context`` positions plus the new row written.
    Each storage is counted once (a bf16 packed weight may share the storage
    of the original parameter); nn.Linear weights are read only through their
    packed form."""
    import torch

    from ppu_amd.integration import _Weight, text_stack

    stack = text_stack(model)
    seen: set[int] = set()
    total = 0

    def add(t):
        nonlocal total
        if t is not None and t.data_ptr() not in seen:
            seen.add(t.data_ptr())
            total += t.numel() * t.element_size()

    for m in model.modules():
        if isinstance(m, _Weight):
            add(m.w)
            add(m.s)
    from ppu_amd.integration import lm_head_screen

    screen = lm_head_screen(model)
    if screen is None:
        add(model.lm_head.weight)
    else:
        for t in screen:
            add(t)
        total += 2 * 4 * screen[1].numel()  # per-row upper bounds written and read
        seen.add(model.lm_head.weight.data_ptr())  # the tied embedding is not re-counted below
    total += stack.config.hidden_size * 2  # the embedding row of the token
    for mod in stack.modules():
        if isinstance(mod, torch.nn.Linear) or mod is stack.embed_tokens:
            continue
        for p in mod.parameters(recurse=False):
            add(p)
    for layer in stack.layers:
        if hasattr(layer, "linear_attn"):
            m = layer.linear_attn
            total += 2 * m.num_v_heads * m.head_k_dim * m.head_v_dim * 4
            total += 2 * m.conv_dim * m.conv_kernel_size * 2
        else:
            a = layer.self_attn
            kv = a.config.num_key_value_heads * a.head_dim * 2
            total += int(2 * kv * context) + 2 * kv
    return total


def kernel_table(dev) -> dict:
    """Benchmark configs 1-4 as individual launches, rotating distinct buffers.

    Every record also carries its latency floor: ``read_floor_us``, a plain
    streaming read of the record's algorithmic bytes (the faster of
    ``stream_read``'s persistent grid and its one-round grid, which requests
    every byte at once), graph-timed over rotating buffers the same way;
    ``launch_floor_us``, a launch of an empty-work kernel in a graph (one
    16-byte zero fill); ``floor_us`` = the read plus one empty launch for
    every further dependent launch of the record; ``frac_of_floor`` =
    floor_us / us."""
    import torch

    from ppu_amd import kernels as K

    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(20260819)
    out = {}

    def nbuf(nbytes):
        return max(2, (640 << 20) // nbytes + 1)

    tiny = torch.zeros(4, device=dev, dtype=torch.int32)
    launch_us = graph_time_us(lambda i: K.zero_tensors([tiny]), calls=64, reps=10)
    floors: dict[int, float] = {}

    def read_floor(nbytes):
        nbytes = (nbytes + 15) // 16 * 16
        if nbytes not in floors:
            n = nbuf(nbytes)
            bufs = [torch.empty(nbytes, device=dev, dtype=torch.uint8) for _ in range(n)]
            floors[nbytes] = min(
                graph_time_us(lambda i: K.stream_read(bufs[i % n], one_round=r), calls=n, reps=4)
                for r in (False, True))
            del bufs
        return floors[nbytes]

    recorded = []

    def rec(name, us, nbytes, launches=1):
        gbs = nbytes / us / 1e3
        out[name] = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 3)}
        recorded.append((name, us, nbytes, launches))
        log(f"  {name}: {us:.2f} us  {gbs:.0f} GB/s  ({100 * gbs / PEAK_HBM_GBS:.1f}% of 8 TB/s)")

    # config 1: residual add + RMSNorm + GEMV [6144, 2048]
    n = nbuf(6144 * 2048 * 2)
    Ws = [(torch.randn(6144, 2048, device=dev, generator=g) * 0.02).to(bf) for _ in range(n)]
    x = torch.randn(1, 2048, device=dev, generator=g).to(bf)
    r = torch.randn(1, 2048, device=dev, generator=g).to(bf)
    nw = (torch.randn(2048, device=dev, generator=g) * 0.02 + 1).to(bf)
    us = graph_time_us(lambda i: K.residual_norm_linear(r, x, nw, 1e-6, Ws[i % n]), calls=n, reps=4)
    rec("cfg1_resnorm_gemv_6144x2048", us, 25_198_592)
    del Ws
    # config 2: A8W8 GEMV, M = 1, 4, 16
    for (nn, kk) in ((12288, 2048), (2048, 6144)):
        n = nbuf(nn * kk)
        Wq = [torch.randint(-127, 128, (nn, kk), device=dev, generator=g, dtype=torch.int8)
              for _ in range(n)]
        sw = torch.rand(nn, 1, device=dev, generator=g) * 1e-3
        for m in (1, 4, 16):
            xm = torch.randn(m, kk, device=dev, generator=g).to(bf)
            us = graph_time_us(lambda i: K.a8w8_linear(xm, Wq[i % n], sw), calls=n, reps=4)
            rec(f"cfg2_a8w8_{nn}x{kk}_m{m}", us, nn * kk + 4 * nn + 2 * kk * m + 2 * nn * m)
        del Wq
    # config 3: GQA decode attention (8 q / 2 kv heads, D 256)
    for ctx in (512, 2048, 8192):
        n = nbuf(2 * 2 * ctx * 256 * 2)
        Kc = [torch.randn(1, 2, ctx, 256, device=dev, generator=g).to(bf) for _ in range(n)]
        Vc = [torch.randn(1, 2, ctx, 256, device=dev, generator=g).to(bf) for _ in range(n)]
        q = torch.randn(1, 8, 1, 256, device=dev, generator=g).to(bf)
        ln = torch.tensor(ctx, device=dev, dtype=torch.int64)
        us = graph_time_us(lambda i: K.gqa_decode_attention(q, Kc[i % n], Vc[i % n], ln, 1 / 16),
                           calls=n, reps=4)
        rec(f"cfg3_gqa_decode_L{ctx}", us, 2048 * ctx + 8192, launches=2)
        del Kc, Vc
    # config 4: one decode token of a DeltaNet layer through the kernels the
    # model runs (conv update, the 256-wave delta step, packed gated norm),
    # and the delta step alone
    n = nbuf(16 * 128 * 128 * 4)
    St = [torch.randn(1, 16, 128, 128, device=dev, generator=g) * 0.1 for _ in range(n)]
    packed = torch.randn(1, 1, 8320, device=dev, generator=g).to(bf)
    cw = (torch.randn(6144, 4, device=dev, generator=g) * 0.02).to(bf)
    cs = torch.zeros(1, 6144, 4, device=dev, dtype=bf)
    z16 = torch.zeros(16, device=dev, dtype=bf)
    gw = torch.ones(128, device=dev, dtype=bf)

    def chain(i):
        qkv = K.causal_conv1d_fused(packed, cw, cs)
        core = K.delta_recurrent_fused(qkv, packed, z16, z16, St[i % n])
        return K.gated_rms_norm_packed(core.reshape(-1, 128), packed, 6144, 16, gw, 1e-6)

    us = graph_time_us(chain, calls=n, reps=4)
    rec("cfg4_delta_decode_chain_3_launches", us, 2_265_216, launches=3)
    qkv = K.causal_conv1d_fused(packed, cw, cs)
    us = graph_time_us(lambda i: K.delta_recurrent_fused(qkv, packed, z16, z16, St[i % n]),
                       calls=n, reps=4)
    rec("cfg4_delta_step_kernel", us, 2 * 16 * 128 * 128 * 4 + 6144 * 2 + 64 + 4096)
    del St
    # The floors are measured after every config: allocating their rotating
    # buffers (even without touching them) left the later skinny A8W8
    # launches ~0.8 us slower for the rest of the process, on the same
    # weights, inputs and outputs.
    torch.cuda.empty_cache()
    for name, us, nbytes, launches in recorded:
        rf = read_floor(nbytes)
        floor = rf + (launches - 1) * launch_us
        out[name].update({"launches": launches, "read_floor_us": round(rf, 2),
                          "launch_floor_us": round(launch_us, 2), "floor_us": round(floor, 2),
                          "frac_of_floor": round(floor / us, 3)})
        log(f"  {name}: floor {floor:.2f} us ({launches} launch(es): read {rf:.2f} + empty launch "
            f"{launch_us:.2f}) = {100 * floor / us:.0f}% of the time")
    return out


def gemm_sweep(dev, quick: bool = False) -> None:
    """The prefill GEMM shapes of the 2B decoder at M = 1024: the ROCm library
    (F.linear bf16, + silu_and_mul for the packed gate/up; torch._int_mm + the
    dequant kernel for int8) against the hand-written matrix-core GEMM
    (q35_gemm) for its default plan and the other tile plans, each
    graph-timed over rotating weights (>= 512 MB, so the MALL does not serve
    them). Prints one table row per (shape, implementation, plan) on stdout.
    ``quick``: the default plans only."""
    import torch
    import torch.nn.functional as F

    from ppu_amd import _lib
    from ppu_amd import kernels as K

    g = torch.Generator(device=dev).manual_seed(1)
    m = PROMPT_LEN
    stream = torch.cuda.current_stream().cuda_stream
    # (N, K, count per prefill, packed SwiGLU)
    shapes = [(8320, 2048, 18, False), (2048, 2048, 24, False), (5120, 2048, 6, False),
              (12288, 2048, 24, True), (2048, 6144, 24, False)]
    stage = {t: 128 for t in range(9)}
    print("# N x K (per prefill) | implementation | plan (tile, K splits) | us | TFLOP/s (TOP/s)")
    for n, k, count, swiglu in shapes:
        flops = 2 * m * n * k

        nset = max(2, (512 << 20) // (n * k * 2) + 1)
        w = [(torch.randn(n, k, device=dev, generator=g) * 0.02).to(torch.bfloat16) for _ in range(nset)]
        x = torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16)

        def row(impl, plan, us):
            print(f"{n} x {k} ({count}) | {impl} | {plan} | {us:.2f} | {flops / us / 1e6:.0f}",
                  flush=True)

        if swiglu:
            row("library bf16 (F.linear) + silu_and_mul", "-",
                graph_time_us(lambda i: K.silu_and_mul(F.linear(x, w[i % nset])), nset, 5))
        row("library bf16 (F.linear)", "-", graph_time_us(lambda i: F.linear(x, w[i % nset]), nset, 5))
        plans = [None] if quick else [None, (0, 1), (5, 1), (1, 1), (6, 1), (7, 1), (8, 1), (2, 1), (3, 1), (6, 2), (7, 2)]
        for plan in plans:
            if plan and ((2 * k // stage[plan[0]]) % plan[1] or (swiglu and plan[1] > 1)):
                continue
            if swiglu and (plan is None or plan[0] not in (5, 6, 7, 8)):
                us = graph_time_us(lambda i: K.gemm_bf16(x, w[i % nset], swiglu=True, plan=plan), nset, 5)
                row("own bf16 + SwiGLU epilogue (q35_gemm kind 1)", plan or "default plan", us)
            us = graph_time_us(lambda i: K.gemm_bf16(x, w[i % nset], plan=plan), nset, 5)
            row("own bf16 (q35_gemm kind 0)", plan or "default plan", us)
        del w
        nset8 = max(2, (512 << 20) // (n * k) + 1)
        wq = [torch.randint(-127, 128, (n, k), device=dev, dtype=torch.int8, generator=g)
              for _ in range(nset8)]
        sw = torch.rand(n, device=dev, generator=g) * 1e-3
        xq, sx = K.quantize_act_i8(x)
        y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
        acc = torch.empty(m, n, device=dev, dtype=torch.int32)

        def lib_i8(i):
            a = torch._int_mm(xq, wq[i % nset8].t())
            _lib.call("q35_dequant_i32", a.data_ptr(), sx.data_ptr(), sw.data_ptr(), y.data_ptr(),
                      m, n, stream)

        row("library int8 (_int_mm)", "-", graph_time_us(lambda i: torch._int_mm(xq, wq[i % nset8].t()),
                                                        nset8, 5))
        row("library int8 (_int_mm) + dequant", "-", graph_time_us(lib_i8, nset8, 5))
        plans = [None] if quick else [None, (0, 1), (5, 1), (1, 1), (6, 1), (7, 1), (8, 1), (2, 1), (3, 1), (6, 2), (7, 2)]
        for plan in plans:
            if plan and (k // stage[plan[0]]) % plan[1]:
                continue
            us = graph_time_us(lambda i: K.gemm_into(xq, wq[i % nset8], acc, K.GEMM_I32, plan=plan),
                               nset8, 5)
            row("own int8 -> int32 (q35_gemm kind 2)", plan or "default plan", us)
            if plan is not None and plan[0] in (5, 6, 7, 8):
                continue
            us = graph_time_us(lambda i: K.gemm_a8w8(xq, sx, wq[i % nset8], sw, plan=plan), nset8, 5)
            row("own int8 + fused dequant (q35_gemm kind 3)", plan or "default plan", us)
        del wq
        torch.cuda.empty_cache()


def counter_probe(dev) -> None:
    """A short fixed workload for ``rocprofv3 --pmc`` passes (one counter set
    per run), so that per-dispatch counters can be read for:

    * 5 calibration launches of a plain elementwise kernel (``neg``) that reads
      exactly 1 GiB and writes exactly 1 GiB, the yardstick that turns the
      FETCH_SIZE / WRITE_SIZE counters into bytes;
    * 5 launches of the lm_head GEMV + top-1 on a [248320, 2048] bf16 weight,
      then 5 of the screened top-1 (int8 screen + exact rescore) on it;
    * 4 replays of the captured decode step of the seeded 2B decoder (bf16
      linears, 1024-token context): every decode kernel with its real
      weights, 129 dispatches per replay;
    * 16 standalone launches of the delta-rule decode step over rotating
      states, as config 4 times it (fp32 gate parameters, so the kernel is
      the ``<true>`` instance and its rows stay apart from the step's);
    * 3 launches of each prefill GEMM of the product path (M = 1024 tokens,
      the hand-written matrix-core kernels: bf16 plain and SwiGLU, int8 with
      the dequant epilogue), for MFMA counters.
    """
    import torch

    from ppu_amd import kernels as K
    from ppu_amd import synth
    from ppu_amd.graph import GreedyDecodeGraph
    from ppu_amd.integration import apply_fusions

    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(20260819)
    src = torch.randn(1 << 28, device=dev, generator=g)  # 2^28 fp32 = 1 GiB
    dst = torch.empty_like(src)
    for _ in range(5):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    w = (torch.randn(248320, 2048, device=dev, generator=g) * 0.02).to(bf)
    h = torch.randn(1, 2048, device=dev, generator=g).to(bf)
    for _ in range(5):
        K.lm_head_argmax(h, w)
    screen = K.lm_head_screen_prep(w)
    for _ in range(5):
        K.lm_head_argmax(h, w, screen=screen)
    torch.cuda.synchronize()
    _, rows = K.lm_head_argmax(h, w, screen=screen, return_candidates=True)
    log(f"counter probe: the screened top-1 rescored {int(rows)} rows")
    del w, screen
    log("counter probe: calibration + lm_head done; decode step ...")
    cfg = synth.config_2b()
    model = synth.build_model(cfg, device=dev)
    apply_fusions(model)
    from transformers.cache_utils import StaticCache

    prompt = synth.prompt_ids(PROMPT_LEN, cfg.vocab_size).to(dev)
    with torch.inference_mode():
        cache = StaticCache(config=cfg, max_cache_len=1152)
        pos = torch.arange(PROMPT_LEN, device=dev).view(1, -1)
        out = model.model(input_ids=prompt, position_ids=pos, past_key_values=cache, use_cache=True)
        tok = K.lm_head_argmax(out.last_hidden_state[:, -1].contiguous(), model.lm_head.weight)
        graph = GreedyDecodeGraph(model, cache, tok, torch.full((1, 1), PROMPT_LEN, device=dev,
                                                                dtype=torch.long))
        for _ in range(4):
            graph.replay()
        torch.cuda.synchronize()
    del graph, cache, model
    torch.cuda.empty_cache()
    log("counter probe: decode step done; standalone delta step ...")
    states = [torch.randn(1, 16, 128, 128, device=dev, generator=g) * 0.1 for _ in range(16)]
    packed = torch.randn(1, 1, 8320, device=dev, generator=g).to(bf)
    qkv = torch.randn(1, 1, 6144, device=dev, generator=g).to(bf)
    z16 = torch.zeros(16, device=dev)
    for st in states:
        K.delta_recurrent_fused(qkv, packed, z16, z16, st)
    torch.cuda.synchronize()
    del states
    log("counter probe: delta step done; prefill GEMMs ...")
    for (n, k, swiglu) in PROBE_GEMMS:
        x = torch.randn(1024, k, device=dev, generator=g).to(bf)
        wt = (torch.randn(n, k, device=dev, generator=g) * 0.02).to(bf)
        xq, sx = K.quantize_act_i8(x)
        wq, sw = K.quantize_weight_i8(wt)
        for _ in range(3):
            K.gemm_bf16(x, wt, swiglu=swiglu)
        for _ in range(3):
            K.gemm_a8w8(xq, sx, wq, sw.reshape(-1), swiglu=swiglu)
    torch.cuda.synchronize()
    log("counter probe done")


# Algorithmic bytes per launch of the decode-step kernels (2B shape, bf16,
# 1024-token context), by the kernel names rocprofv3 reports.
DECODE_ALGO_BYTES = {
    "gemv_fused<4, 2, 4, 2, 1, false>": 2 * 6144 * 2048 * 2 + 4 * 2048 * 2 + 6144 * 2,
    "gemv_fused<4, 1, 12, 0, 0, false>": 2048 * 6144 * 2 + 6144 * 2 + 2048 * 2,
    "gemv_fused<4, 2, 4, 2, 3, false>": 8320 * 2048 * 2 + 4 * 2048 * 2 + 8320 * 2
    + 6144 * 4 * 2 * 3 + 6144 * 2,
    "gemv_fused<4, 2, 4, 3, 0, false>": 2048 * 2048 * 2 + 2 * 2048 * 2 + 128 * 2 + 2048 * 2,
    "gemv_fused<4, 2, 4, 2, 0, false>": 5120 * 2048 * 2 + 4 * 2048 * 2 + 5120 * 2,
    "gemv_fused<4, 2, 4, 0, 0, false>": 2048 * 2048 * 2 + 2 * 2048 * 2,
    "delta_decode_wave<false>": 2 * 16 * 128 * 128 * 4 + 6144 * 2 + 64 + 16 * 128 * 2,
    "delta_decode_wave<true>": 2 * 16 * 128 * 128 * 4 + 6144 * 2 + 64 * 2 + 16 * 128 * 2,
    "lm_head_top1_persist<4, 1, 4>": 248320 * 2048 * 2 + 2048 * 2 + 8,
    # int8 copy, per-row scale and bound factor read, per-row upper bound written
    "lm_head_screen<4, 2, 2>": 248320 * 2048 + 248320 * 12 + 2048 * 2,
    # K/V over the ~1026 cached tokens of the probe's replays, the packed row,
    # the new K/V cache row (the per-split partials are the design's overhead)
    "gqa_decode_split<4, true>": 2 * 2 * 1026 * 256 * 2 + 5120 * 2 + 2 * 2 * 256 * 2,
    # 8 heads x 36 splits of (acc[256], m, l), the gate row, the bf16 output
    "gqa_decode_combine<4>": 8 * 36 * 258 * 4 + 2048 * 2 + 2048 * 2,
}
# The rescore reads the per-row upper bounds and the bf16 rows of its
# candidates (4 KiB each): its algorithmic bytes need the candidate count.
RESCORE_NAME = "lm_head_rescore<4>"


def trace_summary(kind: str, trace_csv: str, bench_json: str) -> None:
    """Print the per-kernel anatomy of a ``rocprofv3 --kernel-trace`` run of
    ``bench.py --no-cpu --no-kernels``: ``decode`` = one graph-replayed decode
    step per linear variant (the second-to-last replay of each), ``prefill``
    = one warm prefill + first token per variant (the last of each); with the
    unprofiled figures of the same run's JSON line."""
    import collections
    import csv
    import re

    d = json.loads(Path(bench_json).read_text().strip().splitlines()[-1])
    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))

    def short(n):
        n = n.replace("(anonymous namespace)::", "").replace("void ", "")
        m = re.match(r"([\w:]+)(<[^(]*>)?", n)
        return ((m.group(1).split("::")[-1] + (m.group(2) or "")) if m else n)[:58]

    def dur(r):
        return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3

    def int8(a, b):
        # int8 GEMV (last template argument true) or an int8 kind (>= 2) of
        # the prefill GEMM (seventh template argument)
        def is_i8(name):
            m = re.search(r"gemm_ring<(?:\s*\d+,){7}\s*\w+,\s*(\d+),", name)
            return ("gemv_fused" in name and ", true>" in name) or (m is not None and int(m.group(1)) >= 2)
        return any(is_i8(rows[i]["Kernel_Name"]) for i in range(a, b))

    def table(seg, grid, top=None):
        t0, t1 = int(seg[0]["Start_Timestamp"]), int(seg[-1]["End_Timestamp"])
        agg = collections.OrderedDict()
        for r in seg:
            k = short(r["Kernel_Name"]) + (f" g{r['Grid_Size_X']}" if grid else "")
            x = agg.setdefault(k, [0, 0.0])
            x[0] += 1
            x[1] += dur(r)
        busy = sum(v[1] for v in agg.values())
        out = [f"#   {len(seg)} kernels, wall {(t1 - t0) / 1e3:.1f} us, sum of kernel durations {busy:.1f} us"]
        items = sorted(agg.items(), key=lambda kv: -kv[1][1])
        for k, (n, t) in items[:top] if top else items:
            out.append(f"#   {k:72s} n={n:3d} total {t:8.1f} us  avg {t / n:7.2f} us")
        return out

    # a greedy token ends with top1_final, or with the rescore of the screened
    # top-1 (which reduces the candidates itself)
    ends = [i for i, r in enumerate(rows)
            if "top1_final" in r["Kernel_Name"] or "lm_head_rescore" in r["Kernel_Name"]]
    v = d.get("variants", {}).get("a8w8", {})
    lines = []
    if kind == "vision":
        # one fused tower call starts with the patch-embedding GEMM right
        # before its position-embedding add; the last call ends the trace of
        # `bench.py --vision-only`
        starts = [i for i, r in enumerate(rows) if "position_embed_add_rows" in r["Kernel_Name"]]
        gemms = [i for i, r in enumerate(rows) if r["Kernel_Name"].startswith("Cijk")]
        if starts and gemms:
            # ... and ends with the merger's second GEMM and the two output copies
            a, b = max(starts[-1] - 1, 0), gemms[-1] + 1
            while b < len(rows) and b <= gemms[-1] + 2 and "copyBuffer" in rows[b]["Kernel_Name"]:
                b += 1
            lines.append("# fused vision tower, one 784-patch image (the last graph replay in the trace):")
            lines += table(rows[a:b], True)
            lines.append("#")
        vt = d.get("vision_tower", d)
        lines.append(f"# bench.py JSON given ({Path(bench_json).name}): Transformers forward "
                     f"{vt.get('transformers_ms')} ms, fused forward {vt.get('fused_graph_ms')} ms per call, "
                     f"pooled output {vt.get('pooler_rel_l2_vs_transformers')} relative L2 from Transformers.")
        print("\n".join(lines))
        return
    if kind == "decode":
        steps = [(a + 1, b + 1) for a, b in zip(ends, ends[1:]) if 60 < b - a < 400]
        for name, pick in (("bf16", False), ("A8W8", True)):
            sel = [s for s in steps if int8(*s) == pick]
            if len(sel) >= 2:
                lines.append(f"# {name} decode step (second-to-last {name} replay in the trace):")
                lines += table(rows[sel[-2][0]:sel[-2][1]], True)
                lines.append("#")
    else:
        preps = [i for i, r in enumerate(rows) if "delta_chunk_prep" in r["Kernel_Name"]]
        wins = []
        for k in range(0, len(preps), 18):
            w = preps[k:k + 18]
            a = max([e for e in ends if e < w[0]], default=-1) + 1
            b = min([e for e in ends if e > w[-1]], default=len(rows) - 1) + 1
            # a generate() prefill: its first top-1 (the screened one, when the
            # model has it) follows the prefill directly, with no decode GEMV
            # in between as in the bench's separate eager setup
            tail = [rows[i]["Kernel_Name"] for i in range(w[-1], b)]
            if not any("gemv_fused" in n for n in tail) and (
                    any("lm_head_screen" in n for n in tail) or not any(
                        "lm_head_screen" in r["Kernel_Name"] for r in rows)):
                wins.append((a, b))
        for name, pick in (("bf16", False), ("A8W8", True)):
            sel = [w for w in wins if int8(*w) == pick]
            # the graph-replayed prefills are the variant's most frequent
            # window length (the eager TTFT timing launches more kernels)
            mode = collections.Counter(b - a for a, b in sel).most_common(1)
            sel = [w for w in sel if w[1] - w[0] == mode[0][0]] if mode else []
            if sel:
                lines.append(f"# {name}: one warm graph-replayed prefill (1024 tokens) + first token, the last in the trace:")
                lines += table(rows[sel[-1][0]:sel[-1][1]], False, top=24)
                lines.append("#")
    lines.append(f"# bench.py JSON given ({Path(bench_json).name}): bf16 decode {d['ms_per_step']} ms/token = "
                 f"{d['value']} tok/s (graph replay alone {d['graph_replay_ms']} ms), TTFT {d['ttft_ms']} ms;")
    if v:
        lines.append(f"#   A8W8 decode {v.get('ms_per_step')} ms/token = {v.get('value')} tok/s "
                     f"(replay {v.get('graph_replay_ms')} ms), TTFT {v.get('ttft_ms')} ms.")
    print("\n".join(lines))


def pmc_summary(fetch_csv: str, write_csv: str, rescore_rows: int | None = None) -> None:
    """Print the HBM-traffic summary of two ``rocprofv3 --pmc`` runs of
    ``--counter-probe`` (FETCH_SIZE, then WRITE_SIZE; their
    ``*_counter_collection.csv`` files): mean KiB per dispatch per kernel,
    scaled by what the counters read for the 1 GiB in / 1 GiB out ``neg``
    calibration kernel, against the kernel's algorithmic bytes."""
    import csv
    from collections import defaultdict

    def load(path, counter):
        per, raw_names = defaultdict(list), {}
        with open(path) as f:
            for row in csv.DictReader(f):
                if row.get("Counter_Name", counter) != counter:
                    continue
                raw = row["Kernel_Name"].replace("(anonymous namespace)::", "")
                raw = raw[5:] if raw.startswith("void ") else raw
                name = raw.split("(")[0].strip()
                per[name].append(float(row["Counter_Value"]))
                raw_names[name] = raw
        return {k: sum(v) / len(v) for k, v in per.items()}, raw_names

    (fetch, raw), (write, _) = load(fetch_csv, "FETCH_SIZE"), load(write_csv, "WRITE_SIZE")
    neg = [k for k in fetch if "neg_kernel" in raw[k]]
    if not neg:
        raise SystemExit("no calibration (neg) kernel in the FETCH_SIZE run")
    f_scale = (1 << 20) / fetch[neg[0]]
    w_scale = (1 << 20) / write[neg[0]]
    print(f"calibration kernel {neg[0]}: FETCH_SIZE {fetch[neg[0]]:.1f} KiB, WRITE_SIZE "
          f"{write[neg[0]]:.1f} KiB per dispatch for 1 GiB in / 1 GiB out -> scale "
          f"fetch x{f_scale:.4f}, write x{w_scale:.4f}")
    print("kernel | fetch KiB | write KiB | traffic bytes per launch | algorithmic bytes | ratio")
    for name in sorted(fetch, key=lambda k: -fetch[k]):
        if name not in write:
            continue
        traffic = int((fetch[name] * f_scale + write[name] * w_scale) * 1024)
        algo = DECODE_ALGO_BYTES.get(name)
        if name == RESCORE_NAME and rescore_rows is not None:
            algo = 248320 * 4 + rescore_rows * 2048 * 2 + 2048 * 2
        ratio = f"{traffic / algo:.4f}" if algo else "-"
        print(f"{name} | {fetch[name]:.1f} | {write[name]:.1f} | {traffic} | {algo or '-'} | {ratio}")


# The prefill GEMM launches of --counter-probe, in program order: per shape
# (N, K, SwiGLU), 3 bf16 launches then 3 int8 launches.
PROBE_GEMMS = ((8320, 2048, False), (2048, 2048, False), (5120, 2048, False), (12288, 2048, True),
               (2048, 6144, False))


def mfma_summary(pmc_csv: str, trace_csv: str) -> None:
    """Print the matrix-core use of the prefill GEMMs of a ``--counter-probe``
    run: one ``rocprofv3 --pmc SQ_INSTS_VALU_MFMA_MOPS_BF16
    SQ_INSTS_VALU_MFMA_MOPS_I8 SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE`` pass
    and one ``--kernel-trace`` pass. The GEMM dispatches of both runs are taken
    in program order and labelled with the probe's shapes (PROBE_GEMMS):
    operations = MOPS x 512, MFMA busy = busy cycles / (GRBM_GUI_ACTIVE / 8
    XCDs x 1024 SIMDs)."""
    import csv
    from collections import defaultdict

    def short(name):
        n = name.replace("(anonymous namespace)::", "")
        return (n[5:] if n.startswith("void ") else n).split("(")[0].strip()

    per = defaultdict(dict)
    names = {}
    with open(pmc_csv) as f:
        for row in csv.DictReader(f):
            if "gemm_ring" in row["Kernel_Name"]:
                d = int(row["Dispatch_Id"])
                per[d][row["Counter_Name"]] = float(row["Counter_Value"])
                names[d] = short(row["Kernel_Name"])
    cnt = [(names[d], per[d]) for d in sorted(per)]
    with open(trace_csv) as f:
        rows = [r for r in csv.DictReader(f) if "gemm_ring" in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    dur = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rows]
    labels = [f"{n}x{k}{' SwiGLU' if sw else ''} {kind}" for n, k, sw in PROBE_GEMMS
              for kind in ("bf16", "int8") for _ in range(3)]
    # the probe's GEMM phase comes last (the model's own prefill GEMMs before it)
    if len(cnt) < len(labels) or len(dur) < len(labels):
        raise SystemExit(f"expected {len(labels)} GEMM dispatches, got {len(cnt)} counted / {len(dur)} traced")
    cnt, dur = cnt[-len(labels):], dur[-len(labels):]
    print("shape (M = 1024) | kernel | T(FL)OPs per launch | us | T(FL)OP/s | of dense peak | MFMA busy")
    for i in range(0, len(labels), 3):
        name = cnt[i][0]
        mean = {c: sum(cnt[j][1].get(c, 0.0) for j in range(i, i + 3)) / 3 for c in cnt[i][1]}
        i8 = "int8" in labels[i]
        ops = 512 * mean.get("SQ_INSTS_VALU_MFMA_MOPS_I8" if i8 else "SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0)
        us = sum(dur[i:i + 3]) / 3
        peak = 5000.0 if i8 else 2500.0
        active = mean.get("GRBM_GUI_ACTIVE", 0.0) / 8
        busy = mean.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (active * 1024) if active else float("nan")
        rate = ops / us / 1e6
        print(f"{labels[i]} | {name} | {ops / 1e12:.4f} | {us:.2f} | {rate:.1f} | {rate / peak:.3f} | {busy:.3f}")


def cpu_baseline(state, cfg, prompt, decode_steps: int, eager: bool = True) -> dict:
    """The reference's PyTorch CPU path on the host cores, on the config-5
    prompt: the oracle decoder (the reference's fused data flow restated,
    ``kind: port``) prefills the whole prompt and decodes ``decode_steps``
    greedy tokens; beside it Transformers' own eager Qwen3.5 forward, which
    the reference runs for CPU tensors (integration.py:51-52), on the same
    weights and thread count (prefill, then cached decode steps)."""
    import torch

    from oracle.model import OracleDecoder

    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch.set_num_threads(threads)
    oracle = OracleDecoder(state, cfg)
    cache = oracle.new_cache(prompt.shape[1] + decode_steps + 8)
    t0 = time.perf_counter()
    h = oracle.forward(prompt, cache)
    tok, _ = oracle.top1(h[:, -1])
    ttft = time.perf_counter() - t0
    tokens = [tok]
    t1 = time.perf_counter()
    for _ in range(decode_steps):
        h = oracle.forward(torch.tensor([[tok]]), cache)
        tok, _ = oracle.top1(h[:, -1])
        tokens.append(tok)
    dt = time.perf_counter() - t1
    del oracle, cache
    out = {"value": round(decode_steps / dt, 3), "unit": "tokens/s", "cores": torch.get_num_threads(),
           "kind": "port", "ttft_ms": round(ttft * 1e3, 1),
           "sample": f"oracle decoder (torch CPU, same seeded weights): prefill of the full "
                     f"{prompt.shape[1]}-token config-5 prompt, then {decode_steps} greedy decode "
                     f"steps (of the 64 the GPU workload decodes)",
           "cpu_model": _cpu_model()}
    log(f"CPU oracle: TTFT {ttft * 1e3:.0f} ms, decode {decode_steps / dt:.2f} tok/s on "
        f"{threads} threads; tokens {tokens[:6]}")
    if not eager:
        return out
    # The headline CPU figure is the reference's own CPU path, Transformers'
    # eager forward (integration.py:51-52 runs it for CPU tensors); the
    # oracle port is kept beside it.
    ref = _eager_cpu(state, cfg, prompt, decode_steps)
    ref.update(kind="reference", cpu_model=out["cpu_model"], port=out)
    return ref


def cpu_kernel_table() -> dict:
    """Benchmark configs 1-4 on the host cores through the oracle's
    restatement of the reference's CPU arithmetic (torch / numpy on the same
    threads as the config-5 leg): the median time per call over a few calls
    and the algorithmic bytes of the GPU table over it. Config 2's int8
    product is numpy's exact int64 matmul; config 4 is one token of the
    model's chain (conv update, delta step, gated norm), timed over 64
    sequential tokens."""
    import statistics

    import numpy as np
    import torch

    from oracle import a8w8 as oa
    from oracle import ops as oo

    g = torch.Generator().manual_seed(20260819)
    bf = torch.bfloat16
    out = {}

    def timed(fn, reps):
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts) * 1e6

    def rec(name, us, nbytes):
        out[name] = {"us": round(us, 1), "GB/s": round(nbytes / us / 1e3, 2)}

    w = (torch.randn(6144, 2048, generator=g) * 0.02).to(bf)
    x, r = torch.randn(1, 2048, generator=g).to(bf), torch.randn(1, 2048, generator=g).to(bf)
    nw = (torch.randn(2048, generator=g) * 0.02 + 1).to(bf)
    rec("cfg1_resnorm_gemv_6144x2048",
        timed(lambda: oo.linear(oo.residual_add_rms_norm(r, x, nw, 1e-6)[1], w), 5), 25_198_592)
    for nn, kk in ((12288, 2048), (2048, 6144)):
        wq, sw = oa.quantize_weight((torch.randn(nn, kk, generator=g) * 0.02).to(bf))
        for m in (1, 4, 16):
            xm = torch.randn(m, kk, generator=g).to(bf)
            rec(f"cfg2_a8w8_{nn}x{kk}_m{m}", timed(lambda: oa.a8w8_linear(xm, wq, sw), 3),
                nn * kk + 4 * nn + 2 * kk * m + 2 * nn * m)
    for ctx in (512, 2048, 8192):
        kc = torch.randn(1, 2, ctx, 256, generator=g).to(bf)
        vc = torch.randn(1, 2, ctx, 256, generator=g).to(bf)
        q = torch.randn(1, 8, 1, 256, generator=g).to(bf)
        rec(f"cfg3_gqa_decode_L{ctx}", timed(lambda: oo.gqa_decode_attention(q, kc, vc, ctx, 1 / 16), 3),
            2048 * ctx + 8192)
    state = torch.randn(1, 16, 128, 128, generator=g) * 0.1
    cw = (torch.randn(6144, 4, generator=g) * 0.02).to(bf)
    cs = torch.zeros(1, 6144, 4, dtype=bf)
    z16 = torch.zeros(16, dtype=bf)
    gw = torch.ones(128, dtype=bf)
    toks = [torch.randn(1, 1, 8320, generator=g).to(bf) for _ in range(64)]

    def chain():
        for packed in toks:
            qkv = oo.causal_conv1d(packed, cw, cs)
            core = oo.delta_recurrent(qkv, packed, z16, z16, state)
            z = packed[..., 6144:8192].reshape(16, 128)
            oo.gated_rms_norm(core.reshape(16, 128), z, gw, 1e-6)

    rec("cfg4_delta_decode_chain_per_token", timed(chain, 1) / 64, 2_265_216)
    log("CPU configs 1-4 (oracle ops): " + ", ".join(f"{k} {v['us']} us" for k, v in out.items()))
    return out


def _eager_cpu(state, cfg, prompt, decode_steps: int) -> dict:
    import torch
    from transformers.cache_utils import DynamicCache
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5ForCausalLM

    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("meta"):
            model = Qwen3_5ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(old)
    model.load_state_dict(state, assign=True, strict=False)
    model.tie_weights()
    rot = model.model.rotary_emb
    inv_freq, _ = rot.compute_default_rope_parameters(cfg, "cpu")
    rot.inv_freq = inv_freq
    rot.original_inv_freq = inv_freq
    model.eval()
    with torch.inference_mode():
        cache = DynamicCache(config=cfg)
        t0 = time.perf_counter()
        out = model(input_ids=prompt, past_key_values=cache, use_cache=True, logits_to_keep=1)
        tok = int(out.logits[0, -1].argmax())
        ttft = time.perf_counter() - t0
        tokens = [tok]
        t1 = time.perf_counter()
        for _ in range(decode_steps):
            out = model(input_ids=torch.tensor([[tok]]), past_key_values=cache, use_cache=True,
                        logits_to_keep=1)
            tok = int(out.logits[0, -1].argmax())
            tokens.append(tok)
        dt = time.perf_counter() - t1
    log(f"CPU Transformers eager: TTFT {ttft * 1e3:.0f} ms, decode {decode_steps / dt:.2f} tok/s; "
        f"tokens {tokens[:6]}")
    return {"value": round(decode_steps / dt, 3), "unit": "tokens/s", "ttft_ms": round(ttft * 1e3, 1),
            "cores": torch.get_num_threads(),
            "sample": f"Transformers 5.15 eager Qwen3_5ForCausalLM (bf16, CPU, DynamicCache), same "
                      f"weights: {prompt.shape[1]}-token prefill, then {decode_steps} greedy steps"}


def _digest_report(digests: dict) -> dict:
    """The run's input digests and whether they equal the committed ones."""
    try:
        golden = json.loads((ROOT / "tests" / "golden" / "digests.json").read_text())
    except (OSError, ValueError):
        golden = {}
    out = dict(digests)
    if "prompt" in digests:
        out["prompt_matches_golden"] = digests["prompt"] == golden.get("prompt_1024")
    if "weights" in digests:
        out["weights_match_golden"] = digests["weights"] == golden.get("weights_2b")
    return out


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def vision_tower_timing(dev) -> dict:
    """The vision tower (Transformers' default Qwen3.5 vision config: 27 blocks,
    1152 wide, 16 heads) on one 448x448 image (28x28 patches), seeded random
    bf16 weights: Transformers' own forward against the fused forward (eager
    first call, then the captured graph), and their output difference."""
    import torch
    from transformers.models.qwen3_5 import modeling_qwen3_5 as impl
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5VisionConfig
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from ppu_amd import integration

    cfg = Qwen3_5VisionConfig()
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(20260625)
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        tower = impl.Qwen3_5VisionModel(cfg)
    finally:
        torch.set_default_dtype(old)
    hd = cfg.hidden_size // cfg.num_heads // 2
    tower.rotary_pos_emb.inv_freq = 1.0 / (10000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    tower = tower.to(dev).eval()
    grid = torch.tensor([[1, 28, 28]], device=dev)
    pix = torch.randn(784, cfg.in_channels * cfg.temporal_patch_size * cfg.patch_size ** 2,
                      device=dev).to(torch.bfloat16)

    def timed(fn, reps=10):
        fn(); torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            out = fn()
        e1.record(); e1.synchronize()
        return e0.elapsed_time(e1) / reps, out

    with torch.inference_mode(), sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        t_ref, ref = timed(lambda: tower(pix, grid_thw=grid).pooler_output)
        integration.install_vision(tower, integration.FusionConfig())
        t_fused, got = timed(lambda: tower(pix, grid_thw=grid).pooler_output)
    rel = ((got.float() - ref.float()).norm() / ref.float().norm()).item()
    log(f"vision tower 784 patches: Transformers {t_ref:.3f} ms, fused {t_fused:.3f} ms, rel diff {rel:.2e}")
    return {"workload": "Qwen3.5 vision tower (27 x 1152, 16 heads), one 448x448 image (784 patches), bf16",
            "transformers_ms": round(t_ref, 3), "fused_graph_ms": round(t_fused, 3),
            "pooler_rel_l2_vs_transformers": round(rel, 5)}


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--variant", choices=("bf16", "a8w8"), default="bf16")
    ap.add_argument("--no-kernels", action="store_true", help="skip the per-kernel table")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-other-variant", action="store_true",
                    help="skip the second (A8W8 or bf16) decode measurement")
    ap.add_argument("--cpu-decode-steps", type=int, default=16)
    ap.add_argument("--cpu-prompt", type=int, default=PROMPT_LEN, help="prompt length of the CPU sample")
    ap.add_argument("--no-eager", action="store_true", help="skip the Transformers-eager CPU timing")
    ap.add_argument("--no-vision", action="store_true", help="skip the vision-tower timing")
    ap.add_argument("--vision-only", action="store_true",
                    help="only time the vision tower (Transformers vs fused), print its JSON, then exit")
    ap.add_argument("--trace-summary", nargs=3, metavar=("decode|prefill|vision", "TRACE_CSV", "BENCH_JSON"),
                    help="per-kernel anatomy of a rocprofv3 kernel trace of this bench, then exit")
    ap.add_argument("--gemm-sweep", action="store_true",
                    help="prefill GEMM shapes: ROCm library vs the hand-written GEMMs, then exit")
    ap.add_argument("--quick", action="store_true", help="--gemm-sweep: default plans only")
    ap.add_argument("--counter-probe", action="store_true",
                    help="only run the short workload profiled with rocprofv3 --pmc, then exit")
    ap.add_argument("--pmc-summary", nargs="+", metavar="CSV",
                    help="FETCH_CSV WRITE_CSV [RESCORE_ROWS]: print the HBM-traffic table of two "
                         "--counter-probe pmc runs, then exit")
    ap.add_argument("--mfma-summary", nargs=2, metavar=("PMC_CSV", "TRACE_CSV"),
                    help="print the prefill GEMMs' matrix-core use from a --counter-probe pmc run "
                         "and a kernel trace of it, then exit")
    args = ap.parse_args()
    if args.pmc_summary:
        fetch, write, *rows = args.pmc_summary
        pmc_summary(fetch, write, int(rows[0]) if rows else None)
        return
    if args.mfma_summary:
        mfma_summary(*args.mfma_summary)
        return
    if args.trace_summary:
        trace_summary(*args.trace_summary)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (a batch-1 decode step "
              "is bound by per-launch latency, which sharding adds to). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if args.counter_probe:
        counter_probe(torch.device("cuda:0"))
        return
    if args.gemm_sweep:
        gemm_sweep(torch.device("cuda:0"), quick=args.quick)
        return
    if args.vision_only:
        print(json.dumps({"vision_tower": vision_tower_timing(torch.device("cuda:0"))}), flush=True)
        return

    from ppu_amd import synth
    from ppu_amd.generate import FusedGreedyGenerator, cache_bucket
    from ppu_amd.graph import GreedyDecodeGraph, decode_tokens
    from ppu_amd.integration import FusionConfig, apply_fusions
    from ppu_amd.kernels import lm_head_argmax

    dev = torch.device("cuda:0")
    cfg = synth.config_2b()
    prompt_cpu = synth.prompt_ids(PROMPT_LEN, cfg.vocab_size)
    prompt = prompt_cpu.to(dev)
    digests = {"prompt": synth.tensor_sha256(prompt_cpu)}

    def measure(variant: str, keep_state: bool):
        """Build the seeded 2B model with ``variant`` linears, then TTFT through
        the generation loop and K timed decode-graph replays."""
        t0 = time.perf_counter()
        wd = []
        model = synth.build_model(cfg, device=dev, digest=wd if keep_state else None)
        if wd:
            digests["weights"] = wd[0]
        seen, weight_bytes = set(), 0
        for p in model.parameters():
            if p.data_ptr() not in seen:
                seen.add(p.data_ptr())
                weight_bytes += p.numel() * p.element_size()
        state = {k: v.detach().cpu() for k, v in model.state_dict().items()} if keep_state else None
        stats = apply_fusions(model, FusionConfig(a8w8=variant == "a8w8"))
        torch.cuda.synchronize()
        log(f"[{variant}] model built + fused in {time.perf_counter() - t0:.1f} s: {stats}")

        # TTFT and the reference's decode formula through the generation loop.
        runner = FusedGreedyGenerator(model)
        first = runner.generate(prompt, NEW_TOKENS)  # builds cache + captures the graph
        warm = [runner.generate(prompt, NEW_TOKENS) for _ in range(7)]  # median of 7 warm runs
        ttft_ms = statistics.median(r.ttft_seconds for r in warm) * 1e3
        loop_tps = statistics.median(r.decode_tokens_per_second for r in warm)
        assert all(r.tokens == first.tokens for r in warm), "greedy decode is not deterministic"
        log(f"[{variant}] TTFT {ttft_ms:.2f} ms (cold {first.ttft_seconds * 1e3:.1f} ms); "
            f"generate-loop decode {loop_tps:.1f} tok/s; first tokens {first.tokens[:8]}")
        # TTFT of prompt lengths this warmed process has not seen: the eager
        # prefill (the prefill graph of a length is captured after that
        # call's first token, outside its timed region); median of 5 lengths
        # (the first also allocates the new bucket's cache)
        fresh = [runner.generate(prompt[:, : PROMPT_LEN - 8 * (i + 1)], 2).ttft_seconds for i in range(5)]
        ttft_eager_ms = statistics.median(fresh) * 1e3
        log(f"[{variant}] TTFT of a first-seen prompt length (eager prefill): {ttft_eager_ms:.2f} ms")
        del runner

        # Timed decode steps: W warmup + K timed replays of the decode graph.
        bucket = cache_bucket(PROMPT_LEN, args.warmup + args.steps + 2)
        from transformers.cache_utils import StaticCache

        with torch.inference_mode():
            cache = StaticCache(config=model.config, max_cache_len=bucket)
            pos = torch.arange(PROMPT_LEN, device=dev).view(1, -1)
            out = model.model(input_ids=prompt, position_ids=pos, past_key_values=cache,
                              use_cache=True)
            tok = lm_head_argmax(out.last_hidden_state[:, -1].contiguous(), model.lm_head.weight)
            graph = GreedyDecodeGraph(model, cache, tok, torch.full((1, 1), PROMPT_LEN, device=dev,
                                                                    dtype=torch.long), pipelined=True)
            # the generation loop's host side: every token read on the host,
            # the next step queued before the previous token is read
            decode_tokens(graph, args.warmup)
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            timed_tokens = decode_tokens(graph, args.steps)
            torch.cuda.synchronize()
            elapsed = time.perf_counter() - t1
            assert len(timed_tokens) == args.steps
            # pure device time per replay (no host read between replays)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            cache.reset()
            out = model.model(input_ids=prompt, position_ids=pos, past_key_values=cache,
                              use_cache=True)
            graph.set_inputs(tok, torch.full((1, 1), PROMPT_LEN, device=dev, dtype=torch.long))
            torch.cuda.synchronize()
            e0.record()
            for _ in range(args.steps):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
            replay_ms = e0.elapsed_time(e1) / args.steps
            del graph, cache
        ms_per_step = elapsed * 1e3 / args.steps
        log(f"[{variant}] decode: {ms_per_step:.3f} ms/token ({args.steps / elapsed:.1f} tok/s); "
            f"graph replay alone {replay_ms:.3f} ms")
        context = PROMPT_LEN + 1 + args.warmup + (args.steps + 1) / 2
        nbytes = step_bytes(model, context)
        gbs = nbytes / (ms_per_step * 1e-3) / 1e9
        res = {"value": round(args.steps / elapsed, 2), "ms_per_step": round(ms_per_step, 4),
               "ttft_ms": round(ttft_ms, 3), "ttft_eager_ms": round(ttft_eager_ms, 3),
               "graph_replay_ms": round(replay_ms, 4),
               "generate_loop_tokens_per_s": round(loop_tps, 2),
               "weights_gb_per_token": round(weight_bytes / 1e9, 4), "cache_bucket": bucket,
               "step_roofline": {"bytes_per_token": nbytes, "mean_context": context,
                                 "achieved_GB/s": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                 "frac": round(gbs / PEAK_HBM_GBS, 4),
                                 "frac_replay_only": round(nbytes / (replay_ms * 1e-3) / 1e9
                                                           / PEAK_HBM_GBS, 4)}}
        log(f"[{variant}] step: {nbytes / 1e9:.4f} GB/token -> {gbs:.0f} GB/s "
            f"({100 * gbs / PEAK_HBM_GBS:.1f}% of 8 TB/s)")
        return model, state, res

    model, state, main_res = measure(args.variant, keep_state=not args.no_cpu)
    value, ms_per_step, bucket = main_res["value"], main_res["ms_per_step"], main_res["cache_bucket"]

    with torch.inference_mode():
        roof = swiglu_roofline(model, args.variant)
        lm = lm_head_roofline(model)
        kernels = {} if args.no_kernels else kernel_table(dev)
    del model
    torch.cuda.empty_cache()

    # The other linear variant of Benchmark config 5 on the same weights.
    variants = {}
    if not args.no_other_variant:
        other = "a8w8" if args.variant == "bf16" else "bf16"
        m2, _, variants[other] = measure(other, keep_state=False)
        variants[other].pop("weights_gb_per_token")  # counted before quantisation
        with torch.inference_mode():
            variants[other]["swiglu_gemv"] = swiglu_roofline(m2, other)
        del m2
        torch.cuda.empty_cache()

    vision = None
    if not args.no_vision:
        vision = vision_tower_timing(dev)
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        log("CPU baseline ...")
        cpu = cpu_baseline(state, cfg, prompt_cpu[:, : args.cpu_prompt], args.cpu_decode_steps,
                           eager=not args.no_eager)
        cpu["per_config"] = cpu_kernel_table()

    result = {
        "metric": "decode tokens/s (batch 1, greedy) + TTFT, 1 GPU",
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if args.variant == "bf16" else "int8 (A8W8 linears, bf16 elsewhere)",
        "data": "synthetic: seeded random-init N(0,0.02) weights, uniform-random token ids",
        "config": {"workload": "Qwen3.5-2B-shaped decoder (24 layers, 18 DeltaNet + 6 GQA), "
                               f"{PROMPT_LEN}-token prefill then greedy decode, batch 1, "
                               f"{args.variant} linears", "cache_bucket": bucket},
        "ttft_ms": main_res["ttft_ms"],
        "ttft_eager_ms": main_res["ttft_eager_ms"],
        "graph_replay_ms": main_res["graph_replay_ms"],
        "generate_loop_tokens_per_s": main_res["generate_loop_tokens_per_s"],
        "weights_gb_per_token": main_res["weights_gb_per_token"],
        "variants": variants,
        "roofline": {**{k: roof[k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic")},
                     **profile_frac(roof)},
        "roofline_detail": {"swiglu_gemv": roof, "lm_head": lm},
        "step_roofline": main_res["step_roofline"],
        "kernels": kernels,
        "vision_tower": vision,
        "cpu_baseline": cpu,
        "inputs_sha256": _digest_report(digests),
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
