"""Fused greedy generation with TTFT / decode-throughput timing.

Text-only restatement of the reference's ``VLMModel._generate_fused_greedy``
(evaluation_wrapper.py:307-441) on the MI355X path: bucketed static cache,
timer started before the cache reset, prefill through the patched model,
lm_head top-1, ``token.item()`` ends TTFT, one eager decode step on a fresh
bucket, then one captured greedy step replayed per token, every token read
on the host before the next is returned. Unlike the reference's loop, which
reads each token with a copy after its replay, the next replay is queued
before the previous token is read (``graph.decode_tokens``; the token reaches
pinned host memory from the top-1 launch itself), so the GPU does not wait
for the host between steps. Throughput follows the reference formula
``(tokens - 1) / (elapsed - ttft)`` (benchmark_public.py:148-153).

Prefill is captured too, per (cache bucket, prompt length): a length seen
before runs the cache reset, the ~230 prefill launches and the first token's
top-1 as one graph replay (``PrefillGraph``), so the host issues one launch
instead of running the integration's Python per op. The graph is captured at
the end of the first call with that length, outside its timed region.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from .capture import prime_capture_state
from .graph import GreedyDecodeGraph, decode_tokens
from .integration import lm_head_screen, text_stack
from .kernels import lm_head_argmax, zero_tensors


@dataclass
class GenerationResult:
    tokens: list[int]
    ttft_seconds: float
    elapsed_seconds: float
    meta: dict = field(default_factory=dict)

    @property
    def decode_tokens_per_second(self) -> float:
        n = len(self.tokens)
        dt = self.elapsed_seconds - self.ttft_seconds
        return (n - 1) / dt if n > 1 and dt > 0 else 0.0


def cache_bucket(input_len: int, max_new_tokens: int) -> int:
    """evaluation_wrapper.py:339-341."""
    required = input_len + max_new_tokens + 1
    return max(512, ((required + 127) // 128) * 128)


def reset_cache(cache) -> None:
    """Transformers' ``Cache.reset()`` (cache_utils: StaticLayer.reset and
    LinearAttentionCacheLayerMixin.reset) with every tensor it zeroes cleared
    by one kernel launch: the K/V of initialised attention layers, the
    initialised conv and recurrent states of linear-attention layers and the
    static layers' cumulative-length tensors; ``has_previous_state`` flags are
    cleared and integer cumulative lengths set to 0 as there."""

    tensors = []
    for layer in cache.layers:
        if hasattr(layer, "number_of_states"):
            for i in range(layer.number_of_states):
                if layer.is_conv_states_initialized[i]:
                    tensors.append(layer.conv_states[i])
                if layer.is_recurrent_states_initialized[i]:
                    tensors.append(layer.recurrent_states[i])
                layer.has_previous_state[i] = False
        if getattr(layer, "is_initialized", False) and getattr(layer, "keys", None) is not None:
            tensors += [layer.keys, layer.values]
        if hasattr(layer, "cumulative_length"):
            if isinstance(layer.cumulative_length, int):
                layer.cumulative_length = 0
            else:
                tensors.append(layer.cumulative_length)
    zero_tensors(tensors)


_FLAG_ATTRS = ("has_previous_state", "is_conv_states_initialized", "is_recurrent_states_initialized",
               "is_initialized", "cumulative_length")


def _cache_flags(cache) -> list:
    """The host-side state of a cache's layers (flags and integer lengths)
    that the Python of a prefill sets; device tensors are left out."""
    state = []
    for layer in cache.layers:
        for name in _FLAG_ATTRS:
            value = getattr(layer, name, None)
            if isinstance(value, (bool, int)):
                state.append((layer, name, value))
            elif isinstance(value, list) and all(isinstance(v, (bool, int)) for v in value):
                state.append((layer, name, list(value)))
    return state


def _restore_flags(state: list) -> None:
    for layer, name, value in state:
        setattr(layer, name, list(value) if isinstance(value, list) else value)


class PrefillGraph:
    """The prefill of one prompt length over one static cache, captured once:
    the cache reset (one zeroing kernel), the patched model's prefill and the
    first token's lm_head top-1 into a static token tensor. ``run`` copies the
    prompt ids into the captured input buffer, replays, and sets the cache's
    host-side flags to what the eager prefill leaves. The cache's tensors must
    already exist (one eager prefill over it first)."""

    def __init__(self, model, cache, input_ids: torch.Tensor) -> None:
        device = input_ids.device
        self.ids = input_ids.clone()
        self.positions = torch.arange(int(input_ids.shape[-1]), device=device).view(1, -1)
        self.token = torch.zeros((1, 1), device=device, dtype=torch.long)
        saved = _cache_flags(cache)
        screen = lm_head_screen(model)
        # the rotary table depends only on the (fixed) positions: for a text
        # model it is computed once, outside the graph, and kept alive with it
        extra = {}
        if text_stack(model) is model.model:
            stack = model.model
            self.rope = stack.rotary_emb(stack.embed_tokens.weight[:1], self.positions)
            extra["position_embeddings"] = self.rope
        prime_capture_state(device)
        torch.cuda.synchronize(device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            reset_cache(cache)
            out = model.model(input_ids=self.ids, position_ids=self.positions, past_key_values=cache,
                              use_cache=True, return_dict=True, **extra)
            lm_head_argmax(out.last_hidden_state[:, -1, :].contiguous(), model.lm_head.weight,
                           out=self.token, screen=screen)
        self.flags = _cache_flags(cache)  # host state after a prefill
        _restore_flags(saved)  # the capture ran no kernel: the cache is as it was

    def run(self, input_ids: torch.Tensor) -> torch.Tensor:
        self.ids.copy_(input_ids)
        self.graph.replay()
        _restore_flags(self.flags)
        return self.token


class FusedGreedyGenerator:
    """Keeps one StaticCache and one captured decode graph per cache bucket,
    and one captured prefill per (bucket, prompt length) seen (at most
    ``max_prefill_graphs``, the oldest dropped first)."""

    def __init__(self, model, eos_ids: set[int] | None = None, max_prefill_graphs: int = 4):
        self.model = model
        self.eos_ids = eos_ids or set()
        self._caches: dict[int, object] = {}
        self._graphs: dict[int, GreedyDecodeGraph] = {}
        self._prefills: dict[tuple[int, int], PrefillGraph] = {}
        self.max_prefill_graphs = int(max_prefill_graphs)

    def _cache(self, bucket: int):
        from transformers.cache_utils import StaticCache

        cache = self._caches.get(bucket)
        fresh = cache is None
        if fresh:
            cache = StaticCache(config=self.model.config, max_cache_len=bucket)
            self._caches[bucket] = cache
        return cache, fresh

    @torch.inference_mode()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int) -> GenerationResult:
        model = self.model
        input_len = int(input_ids.shape[-1])
        max_new_tokens = max(1, int(max_new_tokens))
        bucket = cache_bucket(input_len, max_new_tokens)
        torch.cuda.synchronize()
        start = time.perf_counter()
        cache, fresh = self._cache(bucket)
        screen = lm_head_screen(model)
        captured = self._prefills.get((bucket, input_len))
        if captured is not None:
            token = captured.run(input_ids)
        else:
            if not fresh:
                reset_cache(cache)
            positions = torch.arange(input_len, device=input_ids.device).view(1, -1)
            prefill = model.model(input_ids=input_ids, position_ids=positions, past_key_values=cache,
                                  use_cache=True, return_dict=True)
            token = lm_head_argmax(prefill.last_hidden_state[:, -1, :].contiguous(),
                                   model.lm_head.weight, screen=screen)
        generated = [int(token.item())]
        first_token_at = time.perf_counter()
        position = torch.full((1, 1), input_len, device=input_ids.device, dtype=torch.long)
        runner = self._graphs.get(bucket)
        reused = runner is not None
        if runner is None and len(generated) < max_new_tokens and generated[-1] not in self.eos_ids:
            out = model.model(input_ids=token, position_ids=position, past_key_values=cache,
                              use_cache=True, return_dict=True)
            token = lm_head_argmax(out.last_hidden_state[:, -1, :].contiguous(), model.lm_head.weight,
                                   screen=screen)
            generated.append(int(token.item()))
            position.add_(1)
        if len(generated) < max_new_tokens and generated[-1] not in self.eos_ids:
            if runner is None:
                runner = GreedyDecodeGraph(model, cache, token, position, pipelined=True)
                self._graphs[bucket] = runner
            else:
                runner.set_inputs(token, position)
            generated += decode_tokens(runner, max_new_tokens - len(generated), self.eos_ids)
        end = time.perf_counter()
        if captured is None:
            # outside the timed region: capture this length's prefill for next time
            while len(self._prefills) >= max(self.max_prefill_graphs, 1):
                self._prefills.pop(next(iter(self._prefills)))
            self._prefills[(bucket, input_len)] = PrefillGraph(model, cache, input_ids)
        return GenerationResult(
            tokens=generated,
            ttft_seconds=first_token_at - start,
            elapsed_seconds=end - start,
            meta={"cache_bucket": bucket, "graph_reused": reused, "cache_reused": not fresh,
                  "prefill_graph": captured is not None},
        )
