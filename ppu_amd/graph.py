"""Captured greedy decode for the Qwen3.5 hot path (hipGraph via torch.cuda.graph).

Interface of reference qwen35_fused/graph.py:10-94 (``GreedyDecodeGraph`` with
``set_inputs`` and ``replay``; ``replay`` returns the next token ``[1, 1]`` for
one step per replay, or ``[steps, 1, 1]``), built around a token ring instead
of separate input/output buffers:

* ``_ring`` holds ``steps`` token slots. Captured step ``s`` reads its input
  token from slot ``s - 1`` (step 0 from the last slot, which holds the
  previous replay's final token or the token given to ``set_inputs``) and its
  greedy token lands in slot ``s``. Consecutive replays therefore continue the
  sequence with no copy node and no host work, and with one step per replay
  the single slot is both the input and the output token.
* With ``fused_lm_head`` the lm_head top-1 launch writes the token straight
  into its ring slot and advances the position tensor in the same launch
  (``lm_head_argmax(..., out=, advance=)``); otherwise the logits path of the
  model runs and the argmax and ``position += 1`` are separate captured ops.

Everything the captured kernels read between replays (token, position, cache
length) lives in device memory, so ``replay`` is one graph launch.

With ``pipelined`` (one step per replay, fused lm_head) the step is captured
twice, and capture ``i``'s top-1 launch also stores the token into pinned host
slot ``i`` (``lm_head_argmax(..., mirror=)``, a store written through to
memory). ``launch`` sets the slot to -1 and replays the two captures
alternately; ``result`` polls the slot until the token replaces the -1, so a
host loop keeps the next step queued while it reads the previous token
(``decode_tokens``): the GPU never waits for the host's read, and nothing runs
on the stream between steps (an event recorded after each replay cost 5 µs
per step). At most two launches are outstanding and results are read in
launch order, so a slot is rewritten only after its token was read.
"""

from __future__ import annotations

import time
from collections import deque

import torch

from .capture import prime_capture_state
from .integration import lm_head_screen
from .kernels import lm_head_argmax


class GreedyDecodeGraph:
    """One capture of ``steps`` greedy decode steps of ``model`` over ``cache``.

    ``cache`` must hold the prefill state (static full-attention layers);
    ``token`` is the first decode input ``[1, 1]`` int64 and ``position_ids``
    its position tensor (``[1, 1]`` text positions or a multimodal
    ``[k, 1, 1]`` tensor), both on the GPU.
    """

    def __init__(self, model, cache, token, position_ids, *, fused_lm_head: bool = True,
                 steps: int = 1, pipelined: bool = False) -> None:
        if not (isinstance(token, torch.Tensor) and token.is_cuda and token.dtype == torch.long
                and token.shape[-1] == 1):
            raise ValueError("token must be an int64 GPU tensor whose last dimension is 1")
        if not (isinstance(position_ids, torch.Tensor) and position_ids.is_cuda):
            raise ValueError("position_ids must be a GPU tensor")
        if int(steps) < 1:
            raise ValueError("steps must be at least 1")
        if pipelined and (int(steps) != 1 or not fused_lm_head):
            raise ValueError("pipelined decode needs one step per replay and the fused lm_head")
        self.model = model
        self.cache = cache
        self.fused_lm_head = bool(fused_lm_head)
        self.steps = int(steps)
        self.pipelined = bool(pipelined)
        self._ring = torch.empty((self.steps, *token.shape), dtype=torch.long, device=token.device)
        self._ring[-1].copy_(token)
        self._positions = position_ids.clone()
        self.logits = None
        self._host = ([torch.zeros(1, dtype=torch.long, pin_memory=True) for _ in range(2)]
                      if self.pipelined else [None])
        self._host_view = [None if t is None else t.numpy() for t in self._host]
        self._streams = [None for _ in self._host]
        self._pending: deque[int] = deque()
        self._next = 0
        self._plain_unsynced = False  # a plain replay's mirror store may still be in flight
        prime_capture_state(token.device)
        torch.cuda.synchronize(token.device)
        self._graphs = []
        for host in self._host:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for s in range(self.steps):
                    self._record_step(self._ring[s - 1], self._ring[s], host)
            self._graphs.append(graph)
        self.graph = self._graphs[0]

    def _record_step(self, token_in: torch.Tensor, token_out: torch.Tensor,
                     host: torch.Tensor | None = None) -> None:
        model, positions = self.model, self._positions
        if self.fused_lm_head:
            state = model.model(input_ids=token_in, attention_mask=None, position_ids=positions,
                                past_key_values=self.cache, use_cache=True, return_dict=True)
            last = state.last_hidden_state[:, -1, :].contiguous()
            lm_head_argmax(last, model.lm_head.weight, out=token_out, mirror=host, advance=positions,
                           screen=lm_head_screen(model))
            return
        state = model(input_ids=token_in, attention_mask=None, position_ids=positions,
                      past_key_values=self.cache, use_cache=True, logits_to_keep=1,
                      return_dict=True)
        self.logits = state.logits
        token_out.copy_(state.logits[:, -1, :].argmax(dim=-1, keepdim=True).view_as(token_out))
        positions.add_(1)

    @property
    def token(self) -> torch.Tensor:
        """The most recent greedy token (the next replay's input)."""
        return self._ring[-1]

    @property
    def position_ids(self) -> torch.Tensor:
        """The position tensor the next replay decodes at."""
        return self._positions

    @property
    def output_tokens(self) -> torch.Tensor | None:
        return self._ring if self.steps > 1 else None

    def set_inputs(self, token: torch.Tensor, position_ids: torch.Tensor) -> None:
        """Start the next replay from ``token`` at ``position_ids``."""
        if tuple(token.shape) != tuple(self._ring.shape[1:]) or position_ids.shape != self._positions.shape:
            raise ValueError("graph input shapes do not match the captured buffers")
        if self._pending:
            raise RuntimeError("read the outstanding tokens (result) before setting new inputs")
        self._ring[-1].copy_(token)
        self._positions.copy_(position_ids)

    def replay(self) -> torch.Tensor:
        """Run the captured steps; the token ``[1, 1]`` (one step) or the
        ``[steps, 1, 1]`` tokens of this replay, in order."""
        if self._pending:
            raise RuntimeError("read the outstanding tokens (result) before a plain replay")
        self.graph.replay()
        self._plain_unsynced = self.pipelined
        return self._ring[0] if self.steps == 1 else self._ring

    def launch(self) -> int:
        """Queue one decode step (pipelined graphs) and return its slot; the
        token is read with ``result(slot)``, in launch order. At most two
        launches may be outstanding."""
        if not self.pipelined:
            raise RuntimeError("launch needs a pipelined GreedyDecodeGraph")
        if len(self._pending) >= 2:
            raise RuntimeError("read a token (result) before a third launch")
        if self._plain_unsynced:
            # capture 0 also stores into host slot 0: let a plain replay's
            # store land before the slot is reset
            torch.cuda.current_stream().synchronize()
            self._plain_unsynced = False
        i = self._next
        self._host_view[i][0] = -1  # token ids are >= 0: -1 marks "not written yet"
        self._streams[i] = torch.cuda.current_stream()
        self._graphs[i].replay()
        self._pending.append(i)
        self._next = 1 - i
        return i

    def result(self, slot: int) -> int:
        """Wait for the oldest outstanding launch (``slot``) and return its
        token: polls that capture's pinned host slot. Should the stream run
        dry with the slot still unwritten, raises RuntimeError instead of
        waiting forever."""
        if not self._pending or self._pending[0] != slot:
            raise RuntimeError("results must be read in launch order")
        view, spins, since = self._host_view[slot], 0, None
        while view[0] < 0:
            spins += 1
            if spins % 1024 == 0:
                # a stream query is not free on the GPU side (it can put a
                # marker in the queue): only after 20 ms of polling, far
                # beyond a step's time, is the stream asked whether it ran dry
                now = time.perf_counter()
                since = now if since is None else since
                if now - since > 0.02 and self._streams[slot].query() and view[0] < 0:
                    raise RuntimeError("the decode step ended without its token reaching the host slot")
        self._pending.popleft()
        return int(view[0])


def decode_tokens(runner: GreedyDecodeGraph, count: int, eos_ids=()) -> list[int]:
    """Up to ``count`` greedy tokens from a pipelined ``runner`` (inputs set):
    the next step is queued before the previous token is read, and no step
    past ``count`` is queued. After an EOS token the one step already queued
    behind it is waited for (its token dropped), so the caller's clock covers
    all the GPU work of the call."""
    tokens: list[int] = []
    launched = 0
    pending: deque[int] = deque()
    if count > 0:
        pending.append(runner.launch())
        launched = 1
    while pending:
        if launched < count:
            pending.append(runner.launch())
            launched += 1
        token = runner.result(pending.popleft())
        tokens.append(token)
        if token in eos_ids:
            break
    while pending:
        runner.result(pending.popleft())
    return tokens
