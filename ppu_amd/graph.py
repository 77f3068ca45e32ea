"""hipGraph runner for the single-token greedy Qwen3.5 decode step.

Drop-in for reference qwen35_fused/graph.py:10-94: captures one (or
``steps``) greedy decode step(s) — the patched text forward, the fused
lm_head top-1, the token feedback and ``position_ids += 1`` — with
``torch.cuda.graph`` (a hipGraph on ROCm) and replays it once per token. All
kernels read the valid cache length and the position from device memory, so a
replay needs no host work besides the launch.
"""

from __future__ import annotations

import torch

from .kernels import lm_head_argmax


class GreedyDecodeGraph:
    """Capture model decode, LM head argmax and autoregressive token feedback.

    The supplied cache must already hold the prefill state and use static
    full-attention layers. ``position_ids`` is the first decode token's
    position tensor (``[1, 1]`` text positions, or the multimodal layout).
    """

    def __init__(self, model, cache, token, position_ids, *, fused_lm_head: bool = True,
                 steps: int = 1) -> None:
        if token.shape[-1] != 1 or token.dtype != torch.long or not token.is_cuda:
            raise ValueError("token must be a GPU int64 tensor with sequence length 1")
        if not position_ids.is_cuda:
            raise ValueError("position_ids must be on the GPU")
        if steps < 1:
            raise ValueError("steps must be positive")
        self.model = model
        self.cache = cache
        self.token = token.clone()
        self.position_ids = position_ids.clone()
        self.graph = torch.cuda.CUDAGraph()
        self.logits = None
        self.fused_lm_head = fused_lm_head
        self.steps = steps
        self.output_tokens = None
        if steps > 1:
            self.output_tokens = torch.empty((steps, *self.token.shape), device=self.token.device,
                                             dtype=self.token.dtype)
        torch.cuda.synchronize()
        with torch.cuda.graph(self.graph):
            for step in range(self.steps):
                if self.fused_lm_head:
                    outputs = self.model.model(input_ids=self.token, attention_mask=None,
                                               position_ids=self.position_ids,
                                               past_key_values=self.cache, use_cache=True,
                                               return_dict=True)
                    hidden = outputs.last_hidden_state[:, -1, :].contiguous()
                    # top-1, token feedback and position += 1 in the final-reduce launch
                    lm_head_argmax(hidden, self.model.lm_head.weight, out=self.token,
                                   advance=self.position_ids)
                    if self.output_tokens is not None:
                        self.output_tokens[step].copy_(self.token)
                    continue
                else:
                    outputs = self.model(input_ids=self.token, attention_mask=None,
                                         position_ids=self.position_ids, past_key_values=self.cache,
                                         use_cache=True, logits_to_keep=1, return_dict=True)
                    self.logits = outputs.logits
                    next_token = self.logits[:, -1, :].argmax(dim=-1, keepdim=True)
                if self.output_tokens is not None:
                    self.output_tokens[step].copy_(next_token)
                self.token.copy_(next_token)
                self.position_ids.add_(1)

    def set_inputs(self, token: torch.Tensor, position_ids: torch.Tensor) -> None:
        """Set the first token and position for the next replay."""
        if token.shape != self.token.shape or position_ids.shape != self.position_ids.shape:
            raise ValueError("graph input shapes do not match the captured buffers")
        self.token.copy_(token)
        self.position_ids.copy_(position_ids)

    def replay(self) -> torch.Tensor:
        self.graph.replay()
        if self.steps == 1:
            return self.token
        assert self.output_tokens is not None
        return self.output_tokens
