"""CPU decoder following the reference's fused data flow (test infrastructure only).

Restates PingGuoLiZiJvZi/ppu qwen35_fused/integration.py on the CPU with the
oracle operators:
  * weight packing (:69-140): DeltaNet [qkv | z | a | b] padded to a multiple
    of 128 rows, MLP [gate; up], attention [q(+gate); k; v];
  * text forward (:390-504): embed -> RMSNorm(layer 0) -> per layer mixer ->
    residual_add_rms_norm(post-attention) -> MLP -> residual_add_rms_norm(next
    input norm, or the final norm after the last layer);
  * DeltaNet mixer (:228-272): packed projection -> conv1d -> delta rule ->
    gated RMSNorm with z -> out_proj;
  * attention mixer (:282-359): packed projection -> Q/K norm + RoPE with the
    cache write at the current length -> length += L -> decode attention
    (L == 1) or causal prefill attention -> sigmoid gate -> o_proj;
  * MLP (:169-187): decode SwiGLU GEMV, prefill F.linear + silu_and_mul;
  * greedy step (graph.py:51-79): lm_head top-1 of the last hidden state.

Linear layers use torch's CPU bf16 F.linear (fp32 accumulation, one bf16
round), pinned against the fp32 restatement ``ops.linear`` in the tests.
Pinning of the data flow: tests/test_oracle_model.py compares it with
Transformers' own eager Qwen3.5 forward on the same weights (logit agreement
within the bf16 rounding the fused path differs by) and checks the packing.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import a8w8 as oa
from . import ops


@dataclass
class Shapes:
    hidden: int
    layers: list  # "linear_attention" / "full_attention"
    q_heads: int
    kv_heads: int
    head_dim: int
    rotary_dim: int
    rope_theta: float
    lin_heads: int
    lin_dim: int
    conv_k: int
    eps: float
    vocab: int
    mrope_section: tuple = (11, 11, 10)

    @classmethod
    def from_config(cls, cfg):
        rp = cfg.rope_parameters
        return cls(
            hidden=cfg.hidden_size,
            layers=list(cfg.layer_types),
            q_heads=cfg.num_attention_heads,
            kv_heads=cfg.num_key_value_heads,
            head_dim=cfg.head_dim,
            rotary_dim=int(cfg.head_dim * rp.get("partial_rotary_factor", 1.0)),
            rope_theta=float(rp["rope_theta"]),
            lin_heads=cfg.linear_num_value_heads,
            lin_dim=cfg.linear_value_head_dim,
            conv_k=cfg.linear_conv_kernel_dim,
            eps=cfg.rms_norm_eps,
            vocab=cfg.vocab_size,
            mrope_section=tuple(rp.get("mrope_section", (11, 11, 10))),
        )


def pack_weights(state: dict[str, torch.Tensor], shapes: Shapes, pad: int = 128) -> dict:
    """Packed CPU weights in the reference layouts (integration.py:69-140)."""
    w = {"embed": state["model.embed_tokens.weight"], "final_norm": state["model.norm.weight"]}
    layers = []
    for i, kind in enumerate(shapes.layers):
        p = f"model.layers.{i}."
        lw = {
            "kind": kind,
            "in_norm": state[p + "input_layernorm.weight"],
            "post_norm": state[p + "post_attention_layernorm.weight"],
            "gate_up": torch.cat((state[p + "mlp.gate_proj.weight"], state[p + "mlp.up_proj.weight"])),
            "down": state[p + "mlp.down_proj.weight"],
        }
        if kind == "linear_attention":
            a = p + "linear_attn."
            packed = torch.cat(
                (state[a + "in_proj_qkv.weight"], state[a + "in_proj_z.weight"],
                 state[a + "in_proj_a.weight"], state[a + "in_proj_b.weight"])
            )
            rows = (-packed.shape[0]) % pad
            if rows:
                packed = F.pad(packed, (0, 0, 0, rows))
            lw.update(
                in_proj=packed.contiguous(),
                conv_w=state[a + "conv1d.weight"].squeeze(1).contiguous(),
                a_log=state[a + "A_log"],
                dt_bias=state[a + "dt_bias"],
                gnorm=state[a + "norm.weight"],
                out_proj=state[a + "out_proj.weight"],
            )
        else:
            a = p + "self_attn."
            lw.update(
                qgkv=torch.cat((state[a + "q_proj.weight"], state[a + "k_proj.weight"],
                                state[a + "v_proj.weight"])).contiguous(),
                q_norm=state[a + "q_norm.weight"],
                k_norm=state[a + "k_norm.weight"],
                o_proj=state[a + "o_proj.weight"],
            )
        layers.append(lw)
    w["layers"] = layers
    return w


class Cache:
    """Static per-request state: conv/recurrent states per DeltaNet layer,
    K/V [1, KVH, max_len, D] per attention layer and the filled length."""

    def __init__(self, shapes: Shapes, max_len: int):
        self.max_len = max_len
        self.length = 0
        conv_dim = 3 * shapes.lin_heads * shapes.lin_dim
        self.conv, self.rec, self.k, self.v = {}, {}, {}, {}
        for i, kind in enumerate(shapes.layers):
            if kind == "linear_attention":
                self.conv[i] = torch.zeros(1, conv_dim, shapes.conv_k, dtype=torch.bfloat16)
                self.rec[i] = torch.zeros(1, shapes.lin_heads, shapes.lin_dim, shapes.lin_dim)
            else:
                self.k[i] = torch.zeros(1, shapes.kv_heads, max_len, shapes.head_dim, dtype=torch.bfloat16)
                self.v[i] = torch.zeros_like(self.k[i])


_LINEARS = ("in_proj", "out_proj", "qgkv", "o_proj", "gate_up", "down")


class OracleDecoder:
    """``a8w8``: every linear except the lm_head runs as A8W8 (per-channel int8
    weights quantised here, per-token int8 activations, exact integer products,
    fp32 dequant), as the reference applies PPUA8W8Linear to the MLP,
    attention and DeltaNet projections (explore_runtime_quantization.py:66-84)."""

    def __init__(self, state: dict[str, torch.Tensor], config, *, a8w8: bool = False):
        self.s = Shapes.from_config(config)
        self.w = pack_weights(state, self.s)
        self.a8w8 = a8w8
        if a8w8:
            for lw in self.w["layers"]:
                for name in _LINEARS:
                    if name in lw:
                        q, sc = oa.quantize_weight(lw[name])
                        lw[name + "_q"] = (torch.from_numpy(q).double(), sc)

    def _lin(self, x: torch.Tensor, lw: dict, name: str) -> torch.Tensor:
        if not self.a8w8:
            return F.linear(x, lw[name])
        wq, sw = lw[name + "_q"]
        xq, sx = oa.quantize_act(x)
        # int8 x int8 products summed over K <= 6144 stay below 2^53: fp64 BLAS is exact
        acc = (torch.from_numpy(xq).double() @ wq.t()).to(torch.int64).numpy()
        assert abs(acc).max(initial=0) < 2**31
        y = oa.dequant(acc.astype("int32"), sx, sw)
        return y.reshape(*x.shape[:-1], -1)

    def new_cache(self, max_len: int) -> Cache:
        return Cache(self.s, max_len)

    # ------------------------------------------------------------ mixers
    def _delta(self, i, lw, h, cache: Cache):
        s = self.s
        b, l, _ = h.shape
        packed = self._lin(h, lw, "in_proj")
        qkv = ops.causal_conv1d(packed, lw["conv_w"], cache.conv[i])
        core = ops.delta_recurrent(qkv, packed, lw["a_log"], lw["dt_bias"], cache.rec[i])
        vd = s.lin_heads * s.lin_dim
        conv_dim = 3 * vd
        z = packed[..., conv_dim : conv_dim + vd].reshape(-1, s.lin_dim)
        core = ops.gated_rms_norm(core.reshape(-1, s.lin_dim), z, lw["gnorm"], s.eps)
        return self._lin(core.reshape(b, l, vd), lw, "out_proj")

    def _attn(self, i, lw, h, cos, sin, cache: Cache, start: int):
        s = self.s
        l = h.shape[1]
        packed = self._lin(h, lw, "qgkv")
        q, kc, vc = ops.qgkv_norm_rope(
            packed, lw["q_norm"], lw["k_norm"], cos, sin, q_heads=s.q_heads, kv_heads=s.kv_heads,
            dim=s.head_dim, rotary_dim=s.rotary_dim, cache_key=cache.k[i], cache_value=cache.v[i],
            cache_start=start,
        )
        scale = s.head_dim ** -0.5
        if l == 1:
            o = ops.gqa_decode_attention(q, kc, vc, start + 1, scale)
        else:
            o = ops.prefill_attention(q, kc, vc, scale, kv_start=start)
        o = ops.attention_gate_mul(o, packed, s.head_dim)
        return self._lin(o, lw, "o_proj")

    def _mlp(self, lw, x):
        if x.shape[1] == 1 and not self.a8w8:
            act = ops.swiglu_gemv(x, lw["gate_up"])
        else:
            act = ops.silu_and_mul(self._lin(x, lw, "gate_up"))
        return self._lin(act, lw, "down")

    # ------------------------------------------------------------ forward
    def _layer_states(self, i: int, cache: Cache) -> dict:
        if i in cache.rec:
            return {"conv": cache.conv[i].clone(), "rec": cache.rec[i].clone()}
        return {"k": cache.k[i].clone(), "v": cache.v[i].clone()}

    @torch.no_grad()
    def forward(self, ids: torch.Tensor | None, cache: Cache, trace: list | None = None, *,
                embeds: torch.Tensor | None = None,
                rope_positions: torch.Tensor | None = None) -> torch.Tensor:
        """ids [1, L] (or ``embeds`` [1, L, hidden], the input embeddings of a
        multimodal prompt) written at cache slots cache.length ...; returns the
        final-normed hidden states [1, L, hidden] and advances the cache.
        ``rope_positions`` ([1, L] or multimodal [3, 1, L]) default to the
        cache slots (text-only positions).

        ``trace`` (a list) receives one dict per layer for layer-wise checks:
        ``residual_in`` / ``normalized_in`` (the layer's input stream and its
        input-normed row), ``update`` (mixer output), ``residual_mid`` (stream
        after the mixer add), ``mlp_out``, ``normalized_out`` (the next
        layer's normed input, or the final norm) and ``states`` (the layer's
        conv/recurrent or K/V cache after the layer, cloned)."""
        s = self.s
        l = ids.shape[1] if ids is not None else embeds.shape[1]
        start = cache.length
        if start + l > cache.max_len:
            raise ValueError("cache too short")
        positions = torch.arange(start, start + l).view(1, l) if rope_positions is None else rope_positions
        cos, sin = ops.rotary_cos_sin(positions, s.rotary_dim, s.rope_theta, s.mrope_section)
        residual = self.w["embed"][ids] if ids is not None else embeds.to(torch.bfloat16)
        layers = self.w["layers"]
        normalized = ops.rms_norm(residual, layers[0]["in_norm"], s.eps)
        for i, lw in enumerate(layers):
            rec = {"residual_in": residual, "normalized_in": normalized} if trace is not None else None
            if lw["kind"] == "linear_attention":
                upd = self._delta(i, lw, normalized, cache)
            else:
                upd = self._attn(i, lw, normalized, cos, sin, cache, start)
            residual, mlp_in = ops.residual_add_rms_norm(residual, upd, lw["post_norm"], s.eps)
            mlp_out = self._mlp(lw, mlp_in)
            nxt = layers[i + 1]["in_norm"] if i + 1 < len(layers) else self.w["final_norm"]
            residual_new, normalized = ops.residual_add_rms_norm(residual, mlp_out, nxt, s.eps)
            if rec is not None:
                rec.update(update=upd, residual_mid=residual, mlp_out=mlp_out,
                           normalized_out=normalized, states=self._layer_states(i, cache))
                trace.append(rec)
            if i + 1 < len(layers):
                residual = residual_new
        cache.length = start + l
        return normalized

    def top1(self, hidden_last: torch.Tensor) -> tuple[int, float]:
        """Greedy token of a [1, hidden] state and its top-2 margin (bf16 logits)."""
        logits = ops._f(ops._bf(F.linear(hidden_last.float(), self.w["embed"].float())))
        top = torch.topk(logits[0], 2)
        tok = int(ops.lm_head_argmax(hidden_last, self.w["embed"]))
        return tok, float(top.values[0] - top.values[1])

    @torch.no_grad()
    def teacher_forced(self, prompt: torch.Tensor, forced: list[int], max_len: int,
                       return_hidden: bool = False):
        """Prefill ``prompt`` then feed ``forced`` tokens one at a time.
        Returns per step (oracle argmax, top-2 margin), len(forced) + 1 steps,
        and with ``return_hidden`` also the final-normed hidden state of each step."""
        cache = self.new_cache(max_len)
        h = self.forward(prompt, cache)
        out = [self.top1(h[:, -1])]
        hidden = [h[:, -1].clone()]
        for tok in forced:
            h = self.forward(torch.tensor([[tok]]), cache)
            out.append(self.top1(h[:, -1]))
            hidden.append(h[:, -1].clone())
        return (out, hidden) if return_hidden else out
