"""Write tests/golden/golden.npz: small input/output vectors for the hot-path
operators, computed by Transformers 5.15.0's own eager Qwen3.5 modules on the
CPU (a third-party restatement of the same semantics, not the reference
repository, which is never imported) plus a brute-force lm_head top-1.

Run from the repository root: ``python tests/golden/make_golden.py``.
bf16 arrays are stored as their uint16 bit patterns.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent / "golden.npz"
BF = torch.bfloat16


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main() -> None:
    from transformers.models.qwen3_5 import modeling_qwen3_5 as m

    g = torch.Generator().manual_seed(20260819)
    rn = lambda *s, sc=1.0, mu=0.0: (torch.randn(*s, generator=g) * sc + mu).to(BF)  # noqa: E731
    d: dict[str, np.ndarray] = {}

    x, w = rn(4, 2048), rn(2048, sc=0.1)
    mod = m.Qwen3_5RMSNorm(2048, eps=1e-6)
    mod.weight.data = w.float()
    d.update(rms_x=bits(x), rms_w=bits(w), rms_out=bits(mod(x)))

    gx, gz, gw = rn(16, 128), rn(16, 128), rn(128, sc=0.1, mu=1.0)
    gmod = m.Qwen3_5RMSNormGated(128, eps=1e-6).to(BF)
    gmod.weight.data = gw
    d.update(g_x=bits(gx), g_z=bits(gz), g_w=bits(gw), g_out=bits(gmod(gx, gz)))

    heads, dim, seq = 4, 128, 3
    qkv = rn(1, seq, 3 * heads * dim)
    packed = rn(1, seq, 4 * heads * dim + 2 * heads)
    packed[..., : 3 * heads * dim] = qkv
    a_log, dt = rn(heads), rn(heads)
    st = torch.randn(1, heads, dim, dim, generator=g) * 0.01
    q, k, v = qkv.float().reshape(1, seq, 3, heads, dim).unbind(2)
    a_off = 4 * heads * dim
    a = packed[..., a_off : a_off + heads].float()
    b = packed[..., a_off + heads :].float()
    gg = -a_log.float().exp() * F.softplus(a + dt.float())
    out, final = m.torch_recurrent_gated_delta_rule(q, k, v, g=gg, beta=b.sigmoid(),
                                                    initial_state=st.clone(), output_final_state=True,
                                                    use_qk_l2norm_in_kernel=True)
    d.update(delta_qkv=bits(qkv), delta_packed=bits(packed), delta_alog=bits(a_log),
             delta_dt=bits(dt), delta_state0=st.numpy(), delta_state1=final.numpy(),
             delta_out=bits(out.to(BF)))

    qh, kvh, hd, rot, sl = 8, 2, 256, 64, 3
    pk = rn(1, sl, 2 * qh * hd + 2 * kvh * hd)
    qw, kw = rn(hd, sc=0.1), rn(hd, sc=0.1)
    cos, sin = rn(1, sl, rot), rn(1, sl, rot)
    qn = m.Qwen3_5RMSNorm(hd)
    qn.weight.data = qw.float()
    kn = m.Qwen3_5RMSNorm(hd)
    kn.weight.data = kw.float()
    q_raw = pk[..., : 2 * qh * hd].reshape(1, sl, qh, 2 * hd)[..., :hd]
    k_raw = pk[..., 2 * qh * hd : 2 * qh * hd + kvh * hd].reshape(1, sl, kvh, hd)
    eq, ek = m.apply_rotary_pos_emb(qn(q_raw).transpose(1, 2), kn(k_raw).transpose(1, 2), cos, sin)
    d.update(qg_packed=bits(pk), qg_qw=bits(qw), qg_kw=bits(kw), qg_cos=bits(cos), qg_sin=bits(sin),
             qg_q=bits(eq), qg_k=bits(ek))

    h, lw = rn(1, 256), rn(1000, 256, sc=0.05)
    logits = (h.double() @ lw.double().t()).float().to(BF).float()
    d.update(lm_h=bits(h), lm_w=bits(lw), lm_idx=np.array(int(logits.argmax())))

    np.savez_compressed(OUT, **d)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(d)} arrays)")


if __name__ == "__main__":
    main()
