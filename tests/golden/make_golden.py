"""Writes the golden vectors of tests/golden/*.npz from HF transformers' Qwen2 modules.

The reference kernels (gojosatorukz/esep-soup-kernels solution/body/norm_rope.py) replace HF's
Qwen2RMSNorm, Qwen2RotaryEmbedding and apply_rotary_pos_emb (transformers
models/qwen2/modeling_qwen2.py; pinned 5.16.1 in the reference's requirements.txt:4, 5.15.0
in this image; the three functions are unchanged between them). These vectors are HF's own
forward outputs and torch-autograd gradients on seeded inputs, so they pin the CPU oracle
(oracle/norm_rope_ref.py) independently of its formulas: tests/test_oracle_golden.py checks
the oracle against them.

    python tests/golden/make_golden.py        # rewrites the .npz files next to this script

Contents (all arrays float64 unless noted):
  rmsnorm_f32.npz   HF Qwen2RMSNorm (fp32 module) on x [37, 256] and x [5, 1536]: y, dx, dw
  rmsnorm_bf16.npz  the same module in bf16 (HF's bf16 rounding of xhat before * w): y
  rope.npz          Qwen2RotaryEmbedding(theta 1e6, head_dim 128) + apply_rotary_pos_emb on
                    q [2, 4, 33, 128], k [2, 2, 33, 128] with position_ids up to 32752:
                    cos, sin, q_embed, k_embed and the q / k gradients
  inv_freq.npz      HF default inverse frequencies for head_dim 64/128/256, theta 1e4/1e6 (fp32)
"""

from pathlib import Path

import numpy as np
import torch
from transformers import Qwen2Config
from transformers.models.qwen2.modeling_qwen2 import (Qwen2RMSNorm, Qwen2RotaryEmbedding,
                                                      apply_rotary_pos_emb)

OUT = Path(__file__).resolve().parent
EPS = 1e-6


def rmsnorm_case(T, H, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(T, H, generator=g) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype)
    dy = torch.randn(T, H, generator=g).to(dtype)
    m = Qwen2RMSNorm(H, eps=EPS).to(dtype)
    with torch.no_grad():
        m.weight.copy_(w)
    xr = x.clone().requires_grad_()
    y = m(xr)
    y.backward(dy)
    f = lambda t: t.detach().to(torch.float64).numpy()  # noqa: E731
    return dict(x=f(x), w=f(w), dy=f(dy), y=f(y), dx=f(xr.grad), dw=f(m.weight.grad))


def rope_case(seed):
    B, HQ, HK, S, D = 2, 4, 2, 33, 128
    g = torch.Generator().manual_seed(seed)
    cfg = Qwen2Config(hidden_size=HQ * D, num_attention_heads=HQ, num_key_value_heads=HK,
                      rope_theta=1e6, max_position_embeddings=32768)
    emb = Qwen2RotaryEmbedding(cfg)
    pos = torch.stack([torch.arange(S), torch.arange(S) * 997 + 881])  # row 1 reaches 32785
    pos[1] = pos[1].clamp(max=32752)
    q = torch.randn(B, HQ, S, D, generator=g, requires_grad=True)
    k = torch.randn(B, HK, S, D, generator=g, requires_grad=True)
    cos, sin = emb(q, pos)
    qe, ke = apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=1)
    dq = torch.randn(qe.shape, generator=g)
    dk = torch.randn(ke.shape, generator=g)
    torch.autograd.backward([qe, ke], [dq, dk])
    f = lambda t: t.detach().to(torch.float64).numpy()  # noqa: E731
    return dict(q=f(q), k=f(k), pos=pos.numpy(), inv_freq=emb.inv_freq.numpy(), cos=f(cos),
                sin=f(sin), q_embed=f(qe), k_embed=f(ke), dq=f(dq), dk=f(dk),
                q_grad=f(q.grad), k_grad=f(k.grad))


def inv_freq_cases():
    out = {}
    for d in (64, 128, 256):
        for theta in (1e4, 1e6):
            cfg = Qwen2Config(hidden_size=4 * d, num_attention_heads=4, num_key_value_heads=2,
                              rope_theta=theta)
            inv, scale = Qwen2RotaryEmbedding.compute_default_rope_parameters(cfg)
            assert scale == 1.0
            out[f"d{d}_theta{int(theta)}"] = inv.numpy()
    return out


def main():
    a = rmsnorm_case(37, 256, 1)
    b = rmsnorm_case(5, 1536, 2)
    np.savez_compressed(OUT / "rmsnorm_f32.npz", **{f"a_{k}": v for k, v in a.items()},
                        **{f"b_{k}": v for k, v in b.items()})
    c = rmsnorm_case(9, 512, 3, torch.bfloat16)
    np.savez_compressed(OUT / "rmsnorm_bf16.npz", **c)
    np.savez_compressed(OUT / "rope.npz", **rope_case(4))
    np.savez_compressed(OUT / "inv_freq.npz", **inv_freq_cases())
    for p in sorted(OUT.glob("*.npz")):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
