"""PyTorch-eager restatement of the HF Qwen2 path that the reference's kernels replace:
Qwen2RMSNorm.forward, Qwen2RotaryEmbedding.forward and apply_rotary_pos_emb
(transformers models/qwen2/modeling_qwen2.py; pinned 5.16.1 by the reference's
requirements.txt:4). Forward and torch.autograd backward run on the CPU in fp32.

TEST INFRASTRUCTURE ONLY: this is the CPU baseline that bench.py times beside the GPU path
(kind "port") and a second checker for tests; the product never imports it.
"""

import torch


def rms_norm(x, weight, eps):
    """HF Qwen2RMSNorm.forward (modeling_qwen2.py:247-252)."""
    dt = x.dtype
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    return weight * h.to(dt)


def rotary_cos_sin(inv_freq, position_ids, dtype):
    """HF Qwen2RotaryEmbedding.forward (modeling_qwen2.py:89-102), attention_scaling 1.0:
    freqs = inv_freq (x) positions in fp32 via a K=1 matmul, emb = cat(freqs, freqs)."""
    inv = inv_freq[None, :, None].float().expand(position_ids.shape[0], -1, 1)
    pos = position_ids[:, None, :].float()
    freqs = (inv @ pos).transpose(1, 2)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x):
    """HF rotate_half (modeling_qwen2.py:105-109)."""
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=1):
    """HF apply_rotary_pos_emb (modeling_qwen2.py:112-135)."""
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    return (q * cos) + (rotate_half(q) * sin), (k * cos) + (rotate_half(k) * sin)


def body_step(x_list, w_list, q, k, dy_list, dq, dk, inv_freq, position_ids, eps):
    """One fwd+bwd pass of the decoder-body path on the CPU: every norm in x_list (with its
    weight and output gradient) and one RoPE on q [B, H, S, D] / k. Returns the gradients."""
    outs = []
    for x, w, dy in zip(x_list, w_list, dy_list):
        xr = x.detach().requires_grad_()
        wr = w.detach().requires_grad_()
        y = rms_norm(xr, wr, eps)
        gx, gw = torch.autograd.grad(y, [xr, wr], dy)
        outs += [gx, gw]
    qr, kr = q.detach().requires_grad_(), k.detach().requires_grad_()
    cos, sin = rotary_cos_sin(inv_freq, position_ids, qr.dtype)
    qe, ke = apply_rotary_pos_emb(qr, kr, cos, sin, unsqueeze_dim=1)
    outs += list(torch.autograd.grad([qe, ke], [qr, kr], [dq, dk]))
    return outs
