"""Varlen causal attention with grouped kv heads on the HIP kernels (esep_attn_fwd /
esep_attn_bwd): the consumer of the RoPE output in the packed decoder. It replaces the
reference's per-row loop over torch's scaled_dot_product_attention (solution/body/packed.py:
404-436) with one launch over all rows: q [T, HQ, D] and k, v [T, HK, D] in the packed token
layout, sequences delimited by cu_seqlens, query head h reading kv head h // (HQ // HK).

Forward saves (q, k, v, o, lse); the backward recomputes the probabilities from lse. Both
directions are deterministic (no atomics). fp16 and bf16, D in {64, 128}; other inputs are
rejected (EsepError), never silently computed another way.
"""

import torch

from . import _hip


def cu_seqlens_from_lengths(lengths, device):
    """int32 [len(lengths) + 1] prefix sums of host sequence lengths, on `device`."""
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + int(n))
    return torch.tensor(cu, dtype=torch.int32, device=device)


def supported(q, k, v, dropout=0.0):
    """Whether varlen_attention takes these inputs ([T, H, D] or [1, T, H, D] views)."""
    if dropout != 0.0 or not q.is_cuda:
        return False
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        return False
    D = q.shape[-1]
    return D in (64, 128) and q.shape[-2] % k.shape[-2] == 0 and k.shape == v.shape


def _heads_packed(t):
    if t.stride(2) != 1 or t.stride(1) != t.shape[2] or t.stride(0) % 8 or t.data_ptr() % 16:
        t = t.contiguous()
    return t


class VarlenAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cu_seqlens, max_seqlen, scale):
        q, k, v = _heads_packed(q), _heads_packed(k), _heads_packed(v)
        T, HQ, D = q.shape
        o = torch.empty_like(q)
        lse = torch.empty((HQ, T), device=q.device, dtype=torch.float32)
        _hip.attn_fwd(q, k, v, o, cu_seqlens, max_seqlen, scale, lse=lse)
        ctx.save_for_backward(q, k, v, o, lse, cu_seqlens)
        ctx.max_seqlen, ctx.scale = int(max_seqlen), float(scale)
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, o, lse, cu = ctx.saved_tensors
        do = _heads_packed(do)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        _hip.attn_bwd(q, k, v, o, do, lse, dq, dk, dv, cu, ctx.max_seqlen, ctx.scale)
        return dq, dk, dv, None, None, None


def varlen_attention(q, k, v, cu_seqlens, max_seqlen, scale=None):
    """Causal attention within each sequence of the packed tokens. q [T, HQ, D] (or
    [1, T, HQ, D]), k, v [T, HK, D]; cu_seqlens int32 [n_seq + 1] on q's device; max_seqlen an
    int >= every sequence length. Returns o [T, HQ, D] in q's dtype."""
    if scale is None:
        scale = q.shape[-1] ** -0.5
    if q.dim() == 4:  # [1, T, H, D] views: the Function works on [T, H, D]
        q, k, v = q.squeeze(0), k.squeeze(0), v.squeeze(0)
    return VarlenAttention.apply(q, k, v, cu_seqlens, int(max_seqlen), float(scale))
