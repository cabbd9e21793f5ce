"""NF4 (double-quant) dequantization and the NF4 linear on this repository's HIP kernel: the
reference's solution/nf4 API (dequantize_nf4, dequantize_nf4_multi, supported, nf4_linear,
NF4Linear) with the Triton dequant replaced by esep_nf4_dequant.

A quant state is anything with bitsandbytes' QuantState attributes: quant_type ("nf4"),
blocksize (64), nested (True), shape (N, K), absmax (uint8 [N*K/64]), code (fp32 [16], the NF4
table), offset (fp32 scalar tensor), state2 with absmax (fp32 [ceil(nb/256)]), code (fp32 [256])
and blocksize (256). bitsandbytes is not installed in this build's environment, so the
reference's Linear4bit class patch (solution/nf4/__init__.py: patch, linear4bit,
linear4bit_multi, dequant_multi) has nothing to patch here and is not provided; the
dequantization and the autograd linear are.
"""

import torch

from ..body import _hip

__all__ = ["supported", "dequantize_nf4", "dequantize_nf4_multi", "nf4_linear", "NF4Linear"]


def supported(quant_state) -> bool:
    """True when dequantize_nf4 handles this quant state (NF4, double quant, blocksize 64 / 256,
    2-D shape with N*K a multiple of 64, on the GPU) (reference dequant.py:70-79)."""
    try:
        return (quant_state.quant_type == "nf4" and quant_state.blocksize == 64
                and quant_state.nested and quant_state.state2.blocksize == 256
                and len(quant_state.shape) == 2
                and (quant_state.shape[0] * quant_state.shape[1]) % 64 == 0
                and quant_state.absmax.is_cuda)
    except AttributeError:
        return False


def _offset(qs):
    off = qs.offset
    if not isinstance(off, torch.Tensor):
        off = torch.tensor([float(off)], dtype=torch.float32, device=qs.absmax.device)
    return off.reshape(1).to(torch.float32)


def dequantize_nf4(packed, quant_state, out=None, dtype=torch.float16):
    """W [N, K] (fp16 by default, as the reference; bf16 / fp32 too) from a packed NF4 weight
    (any view of its N*K/2 bytes) and its quant state. Caller guarantees supported(quant_state)."""
    shape = tuple(quant_state.shape)
    if out is None:
        out = torch.empty(shape, dtype=dtype, device=packed.device)
    qs2 = quant_state.state2
    _hip.nf4_dequant(packed.reshape(-1) if packed.is_contiguous() else packed.contiguous().reshape(-1),
                     quant_state.absmax, qs2.absmax.to(torch.float32).contiguous(),
                     qs2.code.to(torch.float32).contiguous(), _offset(quant_state),
                     quant_state.code.to(torch.float32).contiguous(), out.reshape(-1))
    return out


def dequantize_nf4_multi(weights, quant_states, out=None, dtype=torch.float16):
    """W_cat = cat([dequantize_nf4(w, qs) ...], 0) written straight into one [sum N_i, K] buffer
    by one launch (esep_nf4_dequant_multi, up to 8 weights per launch; the reference's
    multi-weight kernel takes 3, dequant.py:116-205); each slice bit-identical to
    dequantize_nf4."""
    K = quant_states[0].shape[1]
    if any(qs.shape[1] != K for qs in quant_states):
        raise ValueError("weights must share K")
    n_total = sum(qs.shape[0] for qs in quant_states)
    if out is None:
        out = torch.empty((n_total, K), dtype=dtype, device=weights[0].device)
    items, r = [], 0
    for w, qs in zip(weights, quant_states):
        qs2 = qs.state2
        items.append((w.reshape(-1) if w.is_contiguous() else w.contiguous().reshape(-1),
                      qs.absmax.contiguous(), qs2.absmax.to(torch.float32).contiguous(),
                      qs2.code.to(torch.float32).contiguous(), _offset(qs),
                      qs.code.to(torch.float32).contiguous(), out[r:r + qs.shape[0]].reshape(-1)))
        r += qs.shape[0]
    for i in range(0, len(items), _hip.NF4_MULTI_MAX):
        _hip.nf4_dequant_multi(items[i:i + _hip.NF4_MULTI_MAX])
    return out


class NF4Linear(torch.autograd.Function):
    """y = x W^T (+ bias) with W dequantized from NF4 in forward and again in backward (frozen
    weight: nothing of W is saved; dx = dy W) (reference solution/nf4/autograd.py)."""

    @staticmethod
    def forward(ctx, x, packed, quant_state, bias):
        w = dequantize_nf4(packed, quant_state, dtype=x.dtype if x.dtype != torch.float32 else torch.float16)
        x2 = x if x.dtype == w.dtype else x.to(w.dtype)
        y = torch.nn.functional.linear(x2, w, None if bias is None else bias.to(w.dtype))
        ctx.packed, ctx.qs, ctx.x_dtype, ctx.w_dtype = packed, quant_state, x.dtype, w.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        dx = None
        if ctx.needs_input_grad[0]:
            w = dequantize_nf4(ctx.packed, ctx.qs, dtype=ctx.w_dtype)
            dx = torch.matmul(dy.to(ctx.w_dtype), w).to(ctx.x_dtype)
        return dx, None, None, None


def nf4_linear(x, packed, quant_state, bias=None):
    return NF4Linear.apply(x, packed, quant_state, bias)
