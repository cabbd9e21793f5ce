"""Fused SwiGLU, silu(gate) * up, for the Qwen2 MLP on this repository's HIP kernels
(esep_swiglu_fwd / esep_swiglu_bwd): the same API as the reference's solution/swiglu.py
(SwiGLU, swiglu, patch_qwen2_mlp), with the example Triton kernels replaced.

fp32 math inside, one rounding at each store. CUDA tensors only: anything else raises
EsepError (no CPU path).
"""

import torch

from .body import _hip


class SwiGLU(torch.autograd.Function):
    """silu(gate) * up in one launch each way (saves gate and up for the backward)."""

    @staticmethod
    def forward(ctx, gate, up):
        gate = gate.contiguous()
        up = up.to(gate.dtype).contiguous()
        out = torch.empty_like(gate)
        _hip.swiglu_fwd(gate, up, out)
        ctx.save_for_backward(gate, up)
        return out

    @staticmethod
    def backward(ctx, grad):
        gate, up = ctx.saved_tensors
        grad = grad.to(gate.dtype).contiguous()
        dgate, dup = torch.empty_like(gate), torch.empty_like(up)
        _hip.swiglu_bwd(grad, gate, up, dgate, dup)
        return dgate, dup


def swiglu(gate, up):
    return SwiGLU.apply(gate, up)


def patch_qwen2_mlp():
    """Send Qwen2MLP.forward through the fused kernel (class patch; idempotent). Models whose
    activation is not silu, or CPU inputs, keep HF's forward."""
    from transformers.models.qwen2 import modeling_qwen2

    cls = modeling_qwen2.Qwen2MLP
    if getattr(cls.forward, "_esep_swiglu", False):
        return
    original = cls.forward

    def forward(self, x):
        act = getattr(getattr(self, "config", None), "hidden_act", "silu")
        if act != "silu" or not x.is_cuda:
            return original(self, x)
        return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x)))

    forward._esep_swiglu = True
    forward.__wrapped__ = original
    cls.forward = forward
