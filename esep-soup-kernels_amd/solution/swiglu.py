"""SwiGLU activation of the Qwen2 MLP, h = silu(gate) * up, on this repository's HIP kernels
(esep_swiglu_fwd / esep_swiglu_bwd). Public names as in the reference's solution/swiglu.py
(`SwiGLU`, `swiglu`, `patch_qwen2_mlp`; reference swiglu.py:38-81); the organizer's example
Triton kernels there are replaced by the gfx950 kernels in csrc/swiglu.hip.

The kernels compute in fp32 and round once at every store. Device tensors only: a CPU tensor
reaching the kernels raises EsepError (there is no CPU path); the patched MLP leaves CPU inputs
and non-silu activations to HF's own forward.
"""

import functools

import torch

from .body import _hip


def _operands(gate, up):
    """gate and up as dense tensors of one element type (gate's): what the kernels stream."""
    return gate.contiguous(), up.to(dtype=gate.dtype).contiguous()


class SwiGLU(torch.autograd.Function):
    """h = silu(gate) * up, one kernel launch each way. Saved for backward: the two dense
    operands (the backward recomputes the sigmoid from gate)."""

    @staticmethod
    def forward(ctx, gate, up):
        g, u = _operands(gate, up)
        h = torch.empty_like(g)
        _hip.swiglu_fwd(g, u, h)
        ctx.save_for_backward(g, u)
        return h

    @staticmethod
    def backward(ctx, dh):
        g, u = ctx.saved_tensors
        dg, du = torch.empty_like(g), torch.empty_like(u)
        _hip.swiglu_bwd(dh.to(dtype=g.dtype).contiguous(), g, u, dg, du)
        return dg, du


def swiglu(gate, up):
    """silu(gate) * up, differentiable, on the HIP kernels."""
    return SwiGLU.apply(gate, up)


def _silu_mlp(mlp):
    config = getattr(mlp, "config", None)
    return getattr(config, "hidden_act", "silu") == "silu"


def patch_qwen2_mlp():
    """Route transformers' Qwen2MLP.forward through `swiglu` (a class patch, so models built
    before or after it both use it; calling it again changes nothing). HF's forward stays
    reachable as forward.__wrapped__ and serves CPU inputs and other activations."""
    from transformers.models.qwen2 import modeling_qwen2

    cls = modeling_qwen2.Qwen2MLP
    if getattr(cls.forward, "_esep_swiglu", False):
        return
    hf_forward = cls.forward

    @functools.wraps(hf_forward)
    def forward(self, x):
        if not (x.is_cuda and _silu_mlp(self)):
            return hf_forward(self, x)
        return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x)))

    forward._esep_swiglu = True
    cls.forward = forward
