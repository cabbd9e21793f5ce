"""LoRA path of q_proj / v_proj on this repository's HIP dropout kernels: the reference's
solution/body/lora.py API (same names, arguments, saved tensors and gradient dtypes), with the
Triton dropout kernels replaced by esep_lora_dropout_fwd / esep_lora_dropout_bwd.

What it computes (peft's LoRA Linear forward under autocast, reference lora.py:1-52):

    out = base + scaling * (dropout(x) @ A^T) @ B^T,   A [r, in], B [out, r], no bias

* dropout(x) = x * keep / (1 - p), keep Bernoulli(1 - p) per element, applied to the LoRA input
  only (the base projection sees the undropped x). p is read from the peft module and dropout
  runs only when that nn.Dropout is in training mode with p > 0.
* A fresh mask on every forward call: each call draws a new 63-bit key from torch's CUDA
  generator (a one-element device tensor; no host sync), so the stream follows
  torch.manual_seed. The mask is a pure function of (key, element): the backward regenerates it
  from the saved key; neither the mask nor the dropped x is stored between the passes.
* Individual bits differ from torch's own dropout (another Philox stream); the law is the same.

Math (x_d = dropout(x)): xa = x_d A^T; out = base + scaling xa B^T; dxa = scaling dout B;
dB = scaling dout^T xa; dA = dxa^T x_d (x_d regenerated); dx = (dxa A) * keep / (1 - p). The
matmuls run on the vendor BLAS (torch.mm); the HIP kernels do the memory-bound parts.

Compute dtype: fp16 as in the reference, or bf16 when x is bf16 (the reference is fp16-only).
Saved for backward: x, xa, the compute-dtype copies of A and B, and the 8-byte key.

Two autograd Functions: LoRAFunction (v_proj: the LoRA term added in place into the fresh base
output) and LoRADeltaFunction (q_proj: the LoRA term alone, added to q inside the RoPE kernel,
norm_rope.rope(q_delta=...)).
"""

import torch

from . import _hip

_KEY_HIGH = 2 ** 63 - 1


def _cdt(x):
    return torch.bfloat16 if x.dtype == torch.bfloat16 else torch.float16


def new_dropout_key(device):
    """One fresh 63-bit key from torch's CUDA generator, kept on the device (no sync)."""
    return torch.randint(0, _KEY_HIGH, (1,), device=device, dtype=torch.int64)


def cast_lora_weights(weight_a, weight_b, dtype=torch.float16):
    """Compute-dtype copies of A [r, in] and B [out, r] (torch casts: the tensors are tiny)."""
    return weight_a.detach().to(dtype), weight_b.detach().to(dtype)


def lora_dropout(x, key, p):
    """dropout(x) for a contiguous fp16 / bf16 x with the mask defined by key (p > 0)."""
    xd = torch.empty_like(x)
    _hip.lora_dropout_fwd(x, key, xd, p)
    return xd


def lora_down_fwd(x, a16, key, p):
    """xa = dropout(x) @ A^T. x [T, in] contiguous -> xa [T, r]."""
    if p > 0.0:
        return torch.mm(lora_dropout(x, key, p), a16.t())
    return torch.mm(x, a16.t())


def lora_down_bwd(x, a16, dxa, key, p, need_dx=True, dx_accum=None):
    """Backward of lora_down_fwd. Returns (dx or None, dA fp32 [r, in]).

    dx_accum: optional contiguous [T, in] buffer (e.g. the dx of the base projection); when
    given, the LoRA part of dx is added into it in place and it is returned as dx."""
    if p > 0.0 and need_dx:
        xd = torch.empty_like(x)
        g = torch.mm(dxa, a16)
        accumulate = dx_accum is not None
        dx = dx_accum if accumulate else g  # g is overwritten in place when not accumulating
        _hip.lora_dropout_bwd(x, g, key, xd, dx, p, accumulate=accumulate)
    elif p > 0.0:
        xd = lora_dropout(x, key, p)  # only the regenerated x_d is needed (for dA)
        dx = None
    else:
        xd = x
        if need_dx:
            dx = dx_accum.addmm_(dxa, a16) if dx_accum is not None else torch.mm(dxa, a16)
        else:
            dx = None
    return dx, _mm_f32(dxa.t(), xd)


def lora_delta(xa, b16, scaling):
    """scaling * xa @ B^T without adding it (fused into the RoPE kernel by the caller)."""
    return torch.mm(xa, b16.t()).mul_(scaling)


def lora_up_bwd(dout, xa, b16, scaling):
    """(dxa [T, r], dB fp32 [out, r]); dbase = dout is the caller's."""
    dxa = torch.mm(dout, b16).mul_(scaling)
    db = _mm_f32(dout.t(), xa).mul_(scaling)
    return dxa, db


_MM_OUT_DTYPE = [True]


def _mm_f32(a, b):
    """a @ b with an fp32 result: the BLAS with fp32 output (torch.mm out_dtype) when
    available, else the 16-bit result cast to fp32 (what autocast gives)."""
    if _MM_OUT_DTYPE[0]:
        try:
            return torch.mm(a, b, out_dtype=torch.float32)
        except (RuntimeError, TypeError):
            _MM_OUT_DTYPE[0] = False
    return torch.mm(a, b).float()


def _prep(x, dt):
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype != dt:
        x2 = x2.to(dt)
    return x2.contiguous()


class LoRAFunction(torch.autograd.Function):
    """out = base + scaling * (dropout(x) @ A^T) @ B^T, written into base's buffer when base is a
    fresh contiguous tensor of the compute dtype."""

    @staticmethod
    def forward(ctx, x, base, weight_a, weight_b, p, scaling):
        dt = _cdt(x)
        x2 = _prep(x, dt)
        a16, b16 = cast_lora_weights(weight_a, weight_b, dt)
        key = new_dropout_key(x2.device) if p > 0.0 else None
        xa = lora_down_fwd(x2, a16, key, p)
        if base.is_contiguous() and base.dtype == dt and not base._is_view():
            out = base
            out.view(-1, out.shape[-1]).addmm_(xa, b16.t(), alpha=scaling)
            ctx.mark_dirty(base)
        else:
            base2 = base.reshape(-1, base.shape[-1]).to(dt)
            out = torch.addmm(base2, xa, b16.t(), alpha=scaling).view(base.shape)
        ctx.save_for_backward(x2, xa, a16, b16, key)
        ctx.p, ctx.scaling, ctx.dt = p, scaling, dt
        ctx.x_shape, ctx.x_dtype, ctx.base_dtype = x.shape, x.dtype, base.dtype
        ctx.w_dtypes = (weight_a.dtype, weight_b.dtype)
        return out

    @staticmethod
    def backward(ctx, dout):
        x2, xa, a16, b16, key = ctx.saved_tensors
        dout2 = _prep(dout, ctx.dt)
        dxa, db = lora_up_bwd(dout2, xa, b16, ctx.scaling)
        dx, da = lora_down_bwd(x2, a16, dxa, key, ctx.p, need_dx=ctx.needs_input_grad[0])
        if dx is not None:
            dx = dx.view(ctx.x_shape).to(ctx.x_dtype)
        dbase = dout.to(ctx.base_dtype) if ctx.needs_input_grad[1] else None
        da = da.to(ctx.w_dtypes[0]) if ctx.needs_input_grad[2] else None
        db = db.to(ctx.w_dtypes[1]) if ctx.needs_input_grad[3] else None
        return dx, dbase, da, db, None, None


class LoRADeltaFunction(torch.autograd.Function):
    """delta = scaling * (dropout(x) @ A^T) @ B^T, the LoRA term alone (for q_proj, added to the
    base projection inside the RoPE kernel). Same math and saved tensors as LoRAFunction."""

    @staticmethod
    def forward(ctx, x, weight_a, weight_b, p, scaling):
        dt = _cdt(x)
        x2 = _prep(x, dt)
        a16, b16 = cast_lora_weights(weight_a, weight_b, dt)
        key = new_dropout_key(x2.device) if p > 0.0 else None
        xa = lora_down_fwd(x2, a16, key, p)
        delta = lora_delta(xa, b16, scaling)
        ctx.save_for_backward(x2, xa, a16, b16, key)
        ctx.p, ctx.scaling, ctx.dt = p, scaling, dt
        ctx.x_shape, ctx.x_dtype = x.shape, x.dtype
        ctx.w_dtypes = (weight_a.dtype, weight_b.dtype)
        return delta.view(*x.shape[:-1], delta.shape[-1])

    @staticmethod
    def backward(ctx, ddelta):
        x2, xa, a16, b16, key = ctx.saved_tensors
        d2 = _prep(ddelta, ctx.dt)
        dxa, db = lora_up_bwd(d2, xa, b16, ctx.scaling)
        dx, da = lora_down_bwd(x2, a16, dxa, key, ctx.p, need_dx=ctx.needs_input_grad[0])
        if dx is not None:
            dx = dx.view(ctx.x_shape).to(ctx.x_dtype)
        da = da.to(ctx.w_dtypes[0]) if ctx.needs_input_grad[1] else None
        db = db.to(ctx.w_dtypes[1]) if ctx.needs_input_grad[2] else None
        return dx, da, db, None, None


def lora_params(module, adapter="default"):
    """(A weight, B weight, dropout p in effect now, scaling) of a peft LoRA layer, or None if
    the layer uses anything this path does not implement (bias, DoRA / variants, several active
    adapters, merged or disabled adapters, a dropout that is not nn.Dropout / nn.Identity)
    (reference lora.py:299-331)."""
    if getattr(module, "disable_adapters", False) or getattr(module, "merged", False):
        return None
    if list(getattr(module, "active_adapters", [adapter])) != [adapter]:
        return None
    if adapter not in module.lora_A or adapter in getattr(module, "lora_variant", {}):
        return None
    lin_a, lin_b = module.lora_A[adapter], module.lora_B[adapter]
    if lin_a.bias is not None or lin_b.bias is not None:
        return None
    drop = module.lora_dropout[adapter]
    if isinstance(drop, torch.nn.Dropout):
        p = float(drop.p) if drop.training else 0.0
    elif isinstance(drop, torch.nn.Identity):
        p = 0.0
    else:
        return None
    if p >= 1.0:
        return None
    scaling = module.scaling[adapter]
    if isinstance(scaling, bool) or not isinstance(scaling, (int, float)):
        return None
    if getattr(module, "use_dora", {}).get(adapter, False):
        return None
    return lin_a.weight, lin_b.weight, p, float(scaling)


def lora_forward(module, x, base_out, adapter="default"):
    """base_out + the LoRA term of a peft LoRA layer on input x (base_out is updated in place
    when it is a fresh tensor of the compute dtype). None when the layer is not supported."""
    params = lora_params(module, adapter)
    if params is None or not x.is_cuda:
        return None
    weight_a, weight_b, p, scaling = params
    return LoRAFunction.apply(x, base_out, weight_a, weight_b, p, scaling)
