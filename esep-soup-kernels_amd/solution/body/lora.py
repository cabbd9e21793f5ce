"""LoRA terms of q_proj / v_proj with dropout on the LoRA input, on this repository's HIP
dropout kernels (esep_lora_dropout_fwd / esep_lora_dropout_bwd) around vendor-BLAS products.

Public API as in the reference's solution/body/lora.py (reference lora.py:140-359):
new_dropout_key, cast_lora_weights, lora_dropout, lora_down_fwd, lora_down_bwd, lora_delta,
lora_up_bwd, LoRAFunction, LoRADeltaFunction, lora_params, lora_forward, with the same
arguments, saved tensors and gradient dtypes.

The term (peft's LoRA Linear under autocast; A [r, in] and B [out, r] without bias):

    term = scaling * (drop(x) @ A^T) @ B^T,   drop(x) = x * keep / (1 - p)

keep is Bernoulli(1 - p) per element of the LoRA input only (the base projection sees the
undropped x); p comes from the peft module and applies only while its nn.Dropout is in
training mode. Every forward call draws a fresh 63-bit key from torch's device generator (no
host sync; torch.manual_seed reproduces it) and the mask is a pure function of (key, element),
so the backward regenerates it from the saved key instead of storing it. The bits differ from
torch's own dropout stream; the law is the same.

Gradients (xa = drop(x) A^T, dterm the incoming gradient):
    dxa = scaling * dterm @ B        dB = scaling * dterm^T @ xa   (fp32)
    dA  = dxa^T @ drop(x)  (fp32)    dx = (dxa @ A) * keep / (1 - p)
The products run on the vendor BLAS; the HIP kernels regenerate the mask and do the
element-wise passes. Compute dtype: fp16 (the reference's), or bf16 when x is bf16.

LoRAFunction adds the term to the base projection's output (in place when that output is a
fresh dense tensor of the compute dtype: v_proj); LoRADeltaFunction returns the term alone
(q_proj: the RoPE kernel adds it to q, norm_rope.rope(q_delta=...)). Saved for backward by
both: x, xa, the compute-dtype A and B, and the key.
"""

import torch

from . import _hip

_KEY_RANGE = 2 ** 63 - 1


def _compute_dtype(x):
    return torch.bfloat16 if x.dtype == torch.bfloat16 else torch.float16


def new_dropout_key(device):
    """A fresh 63-bit dropout key drawn from torch's generator on `device` (stays there)."""
    return torch.randint(0, _KEY_RANGE, (1,), device=device, dtype=torch.int64)


def cast_lora_weights(weight_a, weight_b, dtype=torch.float16):
    """A and B in the compute dtype, detached (they are r x in and out x r: tiny)."""
    return weight_a.detach().to(dtype), weight_b.detach().to(dtype)


def lora_dropout(x, key, p):
    """x * keep / (1 - p) for a dense 16-bit x, the mask given by `key` (p > 0)."""
    out = torch.empty_like(x)
    _hip.lora_dropout_fwd(x, key, out, p)
    return out


_OUT_DTYPE_OK = True


def _mm_fp32(a, b):
    """a @ b returned in fp32: the BLAS writes fp32 where torch.mm takes out_dtype, else the
    16-bit product is widened (autocast's result)."""
    global _OUT_DTYPE_OK
    if _OUT_DTYPE_OK:
        try:
            return torch.mm(a, b, out_dtype=torch.float32)
        except (RuntimeError, TypeError):
            _OUT_DTYPE_OK = False
    return torch.mm(a, b).float()


def lora_down_fwd(x, a16, key, p):
    """xa = drop(x) @ A^T for a dense x [T, in] (no dropout pass when p == 0)."""
    return torch.mm(lora_dropout(x, key, p) if p > 0.0 else x, a16.t())


def lora_down_bwd(x, a16, dxa, key, p, need_dx=True, dx_accum=None):
    """Backward of lora_down_fwd: (dx or None, dA fp32 [r, in]). With dx_accum (a dense
    [T, in] buffer, e.g. the base projection's dx) the LoRA part of dx is added into it in
    place and it is returned as dx."""
    if not need_dx:
        dropped = lora_dropout(x, key, p) if p > 0.0 else x
        return None, _mm_fp32(dxa.t(), dropped)
    if p == 0.0:
        dx = torch.mm(dxa, a16) if dx_accum is None else dx_accum.addmm_(dxa, a16)
        return dx, _mm_fp32(dxa.t(), x)
    # one kernel pass: the regenerated dropped input (for dA) and the masked, scaled dx,
    # written over the product itself unless it accumulates into dx_accum
    g = torch.mm(dxa, a16)
    dropped = torch.empty_like(x)
    dx = g if dx_accum is None else dx_accum
    _hip.lora_dropout_bwd(x, g, key, dropped, dx, p, accumulate=dx_accum is not None)
    return dx, _mm_fp32(dxa.t(), dropped)


def lora_delta(xa, b16, scaling):
    """The term scaling * xa @ B^T on its own."""
    term = torch.mm(xa, b16.t())
    return term.mul_(scaling)


def lora_up_bwd(dout, xa, b16, scaling):
    """(dxa [T, r], dB fp32 [out, r]) for the term's gradient dout."""
    return torch.mm(dout, b16).mul_(scaling), _mm_fp32(dout.t(), xa).mul_(scaling)


def _rows(t, dtype):
    """t [..., k] as a dense [rows, k] tensor of dtype."""
    flat = t.reshape(-1, t.shape[-1])
    return flat.to(dtype).contiguous() if flat.dtype != dtype else flat.contiguous()


def _rows_mm(t, dtype):
    """t [..., k] as a [rows, k] matrix of dtype for torch's products, which take a row stride:
    a 2-D view with unit column stride (such as a column block of a wider gradient) is used as
    it is, anything else as _rows gives it."""
    if t.dim() == 2 and t.dtype == dtype and t.stride(1) == 1 and t.stride(0) >= t.shape[1]:
        return t
    return _rows(t, dtype)


class _LoRATerm:
    """The parts both Functions share: set up the forward (compute dtype, casts, key, xa) and
    turn the term's gradient into (dx, dA, dB) in the dtypes autograd expects."""

    @staticmethod
    def begin(ctx, x, weight_a, weight_b, p, scaling):
        dtype = _compute_dtype(x)
        x2 = _rows(x, dtype)
        a16, b16 = cast_lora_weights(weight_a, weight_b, dtype)
        key = new_dropout_key(x2.device) if p > 0.0 else None
        xa = lora_down_fwd(x2, a16, key, p)
        ctx.save_for_backward(x2, xa, a16, b16, key)
        ctx.p, ctx.scaling, ctx.dtype = p, scaling, dtype
        ctx.x_shape, ctx.x_dtype = x.shape, x.dtype
        ctx.a_dtype, ctx.b_dtype = weight_a.dtype, weight_b.dtype
        return xa, b16

    @staticmethod
    def grads(ctx, dterm, x_index, a_index):
        x2, xa, a16, b16, key = ctx.saved_tensors
        dxa, db = lora_up_bwd(_rows_mm(dterm, ctx.dtype), xa, b16, ctx.scaling)
        dx, da = lora_down_bwd(x2, a16, dxa, key, ctx.p, need_dx=ctx.needs_input_grad[x_index])
        need = ctx.needs_input_grad
        return (dx.view(ctx.x_shape).to(ctx.x_dtype) if dx is not None else None,
                da.to(ctx.a_dtype) if need[a_index] else None,
                db.to(ctx.b_dtype) if need[a_index + 1] else None)


class LoRAFunction(torch.autograd.Function):
    """apply(x, base, weight_a, weight_b, p, scaling) -> base + term. The term is added into
    base's own buffer when base is a fresh dense (non-view) tensor of the compute dtype (it is
    then marked dirty); otherwise a new tensor is returned."""

    @staticmethod
    def forward(ctx, x, base, weight_a, weight_b, p, scaling):
        xa, b16 = _LoRATerm.begin(ctx, x, weight_a, weight_b, p, scaling)
        ctx.base_dtype = base.dtype
        if base.dtype == ctx.dtype and base.is_contiguous() and not base._is_view():
            base.view(-1, base.shape[-1]).addmm_(xa, b16.t(), alpha=scaling)
            ctx.mark_dirty(base)
            return base
        flat = base.reshape(-1, base.shape[-1]).to(ctx.dtype)
        return torch.addmm(flat, xa, b16.t(), alpha=scaling).view(base.shape)

    @staticmethod
    def backward(ctx, dout):
        dx, da, db = _LoRATerm.grads(ctx, dout, 0, 2)
        dbase = dout.to(ctx.base_dtype) if ctx.needs_input_grad[1] else None
        return dx, dbase, da, db, None, None


class LoRADeltaFunction(torch.autograd.Function):
    """apply(x, weight_a, weight_b, p, scaling) -> term alone, shaped [..., out]; its gradient
    is the gradient of q before the rotation (the RoPE kernel adds the term to q)."""

    @staticmethod
    def forward(ctx, x, weight_a, weight_b, p, scaling):
        xa, b16 = _LoRATerm.begin(ctx, x, weight_a, weight_b, p, scaling)
        term = lora_delta(xa, b16, scaling)
        return term.view(*x.shape[:-1], term.shape[-1])

    @staticmethod
    def backward(ctx, dterm):
        dx, da, db = _LoRATerm.grads(ctx, dterm, 0, 1)
        return dx, da, db, None, None


def _dropout_p(drop):
    """The dropout probability in effect for a peft LoRA dropout module, or None when it is a
    module this path does not implement."""
    if isinstance(drop, torch.nn.Identity):
        return 0.0
    if isinstance(drop, torch.nn.Dropout):
        return float(drop.p) if drop.training else 0.0
    return None


def _single_plain_adapter(module, adapter):
    """The adapter is the only active one, present, unmerged, enabled, not a DoRA / variant."""
    if getattr(module, "disable_adapters", False) or getattr(module, "merged", False):
        return False
    if list(getattr(module, "active_adapters", [adapter])) != [adapter]:
        return False
    if adapter not in module.lora_A or adapter in getattr(module, "lora_variant", {}):
        return False
    return not getattr(module, "use_dora", {}).get(adapter, False)


def lora_params(module, adapter="default"):
    """(A weight, B weight, dropout p in effect, scaling) of a peft LoRA layer, or None when the
    layer uses something this path does not implement: a bias on A or B, DoRA or another
    variant, several active adapters, a merged or disabled adapter, a dropout other than
    nn.Dropout / nn.Identity, p >= 1, or a scaling that is not a plain number
    (reference lora.py:319-343)."""
    if not _single_plain_adapter(module, adapter):
        return None
    down, up = module.lora_A[adapter], module.lora_B[adapter]
    if down.bias is not None or up.bias is not None:
        return None
    p = _dropout_p(module.lora_dropout[adapter])
    scale = module.scaling[adapter]
    if p is None or p >= 1.0 or isinstance(scale, bool) or not isinstance(scale, (int, float)):
        return None
    return down.weight, up.weight, p, float(scale)


def lora_forward(module, x, base_out, adapter="default"):
    """base_out + the LoRA term of a peft LoRA layer for input x (base_out, the base
    projection's fresh output, is updated in place when it can be); None when the layer or
    the input is not supported (the caller then runs peft's own forward)."""
    params = lora_params(module, adapter)
    if params is None or not x.is_cuda:
        return None
    weight_a, weight_b, p, scaling = params
    return LoRAFunction.apply(x, base_out, weight_a, weight_b, p, scaling)
