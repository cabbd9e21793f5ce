"""NF4 (double-quant) dequantization and the NF4 linear on this repository's HIP kernel: the
reference's solution/nf4 API with the Triton dequant replaced by esep_nf4_dequant(_multi).

  supported, dequantize_nf4, dequantize_nf4_multi   the dequantization (reference dequant.py)
  NF4Linear, nf4_linear, NF4MultiLinear             the autograd linears (reference autograd.py)
  linear4bit, linear4bit_multi, dequant_multi       bitsandbytes Linear4bit.forward semantics on
                                                    the kernels, for one module or 2-8 modules
                                                    reading the same input (reference
                                                    __init__.py:80-226)
  patch                                             Linear4bit.forward routed through linear4bit

A quant state is anything with bitsandbytes' QuantState attributes: quant_type ("nf4"),
blocksize (64), nested (True), shape (N, K), absmax (uint8 [N*K/64]), code (fp32 [16], the NF4
table), offset (fp32 scalar tensor), state2 with absmax (fp32 [ceil(nb/256)]), code (fp32 [256])
and blocksize (256). A Linear4bit module is one with bitsandbytes' Linear4bit interface: the
packed weight with its quant_state, compute_dtype, compute_type_is_set and bias. With
bitsandbytes installed that is an instance of bitsandbytes.nn.Linear4bit; bitsandbytes is not
installed in this build's environment, where a module whose class is named Linear4bit with those
attributes is taken as one (is_linear4bit), and patch() has no class to patch.
"""

import functools

import torch

from ..body import _hip

__all__ = ["patch", "linear4bit", "linear4bit_multi", "dequant_multi", "is_linear4bit",
           "supported", "dequantize_nf4", "dequantize_nf4_multi", "nf4_linear", "NF4Linear",
           "NF4MultiLinear", "MIN_ROWS", "MULTI_MAX"]


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
    """y = x W^T + bias with W dequantized from NF4 in forward and again in backward (frozen
    weight: nothing of W is kept; dx = dy W) (reference autograd.py:24-48). x and W in x's
    16-bit dtype (fp16 as the reference; an fp32 x computes with an fp16 W and returns fp16);
    the bias gets its gradient (the sum of dy over the rows, in the bias dtype) when it needs one."""

    @staticmethod
    def forward(ctx, x, packed, bias, quant_state):
        w_dtype = x.dtype if x.dtype != torch.float32 else torch.float16
        w = dequantize_nf4(packed, quant_state, dtype=w_dtype)
        x2 = x if x.dtype == w_dtype else x.to(w_dtype)
        y = torch.nn.functional.linear(x2, w, None if bias is None else bias.to(w_dtype))
        ctx.packed, ctx.qs, ctx.x_dtype, ctx.w_dtype = packed, quant_state, x.dtype, w_dtype
        ctx.bias_dtype = None if bias is None else bias.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        dx = dbias = None
        if ctx.needs_input_grad[2]:
            dbias = dy.reshape(-1, dy.shape[-1]).sum(0, dtype=ctx.bias_dtype)
        if ctx.needs_input_grad[0]:
            w = dequantize_nf4(ctx.packed, ctx.qs, dtype=ctx.w_dtype)
            dx = torch.matmul(dy.to(ctx.w_dtype), w).to(ctx.x_dtype)
        return dx, None, dbias, None


def nf4_linear(x, packed, bias, quant_state):
    """x (any leading dims) -> x W^T + bias for an NF4 weight (reference autograd.py:51-53)."""
    return NF4Linear.apply(x, packed, bias, quant_state)


class NF4MultiLinear(torch.autograd.Function):
    """Y_cat = x W_cat^T + bias_cat for several NF4 weights reading the same x (fused q/k/v, or
    gate/up): W_cat from one esep_nf4_dequant_multi launch, one GEMM; backward re-dequantizes
    W_cat (one launch) for one dX GEMM (reference autograd.py:56-92). group = (packed weights,
    quant states, bias dtype), not differentiable; x fp16."""

    @staticmethod
    def forward(ctx, x, bias_cat, group):
        weights, states, _ = group
        w = dequantize_nf4_multi(weights, states)
        ctx.group = group
        return torch.nn.functional.linear(x, w, bias_cat)

    @staticmethod
    def backward(ctx, dy):
        weights, states, bias_dtype = ctx.group
        dx = dbias = None
        if ctx.needs_input_grad[1]:
            dbias = dy.reshape(-1, dy.shape[-1]).sum(0, dtype=bias_dtype)
        if ctx.needs_input_grad[0]:
            w = dequantize_nf4_multi(weights, states)
            dx = torch.matmul(dy if dy.dtype == w.dtype else dy.to(w.dtype), w)
        return dx, dbias, None


# ----------------------------------------------------------------------------------------------
# bitsandbytes Linear4bit.forward on the kernels (reference solution/nf4/__init__.py:41-245)
# ----------------------------------------------------------------------------------------------
# Below this many rows bitsandbytes runs its own small-batch kernels; those calls stay with it.
MIN_ROWS = 8
# Modules per fused call: one esep_nf4_dequant_multi launch takes up to this many weights.
MULTI_MAX = _hip.NF4_MULTI_MAX

_FP16, _FP32 = torch.float16, torch.float32
_orig_forward = None  # Linear4bit.forward as it was before patch()


@functools.cache
def _bnb_class():
    """bitsandbytes.nn.Linear4bit, or None where bitsandbytes is not installed. Looked up once
    per process: Python does not remember a failed import, so without bitsandbytes every
    lookup would search sys.path again (the packed decoder asks ten times per layer)."""
    try:
        from bitsandbytes.nn import Linear4bit
    except Exception:
        return None
    return Linear4bit


def _qs_ok(qs):
    """supported(qs), memoized on the state object."""
    ok = getattr(qs, "_esep_nf4_ok", None)
    if ok is None:
        ok = supported(qs)
        try:
            qs._esep_nf4_ok = ok
        except AttributeError:
            pass
    return ok


def is_linear4bit(module):
    """True for a module with bitsandbytes' Linear4bit interface whose weight this package
    decodes (see the module docstring for what counts as one without bitsandbytes)."""
    cls = _bnb_class()
    if cls is not None:
        if not isinstance(module, cls):
            return False
    elif type(module).__name__ != "Linear4bit":
        return False
    qs = getattr(getattr(module, "weight", None), "quant_state", None)
    return (qs is not None and hasattr(module, "compute_dtype")
            and hasattr(module, "compute_type_is_set") and _qs_ok(qs))


def _original(module, x):
    """The module's own forward: bitsandbytes' (the one patch() replaced, if it did)."""
    if _orig_forward is not None:
        return _orig_forward(module, x)
    return type(module).forward(module, x)


def _fallback(module, x, keep_fp16):
    out = _original(module, x)
    return out.to(_FP16) if keep_fp16 else out


def _fp16_autocast():
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") is _FP16


def linear4bit(x, module, keep_fp16=False):
    """bitsandbytes Linear4bit.forward(module, x) with the NF4 matmul on the HIP dequant
    (NF4Linear): x cast to the compute dtype fp16 (bitsandbytes' in-place bias.data cast
    included), or, for compute dtype fp32 under fp16 CUDA autocast, the fp16 GEMM autocast would
    run on bitsandbytes' fp32 dequant (the same fp16 W). Output in x's dtype, or with keep_fp16
    the fp16 output before that cast. Anything else (no quant state or one the kernel does not
    decode, compute dtype not set, a CPU x, fewer than MIN_ROWS rows, another compute dtype) runs
    the module's own forward (.to(fp16) with keep_fp16). Reference __init__.py:80-118."""
    qs = getattr(module.weight, "quant_state", None)
    if (qs is None or not getattr(module, "compute_type_is_set", False) or not x.is_cuda
            or not _qs_ok(qs)):
        return _fallback(module, x, keep_fp16)
    K = x.shape[-1]
    if K != qs.shape[1] or x.numel() < MIN_ROWS * K:
        return _fallback(module, x, keep_fp16)
    cd, inp_dtype, bias = module.compute_dtype, x.dtype, module.bias
    if cd is _FP16:
        x = x.to(_FP16)
        if bias is not None and bias.dtype != _FP16:
            bias.data = bias.data.to(_FP16)  # what bitsandbytes' forward does to the bias
    elif cd is _FP32 and _fp16_autocast():
        x = x.to(_FP16)
        if bias is not None:
            if bias.dtype != _FP32:
                bias.data = bias.data.to(_FP32)
            bias = bias.to(_FP16)  # the cast autocast makes inside F.linear
    else:
        return _fallback(module, x, keep_fp16)
    out = NF4Linear.apply(x, module.weight, bias, qs)
    return out if keep_fp16 else out.to(inp_dtype)


_GROUP_ATTR = "_esep_nf4_group"


def _group_cache(modules):
    """Per-group cache (fp16 bias_cat of frozen biases), kept on the first module."""
    d = modules[0].__dict__.setdefault(_GROUP_ATTR, {})
    return d.setdefault(tuple(id(m) for m in modules), {})


def _multi_states(modules, K=None):
    """The modules' quant states when one multi-weight dequant serves them all, else None."""
    if not 2 <= len(modules) <= MULTI_MAX:
        return None
    states = []
    for m in modules:
        qs = getattr(m.weight, "quant_state", None)
        if qs is None or not _qs_ok(qs):
            return None
        states.append(qs)
    K = states[0].shape[1] if K is None else K
    return states if all(qs.shape[1] == K for qs in states) else None


def dequant_multi(modules):
    """fp16 W_cat [sum N_i, K] = cat of the modules' dequantized NF4 weights, row-major, from one
    esep_nf4_dequant_multi launch (each row block bit-exact with dequantize_nf4 of its module);
    weights the kernel does not decode come from the module's own dequantization (bitsandbytes'
    dequantize_4bit) instead. No autograd. Reference __init__.py:136-158."""
    modules = tuple(modules)
    states = _multi_states(modules)
    if states is not None:
        return dequantize_nf4_multi([m.weight for m in modules], states)
    parts = []
    for m in modules:
        qs = m.weight.quant_state
        if _qs_ok(qs):
            parts.append(dequantize_nf4(m.weight, qs))
        else:
            import bitsandbytes.functional as bnb_f

            parts.append(bnb_f.dequantize_4bit(m.weight, qs).to(_FP16))
    return torch.cat(parts, 0)


def _multi_fallback(x, modules, split):
    outs = [linear4bit(x, m, keep_fp16=True) for m in modules]
    return tuple(outs) if split else torch.cat(outs, -1)


def linear4bit_multi(x, modules, split=True):
    """cat([linear4bit(x, m, keep_fp16=True) for m in modules], -1) for 2-8 Linear4bit modules
    reading the same x, as one dequant launch into W_cat and one GEMM (NF4MultiLinear; backward
    one re-dequant and one dX GEMM). fp16 out; split=True gives one column view of Y_cat per
    module (autograd's split backward cats their grads into one dY_cat), split=False Y_cat.
    Conditions per module as linear4bit's, one K, and all or none with a bias (bias_cat cached
    per group while the biases are frozen and unchanged; built per call when one trains). Else
    the separate linear4bit calls. Reference __init__.py:165-226."""
    modules = tuple(modules)
    K = x.shape[-1]
    if len(modules) < 2 or not x.is_cuda or x.numel() < MIN_ROWS * K:
        return _multi_fallback(x, modules, split)
    states = _multi_states(modules, K)
    if states is None:
        return _multi_fallback(x, modules, split)
    biases = []
    for m in modules:
        if not getattr(m, "compute_type_is_set", False):
            return _multi_fallback(x, modules, split)
        if not (m.compute_dtype is _FP16 or (m.compute_dtype is _FP32 and _fp16_autocast())):
            return _multi_fallback(x, modules, split)
        biases.append(m.bias)
    with_bias = [b is not None for b in biases]
    if any(with_bias) and not all(with_bias):
        return _multi_fallback(x, modules, split)
    bias_cat = None
    if with_bias[0]:
        for m, b in zip(modules, biases):  # bitsandbytes' in-place casts, as in linear4bit
            want = _FP16 if m.compute_dtype is _FP16 else _FP32
            if b.dtype != want:
                b.data = b.data.to(want)
        if any(b.requires_grad for b in biases):
            bias_cat = torch.cat([b.to(_FP16) for b in biases])  # gradients reach each bias
        else:
            cache = _group_cache(modules)
            key = tuple((b.data_ptr(), b._version, b.dtype) for b in biases)
            hit = cache.get("bias")
            if hit is None or hit[0] != key:
                with torch.no_grad():
                    hit = cache["bias"] = (key, torch.cat([b.to(_FP16) for b in biases]))
            bias_cat = hit[1]
    group = ([m.weight for m in modules], states, None if bias_cat is None else bias_cat.dtype)
    y = NF4MultiLinear.apply(x.to(_FP16), bias_cat, group)
    return y.split([qs.shape[0] for qs in states], -1) if split else y


def _forward(self, x):
    return linear4bit(x, self)


_forward._esep_nf4 = True


def patch():
    """Route bitsandbytes' Linear4bit.forward through linear4bit (a class patch, so peft's LoRA
    wrapper, which calls its base layer, takes it too). Idempotent; False without bitsandbytes.
    Reference __init__.py:233-245."""
    global _orig_forward
    cls = _bnb_class()
    if cls is None:
        return False
    if getattr(cls.forward, "_esep_nf4", False):
        return True
    _orig_forward = cls.forward
    cls.forward = _forward
    return True
