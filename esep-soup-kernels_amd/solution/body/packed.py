"""The reference's patch point (solution/body/packed.py): Qwen2Model.forward replaced by a
pad-free decoder whose norms, RoPE, attention and SwiGLU run on this repository's HIP kernels.

`patch()` swaps Qwen2Model.forward (a class patch; the original stays reachable as
forward.__wrapped__). For a training-style call (2-D CUDA input_ids and attention mask, no
cache, no captured hidden states or attentions) the real tokens of all rows are gathered into
one packed [1, T, H] stream, every token-wise piece of the decoder layers runs on those T
tokens, attention runs causally within each original row, and the final hidden states are
scattered back to [B, L, H] with zeros at the pads. Any other call runs the original forward.

Per decoder layer, each piece has a guard and an HF / torch fallback (warned once per
(piece, reason) while training; reference packed.py:62-96):
  norms       norm_rope.add_rmsnorm: residual add fused into the RMSNorm on an fp32 residual
              stream; the decoder-layer norms return one copy of their output per consumer (5 after
              the input norm: q / k / v projections and the q / v LoRA inputs; 2 after the
              post-attention norm: gate and up) so their gradients are summed in the norm
              backward. A trainable norm weight stays on the kernel (its gradient comes from the
              kernel's two-stage reduction); the reference hands it to HF (its packed.py:129).
  q/k/v/o     the model's projections; a peft-style LoRA projection (base_layer + lora_A /
              lora_B / lora_dropout / scaling, one active adapter) runs its base layer directly
              and its LoRA term on lora.py: v's added into the base output, q's passed to the
              RoPE kernel as q_delta (reference packed.py:240-352). NF4 base layers
              (bitsandbytes' Linear4bit interface, solution.nf4) run through nf4.linear4bit on
              the HIP dequant, and q/k/v on NF4 bases as one nf4.linear4bit_multi call (one
              dequant launch and one GEMM) on the input norm's output (reference :184-352);
              q/k/v on plain nn.Linear bases likewise as one GEMM against their concatenated
              weights (FUSE_QKV; the reference runs those three apart).
  RoPE        norm_rope.rope on the packed positions with the model's inv_freq.
  attention   attention.varlen_attention over all rows in one launch per direction; else a
              per-row SDPA loop (reference packed.py:404-436).
  MLP         frozen plain or NF4 projections: _RecomputeMLP (no [T, intermediate] tensor
              saved; NF4 weights dequantized on the HIP kernel, gate and up in one launch);
              otherwise the projections with the HIP SwiGLU, gate and up fed from their own
              copies of the norm output.
"""

import contextlib
import functools
import logging

import torch
import torch.nn.functional as F

log = logging.getLogger(__name__)

# Switches read at call time (never from the environment), as the reference's: USE_KERNELS
# (packed.py:106) turns every HIP piece off (the packed layout on torch ops);
# NORM_SAVE_OUTPUT (:149) makes the decoder-layer norms save their 16-bit output instead of
# the fp32 residual; USE_LORA_KERNELS (:186) runs LoRA projections as modules when off;
# RECOMPUTE_MLP (:448) sends frozen MLPs through _RecomputeMLP. FUSE_QKV (this build's) runs
# plain nn.Linear q / k / v bases as one GEMM against their concatenated weights (_qkv).
USE_KERNELS = True
NORM_SAVE_OUTPUT = True
USE_LORA_KERNELS = True
RECOMPUTE_MLP = True
FUSE_QKV = True

_KERNEL_FLOATS = (torch.float16, torch.bfloat16, torch.float32)

# Keyword arguments of Qwen2Model.forward that a training step may pass and that the packed
# path can ignore (reference packed.py:59-60); any other one selects the original forward.
_IGNORED_KWARGS = {"num_items_in_batch", "return_dict", "output_attentions",
                   "output_hidden_states", "is_causal"}

# Messages already logged by this process (keys: "active", a full-fallback reason, or
# "piece: reason"); a module-level set so that tests can reset it.
_warned = set()


class _Report:
    """Where the packed forward is (training or not, which layer) for the warn-once log."""

    training = False
    where = None

    @classmethod
    def once(cls, key, message, *args):
        if key not in _warned:
            _warned.add(key)
            log.warning(message, *args)


def _warn_once(reason):
    """The whole call went to the original forward."""
    _Report.once(reason, "solution.body.packed: original Qwen2Model.forward used (%s)", reason)


def _fallback(piece, reason):
    """A guard sent one piece of the packed forward to its HF / torch op. Logged once per
    (piece, reason) and only while training, naming the first layer it happened at. Returns
    None so that guards can `return _fallback(...)`."""
    if _Report.training:
        _Report.once(f"{piece}: {reason}", "solution.body.packed: %s not used (%s; first at layer %s)",
                     piece, reason, _Report.where)
    return None


def _note_active():
    _Report.once("active", "solution.body: packed decoder active (pad removal + own kernels)")


def _has_hooks(module):
    return bool(module._forward_hooks or module._forward_pre_hooks
                or getattr(module, "_forward_hooks_with_kwargs", None))


# ----------------------------------------------------------------------------------------
# norms
# ----------------------------------------------------------------------------------------
def _is_rmsnorm(norm):
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    from .norm_rope import FusedRMSNorm

    return type(norm) in (Qwen2RMSNorm, FusedRMSNorm)


def _norm_eps(norm, residual, delta):
    """The eps add_rmsnorm runs with when it can stand in for norm(residual + delta), else None
    after a logged fallback (the conditions of reference packed.py:111-140; this build also
    takes a trainable weight, whose gradient the kernel's weight-gradient reduction gives)."""
    if not USE_KERNELS:
        return None
    from .norm_rope import NORM_BLOCK

    w = getattr(norm, "weight", None)
    eps = getattr(norm, "variance_epsilon", None)
    # (condition the kernel needs, why not) in order; each condition may rely on the ones before
    needs = (
        (lambda: _is_rmsnorm(norm) and not _has_hooks(norm),
         lambda: "not a plain Qwen2RMSNorm or hooks"),
        (lambda: isinstance(w, torch.Tensor) and eps is not None,
         lambda: "no weight tensor or no variance_epsilon"),
        (lambda: w.dim() == 1 and w.is_cuda and w.dtype in _KERNEL_FLOATS,
         lambda: f"weight {w.dtype} {tuple(w.shape)} on {w.device}"),
        (lambda: (residual.is_cuda and residual.dtype == torch.float32
                  and residual.shape[-1] == w.shape[0]),
         lambda: f"residual stream {residual.dtype} on {residual.device}"),
        (lambda: w.shape[0] <= NORM_BLOCK,
         lambda: f"hidden size {w.shape[0]} above {NORM_BLOCK}"),
        (lambda: delta is None or (delta.dtype in _KERNEL_FLOATS and delta.device == residual.device
                                   and delta.shape == residual.shape),
         lambda: f"delta {delta.dtype} {tuple(delta.shape)}"),
    )
    for ok, why in needs:
        if not ok():
            return _fallback("norm kernel", why())
    return float(eps)


def _normed_dtype(norm, residual, final):
    """dtype of a kernel norm's output: what its consumers compute in. A decoder-layer norm
    feeds projections, which run in the autocast dtype under autocast; the final norm returns
    HF's dtype, promote(weight, residual)."""
    if not final and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return torch.promote_types(norm.weight.dtype, residual.dtype)


def _add_norm(norm, residual, delta, final=False, with_eps=False, n_out=1, save_output=False):
    """(r, normed) for r = residual (+ delta); with_eps appends the eps the kernel ran with
    (None on HF's norm: the MLP recompute needs to know which ran). n_out > 1 gives one output
    per consumer: distinct views of the kernel's single buffer (its backward adds their
    gradients in fp32), or HF's tensor n_out times. The kernel keeps r in fp32. Reference
    packed.py:152-181."""
    eps = _norm_eps(norm, residual, delta)
    out_dtype = None if eps is None else _normed_dtype(norm, residual, final)
    if out_dtype in _KERNEL_FLOATS:
        from .norm_rope import add_rmsnorm

        r, normed = add_rmsnorm(residual, delta, norm.weight, eps, out_dtype, n_out,
                                save_output=save_output and not final)
    else:
        eps = None
        r = residual if delta is None else residual + delta
        normed = norm(r)
        if n_out > 1:
            normed = tuple(normed for _ in range(n_out))
    return (r, normed, eps) if with_eps else (r, normed)


# ----------------------------------------------------------------------------------------
# projections and their LoRA terms
# ----------------------------------------------------------------------------------------
def _nf4():
    from .. import nf4

    return nf4


def _fp16_under_autocast(x):
    return (x.dtype == torch.float16 and x.is_cuda and torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") == torch.float16)


def _lora_route(module, x):
    """How a projection runs on the packed 16-bit x [1, T, in]:
      (base layer, None)              the base layer alone: an NF4 Linear4bit itself, or a LoRA
                                      wrapper with no adapter active;
      (base layer, (A, B, p, scale))  a LoRA wrapper this path runs (lora.lora_params);
      None                            anything else, or a guard failed: module(x).
    A LoRA wrapper is any module with peft's LoRA layer attributes (base_layer, lora_A, lora_B,
    lora_dropout, scaling, active_adapters) whose base is a plain nn.Linear or an NF4 Linear4bit
    (nf4.is_linear4bit). The path needs the kernels on, a device x in fp16 / bf16 under autocast
    to that dtype (peft computes the term in the autocast dtype then; fp16 for an NF4 base, whose
    linear4bit computes in fp16), and no hooks (reference packed.py:240-290)."""
    if not (USE_KERNELS and USE_LORA_KERNELS):
        return None
    nf4 = _nf4()
    if nf4.is_linear4bit(module):
        if not _fp16_under_autocast(x) or _has_hooks(module):
            return _fallback("NF4 path", f"x {x.dtype}, no fp16 autocast, or hooks")
        return module, None
    base = getattr(module, "base_layer", None)
    if base is None or not hasattr(module, "lora_A"):
        return None
    if x.dtype not in (torch.float16, torch.bfloat16) or not x.is_cuda:
        return _fallback("LoRA path", f"x {x.dtype} {x.device}")
    if not torch.is_autocast_enabled("cuda") or torch.get_autocast_dtype("cuda") != x.dtype:
        return _fallback("LoRA path", f"no autocast to {x.dtype}")
    nf4_base = nf4.is_linear4bit(base)
    if _has_hooks(module) or not (type(base) is torch.nn.Linear or nf4_base) or _has_hooks(base):
        return _fallback("LoRA path", f"{type(module).__name__} / {type(base).__name__} or hooks")
    if nf4_base and x.dtype != torch.float16:
        return _fallback("LoRA path", f"NF4 base under {x.dtype} autocast")
    if getattr(module, "disable_adapters", False) or getattr(module, "merged", False):
        return _fallback("LoRA path", "adapters disabled or merged")
    if not any(name in module.lora_A for name in getattr(module, "active_adapters", ())):
        return base, None
    from .lora import lora_params

    params = lora_params(module)
    if params is None:
        return _fallback("LoRA path", "adapter config (lora.lora_params)")
    return base, params


def _base(base, x2):
    """The base projection on the 2-D x (a fresh output): an NF4 Linear4bit through
    nf4.linear4bit (its fp16 output), anything else through its own forward."""
    nf4 = _nf4()
    if nf4.is_linear4bit(base):
        return nf4.linear4bit(x2, base, keep_fp16=True)
    return base(x2)


def _project(module, x, x_lora=None):
    """module(x) for x [1, T, in] -> [1, T, out]. A routed projection runs its base on the 2-D x
    (a fresh output: F.linear with a bias on a 3-D input can return a view) and adds its LoRA
    term into that output; x_lora is the LoRA term's own copy of the norm output (same values),
    so the two input gradients reach the norm backward apart."""
    route = _lora_route(module, x)
    if route is None:
        return module(x)
    base, params = route
    x2 = x.reshape(-1, x.shape[-1])
    out = _base(base, x2)
    if params is not None:
        from .lora import LoRAFunction

        xl = x2 if x_lora is None else x_lora.reshape(-1, x_lora.shape[-1])
        out = LoRAFunction.apply(xl, out, *params)
    return out.view(1, x2.shape[0], -1)


def _project_q(module, x, x_lora=None):
    """(q [1, T, out], LoRA term [1, T, out] or None) for q_proj. The term is not added here:
    the RoPE kernel adds it to q before rotating, and its backward hands the same pre-rotation
    gradient to both. Without a routed LoRA, q is module(x) (its LoRA included)."""
    route = _lora_route(module, x)
    if route is None or route[1] is None:
        return _project(module, x), None
    base, params = route
    from .lora import LoRADeltaFunction

    x2 = x.reshape(-1, x.shape[-1])
    q = _base(base, x2)
    xl = x2 if x_lora is None else x_lora.reshape(-1, x_lora.shape[-1])
    term = LoRADeltaFunction.apply(xl, *params)
    return q.view(1, x2.shape[0], -1), term.view(1, x2.shape[0], -1)


def _qkv_route(module, x):
    """_lora_route's answer for one of q / k / v, except that a plain nn.Linear without hooks
    (which _lora_route leaves to module(x)) is (module, None) when FUSE_QKV is on."""
    route = _lora_route(module, x)
    if (route is None and FUSE_QKV and USE_KERNELS and type(module) is torch.nn.Linear
            and not _has_hooks(module)):
        return module, None
    return route


def _linear_multi(x2, bases):
    """The outputs of plain nn.Linear layers that read the same 2-D x2, side by side in the
    columns of ONE GEMM's output against their concatenated weights and biases, or None when
    they differ in weight dtype, device, input width or bias presence, or would not compute in
    x2's dtype (autocast to it, or weights of it). Under autocast the concatenation is cast
    once (the bits of autocast's per-weight casts). Autograd reaches each weight through the
    cast and the concatenation (one dW GEMM for all trainable ones, sliced by the cat's
    backward), and one dX GEMM reads the output's whole gradient."""
    ws = [b.weight for b in bases]
    bs = [b.bias for b in bases]
    if (len({(w.dtype, w.device, w.dim(), w.shape[-1]) for w in ws}) != 1 or ws[0].dim() != 2
            or (any(b is None for b in bs) and not all(b is None for b in bs))):
        return _fallback("fused q/k/v", "projections differ in weight dtype, shape or bias")
    if torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
    else:
        dt = ws[0].dtype
    if dt != x2.dtype:
        return _fallback("fused q/k/v", f"x {x2.dtype} against compute dtype {dt}")
    w = torch.cat(ws).to(dt)
    if bs[0] is None:
        b = None
    elif any(t.requires_grad for t in bs):
        b = torch.cat(bs).to(dt)  # gradients reach each bias
    else:
        b = _frozen_bias_cat(bases, bs, dt)
    return F.linear(x2, w, b)


def _frozen_bias_cat(bases, bs, dt):
    """The concatenation of frozen biases in dtype dt, kept on the first layer and rebuilt when
    a bias is replaced, re-pointed or changed in place (identity, data pointer and version of
    each; the NF4 path caches its bias_cat the same way, reference nf4/__init__.py:165-226):
    two launches per layer and forward less for a few KB."""
    stamp = [(t.data_ptr(), t._version) for t in bs]
    cache = bases[0].__dict__.setdefault("_esep_bias_cat", {})
    slot = tuple(id(m) for m in bases)
    hit = cache.get(slot)
    fresh = (hit is not None and hit[0] == dt and len(hit[1]) == len(bs)
             and all(a is t for a, t in zip(hit[1], bs)) and hit[2] == stamp)
    if not fresh:
        with torch.no_grad():
            hit = cache[slot] = (dt, list(bs), stamp, torch.cat(bs).to(dt))
    return hit[3]


def _rope_kernel_ok(rope_in, q, q_delta):
    """The RoPE kernel takes q (and a k of q's dtype) with these rotary inputs."""
    return (rope_in.positions is not None and q.dtype in _KERNEL_FLOATS and q.is_cuda
            and (q_delta is None or q_delta.dtype == q.dtype))


class _QKVRope(torch.autograd.Function):
    """RoPE on the q and k columns of the fused q / k / v output y [T, nq + nk + nv], and v
    copied out of it: apply(y, nq, nk, head_dim, positions [T], inv_freq, q_delta [T, nq] or
    None) -> (q rotated [1, T, nq / D, D], k rotated [1, T, nk / D, D], v [T, nv]), q_delta
    added to q inside the kernel before the rotation. The backward writes the inverse
    rotations of dq and dk and a copy of dv straight into the columns of one gradient of y,
    which the fused GEMM's backward reads whole; with column views of y instead, the split's
    backward concatenates three separate gradients (a copy of all of them: 19 us per layer at
    the Qwen2.5-1.5B shape against a copy of v's columns). q_delta gets the gradient of q's
    columns, as Rope gives it. v is a copy so that y is freed once RoPE has read it."""

    @staticmethod
    def forward(ctx, y, nq, nk, head_dim, positions, inv_freq, q_delta):
        from . import _hip

        T = y.shape[0]
        q4 = y[:, :nq].view(1, T, nq // head_dim, head_dim)
        k4 = y[:, nq:nq + nk].view(1, T, nk // head_dim, head_dim)
        qd4 = None if q_delta is None else q_delta.reshape(q4.shape)
        qo = torch.empty(q4.shape, device=y.device, dtype=y.dtype)
        ko = torch.empty(k4.shape, device=y.device, dtype=y.dtype)
        pos2 = positions.view(1, -1)
        if T > 0:
            _hip.rope(q4, k4, qo, ko, inv_freq, 1.0, q_delta=qd4, positions=pos2)
        v = y[:, nq + nk:].contiguous()
        ctx.save_for_backward(positions, inv_freq)
        ctx.dims, ctx.dtype = (T, nq, nk, y.shape[1], head_dim), y.dtype
        ctx.has_qd = q_delta is not None
        return qo, ko, v

    @staticmethod
    def backward(ctx, dqo, dko, dv):
        from . import _hip

        positions, inv_freq = ctx.saved_tensors
        T, nq, nk, n, head_dim = ctx.dims
        dy = torch.empty((T, n), device=inv_freq.device, dtype=ctx.dtype)
        dq4 = dy[:, :nq].view(1, T, nq // head_dim, head_dim)
        dk4 = dy[:, nq:nq + nk].view(1, T, nk // head_dim, head_dim)
        # an unused output's gradient is zero (as in Rope)
        dqo = torch.zeros_like(dq4) if dqo is None else dqo.contiguous()
        dko = torch.zeros_like(dk4) if dko is None else dko.contiguous()
        if T > 0:
            _hip.rope(dqo, dko, dq4, dk4, inv_freq, -1.0, positions=positions.view(1, -1))
        if dv is None:
            dy[:, nq + nk:].zero_()
        else:
            dy[:, nq + nk:].copy_(dv)
        dqd = dy[:, :nq] if ctx.has_qd and ctx.needs_input_grad[6] else None
        return dy, None, None, None, None, None, dqd


def _qkv(attn, x_q, x_ql, x_vl, rope_in):
    """(q, q term, k, v, rotated) as _project_q / _project give them, with the three base
    projections as ONE GEMM on x_q when q, k and v all take this path, k without a LoRA term of
    its own: NF4 bases through nf4.linear4bit_multi (one dequant launch into W_cat, one GEMM;
    backward one re-dequant and one dX GEMM; reference packed.py:321-352), plain nn.Linear
    bases (or plain layers themselves, FUSE_QKV) through _linear_multi. Else None (the separate
    calls run). The fused output goes through _QKVRope when the RoPE kernel takes it
    (rotated True: q and k come back rotated, q's LoRA term added inside); otherwise q, k, v
    are column views of the one output (rotated False). v's LoRA term is added out of place.
    The norm backward then gets one base gradient (through x_q) beside the q and v LoRA
    gradients (x_ql, x_vl); the k and v base copies of the norm output get none."""
    routes = [_qkv_route(m, x_q) for m in (attn.q_proj, attn.k_proj, attn.v_proj)]
    if any(r is None for r in routes) or routes[1][1] is not None:
        return None
    nf4 = _nf4()
    bases = [r[0] for r in routes]
    x2 = x_q.reshape(-1, x_q.shape[-1])
    n_tok = x2.shape[0]
    if all(nf4.is_linear4bit(b) for b in bases):
        y = nf4.linear4bit_multi(x2, bases, split=False)
        sizes = [b.weight.quant_state.shape[0] for b in bases]
    elif FUSE_QKV and all(type(b) is torch.nn.Linear for b in bases):
        y = _linear_multi(x2, bases)
        if y is None:
            return None
        sizes = [b.weight.shape[0] for b in bases]
    else:
        return None
    from .lora import LoRADeltaFunction, LoRAFunction

    q_term = None
    if routes[0][1] is not None:
        q_term = LoRADeltaFunction.apply(x_ql.reshape(-1, x_ql.shape[-1]), *routes[0][1])
    rotated = _rope_kernel_ok(rope_in, y, q_term)
    if rotated:
        q, k, v = _QKVRope.apply(y, sizes[0], sizes[1], attn.head_dim, rope_in.positions,
                                 rope_in.inv_freq, q_term)
        q_term = None  # added inside the kernel
    else:
        q, k, v = y.split(sizes, dim=-1)
    if q_term is not None:
        q_term = q_term.view(1, n_tok, -1)
    if routes[2][1] is not None:
        v = LoRAFunction.apply(x_vl.reshape(-1, x_vl.shape[-1]), v, *routes[2][1])
    elif not rotated:
        # v as a view would keep the whole fused output (q's and k's columns too; RoPE writes
        # new tensors) alive until the attention backward: 21 MB per layer at the Qwen2.5-1.5B
        # shape, against a copy of v's 3 MB
        v = v.contiguous()
    if rotated:
        return q, None, k, v.view(1, n_tok, -1), True
    return q.view(1, n_tok, -1), q_term, k.view(1, n_tok, -1), v.view(1, n_tok, -1), False


# ----------------------------------------------------------------------------------------
# rotary embedding
# ----------------------------------------------------------------------------------------
class _RopeInputs:
    """The rotary inputs of one packed forward (reference packed.py:355-379): the kernel's
    (positions [T] int64, fp32 inv_freq) when the model's rotary embedding is HF's default type
    with attention_scaling 1 and a head dim the kernel takes, else HF's cos / sin, built once
    on first use."""

    def __init__(self, model, hidden, pos):
        rotary = model.rotary_emb
        self._rotary, self._hidden, self._pos = rotary, hidden, pos
        self._cos_sin = None
        self.positions = self.inv_freq = None
        cfg = model.config
        head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        inv = getattr(rotary, "inv_freq", None)
        kernel_ok = (USE_KERNELS and type(rotary).__name__ == "Qwen2RotaryEmbedding"
                     and not _has_hooks(rotary) and getattr(rotary, "rope_type", None) == "default"
                     and getattr(rotary, "attention_scaling", None) == 1.0
                     and isinstance(inv, torch.Tensor) and inv.is_cuda and inv.dim() == 1
                     and head_dim in (64, 128, 256) and inv.shape[0] == head_dim // 2)
        if kernel_ok:
            self.positions = pos.reshape(-1)
            self.inv_freq = inv.detach().to(torch.float32).contiguous()

    def cos_sin(self):
        if self._cos_sin is None:
            self._cos_sin = self._rotary(self._hidden, self._pos)
        return self._cos_sin


def _rope(q, k, rope_in, q_delta=None):
    """Rotated (q + q_delta, k) for q [1, T, Hq, D], k [1, T, Hk, D] (reference
    packed.py:382-401): on the kernel when it takes these inputs (the add happens inside it,
    in q's dtype), else HF's apply_rotary_pos_emb after the add."""
    if _rope_kernel_ok(rope_in, q, q_delta) and k.dtype == q.dtype:
        from .norm_rope import rope

        # squeeze, not indexing: its backward is a view too
        qo, ko = rope(q.squeeze(0), k.squeeze(0), rope_in.positions, rope_in.inv_freq,
                      q_delta=None if q_delta is None else q_delta.squeeze(0))
        return qo.unsqueeze(0), ko.unsqueeze(0)
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    if q_delta is not None:
        q = q + q_delta.view_as(q)
    cos, sin = rope_in.cos_sin()
    return apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=2)


# ----------------------------------------------------------------------------------------
# attention
# ----------------------------------------------------------------------------------------
@functools.lru_cache(maxsize=4)
def _cu_seqlens(lens, device):
    """int32 [n + 1] sequence offsets of the packed rows (cached for the few recent batches)."""
    from .attention import cu_seqlens_from_lengths

    return cu_seqlens_from_lengths(list(lens), device)


def _attention(attn, q, k, v, lens):
    """Causal attention within each original row of the packed q [1, T, Hq, D] and k, v
    [1, T, Hk, D] -> [1, T, Hq * D]; query head h reads kv head h // (Hq / Hk) (HF's repeat_kv).
    One varlen kernel launch per direction when it applies, else torch's SDPA per row
    (reference packed.py:404-436)."""
    if torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        q, k, v = q.to(dt), k.to(dt), v.to(dt)
    n_tok, hq, d = q.shape[1], q.shape[2], q.shape[3]
    dropout = attn.attention_dropout if attn.training else 0.0
    if USE_KERNELS:
        from . import attention

        if attention.supported(q, k, v, dropout):
            o = attention.varlen_attention(q, k, v, _cu_seqlens(tuple(lens), q.device), max(lens),
                                           attn.scaling)
            return o.view(1, n_tok, hq * d)
        _fallback("attention kernel", f"dtype {q.dtype}, head_dim {d}, dropout {dropout}")
    rows = []
    for qs, ks, vs in zip(q[0].split(lens), k[0].split(lens), v[0].split(lens)):
        # [n, H, D] row slices as [1, H, n, D]; SDPA's grouped-query mode maps query head h to
        # kv head h // (Hq / Hk)
        o = F.scaled_dot_product_attention(qs.transpose(0, 1)[None], ks.transpose(0, 1)[None],
                                           vs.transpose(0, 1)[None], dropout_p=dropout,
                                           is_causal=True, scale=attn.scaling, enable_gqa=True)
        rows.append(o[0].transpose(0, 1))  # [n, Hq, D]
    return torch.cat(rows).reshape(1, n_tok, hq * d)


# ----------------------------------------------------------------------------------------
# MLP
# ----------------------------------------------------------------------------------------
def _plain_silu_mlp(mlp, x):
    """An unmodified silu Qwen2MLP without hooks, on a device input."""
    from transformers.models.qwen2.modeling_qwen2 import Qwen2MLP

    act = getattr(getattr(mlp, "config", None), "hidden_act", None)
    return type(mlp) is Qwen2MLP and not _has_hooks(mlp) and x.is_cuda and act == "silu"


def _mlp_layers(mlp, x):
    """(gate, up, down) when mlp(x) can run as _RecomputeMLP, else None (reference
    packed.py:493-524): the kernels and RECOMPUTE_MLP on, grad mode on, a plain silu Qwen2MLP
    without hooks whose three projections are all frozen NF4 Linear4bit (nf4.is_linear4bit)
    without bias or hooks, with a fp16 device x under fp16 autocast (linear4bit computes in
    fp16), or all bias-free nn.Linear without hooks with a 16-bit device x that they compute in
    (autocast to x's dtype, or weights of x's dtype); nothing in the MLP trainable."""
    if not (USE_KERNELS and RECOMPUTE_MLP) or not torch.is_grad_enabled():
        return None
    piece = "recompute MLP"
    if x.dtype not in (torch.float16, torch.bfloat16) or not _plain_silu_mlp(mlp, x):
        return _fallback(piece, f"x {x.dtype}, {type(mlp).__name__}, hooks or activation")
    projections = (mlp.gate_proj, mlp.up_proj, mlp.down_proj)
    if any(prm.requires_grad for prm in mlp.parameters()):
        return _fallback(piece, "trainable parameter in the MLP")
    nf4 = _nf4()
    if all(nf4.is_linear4bit(lin) for lin in projections):
        if not _fp16_under_autocast(x):
            return _fallback(piece, f"NF4 projections with x {x.dtype} / no fp16 autocast")
        if any(_has_hooks(lin) or lin.bias is not None for lin in projections):
            return _fallback(piece, "NF4 projection with a bias or hooks")
        return projections
    autocast_to_x = (torch.is_autocast_enabled("cuda")
                     and torch.get_autocast_dtype("cuda") == x.dtype)
    for lin in projections:
        if type(lin) is not torch.nn.Linear or _has_hooks(lin) or lin.bias is not None:
            return _fallback(piece, "projections not all bias-free nn.Linear or NF4 Linear4bit")
        if not autocast_to_x and lin.weight.dtype != x.dtype:
            return _fallback(piece, f"weights {lin.weight.dtype} without autocast to {x.dtype}")
    return projections


class _RecomputeMLP(torch.autograd.Function):
    """down(silu(gate(x)) * up(x)) for frozen projections without saving any [T, intermediate]
    tensor (the reference's activation-memory trade, packed.py:562-643): frozen NF4 Linear4bit
    projections as in the reference, or frozen 16-bit nn.Linear (a LoRA run on an unquantized
    base).

    apply(x_gate, x_up, r, w_norm, eps, gate, up, down). Saved: x itself, or (when the norm
    that produced x did not keep its output) the norm's fp32 input r and weight, x then being
    recomputed bit-exactly by the same norm kernel in backward; for nn.Linear also the three
    weights in the dtype the projections compute in (the casts HF's autograd holds as well;
    casting again in backward cost five weight casts per layer). Forward: g, u from the two
    projections (NF4: nf4.linear4bit, dequant on the HIP kernel + fp16 GEMM), h = silu(g) * u on
    the HIP kernel (into g), out from the down projection. Backward: dh = dout W_down, g and u
    recomputed, (dg, du) by the HIP kernel in place. NF4: W_down from one dequant launch, W_gate
    and W_up from one esep_nf4_dequant_multi launch (row blocks bit-exact with the forward's
    dequants, so g and u recompute bit-exactly), and dx = dg W_gate + du W_up formed as mm +
    addmm into one buffer, returned as x_gate's gradient (x_up gets none). nn.Linear: dx_gate =
    dg gate and dx_up = du up, returned for the two fan-out copies (the norm backward sums
    them)."""

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, x, x_up, r, w_norm, eps, gate, up, down):
        from . import _hip

        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        nf4 = _nf4()
        ctx.nf4 = nf4.is_linear4bit(gate)
        if ctx.nf4:
            h = nf4.linear4bit(x2, gate, keep_fp16=True).contiguous()
            u = nf4.linear4bit(x2, up, keep_fp16=True).contiguous()
            _hip.swiglu_fwd(h, u, h)
            out = nf4.linear4bit(h, down, keep_fp16=True)
            weights = ()
        else:
            # The weights in the dtype the projections compute in, cast once and kept for the
            # backward (the bits autocast's own cast gives): autocast caches casts only of
            # leaves that require grad, so frozen fp32 weights would be cast again at each of
            # their five uses in backward. Weights already in that dtype are kept as they are.
            dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else None
            weights = tuple(lin.weight if dt is None else lin.weight.to(dt)
                            for lin in (gate, up, down))
            h = F.linear(x2, weights[0]).contiguous()
            u = F.linear(x2, weights[1]).contiguous()
            _hip.swiglu_fwd(h, u, h)
            out = F.linear(h, weights[2])
        del h, u
        saved = (x2,) if r is None else (r, w_norm)
        ctx.n_x = len(saved)
        ctx.save_for_backward(*saved, *weights)
        ctx.from_residual, ctx.eps = r is not None, eps
        ctx.shape, ctx.x_dtype, ctx.proj = shape, x.dtype, (gate, up, down)
        return out.view(*shape[:-1], out.shape[-1])

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        from . import _hip

        gate, up, down = ctx.proj
        saved = ctx.saved_tensors
        if ctx.from_residual:
            from .norm_rope import rmsnorm_recompute

            r, w_norm = saved[:2]
            x2 = rmsnorm_recompute(r.reshape(-1, r.shape[-1]), w_norm, ctx.eps, ctx.x_dtype)
        else:
            x2 = saved[0]
        weights = saved[ctx.n_x:]
        del saved
        dout2 = dout.reshape(-1, dout.shape[-1])
        if ctx.nf4:
            nf4 = _nf4()
            w = nf4.dequantize_nf4(down.weight, down.weight.quant_state)
            dh = torch.matmul(dout2.to(w.dtype), w)
            del w
            w_gu = nf4.dequant_multi([gate, up])
            n_gate = gate.weight.quant_state.shape[0]
            w_gate, w_up = w_gu[:n_gate], w_gu[n_gate:]
            g = F.linear(x2, w_gate).contiguous()
            u = F.linear(x2, w_up).contiguous()
            del x2
            _hip.swiglu_bwd(dh.contiguous(), g, u, g, u)  # dg into g, du into u
            del dh
            dx = torch.mm(g, w_gate)
            dx.addmm_(u, w_up)
            return dx.view(ctx.shape), None, None, None, None, None, None, None
        w_gate, w_up, w_down = weights
        dh = torch.matmul(dout2, w_down)
        g = F.linear(x2, w_gate).contiguous()
        u = F.linear(x2, w_up).contiguous()
        del x2
        _hip.swiglu_bwd(dh.to(g.dtype).contiguous(), g, u, g, u)  # dg into g, du into u
        del dh
        dx_gate = torch.matmul(g, w_gate).to(ctx.x_dtype)
        del g
        dx_up = torch.matmul(u, w_up).to(ctx.x_dtype)
        return dx_gate.view(ctx.shape), dx_up.view(ctx.shape), None, None, None, None, None, None


def _mlp(mlp, xs, norm=None, residual=None, eps=None, norm_saves_y=False):
    """The layer's MLP on the post-attention norm's output (reference packed.py:676-693). xs is
    a tensor or the pair (x_gate, x_up) of fan-out copies. Frozen plain projections:
    _RecomputeMLP (x recomputed from the norm's fp32 residual when the norm did not save its
    output: eps given and norm_saves_y False). A plain silu MLP otherwise: the model's
    projections with the HIP SwiGLU (HF's silu with the kernels off), gate and up reading their
    own copies. Anything else (hooks, another MLP class or activation): mlp(x_gate)."""
    x_gate, x_up = xs if isinstance(xs, tuple) else (xs, xs)
    projections = _mlp_layers(mlp, x_gate)
    if projections is not None:
        from_residual = (eps is not None and not norm_saves_y and residual is not None
                         and residual.dtype == torch.float32 and residual.is_contiguous())
        r = residual if from_residual else None
        w_norm = norm.weight.detach().to(torch.float32) if from_residual else None
        return _RecomputeMLP.apply(x_gate, x_up, r, w_norm, eps, *projections)
    if not _plain_silu_mlp(mlp, x_gate):
        return mlp(x_gate)  # its own forward (and hooks); the copy x_up gets no gradient
    if USE_KERNELS:
        from ..swiglu import swiglu

        return mlp.down_proj(swiglu(mlp.gate_proj(x_gate), mlp.up_proj(x_up)))
    return mlp.down_proj(mlp.act_fn(mlp.gate_proj(x_gate)) * mlp.up_proj(x_up))


# ----------------------------------------------------------------------------------------
# one decoder layer and the patched forward
# ----------------------------------------------------------------------------------------
def _layer(layer, residual, delta, rope_in, lens):
    """One Qwen2DecoderLayer on the packed tokens (reference packed.py:696-724). Returns
    (residual, delta): the layer's output is residual + delta, the add left to the next norm.
    The input norm's output goes to five consumers, each with its own copy: q, k and v
    projections and the q and v LoRA terms (a copy nothing consumes gets no gradient; with the
    fused NF4 q/k/v call, the k and v base copies)."""
    attn = layer.self_attn
    residual, (x_q, x_ql, x_k, x_v, x_vl) = _add_norm(layer.input_layernorm, residual, delta,
                                                      n_out=5, save_output=NORM_SAVE_OUTPUT)
    n_tok, head_dim = x_q.shape[1], attn.head_dim
    fused = _qkv(attn, x_q, x_ql, x_vl, rope_in)
    rotated = False
    if fused is not None:
        q, q_term, k, v, rotated = fused
    else:
        q, q_term = _project_q(attn.q_proj, x_q, x_ql)
        k = _project(attn.k_proj, x_k)
        v = _project(attn.v_proj, x_v, x_vl)
    if not rotated:
        q, k = _rope(q.view(1, n_tok, -1, head_dim), k.view(1, n_tok, -1, head_dim), rope_in,
                     q_term)
    o = _project(attn.o_proj, _attention(attn, q, k, v.view(1, n_tok, -1, head_dim), lens))
    post = layer.post_attention_layernorm
    residual, xs, eps = _add_norm(post, residual, o, with_eps=True, n_out=2,
                                  save_output=NORM_SAVE_OUTPUT)
    return residual, _mlp(layer.mlp, xs, post, residual, eps, norm_saves_y=NORM_SAVE_OUTPUT)


def _unsupported(model, input_ids, attention_mask, past_key_values, inputs_embeds, use_cache,
                 kwargs):
    """None when the packed path takes this call, else the reason it does not (reference
    packed.py:736-771)."""
    if not isinstance(model, torch.nn.Module) or not hasattr(model, "layers"):
        return "not a real model"
    config = getattr(model, "config", None)
    if config is None:
        return "no config"
    checks = (
        (inputs_embeds is not None, "inputs_embeds"),
        (not (isinstance(input_ids, torch.Tensor) and input_ids.dim() == 2 and input_ids.is_cuda),
         "input_ids not 2D CUDA"),
        (not (isinstance(attention_mask, torch.Tensor)
              and attention_mask.shape == getattr(input_ids, "shape", None)),
         "attention_mask missing or not 2D"),
        (past_key_values is not None, "past_key_values"),
        (getattr(config, "use_cache", False) if use_cache is None else use_cache, "use_cache"),
    )
    for failed, reason in checks:
        if failed:
            return reason
    extra = [key for key in kwargs if key not in _IGNORED_KWARGS]
    if extra:
        return f"kwarg {extra[0]}"
    for key in ("output_attentions", "output_hidden_states"):
        if kwargs.get(key, getattr(config, key, False)):
            return key
    if getattr(config, "_attn_implementation", None) != "sdpa":
        return "attn_implementation is not sdpa"
    if any(kind != "full_attention" for kind in getattr(config, "layer_types", ["full_attention"])):
        return "sliding window layers"
    if model.training and getattr(model, "gradient_checkpointing", False):
        return "gradient checkpointing"
    if any(_has_hooks(lyr) or _has_hooks(lyr.self_attn)
           for lyr in model.layers[: config.num_hidden_layers]):
        return "hooks on decoder layers"
    return None


class _Packing:
    """Geometry of one padded [B, L] batch: the row lengths (the forward's one host sync), the
    flat indices of the real tokens in row-major order (rows stay in order, so each row is one
    slice of the packed stream) and their positions: the column index, which is HF's default
    arange(L) per row also under left padding, or the caller's position_ids gathered
    (reference packed.py:800-814)."""

    def __init__(self, attention_mask, position_ids):
        real = attention_mask.bool()
        self.B, self.L = real.shape
        self.lens = real.sum(1).tolist()
        self.T = sum(self.lens)
        self.index = torch.nonzero_static(real.reshape(-1), size=self.T).squeeze(1)
        if position_ids is None:
            pos = self.index % self.L
        else:
            pos = position_ids.expand(self.B, self.L).reshape(-1).index_select(0, self.index)
        self.positions = pos.to(torch.int64).unsqueeze(0)

    def gather(self, t):
        """[B, L, ...] -> the packed [1, T, ...]."""
        return t.reshape(self.B * self.L, *t.shape[2:]).index_select(0, self.index).unsqueeze(0)

    def scatter(self, packed):
        """The packed [1, T, H] back to [B, L, H] with zeros at the pads. The copy goes into a
        fresh zero tensor in place (autograd records it; the gradient gathers back)."""
        full = packed.new_zeros(self.B * self.L, packed.shape[-1])
        full.index_copy_(0, self.index, packed.squeeze(0))
        return full.view(self.B, self.L, -1)


def packed_forward(model, input_ids, attention_mask, position_ids, kwargs):
    """The packed decoder body (reference packed.py:800-840): [B, L, H] hidden states, or None
    when a row has no token (the caller then runs the original forward)."""
    pack = _Packing(attention_mask, position_ids)
    if min(pack.lens) == 0:
        return None
    hidden = model.embed_tokens(pack.gather(input_ids))
    _Report.training, _Report.where = bool(model.training), "embedding"
    emb_w = getattr(model.embed_tokens, "weight", None)
    if (hidden.dtype != torch.float32 and isinstance(emb_w, torch.Tensor)
            and emb_w.dtype == torch.float32):
        _fallback("fp32 residual stream", f"embedding output is {hidden.dtype}")
    rope_in = _RopeInputs(model, hidden, pack.positions)
    residual, delta = hidden, None
    try:
        for i, layer in enumerate(model.layers[: model.config.num_hidden_layers]):
            _Report.where = i
            residual, delta = _layer(layer, residual, delta, rope_in, pack.lens)
        _Report.where = "final norm"
        _, out = _add_norm(model.norm, residual, delta, final=True)
    finally:
        _Report.training = False
    return pack.scatter(out)


def patch():
    """Replace Qwen2Model.forward by the packed decoder (idempotent). The original forward
    stays at forward.__wrapped__ and serves every call the packed path does not take
    (reference packed.py:843-875)."""
    from transformers.modeling_outputs import BaseModelOutputWithPast
    from transformers.models.qwen2 import modeling_qwen2

    cls = modeling_qwen2.Qwen2Model
    if getattr(cls.forward, "_solution_body_packed", False):
        return
    original = cls.forward

    @functools.wraps(original)
    def forward(self, input_ids=None, attention_mask=None, position_ids=None,
                past_key_values=None, inputs_embeds=None, use_cache=None, **kwargs):
        reason = _unsupported(self, input_ids, attention_mask, past_key_values, inputs_embeds,
                              use_cache, kwargs)
        hidden = None
        if reason is None:
            hidden = packed_forward(self, input_ids, attention_mask, position_ids, kwargs)
            reason = None if hidden is not None else "a row without tokens"
        training = getattr(self, "training", False)
        if hidden is None:
            if training and reason != "not a real model":
                _warn_once(reason)
            return original(self, input_ids=input_ids, attention_mask=attention_mask,
                            position_ids=position_ids, past_key_values=past_key_values,
                            inputs_embeds=inputs_embeds, use_cache=use_cache, **kwargs)
        if training:
            _note_active()
        result = BaseModelOutputWithPast(last_hidden_state=hidden, past_key_values=None)
        return_dict = kwargs.get("return_dict", getattr(self.config, "return_dict", True))
        return result.to_tuple() if return_dict is False else result

    forward._solution_body_packed = True
    cls.forward = forward


@contextlib.contextmanager
def kernels_enabled(on):
    """USE_KERNELS set to `on` for the duration of the block (tests, benchmarks)."""
    global USE_KERNELS
    saved, USE_KERNELS = USE_KERNELS, on
    try:
        yield
    finally:
        USE_KERNELS = saved
