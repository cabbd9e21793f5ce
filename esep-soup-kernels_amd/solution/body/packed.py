"""Pad removal inside one batch for the Qwen2 decoder, with the norms and RoPE on this
repository's HIP kernels: the reference's patch point (gojosatorukz/esep-soup-kernels,
solution/body/packed.py), rebuilt around norm_rope.py.

`Qwen2Model.forward` is class-patched (`patch()`, reference packed.py:843-875). For a normal
training batch (2-D attention mask, no cache, no captured outputs) the real tokens of all rows
are packed into one [1, T, H] sequence, every token-wise op of the decoder layers runs on the
T real tokens only, attention runs per row on that row's slice with a causal mask, and the
final hidden states are scattered back to [B, L, H] with zeros at the pad positions
(reference packed.py:800-840). Anything unusual goes to the original forward.

Pieces and their guards (each falls back to the HF / torch op when its inputs are not what the
kernel takes, as the reference's do):
  _add_norm   residual add + RMSNorm on norm_rope.add_rmsnorm (fp32 residual stream, a plain
              Qwen2RMSNorm without hooks, row width <= NORM_BLOCK). Unlike the reference, a
              trainable norm weight stays on the kernel: it gets its gradient from the kernel's
              deterministic two-stage reduction (the reference sends it to HF, packed.py:129).
  _rope       norm_rope.rope on the packed positions and the model's inv_freq (HF default rope
              type with attention_scaling 1.0), fp16 / bf16 / fp32 q and k.
  _attention  attention.varlen_attention: causal attention over all rows in one launch per
              direction (fp16 / bf16, head_dim 64 or 128, no dropout); else the reference's
              per-row SDPA loop.
  _mlp        frozen projections: _RecomputeMLP (saves no [T, intermediate] tensor, recomputes
              the gate / up projections and, when the norm did not save its output, the norm
              itself in backward); otherwise the model's projections with silu(g) * u on the
              HIP SwiGLU kernel (solution/swiglu.py).
The q/k/v/o projections call the model's own modules: the reference's NF4 / LoRA routes
(packed.py:184-352, :440-524) are other workstreams and are not part of this build; their flags
exist for API compatibility.
"""

import contextlib
import logging

import torch
import torch.nn.functional as F

log = logging.getLogger(__name__)

# Keyword arguments that may reach Qwen2Model.forward in a training step and that the packed
# path can ignore (reference packed.py:59-60). Anything else -> original forward.
_IGNORED_KWARGS = {"num_items_in_batch", "return_dict", "output_attentions",
                   "output_hidden_states", "is_causal"}

# In-process switches (never read from the environment), as in the reference: USE_KERNELS
# (packed.py:106) turns the HIP norm / RoPE off (packed layout on torch ops);
# NORM_SAVE_OUTPUT (:149) makes the decoder-layer norms save their 16-bit output instead of the
# fp32 residual; RECOMPUTE_MLP (:448) sends an MLP with frozen projections through
# _RecomputeMLP; USE_LORA_KERNELS (:186) selects a route this build does not have (kept so code
# that sets it keeps working).
USE_KERNELS = True
NORM_SAVE_OUTPUT = True
USE_LORA_KERNELS = True
RECOMPUTE_MLP = True

_KERNEL_FLOATS = (torch.float16, torch.bfloat16, torch.float32)

_warned = set()
# [training, layer index or "final norm"], set by packed_forward for the warn-once messages.
_WHERE = [False, None]


def _warn_once(reason):
    if reason not in _warned:
        _warned.add(reason)
        log.warning("solution.body.packed: original Qwen2Model.forward used (%s)", reason)


def _fallback(piece, reason):
    """A guard sent `piece` to the HF / torch op: one warning per (piece, reason) in training,
    naming the first layer seen (reference packed.py:76-87). Returns None."""
    if _WHERE[0]:
        key = f"{piece}: {reason}"
        if key not in _warned:
            _warned.add(key)
            log.warning("solution.body.packed: %s not used (%s; first at layer %s)", piece,
                        reason, _WHERE[1])
    return None


def _note_active():
    if "active" not in _warned:
        _warned.add("active")
        log.warning("solution.body: packed decoder active (pad removal + own kernels)")


def _has_hooks(module):
    return bool(module._forward_hooks or module._forward_pre_hooks
                or getattr(module, "_forward_hooks_with_kwargs", None))


def _is_rmsnorm(norm):
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    from .norm_rope import FusedRMSNorm

    return type(norm) in (Qwen2RMSNorm, FusedRMSNorm)


def _norm_eps(norm, residual, delta):
    """`variance_epsilon` if add_rmsnorm can replace `norm(residual + delta)`, else None
    (reference packed.py:111-140): a plain Qwen2RMSNorm without hooks, a 1-D float weight on the
    residual's device, an fp32 device residual (a 16-bit residual stream keeps HF's rounding by
    falling back), row width <= NORM_BLOCK, and a float delta of the residual's shape."""
    if not USE_KERNELS:
        return None
    from .norm_rope import NORM_BLOCK

    if not _is_rmsnorm(norm) or _has_hooks(norm):
        return _fallback("norm kernel", "not a plain Qwen2RMSNorm or hooks")
    w = getattr(norm, "weight", None)
    eps = getattr(norm, "variance_epsilon", None)
    if not isinstance(w, torch.Tensor) or eps is None:
        return _fallback("norm kernel", "missing weight / eps")
    if w.dim() != 1 or w.dtype not in _KERNEL_FLOATS or not w.is_cuda:
        return _fallback("norm kernel", f"weight {w.dtype} {tuple(w.shape)}")
    if residual.dtype != torch.float32 or not residual.is_cuda or residual.shape[-1] != w.shape[0]:
        return _fallback("norm kernel", f"residual {residual.dtype} {residual.device}")
    if w.shape[0] > NORM_BLOCK:
        return _fallback("norm kernel", f"hidden {w.shape[0]} > {NORM_BLOCK}")
    if delta is not None and (delta.dtype not in _KERNEL_FLOATS or delta.shape != residual.shape
                              or delta.device != residual.device):
        return _fallback("norm kernel", f"delta {delta.dtype} {tuple(delta.shape)}")
    return float(eps)


def _add_norm(norm, residual, delta, final=False, with_eps=False, n_out=1, save_output=False):
    """`r = residual + delta` (delta may be None); returns (r, norm(r)) (+ eps with with_eps:
    the eps the kernel used, or None when HF's norm ran). Kernel path: r stays fp32; the normed
    output of a decoder-layer norm is stored in the autocast dtype (it only feeds projections,
    which compute in it); the final norm's output has HF's dtype promote(weight, residual).
    n_out > 1: n_out outputs, one per consumer (kernel: views whose gradients the norm backward
    sums; HF: the same tensor n_out times). Reference packed.py:152-181."""
    eps = _norm_eps(norm, residual, delta)
    if eps is not None:
        out_dtype = torch.promote_types(norm.weight.dtype, residual.dtype)
        if not final and torch.is_autocast_enabled("cuda"):
            out_dtype = torch.get_autocast_dtype("cuda")
        if out_dtype in _KERNEL_FLOATS:
            from .norm_rope import add_rmsnorm

            r, y = add_rmsnorm(residual, delta, norm.weight, eps, out_dtype, n_out,
                               save_output=save_output and not final)
            return (r, y, eps) if with_eps else (r, y)
    if delta is not None:
        residual = residual + delta
    y = norm(residual)
    if n_out > 1:
        y = (y,) * n_out
    return (residual, y, None) if with_eps else (residual, y)


class _RopeInputs:
    """What RoPE needs for one packed forward (reference packed.py:355-379): the kernel's
    (positions [T] int64, inv_freq fp32) when the rotary embedding is HF's default type with
    attention_scaling 1.0 (Qwen2.5), else HF's cos/sin, built lazily once."""

    def __init__(self, model, hidden, pos):
        self.rotary, self.hidden, self.pos = model.rotary_emb, hidden, pos  # pos [1, T] int64
        self.positions = self.inv_freq = None
        self._cos_sin = None
        rot = self.rotary
        inv = getattr(rot, "inv_freq", None)
        hd = getattr(model.config, "head_dim", None) or \
            model.config.hidden_size // model.config.num_attention_heads
        if (USE_KERNELS and type(rot).__name__ == "Qwen2RotaryEmbedding" and not _has_hooks(rot)
                and getattr(rot, "rope_type", None) == "default"
                and getattr(rot, "attention_scaling", None) == 1.0
                and isinstance(inv, torch.Tensor) and inv.is_cuda and inv.dim() == 1
                and hd in (64, 128, 256) and inv.shape[0] == hd // 2):
            self.positions = pos.reshape(-1)
            self.inv_freq = inv.detach().to(torch.float32).contiguous()

    def cos_sin(self):
        if self._cos_sin is None:
            self._cos_sin = self.rotary(self.hidden, self.pos)
        return self._cos_sin


def _rope(q, k, rope_in, q_delta=None):
    """RoPE on q [1, T, Hq, D] and k [1, T, Hk, D] -> same shapes (reference packed.py:382-401).
    squeeze(0), not [0]: a view whose backward is a view too."""
    if (rope_in.positions is not None and q.dtype in _KERNEL_FLOATS and k.dtype == q.dtype
            and q.is_cuda and (q_delta is None or q_delta.dtype == q.dtype)):
        from .norm_rope import rope

        qo, ko = rope(q.squeeze(0), k.squeeze(0), rope_in.positions, rope_in.inv_freq,
                      q_delta=None if q_delta is None else q_delta.squeeze(0))
        return qo.unsqueeze(0), ko.unsqueeze(0)
    if q_delta is not None:
        q = q + q_delta.view_as(q)
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    cos, sin = rope_in.cos_sin()
    return apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=2)


_CU_CACHE = {}  # (device, lens) -> cu_seqlens of the current batch (one entry)


def _cu_seqlens(lens, device):
    key = (device, tuple(lens))
    cu = _CU_CACHE.get(key)
    if cu is None:
        from .attention import cu_seqlens_from_lengths

        _CU_CACHE.clear()
        cu = _CU_CACHE[key] = cu_seqlens_from_lengths(lens, device)
    return cu


def _attention(attn, q, k, v, lens):
    """Causal attention per original row on its packed slice. q [1, T, Hq, D], k/v [1, T, Hk, D]
    -> [1, T, Hq * D]. GQA: query head h uses kv head h // (Hq / Hk), as HF's repeat_kv.
    With the kernels on (fp16 / bf16, D in {64, 128}, no dropout) every row runs in one varlen
    launch (attention.varlen_attention); otherwise per row through torch's SDPA with the kv
    heads broadcast by a zero stride (reference packed.py:404-436)."""
    if torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        q, k, v = q.to(dt), k.to(dt), v.to(dt)
    hq, hk, d = q.shape[2], k.shape[2], q.shape[3]
    groups = hq // hk
    dropout = attn.attention_dropout if attn.training else 0.0
    if USE_KERNELS:
        from . import attention

        if attention.supported(q, k, v, dropout):
            o = attention.varlen_attention(q, k, v, _cu_seqlens(lens, q.device), max(lens),
                                           attn.scaling)
            return o.view(1, o.shape[0], hq * d)
        _fallback("attention kernel", f"dtype {q.dtype}, head_dim {d}, dropout {dropout}")
    outs = []
    for qr, kr, vr in zip(q.squeeze(0).split(lens), k.squeeze(0).split(lens),
                          v.squeeze(0).split(lens)):
        n = qr.shape[0]
        qh = qr.reshape(n, hk, groups, d).permute(1, 2, 0, 3)               # [Hk, G, n, D]
        kh = kr.permute(1, 0, 2).unsqueeze(1).expand(hk, groups, n, d)
        vh = vr.permute(1, 0, 2).unsqueeze(1).expand(hk, groups, n, d)
        o = F.scaled_dot_product_attention(qh, kh, vh, dropout_p=dropout, is_causal=True,
                                           scale=attn.scaling)
        outs.append(o.permute(2, 0, 1, 3))                                  # [n, Hk, G, D]
    out = torch.cat(outs, dim=0) if len(outs) > 1 else outs[0].contiguous()
    return out.reshape(1, out.shape[0], hq * d)


def _plain_silu_mlp(mlp, x):
    """An unmodified Qwen2MLP with silu and no hooks, on a CUDA input."""
    from transformers.models.qwen2.modeling_qwen2 import Qwen2MLP

    return (type(mlp) is Qwen2MLP and not _has_hooks(mlp) and x.is_cuda
            and getattr(getattr(mlp, "config", None), "hidden_act", None) == "silu")


def _mlp_layers(mlp, x):
    """(gate, up, down) when the recompute MLP applies to mlp(x), else None (reference
    packed.py:493-524, there for frozen NF4 projections): kernels and RECOMPUTE_MLP on, grad
    mode on, an unmodified silu Qwen2MLP whose projections are exactly nn.Linear without bias
    or hooks, no trainable parameter in the block, and an fp16 / bf16 CUDA x that the
    projections compute in (autocast to x's dtype, or weights of x's dtype)."""
    if not (USE_KERNELS and RECOMPUTE_MLP) or not torch.is_grad_enabled():
        return None
    why = "recompute MLP"
    if x.dtype not in (torch.float16, torch.bfloat16) or not _plain_silu_mlp(mlp, x):
        return _fallback(why, f"x {x.dtype}, {type(mlp).__name__}, hooks or activation")
    layers = (getattr(mlp, "gate_proj", None), getattr(mlp, "up_proj", None),
              getattr(mlp, "down_proj", None))
    autocast = torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == x.dtype
    for lin in layers:
        if type(lin) is not torch.nn.Linear or _has_hooks(lin) or lin.bias is not None:
            return _fallback(why, "projection not a plain bias-free nn.Linear")
        if not autocast and lin.weight.dtype != x.dtype:
            return _fallback(why, f"weights {lin.weight.dtype} without autocast to {x.dtype}")
    if any(q.requires_grad for q in mlp.parameters()):
        return _fallback(why, "trainable parameter in the MLP")
    return layers


class _RecomputeMLP(torch.autograd.Function):
    """down(silu(gate(x)) * up(x)) for frozen projections, saving nothing of size
    [T, intermediate] (reference packed.py:562-643; there the projections are frozen NF4, here
    frozen fp16 / bf16 nn.Linear, as in a LoRA run on an unquantized base).

    forward: g = x Wg^T, u = x Wu^T, h = silu(g) * u (HIP kernel, in place into g), out = h Wd^T.
    Saved: x itself (when the norm saves its output, the same tensor: no extra memory), or the
    norm's fp32 input r and weight, x then recomputed in backward by the same norm kernel
    (bit-exact, norm_rope.rmsnorm_recompute).
    backward: dh = dout Wd; g, u recomputed; (dg, du) = swiglu backward (HIP kernel, in place
    into g, u); dx_gate = dg Wg, dx_up = du Wu, returned as the grads of the two fan-out copies
    x_gate, x_up (the norm backward sums them; one tensor for both: autograd sums them).
    """

    @staticmethod
    @torch.amp.custom_fwd(device_type="cuda")
    def forward(ctx, x, x_up, r, w_norm, eps, gate, up, down):
        from . import _hip

        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        g = F.linear(x2, gate.weight).contiguous()
        u = F.linear(x2, up.weight).contiguous()
        _hip.swiglu_fwd(g, u, g)
        del u
        out = F.linear(g, down.weight)
        del g
        if r is not None:
            ctx.save_for_backward(r, w_norm)
        else:
            ctx.save_for_backward(x2)
        ctx.recompute_x = r is not None
        ctx.eps, ctx.shape, ctx.dtype, ctx.layers = eps, shape, x.dtype, (gate, up, down)
        return out.view(*shape[:-1], out.shape[-1])

    @staticmethod
    @torch.amp.custom_bwd(device_type="cuda")
    def backward(ctx, dout):
        from . import _hip

        gate, up, down = ctx.layers
        if ctx.recompute_x:
            from .norm_rope import rmsnorm_recompute

            r, w_norm = ctx.saved_tensors
            x2 = rmsnorm_recompute(r.reshape(-1, r.shape[-1]), w_norm, ctx.eps, ctx.dtype)
        else:
            (x2,) = ctx.saved_tensors
        dh = torch.matmul(dout.reshape(-1, dout.shape[-1]), down.weight)
        g = F.linear(x2, gate.weight).contiguous()
        u = F.linear(x2, up.weight).contiguous()
        del x2
        dh = dh.to(g.dtype).contiguous()
        _hip.swiglu_bwd(dh, g, u, g, u)  # dg into g, du into u
        del dh
        dx_gate = torch.matmul(g, gate.weight).to(ctx.dtype)
        del g
        dx_up = torch.matmul(u, up.weight).to(ctx.dtype)
        return dx_gate.view(ctx.shape), dx_up.view(ctx.shape), None, None, None, None, None, None


def _mlp(mlp, xs, norm=None, residual=None, eps=None, norm_saves_y=False):
    """Qwen2MLP on the post-attention norm's two outputs (gate, up): each projection takes its
    own copy, so the norm backward sums their input gradients (reference packed.py:676-693).
    Frozen projections: _RecomputeMLP (x recomputed from the norm's residual when the norm did
    not save its output). Otherwise, with the kernels on, the projections as the model's modules
    and silu(g) * u on the HIP kernel; else HF's ops."""
    x_gate, x_up = xs if isinstance(xs, tuple) else (xs, xs)
    layers = _mlp_layers(mlp, x_gate)
    if layers is not None:
        r = w_norm = None
        if (eps is not None and not norm_saves_y and residual is not None
                and residual.dtype == torch.float32 and residual.is_contiguous()):
            r, w_norm = residual, norm.weight.detach().to(torch.float32)
        return _RecomputeMLP.apply(x_gate, x_up, r, w_norm, eps, *layers)
    if USE_KERNELS and _plain_silu_mlp(mlp, x_gate):
        from ..swiglu import swiglu

        return mlp.down_proj(swiglu(mlp.gate_proj(x_gate), mlp.up_proj(x_up)))
    return mlp.down_proj(mlp.act_fn(mlp.gate_proj(x_gate)) * mlp.up_proj(x_up))


def _layer(layer, residual, delta, rope_in, lens):
    """One Qwen2DecoderLayer on packed tokens (reference packed.py:696-724). Returns
    (residual, delta) with the layer output residual + delta (the add is left pending so that it
    fuses with the next norm)."""
    attn = layer.self_attn
    residual, (x_q, x_k, x_v) = _add_norm(layer.input_layernorm, residual, delta, n_out=3,
                                          save_output=NORM_SAVE_OUTPUT)
    n = x_q.shape[1]
    hd = attn.head_dim
    q = attn.q_proj(x_q).view(1, n, -1, hd)
    k = attn.k_proj(x_k).view(1, n, -1, hd)
    v = attn.v_proj(x_v).view(1, n, -1, hd)
    q, k = _rope(q, k, rope_in)
    o = attn.o_proj(_attention(attn, q, k, v, lens))
    norm = layer.post_attention_layernorm
    residual, xs, eps = _add_norm(norm, residual, o, with_eps=True, n_out=2,
                                  save_output=NORM_SAVE_OUTPUT)
    return residual, _mlp(layer.mlp, xs, norm, residual, eps, norm_saves_y=NORM_SAVE_OUTPUT)


def _unsupported(model, input_ids, attention_mask, past_key_values, inputs_embeds, use_cache,
                 kwargs):
    """None if the packed path applies, else a short reason (reference packed.py:736-771)."""
    if not isinstance(model, torch.nn.Module) or not hasattr(model, "layers"):
        return "not a real model"
    config = getattr(model, "config", None)
    if config is None:
        return "no config"
    if inputs_embeds is not None:
        return "inputs_embeds"
    if not isinstance(input_ids, torch.Tensor) or input_ids.dim() != 2 or not input_ids.is_cuda:
        return "input_ids not 2D CUDA"
    if not isinstance(attention_mask, torch.Tensor) or attention_mask.shape != input_ids.shape:
        return "attention_mask missing or not 2D"
    if past_key_values is not None:
        return "past_key_values"
    if use_cache is None:
        use_cache = getattr(config, "use_cache", False)
    if use_cache:
        return "use_cache"
    for key in kwargs:
        if key not in _IGNORED_KWARGS:
            return f"kwarg {key}"
    for key in ("output_attentions", "output_hidden_states"):
        if kwargs.get(key, getattr(config, key, False)):
            return key
    if getattr(config, "_attn_implementation", None) != "sdpa":
        return "attn_implementation is not sdpa"
    if any(t != "full_attention" for t in getattr(config, "layer_types", ["full_attention"])):
        return "sliding window layers"
    if getattr(model, "gradient_checkpointing", False) and model.training:
        return "gradient checkpointing"
    for layer in model.layers[: config.num_hidden_layers]:
        if _has_hooks(layer) or _has_hooks(layer.self_attn):
            return "hooks on decoder layers"
    return None


def packed_forward(model, input_ids, attention_mask, position_ids, kwargs):
    """The packed decoder (reference packed.py:800-840). Returns [B, L, H] hidden states, or None
    for a batch with an empty row (the caller then runs the original forward)."""
    B, L = input_ids.shape
    mask = attention_mask.bool()
    lens = mask.sum(1).tolist()  # the one host sync of the forward
    if min(lens) == 0:
        return None
    T = sum(lens)
    flat_mask = mask.reshape(-1)
    idx = torch.nonzero_static(flat_mask, size=T).squeeze(1)  # row-major: rows stay in order

    if position_ids is None:
        pos = idx % L  # HF default: arange(L) for every row (left padding keeps it)
    else:
        pos = position_ids.expand(B, L).reshape(-1).index_select(0, idx)
    pos = pos.to(torch.int64).unsqueeze(0)

    hidden = model.embed_tokens(input_ids.reshape(-1).index_select(0, idx).unsqueeze(0))
    _WHERE[0], _WHERE[1] = bool(model.training), "embedding"
    rope_in = _RopeInputs(model, hidden, pos)

    residual, delta = hidden, None
    for i, layer in enumerate(model.layers[: model.config.num_hidden_layers]):
        _WHERE[1] = i
        residual, delta = _layer(layer, residual, delta, rope_in, lens)
    _WHERE[1] = "final norm"
    _, out = _add_norm(model.norm, residual, delta, final=True)
    _WHERE[0] = False

    # In place into fresh zeros (autograd records the copy; the source grad is
    # grad.index_select(0, idx)).
    full = out.new_zeros(B * L, out.shape[-1])
    full.index_copy_(0, idx, out.squeeze(0))
    return full.view(B, L, -1)


def patch():
    """Class-patch Qwen2Model.forward (idempotent; the original stays at forward.__wrapped__).
    Reference packed.py:843-875."""
    from transformers.modeling_outputs import BaseModelOutputWithPast
    from transformers.models.qwen2 import modeling_qwen2

    cls = modeling_qwen2.Qwen2Model
    if getattr(cls.forward, "_solution_body_packed", False):
        return
    original = cls.forward

    def forward(self, input_ids=None, attention_mask=None, position_ids=None,
                past_key_values=None, inputs_embeds=None, use_cache=None, **kwargs):
        reason = _unsupported(self, input_ids, attention_mask, past_key_values, inputs_embeds,
                              use_cache, kwargs)
        hidden = None
        if reason is None:
            hidden = packed_forward(self, input_ids, attention_mask, position_ids, kwargs)
            if hidden is None:
                reason = "a row without tokens"
        if hidden is not None and getattr(self, "training", False):
            _note_active()
        if hidden is None:
            if getattr(self, "training", False) and reason != "not a real model":
                _warn_once(reason)
            return original(self, input_ids=input_ids, attention_mask=attention_mask,
                            position_ids=position_ids, past_key_values=past_key_values,
                            inputs_embeds=inputs_embeds, use_cache=use_cache, **kwargs)
        out = BaseModelOutputWithPast(last_hidden_state=hidden, past_key_values=None)
        return_dict = kwargs.get("return_dict", getattr(self.config, "return_dict", True))
        return out.to_tuple() if return_dict is False else out

    forward._solution_body_packed = True
    forward.__wrapped__ = original
    cls.forward = forward


@contextlib.contextmanager
def kernels_enabled(on):
    """Temporarily set USE_KERNELS (tests, benchmarks)."""
    global USE_KERNELS
    old = USE_KERNELS
    USE_KERNELS = on
    try:
        yield
    finally:
        USE_KERNELS = old
