"""Residual-add + RMSNorm (K1) and rotary embedding (K2) of the Qwen2 decoder body, on
hand-written HIP kernels for MI355X (gfx950) behind the C ABI of libesep_body.so.

Drop-in for the reference module solution/body/norm_rope.py (gojosatorukz/esep-soup-kernels):
the public names, signatures, saved tensors, gradient dtypes and launch counts are the
reference's; the kernels underneath are this repository's (csrc/*.hip). Citations below are
file:line in the reference.

K1 add_rmsnorm(r_in, delta, w, eps, out_dtype, n_out=1, save_output=False) -> (r_out, y)
    r_out = r_in + delta (fp32), y = w * (r_out * rsqrt(mean(r_out^2) + eps)) stored as
    out_dtype (fp32 math, one rounding). Reference: norm_rope.py:7-37, :83-109, :289-306.
    Saved for backward: (r_out, rstd, w), or with save_output (a delta and a 16-bit y):
    (y, rstd, w, slots[, xs]) where xs holds the exact xhat of the channels whose |w| makes
    y / w ill-conditioned (special_channels). n_out > 1 returns n_out views of one y, whose
    gradients the backward kernel sums in fp32 (one launch).
    Weight gradient: the reference treats the norm weight as frozen (norm_rope.py:12-14, :304)
    and returns None for it. Here the weight gets a gradient exactly when it requires one
    (weight.requires_grad under grad mode): dw_j = sum_t dy_tj * xhat_tj, reduced in two fixed
    stages in fp32, so it is bitwise reproducible. A frozen weight (the reference's use, a
    QLoRA base model) behaves as in the reference.

K2 rope(q, k, positions, inv_freq, q_delta=None, cu_seqlens=None) -> (q_rot, k_rot)
    q [T, HQ, D], k [T, HK, D] (any token/head strides, unit last stride), positions [T]
    int32/int64, or cu_seqlens int32 [n_seq + 1] for positions restarting at every packed
    sequence. angle = float(pos) * inv_freq[j] (one fp32 multiply), cos/sin computed in the
    kernel, rotate_half convention; q_delta is added to q in the storage dtype first.
    Reference: norm_rope.py:39-50, :330-445 (positions only).
    rope_bhsd(q, k, inv_freq, position_ids=None) is the same rotation for HF's padded
    [B, H, S, D] layout (HF apply_rotary_pos_emb with unsqueeze_dim=1).

rmsnorm(x, weight, eps, out_dtype=None, recompute_rstd=False) -> y
    Plain RMSNorm of a 16-bit or fp32 activation (the north star's input / post-attention /
    final norm without a residual stream): y in x's dtype, dx in x's dtype, dw when the weight
    requires a gradient, rstd saved or recomputed in backward.
"""

import math
import threading
import weakref

import torch

from . import _hip

# Widest row the K1 kernels take (columns). The reference caps at 2048 (norm_rope.py:73).
NORM_BLOCK = 16384
# Most gradients of one norm output summed by the backward kernel (norm_rope.py:113).
MAX_DY = 5
# save_output mode: channels with |w| < SPECIAL_W_MIN, |w| > 65504 / sqrt(H) or a non-finite w
# keep an exact fp32 xhat (norm_rope.py:165-170). Read at call time (tests monkeypatch it).
SPECIAL_W_MIN = 2.0 ** -10

_FLOATS = (torch.float32, torch.float16, torch.bfloat16)

# Attribute under which special_channels memoizes its answer on the weight tensor itself.
_MEMO_ATTR = "_esep_exact_channels"


def special_channels(weight):
    """(slots int32 [H], K) for a frozen norm weight [H]: slots[j] = 0..K-1 (ascending channel
    order) for the channels whose xhat is saved exactly, -1 elsewhere. Reference:
    norm_rope.py:183-205.

    A channel is well-conditioned for the y / w recovery when SPECIAL_W_MIN <= |w| <=
    65504 / sqrt(H); every other channel (tiny, huge, NaN or infinite weight) is exact. The
    answer is memoized on the weight tensor, tagged with its storage address, version counter,
    size, dtype and the threshold in force: an in-place edit (which bumps the version) or a
    new threshold recomputes it, and the memo dies with the tensor. Computing it costs one
    host sync (the count K)."""
    thr = float(SPECIAL_W_MIN)
    tag = (weight.data_ptr(), weight._version, weight.numel(), weight.dtype, thr)
    memo = getattr(weight, _MEMO_ATTR, None)
    if memo is not None and memo[0] == tag:
        return memo[1], memo[2]
    mag = weight.detach().to(torch.float32).abs()
    limit = 65504.0 / math.sqrt(weight.shape[0])
    exact = ~((mag >= thr) & (mag <= limit))  # NaN fails both comparisons
    rank = torch.cumsum(exact, 0, dtype=torch.int32) - 1
    slots = torch.where(exact, rank, torch.full_like(rank, -1))
    count = int(exact.sum())
    try:
        setattr(weight, _MEMO_ATTR, (tag, slots, count))
    except (AttributeError, TypeError):  # a tensor subclass without attributes: no memo
        pass
    return slots, count


def _weight_f32(weight, grad):
    """The norm weight as the kernels read it: contiguous fp32 [H]. Differentiable when the
    weight gets a gradient (the cast's backward returns dw in the weight's dtype)."""
    w = weight if grad else weight.detach()
    return w.to(torch.float32).contiguous()


def _wants_weight_grad(weight):
    return bool(weight.requires_grad and torch.is_grad_enabled())


def _rows_of(t, dtype=None):
    """t [..., n] as a dense [rows, n] tensor (optionally cast): the kernels' row layout."""
    n = t.shape[-1]
    flat = t.reshape(-1, n)
    if dtype is not None and flat.dtype != dtype:
        flat = flat.to(dtype)
    return flat.contiguous()


# ----------------------------------------------------------------------------------------
# Weight gradient: stage 2 deferred to the end of the backward pass
# ----------------------------------------------------------------------------------------
# A trainable norm weight's gradient is reduced in two fixed-order stages: the backward kernel
# writes [P, n] fp32 partials (P depends on the shape only) and stage 2 sums them over P. With
# DEFER_WEIGHT_GRAD on (read at call time), a backward pass that accumulates into the weight's
# .grad (loss.backward(), not autograd.grad) keeps each norm's partials and runs stage 2 once
# at the end of the pass for every norm (esep_dgamma_reduce_batch: one launch per 64 norms
# instead of one per norm), then accumulates the results into .grad. The gradients are the same
# bits either way. It is not used (each backward reduces its own partials and returns dw as
# usual) under autograd.grad or backward(inputs=...) without the weight, with hooks on the
# weight, for a double backward (create_graph=True), inside a torch.distributed job (whose
# gradient hooks expect every gradient through autograd), for a weight that is not a parameter
# or its dtype cast (p * 0.5, a row of a stacked parameter: autograd applies their chain rule),
# and whenever the autograd engine's entry points it relies on are missing or fail. Partials of a
# pass that ends in an exception are dropped with the pass.
DEFER_WEIGHT_GRAD = True

_defer_lock = threading.Lock()
_deferred = {}  # autograd graph task id -> [(weight leaf, partials, stream)]

# grad_fn types of the chain _weight_f32 builds between a trainable weight and the kernel's
# fp32 weight: a dtype cast and a contiguous copy, whose chain rule is a cast back / identity
_CAST_NODES = ("ToCopyBackward0", "CloneBackward0")


def _weight_leaf(w):
    """The trainable leaf parameter behind the kernel weight w, when w is that leaf or comes from
    it through the casts _weight_f32 makes (dtype cast, contiguous copy: nothing else) with the
    same shape and device; else None. Only such a leaf can take the deferred gradient, which is
    written into its .grad directly (cast to its dtype: the casts' own chain rule); any other
    weight (p * 0.5, a row of a stacked parameter, a view) takes the per-call path and gets its
    gradient through autograd."""
    if w.is_leaf:
        return w if w.requires_grad else None
    node, hops = w.grad_fn, 0
    while node is not None and type(node).__name__ in _CAST_NODES and hops < 2:
        nxt = [f for f, _ in node.next_functions if f is not None]
        if len(nxt) != 1:
            return None
        node, hops = nxt[0], hops + 1
    if node is None or type(node).__name__ != "AccumulateGrad":
        return None
    leaf = getattr(node, "variable", None)
    if leaf is None or leaf.shape != w.shape or leaf.device != w.device:
        return None
    return leaf


def _engine():
    """The autograd engine's entry points the deferral uses (looked up at each call), or None
    when this torch lacks one of them: the per-call path then serves every backward."""
    try:
        return (torch.autograd.graph.get_gradient_edge, torch._C._will_engine_execute_node,
                torch._C._current_graph_task_id,
                torch.autograd.Variable._execution_engine.queue_callback)
    except AttributeError:
        return None


def _can_defer(leaf):
    if not DEFER_WEIGHT_GRAD or leaf is None or not leaf.requires_grad or torch.is_grad_enabled():
        return False
    if leaf._backward_hooks or getattr(leaf, "_post_accumulate_grad_hooks", None):
        return False
    if torch.distributed.is_available() and torch.distributed.is_initialized():
        return False
    eng = _engine()
    if eng is None:
        return False
    get_edge, will_execute = eng[0], eng[1]
    try:
        return bool(will_execute(get_edge(leaf).node))
    except Exception:  # outside a backward pass, or an engine that changed: per call
        return False


class _PassToken:
    """Held by the end-of-pass callback of one backward pass (graph task). The engine drops its
    callbacks when the pass ends, normally or by an exception; the token then dies and takes the
    pass's entries (partials included) out of _deferred if the callback never ran."""

    __slots__ = ("task", "__weakref__")

    def __init__(self, task):
        self.task = task


def _drop_task(task):
    with _defer_lock:
        _deferred.pop(task, None)


def _defer(leaf, partials):
    """Keep one norm's partials for the end of the current backward pass. Returns False (nothing
    kept: the caller reduces them itself) when the engine's entry points are missing or fail."""
    eng = _engine()
    if eng is None:
        return False
    current_task, queue_callback = eng[2], eng[3]
    try:
        task = current_task()
        stream = torch.cuda.current_stream(partials.device)
    except Exception:
        return False
    with _defer_lock:
        entries = _deferred.get(task)
        first = entries is None
        if first:
            entries = _deferred[task] = []
    if first:
        token = _PassToken(task)
        weakref.finalize(token, _drop_task, task)
        try:
            queue_callback(lambda: _finish_deferred(token))
        except Exception:
            _drop_task(task)
            return False
    with _defer_lock:
        entries.append((leaf, partials, stream))
    return True


def _weight_grad_or_defer(ctx, partials):
    """After a backward kernel wrote a deferred norm's partials: None when they were queued for
    the end of the pass, else their stage 2 now (the per-call gradient)."""
    if _defer(ctx.weight_leaf, partials):
        return None
    dw = torch.empty((partials.shape[1],), device=partials.device, dtype=torch.float32)
    _hip.dgamma_reduce(partials, dw)
    return dw


def _finish_deferred(token):
    """End of a backward pass: stage 2 of every deferred norm, batched per (device, dtype, n),
    accumulated into the weights' .grad on the caller's current stream (the engine has made it
    wait for the leaf streams; the streams the partials were written on are waited for too)."""
    with _defer_lock:
        items = _deferred.pop(token.task, [])
    groups = {}
    for leaf, part, stream in items:
        key = (part.device, leaf.dtype, part.shape[1])
        groups.setdefault(key, []).append((leaf, part, stream))
    with torch.no_grad():
        for (dev, dtype, n), grp in groups.items():
            cur = torch.cuda.current_stream(dev)
            for st in {st for _, _, st in grp}:
                if st != cur:
                    cur.wait_stream(st)
            out_dtype = dtype if dtype in _FLOATS else torch.float32
            for i in range(0, len(grp), _hip.DGAMMA_BATCH_MAX):
                chunk = grp[i:i + _hip.DGAMMA_BATCH_MAX]
                dws = [torch.empty((n,), device=dev, dtype=out_dtype) for _ in chunk]
                _hip.dgamma_reduce_batch([part for _, part, _ in chunk], dws)
                for (leaf, part, _), dw in zip(chunk, dws):
                    part.record_stream(cur)
                    g = dw if dw.dtype == leaf.dtype else dw.to(leaf.dtype)
                    if leaf.grad is None:
                        leaf.grad = g
                    else:
                        leaf.grad.add_(g)


def _weight_grad_target(ctx, w, rows, w_index):
    """(dw buffer or None, partials or None) for a backward: partials when stage 2 is deferred
    (dw is then not returned: it reaches .grad at the end of the pass), else a dw buffer when
    the weight (apply() argument w_index) needs a gradient."""
    if not ctx.needs_input_grad[w_index]:
        return None, None
    n = w.shape[0]
    if rows > 0 and _can_defer(ctx.weight_leaf):
        P = _hip.rmsnorm_partials(rows, n)
        return None, torch.empty((P, n), device=w.device, dtype=torch.float32)
    return torch.empty((n,), device=w.device, dtype=torch.float32), None


class AddRMSNorm(torch.autograd.Function):
    """Reference: norm_rope.py:208-286 (same apply() arguments and saved tensors).

    apply(r_in, delta, w, eps, out_dtype, n_out, slots, n_special) -> (r_out, y_1 .. y_n_out)

    Saved for backward: (r_out, rstd, w); with slots given (save-output mode), (y, rstd, w,
    slots, xs) where xs [rows, K] holds the exact xhat of the K special channels. Outputs whose
    gradient nothing produces arrive in backward as None (no zero tensors)."""

    @staticmethod
    def forward(ctx, r_in, delta, w, eps, out_dtype, n_out, slots, n_special):
        shape = r_in.shape
        n = shape[-1]
        assert n <= NORM_BLOCK, f"row of {n} columns is wider than NORM_BLOCK={NORM_BLOCK}"
        assert 1 <= n_out <= MAX_DY, f"n_out={n_out} outside 1..{MAX_DY}"
        resid_in = _rows_of(r_in, torch.float32)
        rows, dev = resid_in.shape[0], resid_in.device
        save_y = slots is not None
        k_exact = n_special if save_y else 0

        y = torch.empty((rows, n), device=dev, dtype=out_dtype)
        rstd = torch.empty((rows,), device=dev, dtype=torch.float32)
        xs = torch.empty((rows, k_exact), device=dev, dtype=torch.float32) if k_exact else None
        # Without a delta the residual passes through unchanged (r_out aliases r_in) and its
        # gradient comes back to backward as dr_out; with one, the kernel writes the sum.
        add = None if delta is None else _rows_of(delta)
        resid_out = resid_in if add is None else torch.empty_like(resid_in)
        if rows:
            _hip.rmsnorm_fwd(resid_in, w, y, eps, delta=add,
                             r_out=None if add is None else resid_out, rstd=rstd,
                             slot=slots if k_exact else None, xs=xs, n_special=k_exact)

        ctx.save_for_backward(*((y, rstd, w, slots, xs) if save_y else (resid_out, rstd, w)))
        ctx.weight_leaf = _weight_leaf(w) if w.requires_grad else None
        ctx.from_y, ctx.n_special, ctx.eps, ctx.shape = save_y, k_exact, eps, shape
        ctx.has_delta = add is not None
        ctx.delta_dtype = None if delta is None else delta.dtype
        ctx.set_materialize_grads(False)
        # One buffer, n_out distinct views: each consumer's gradient reaches backward on its
        # own and the kernel sums them there.
        return (resid_out.view(shape),) + tuple(y.view(shape) for _ in range(n_out))

    @staticmethod
    def backward(ctx, dr_out, *dys):
        if ctx.from_y:
            x, rstd, w, slots, xs = ctx.saved_tensors
        else:
            (x, rstd, w), slots, xs = ctx.saved_tensors, None, None
        n = x.shape[-1]
        rows = x.shape[0]
        dys = [d.reshape(-1, n).contiguous() for d in dys if d is not None]
        has_dr = dr_out is not None
        want_r = ctx.needs_input_grad[0]
        write_dd = ctx.has_delta and ctx.needs_input_grad[1]
        want_w = ctx.needs_input_grad[2]
        if not dys and not has_dr:
            dw = torch.zeros_like(w) if want_w else None
            return None, None, dw, None, None, None, None, None
        dev = x.device
        dr = torch.empty((rows, n), device=dev, dtype=torch.float32) if want_r else None
        ddelta = torch.empty((rows, n), device=dev, dtype=ctx.delta_dtype) if write_dd else None
        dw, partials = _weight_grad_target(ctx, w, rows, 2)
        dr2 = dr_out.reshape(-1, n).to(torch.float32).contiguous() if has_dr else None
        if rows > 0 and (dr is not None or ddelta is not None or want_w):
            _hip.rmsnorm_bwd(dys, x, w, ctx.eps, from_y=ctx.from_y, rstd=rstd, dr_out=dr2,
                             slot=slots if ctx.n_special else None, xs=xs,
                             n_special=ctx.n_special, dr=dr, dx=ddelta, dw=dw, partials=partials)
            if partials is not None:
                dw = _weight_grad_or_defer(ctx, partials)
        elif dw is not None:
            dw.zero_()
        d_rin = dr.view(ctx.shape) if want_r else None
        d_delta = ddelta.view(ctx.shape) if write_dd else None
        return d_rin, d_delta, dw, None, None, None, None, None


def add_rmsnorm(r_in, delta, weight, eps=1e-6, out_dtype=torch.float16, n_out=1,
                save_output=False):
    """r_out = r_in + delta; y = weight * rmsnorm(r_out). Returns (r_out fp32, y out_dtype);
    with n_out > 1, (r_out, (y_1, ..., y_n_out)): views of one y, one per consumer, whose
    gradients the backward kernel sums (no autograd add kernels).

    r_in: fp32 [..., H]; delta: fp16/bf16/fp32 [..., H] or None (then r_out is r_in);
    weight: [H]; gets a gradient only if it requires one (see the module docstring).
    save_output: backward from the saved y (+ exact xhat of the ill-conditioned channels)
    instead of the fp32 r_out; applies only with a delta and a 16-bit y, else ignored.
    Reference: norm_rope.py:289-306.
    """
    if out_dtype not in _FLOATS:
        raise TypeError(f"out_dtype {out_dtype} not supported")
    # y stands in for the residual in backward only where it is worth it and well defined: a
    # residual add happened and y is a 16-bit copy (else the fp32 r_out is saved)
    keep_y = save_output and delta is not None and out_dtype != torch.float32
    slots, n_exact = special_channels(weight) if keep_y else (None, 0)
    w = _weight_f32(weight, _wants_weight_grad(weight))
    r_out, *ys = AddRMSNorm.apply(r_in, delta, w, float(eps), out_dtype, int(n_out), slots,
                                  n_exact)
    return r_out, (ys[0] if n_out == 1 else tuple(ys))


def rmsnorm_recompute(r, w, eps, out_dtype=torch.float16):
    """y = w * rmsnorm(r) for fp32 r [T, H] (contiguous) and fp32 w [H], no autograd.

    The same forward kernel as add_rmsnorm on its saved fp32 residual: bit-for-bit the y that
    add_rmsnorm returned for it. Reference: norm_rope.py:309-323.
    """
    y = torch.empty(r.shape, device=r.device, dtype=out_dtype)
    if r.shape[0]:
        w32 = w.detach().to(torch.float32).contiguous()
        _hip.rmsnorm_fwd(r, w32, y, eps)  # no rstd, no residual add: the forward's y only
    return y


# ----------------------------------------------------------------------------------------
# Plain RMSNorm (no residual stream), with weight gradient and saved or recomputed rstd
# ----------------------------------------------------------------------------------------
class RMSNorm(torch.autograd.Function):
    """y = w * rmsnorm(x) for x [rows, n] in fp32/fp16/bf16. Saved: (x, w, rstd) or, with
    recompute_rstd, (x, w) and backward recomputes rstd from x (bitwise what the forward
    computed). Gradients: dx in x's dtype; dw (fp32, cast by the caller) if w requires it."""

    @staticmethod
    def forward(ctx, x, w, eps, out_dtype, recompute_rstd):
        shape = x.shape
        n = shape[-1]
        assert n <= NORM_BLOCK, "row wider than NORM_BLOCK"
        x2 = x.reshape(-1, n)
        # the kernels take rows with a unit column stride that do not overlap
        if (n > 1 and x2.stride(1) != 1) or (x2.shape[0] > 1 and x2.stride(0) < n):
            x2 = x2.contiguous()
        rows = x2.shape[0]
        y = torch.empty((rows, n), device=x.device, dtype=out_dtype)
        rstd = None if recompute_rstd else torch.empty((rows,), device=x.device,
                                                       dtype=torch.float32)
        if rows > 0:
            _hip.rmsnorm_fwd(x2, w, y, eps, rstd=rstd)
        if recompute_rstd:
            ctx.save_for_backward(x2, w)
        else:
            ctx.save_for_backward(x2, w, rstd)
        ctx.eps, ctx.shape, ctx.recompute = eps, shape, recompute_rstd
        ctx.weight_leaf = _weight_leaf(w) if w.requires_grad else None
        return y.view(shape)

    @staticmethod
    def backward(ctx, dy):
        if ctx.recompute:
            (x2, w), rstd = ctx.saved_tensors, None
        else:
            x2, w, rstd = ctx.saved_tensors
        rows, n = x2.shape
        want_x, want_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dx = torch.empty((rows, n), device=x2.device, dtype=x2.dtype) if want_x else None
        dw, partials = _weight_grad_target(ctx, w, rows, 1)
        if rows > 0 and (want_x or want_w):
            dy2 = dy.reshape(-1, n).contiguous()
            out = dict(dr=dx) if x2.dtype == torch.float32 else dict(dx=dx)
            _hip.rmsnorm_bwd([dy2], x2, w, ctx.eps, rstd=rstd, dw=dw, partials=partials, **out)
            if partials is not None:
                dw = _weight_grad_or_defer(ctx, partials)
        elif dw is not None:
            dw.zero_()
        return (dx.view(ctx.shape) if want_x else None), dw, None, None, None


def rmsnorm(x, weight, eps=1e-6, out_dtype=None, recompute_rstd=False):
    """y = weight * rmsnorm(x) over the last dim, fp32 math, one rounding to out_dtype
    (default: x's dtype). HF Qwen2RMSNorm.forward semantics for the input / post-attention /
    final norms without a residual stream; weight gets a gradient if it requires one.
    recompute_rstd: do not save rstd; backward recomputes it from x."""
    if x.dtype not in _FLOATS:
        raise TypeError(f"x dtype {x.dtype} not supported")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    w = _weight_f32(weight, _wants_weight_grad(weight))
    return RMSNorm.apply(x, w, float(eps), out_dtype, bool(recompute_rstd))


class FusedRMSNorm(torch.nn.Module):
    """Module form of rmsnorm, interchangeable with HF Qwen2RMSNorm (weight, variance_epsilon)."""

    def __init__(self, hidden_size, eps=1e-6, device=None, dtype=None, recompute_rstd=False):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(hidden_size, device=device, dtype=dtype))
        self.variance_epsilon = eps
        self.recompute_rstd = recompute_rstd

    def forward(self, hidden_states):
        return rmsnorm(hidden_states, self.weight, self.variance_epsilon,
                       recompute_rstd=self.recompute_rstd)


# ----------------------------------------------------------------------------------------
# K2: rotary embedding for q and k in one launch
# ----------------------------------------------------------------------------------------
def _unit_last(t):
    return t if t.shape[-1] <= 1 or t.stride(-1) == 1 else t.contiguous()


def _launch_rope(q4, k4, inv_freq, sign, qd4=None, positions=None, cu_seqlens=None, bhsd=False):
    """q4 / k4 / qd4: (B, S, H, D) views. Outputs: for the packed layout fresh contiguous
    [T, H, D] tensors (as (1, T, H, D) views); for [B, H, S, D] tensors laid out like the
    input (empty_like keeps a dense input's stride order)."""
    if bhsd:
        qo = torch.empty_like(q4.transpose(1, 2)).transpose(1, 2)
        ko = torch.empty_like(k4.transpose(1, 2)).transpose(1, 2)
    else:
        qo = torch.empty(q4.shape, device=q4.device, dtype=q4.dtype)
        ko = torch.empty(k4.shape, device=k4.device, dtype=k4.dtype)
    if q4.shape[0] * q4.shape[1] > 0:
        _hip.rope(q4, k4, qo, ko, inv_freq, sign, q_delta=qd4, positions=positions,
                  cu_seqlens=cu_seqlens)
    return qo, ko


class Rope(torch.autograd.Function):
    """Reference: norm_rope.py:396-420. apply(q, k, positions, inv_freq, q_delta) for the packed
    [T, H, D] layout, plus cu_seqlens (positions None) and the [B, H, S, D] layout (bhsd)."""

    @staticmethod
    def forward(ctx, q, k, positions, inv_freq, q_delta, cu_seqlens=None, bhsd=False):
        q, k = _unit_last(q), _unit_last(k)
        if bhsd:
            q4, k4 = q.transpose(1, 2), k.transpose(1, 2)
            pos2 = positions
        else:
            q4, k4 = q.unsqueeze(0), k.unsqueeze(0)
            pos2 = positions.view(1, -1) if positions is not None else None
        qd4 = None
        if q_delta is not None:
            qd = _unit_last(q_delta.reshape(q.shape))
            qd4 = qd.transpose(1, 2) if bhsd else qd.unsqueeze(0)
        qo4, ko4 = _launch_rope(q4, k4, inv_freq, 1.0, qd4, pos2, cu_seqlens, bhsd)
        ctx.save_for_backward(*(t for t in (positions, inv_freq, cu_seqlens) if t is not None))
        ctx.has_pos, ctx.has_cu, ctx.bhsd = positions is not None, cu_seqlens is not None, bhsd
        ctx.q_shape, ctx.q_dtype = q.shape, q.dtype
        ctx.k_shape, ctx.k_dtype = k.shape, k.dtype
        ctx.has_qd = q_delta is not None
        ctx.qd_shape = q_delta.shape if q_delta is not None else None
        if bhsd:
            return qo4.transpose(1, 2), ko4.transpose(1, 2)
        return qo4.squeeze(0), ko4.squeeze(0)

    @staticmethod
    def backward(ctx, dqo, dko):
        saved = list(ctx.saved_tensors)
        positions = saved.pop(0) if ctx.has_pos else None
        inv_freq = saved.pop(0)
        cu_seqlens = saved.pop(0) if ctx.has_cu else None
        dev = inv_freq.device
        # A None gradient (output unused) becomes zeros (reference norm_rope.py:411-415).
        if dqo is None:
            dqo = torch.zeros(ctx.q_shape, device=dev, dtype=ctx.q_dtype)
        if dko is None:
            dko = torch.zeros(ctx.k_shape, device=dev, dtype=ctx.k_dtype)
        dqo, dko = _unit_last(dqo), _unit_last(dko)
        if ctx.bhsd:
            q4, k4, pos2 = dqo.transpose(1, 2), dko.transpose(1, 2), positions
        else:
            q4, k4 = dqo.unsqueeze(0), dko.unsqueeze(0)
            pos2 = positions.view(1, -1) if positions is not None else None
        dq4, dk4 = _launch_rope(q4, k4, inv_freq, -1.0, None, pos2, cu_seqlens, ctx.bhsd)
        if ctx.bhsd:
            dq, dk = dq4.transpose(1, 2), dk4.transpose(1, 2)
        else:
            dq, dk = dq4.squeeze(0), dk4.squeeze(0)
        # d(q_delta) == d(q): the delta is added before the rotation.
        dqd = dq.reshape(ctx.qd_shape) if ctx.has_qd and ctx.needs_input_grad[4] else None
        return dq, dk, None, None, dqd, None, None


def default_inv_freq(head_dim=128, theta=1e6, device=None):
    """HF default-rope inverse frequencies, computed exactly as transformers does (fp32, on the
    CPU, then moved). Reference: norm_rope.py:423-426."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    return inv.to(device)


def _check_head_dim(d):
    assert d % 2 == 0, "head dim must be even"
    assert (d // 2) & (d // 2 - 1) == 0, "D/2 must be a power of two"


def rope(q, k, positions, inv_freq, q_delta=None, cu_seqlens=None):
    """Rotate q [T, HQ, D] and k [T, HK, D] by per-token angles pos * inv_freq.

    positions: int32/int64 [T] on the device; or None with cu_seqlens (int32 [n_seq + 1],
    cu_seqlens[0] = 0, cu_seqlens[-1] = T): position = token index - start of its sequence.
    q_delta: optional [T, HQ*D] or [T, HQ, D] in q's dtype, added to q in that dtype before the
    rotation; its gradient is q's gradient. inv_freq: fp32 [D/2] (the model's
    rotary_emb.inv_freq). Returns fresh contiguous (q_rot, k_rot) in q's / k's dtype.
    Reference: norm_rope.py:429-445.
    """
    assert q.dim() == 3 and k.dim() == 3 and q.shape[0] == k.shape[0]
    assert q.shape[-1] == k.shape[-1]
    _check_head_dim(q.shape[-1])
    assert (positions is None) != (cu_seqlens is None), "give positions or cu_seqlens"
    if positions is not None:
        assert positions.shape[0] == q.shape[0]
        positions = positions.contiguous()
    else:
        cu_seqlens = cu_seqlens.to(torch.int32).contiguous()
    inv_freq = inv_freq.detach().to(torch.float32).contiguous()
    return Rope.apply(q, k, positions, inv_freq, q_delta, cu_seqlens, False)


def rope_bhsd(q, k, inv_freq, position_ids=None, q_delta=None):
    """HF apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=1) for q [B, HQ, S, D] and
    k [B, HK, S, D] (any strides with a unit last stride, e.g. HF's transposed projection
    views), with cos/sin computed in the kernel from position_ids ([B, S] or [1, S], int32 or
    int64; None: 0..S-1 per row) and inv_freq."""
    assert q.dim() == 4 and k.dim() == 4 and q.shape[0] == k.shape[0] and q.shape[2] == k.shape[2]
    assert q.shape[-1] == k.shape[-1]
    _check_head_dim(q.shape[-1])
    if position_ids is not None:
        assert position_ids.dim() == 2 and position_ids.shape[1] == q.shape[2]
        assert position_ids.shape[0] in (1, q.shape[0])
    inv_freq = inv_freq.detach().to(torch.float32).contiguous()
    return Rope.apply(q, k, position_ids, inv_freq, q_delta, None, True)
