"""Fused LM-head linear + cross-entropy on this repository's HIP row kernel
(esep_head_row_softmax). Public API as in the reference's solution/head/op.py
(fused_linear_ce, FusedLinearCE, warmup, CHUNK_ROWS, G_SCALE, VOCAB; reference op.py:34-175).

    loss, stats = fused_linear_ce(x, w16, target, ce_weight)

x [N, H] (fp16, bf16 or fp32; cast to the weight's dtype for the products, its gradient comes
back in x's dtype); w16 [V, H] the frozen head weight (fp16 as the reference, or bf16; no
gradient); target [N] ints, anything outside [0, V) (e.g. -100) meaning "no CE term";
ce_weight [N] fp32 weight of each row's term (0 for rows without a target).
loss = sum_i ce_weight_i * (lse_i - z_i[target_i]), a 0-dim fp32 tensor, differentiable in x.
stats: detached [N] tensors "lse", "target_logit" (0 where ignored), "ce" (0 where ignored),
"entropy" (fp32) and "argmax" (int64), for every row.

Never materializes all N x V logits. Rows go through in chunks of `chunk_rows`: the chunk's
logits z = x_c W^T (hipBLASLt, the weight's dtype, fp32 accumulation) land in one reused
[chunk, V] buffer; the row kernel reads them once for the statistics and, when a gradient is
wanted, rewrites the rows that carry a loss with g = (softmax - onehot) * G_SCALE; then
dX_c = g W (hipBLASLt, fp32 out) for those rows, scaled by ce_weight / G_SCALE. The rows that
carry a loss are moved to the front first (a stable partition), so the g pass and the dX
product work on a prefix of each chunk. dX is finished in the forward; the backward only
scales it by the incoming gradient.
"""

import torch

from ..body import _hip

# Rows per chunk (the reference uses 256 for a 16 GB T4). The logits buffer is
# [CHUNK_ROWS, V] in the weight's dtype: 4096 x 151936 x 2 B = 1.16 GiB. On MI355X (Qwen2.5
# head, 8192 rows, forward + dX) 4096-row chunks take 7.9 ms against 21.6 ms at 256: the two
# products need the larger M to fill 256 CUs. (One 8192-row chunk measured 8.0 ms with every
# row weighted but 9.0 ms with every 7th row ignored: the dX product then runs at M = 7021, for
# which hipBLASLt picks a slower kernel than for 4096 + 2925.)
CHUNK_ROWS = 4096
# The probabilities are stored as (softmax - onehot) * G_SCALE in the 16-bit logits buffer so
# that small ones stay clear of the fp16 subnormal range; the dX product's fp32 result is
# divided by it again.
G_SCALE = 1024.0
# Qwen2.5 vocabulary size.
VOCAB = 151936

_KEYS = ("lse", "target_logit", "ce", "entropy", "argmax")


def warmup(device=None, vocab=VOCAB):
    """The reference compiles its Triton kernel here ahead of the first step; the HIP kernels
    are compiled ahead of time, so this only loads libesep_body.so."""
    _hip.lib()


class _RowOrder:
    """A stable partition of the rows: those with a nonzero loss weight first, in their
    original order, then the rest. `take` permutes per-row tensors into that order and `undo`
    brings results back. The identity (no copy) when no gradient pass is wanted."""

    def __init__(self, cew, partition):
        self.perm = self.inv = None
        self.n_live = 0
        if partition:
            live = cew != 0
            self.perm = torch.cat((live.nonzero().squeeze(1), (~live).nonzero().squeeze(1)))
            self.n_live = int(live.sum())  # the one host sync of the call
            self.inv = torch.empty_like(self.perm)
            self.inv[self.perm] = torch.arange(self.perm.numel(), device=self.perm.device)

    def take(self, t):
        return t.contiguous() if self.perm is None else t.index_select(0, self.perm)

    def undo(self, t):
        return t if self.inv is None else t.index_select(0, self.inv)


class _Chunks:
    """Statistics (and dX) of rows already in partition order, chunk by chunk."""

    def __init__(self, x16, w16, target, cew, n_live, want_dx, chunk_rows):
        self.x16, self.w16, self.target, self.cew = x16, w16, target, cew
        self.n_live, self.want_dx = n_live, want_dx
        n, h = x16.shape
        dev = x16.device
        self.rows = max(1, min(chunk_rows, n))
        self.z = torch.empty(self.rows, w16.shape[0], device=dev, dtype=w16.dtype)
        self.lse, self.tlogit, self.ent = (torch.empty(n, device=dev, dtype=torch.float32)
                                           for _ in range(3))
        self.amax = torch.empty(n, device=dev, dtype=torch.int32)
        self.dx = torch.zeros(n, h, device=dev, dtype=torch.float32) if want_dx else None
        self._full = None  # dX product over a whole chunk (see _dx)

    def run(self):
        n = self.x16.shape[0]
        for r0 in range(0, n, self.rows):
            self._chunk(r0, min(self.rows, n - r0))
        return self.lse, self.tlogit, self.ent, self.amax, self.dx

    def _chunk(self, r0, nr):
        rows = slice(r0, r0 + nr)
        z = self.z[:nr]
        torch.mm(self.x16[rows], self.w16.t(), out=z)
        _hip.head_row_softmax(z, self.target[rows], self.cew[rows], self.lse[rows],
                              self.tlogit[rows], self.ent[rows], self.amax[rows],
                              self.want_dx, G_SCALE)
        live = max(0, min(self.n_live - r0, nr))
        if self.want_dx and live:
            self._dx(r0, nr, live)

    def _dx(self, r0, nr, live):
        scale = (self.cew[r0:r0 + live] * (1.0 / G_SCALE)).unsqueeze(1)
        out = self.dx[r0:r0 + live]
        if live < self.rows <= 2 * live:
            # hipBLASLt runs this product much faster at the chunk's full row count than at a
            # ragged one (MI355X, K = 151936, N = 1536: M = 2925 2.06 ms, M = 4096 1.67 ms), so
            # it covers the whole buffer and keeps the first `live` rows (the others hold
            # logits or an earlier chunk's g and are dropped)
            if self._full is None:
                self._full = torch.empty(self.rows, self.x16.shape[1], device=self.x16.device,
                                         dtype=torch.float32)
            torch.mm(self.z, self.w16, out_dtype=torch.float32, out=self._full)
            torch.mul(self._full[:live], scale, out=out)
        else:
            torch.mm(self.z[:live], self.w16, out_dtype=torch.float32, out=out)
            out.mul_(scale)


def _forward(x, w16, target, ce_weight, want_dx, chunk_rows):
    """(loss, stats tuple in _KEYS order, dX fp32 or None) for the given rows."""
    vocab = w16.shape[0]
    has_target = (target >= 0) & (target < vocab)
    cew = torch.where(has_target, ce_weight.to(torch.float32), 0.0)
    tgt = torch.where(has_target, target, -1)
    order = _RowOrder(cew, want_dx)
    lse, tlogit, ent, amax, dx = _Chunks(order.take(x.to(w16.dtype)), w16, order.take(tgt),
                                         order.take(cew), order.n_live, want_dx,
                                         chunk_rows).run()
    lse, tlogit, ent, amax = (order.undo(t) for t in (lse, tlogit, ent, amax))
    dx = order.undo(dx) if dx is not None else None
    tlogit = torch.where(has_target, tlogit, 0.0)
    ce = torch.where(has_target, lse - tlogit, 0.0)
    return (cew * ce).sum(), (lse, tlogit, ce, ent, amax.to(torch.int64)), dx


class FusedLinearCE(torch.autograd.Function):
    """apply(x, w16, target, ce_weight, chunk_rows) -> (loss, lse, target_logit, ce, entropy,
    argmax). Only the loss is differentiable, in x; its dX comes from the forward."""

    @staticmethod
    def forward(ctx, x, w16, target, ce_weight, chunk_rows):
        loss, stats, dx = _forward(x, w16, target, ce_weight, True, chunk_rows)
        ctx.save_for_backward(dx)
        ctx.x_dtype = x.dtype
        ctx.mark_non_differentiable(*stats)
        return (loss, *stats)

    @staticmethod
    def backward(ctx, dloss, *_stat_grads):
        (dx,) = ctx.saved_tensors
        return (dx * dloss).to(ctx.x_dtype), None, None, None, None


def _check_args(x, w16, target, ce_weight):
    if x.dim() != 2 or w16.dim() != 2 or x.shape[1] != w16.shape[1]:
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, w16 {tuple(w16.shape)}")
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("x must be fp16, bf16 or fp32")
    if w16.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("w16 must be fp16 or bf16")
    if tuple(target.shape) != (x.shape[0],) or tuple(ce_weight.shape) != (x.shape[0],):
        raise ValueError("target and ce_weight must be [N]")
    if not (x.is_cuda and w16.is_cuda):
        raise ValueError("fused_linear_ce runs on the GPU (HIP tensors)")


def fused_linear_ce(x, w16, target, ce_weight, need_grad=None, chunk_rows=CHUNK_ROWS):
    """loss = sum_i ce_weight_i * CE(x_i @ w16^T, target_i) and the per-row stats dict.
    need_grad None means "grad mode is on and x requires grad"; without a gradient the g pass
    and the dX product are skipped."""
    _check_args(x, w16, target, ce_weight)
    if need_grad is None:
        need_grad = torch.is_grad_enabled() and x.requires_grad
    w16, target = w16.contiguous(), target.to(torch.int64)
    if x.shape[0] == 0:
        empty = torch.zeros(0, device=x.device, dtype=torch.float32)
        loss = torch.zeros((), device=x.device, dtype=torch.float32)
        if need_grad:
            loss = loss + x.float().sum()  # a zero that still reaches x
        return loss, dict(zip(_KEYS, (empty, empty, empty, empty, empty.to(torch.int64))))
    if need_grad:
        loss, *stats = FusedLinearCE.apply(x, w16, target, ce_weight, chunk_rows)
    else:
        with torch.no_grad():
            loss, stats, _ = _forward(x, w16, target, ce_weight, False, chunk_rows)
    return loss, dict(zip(_KEYS, stats))
