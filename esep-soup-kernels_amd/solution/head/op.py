"""Fused linear + cross-entropy over the LM head on this repository's HIP row kernel: the
reference's solution/head/op.py API (fused_linear_ce, FusedLinearCE, warmup) with the Triton
row kernel replaced by esep_head_row_softmax.

``loss, stats = fused_linear_ce(x, w16, target, ce_weight)``

- x:         [N, H] fp16 / bf16 / fp32 hidden states (after the final norm). Cast to the head
             weight's dtype inside; the gradient comes back in x.dtype.
- w16:       [V, H] frozen LM head weight, fp16 (the reference's) or bf16; gets no gradient.
- target:    [N] int, -100 (or any id outside [0, V)) = no CE term for the row
- ce_weight: [N] fp32 weight of each row's CE term (forced to 0 for ignored rows)
- loss:      0-dim fp32, sum_i ce_weight_i * (lse_i - z_i[target_i]); differentiable w.r.t. x
- stats:     dict of detached [N] tensors for every row: "lse", "target_logit" (0 where ignored),
             "ce" (0 where ignored), "entropy" (fp32) and "argmax" (int64)

Per chunk of rows (reference op.py:63-93): z = x_c W^T by hipBLASLt (logits in the weight's
dtype, fp32 accumulation) into one reused [chunk, V] buffer; esep_head_row_softmax computes the
row statistics and overwrites the weighted rows with g = (softmax - onehot) * G_SCALE in place;
dX_c = g W by hipBLASLt with fp32 output, for the weighted rows only (computed over the whole
chunk when at least half of it is weighted: a faster GEMM shape), scaled by ce_weight / G_SCALE
in fp32. Rows that carry a loss are moved to the front first (stable), so
the g pass and the second GEMM run on a prefix. dX is computed in the forward (when a gradient
is wanted) and the backward only scales it by the incoming gradient.
"""

import torch

from ..body import _hip

# Rows per chunk (reference op.py:34 uses 256). The chunk buffer is [CHUNK_ROWS, V] in the
# weight's dtype: 4096 x 151936 x 2 B = 1.16 GiB, small against the 288 GB of an MI355X. On
# MI355X (Qwen2.5 head, 8192 rows, forward + dX) 4096-row chunks take 7.9 ms against 21.6 ms
# with 256: the two GEMMs need the larger M to fill 256 CUs. (One 8192-row chunk measured 8.0 ms
# with every row weighted but 9.0 ms with every 7th row ignored: the dX GEMM then runs at
# M = 7021, for which hipBLASLt picks a slower kernel than for 4096 + 2925.)
CHUNK_ROWS = 4096
# g = (softmax - onehot) * G_SCALE in fp16 keeps small probabilities out of the fp16 subnormal
# range (reference op.py:36); undone in fp32 after the g @ W GEMM.
G_SCALE = 1024.0
# Qwen2.5 vocabulary size (reference op.py:41).
VOCAB = 151936

_KEYS = ("lse", "target_logit", "ce", "entropy", "argmax")


def warmup(device=None, vocab=VOCAB):
    """Kept for the reference's API (op.py:44-61 compiles the Triton kernel ahead of time). The
    HIP kernels are compiled ahead of time, so this only loads libesep_body.so."""
    _hip.lib()


def _run(x16, w16, target, cew, n_live, need_grad, chunk_rows=CHUNK_ROWS):
    """Chunks over rows as given; rows [0, n_live) are the weighted ones (cew != 0); target is
    -1 and cew 0 on rows without a valid target. Returns (lse, tlogit, ent, amax, dx)."""
    n, h = x16.shape
    v = w16.shape[0]
    dev = x16.device
    lse = torch.empty(n, device=dev, dtype=torch.float32)
    ent = torch.empty(n, device=dev, dtype=torch.float32)
    tlogit = torch.empty(n, device=dev, dtype=torch.float32)
    amax = torch.empty(n, device=dev, dtype=torch.int32)
    dx = torch.zeros(n, h, device=dev, dtype=torch.float32) if need_grad else None
    nc = max(1, min(chunk_rows, n))
    z = torch.empty(nc, v, device=dev, dtype=w16.dtype)
    dxt = None
    wt = w16.t()
    for r0 in range(0, n, nc):
        nr = min(nc, n - r0)
        zc = z[:nr]
        torch.mm(x16[r0:r0 + nr], wt, out=zc)
        _hip.head_row_softmax(zc, target[r0:r0 + nr], cew[r0:r0 + nr], lse[r0:r0 + nr],
                              tlogit[r0:r0 + nr], ent[r0:r0 + nr], amax[r0:r0 + nr],
                              need_grad, G_SCALE)
        nl = min(max(n_live - r0, 0), nr)
        if need_grad and nl:
            scale = (cew[r0:r0 + nl] * (1.0 / G_SCALE))[:, None]
            if 2 * nl >= nc and nl < nc:
                # hipBLASLt runs this GEMM much faster at the chunk's row count than at a ragged
                # count of weighted rows (MI355X, K = 151936, N = 1536: M = 2925 2.06 ms,
                # M = 4096 1.67 ms), so it covers the whole chunk buffer and the rows past the
                # weighted ones (logits, or a previous chunk's rows) are computed and dropped
                if dxt is None:
                    dxt = torch.empty(nc, h, device=dev, dtype=torch.float32)
                torch.mm(z, w16, out_dtype=torch.float32, out=dxt)
                torch.mul(dxt[:nl], scale, out=dx[r0:r0 + nl])
            else:
                dxc = dx[r0:r0 + nl]
                torch.mm(zc[:nl], w16, out_dtype=torch.float32, out=dxc)
                dxc.mul_(scale)
    return lse, tlogit, ent, amax, dx


def _forward(x, w16, target, ce_weight, need_grad, chunk_rows):
    """Reference op.py:96-128."""
    v = w16.shape[0]
    valid = (target >= 0) & (target < v)
    cew = torch.where(valid, ce_weight.to(torch.float32), 0.0)
    target = torch.where(valid, target, -1)
    x16 = x.to(w16.dtype)
    perm = None
    n_live = 0
    if need_grad:
        live = cew != 0
        perm = torch.argsort((~live).to(torch.int8), stable=True)
        n_live = int(live.sum())  # one host sync per call
        x16, target_p, cew_p = x16[perm], target[perm], cew[perm]
    else:
        x16, target_p, cew_p = x16.contiguous(), target.contiguous(), cew.contiguous()
    lse, tlogit, ent, amax, dx = _run(x16, w16, target_p, cew_p, n_live, need_grad, chunk_rows)
    if perm is not None:
        inv = torch.empty_like(perm)
        inv[perm] = torch.arange(perm.numel(), device=perm.device)
        lse, tlogit, ent, amax, dx = lse[inv], tlogit[inv], ent[inv], amax[inv], dx[inv]
    tlogit = torch.where(valid, tlogit, 0.0)
    ce = torch.where(valid, lse - tlogit, 0.0)
    loss = (cew * ce).sum()
    return loss, (lse, tlogit, ce, ent, amax.long()), dx


class FusedLinearCE(torch.autograd.Function):
    """Loss differentiable w.r.t. x; dX precomputed in the forward (reference op.py:131-145)."""

    @staticmethod
    def forward(ctx, x, w16, target, ce_weight, chunk_rows):
        loss, stats, dx = _forward(x, w16, target, ce_weight, True, chunk_rows)
        ctx.save_for_backward(dx)
        ctx.x_dtype = x.dtype
        ctx.mark_non_differentiable(*stats)
        return (loss, *stats)

    @staticmethod
    def backward(ctx, grad_loss, *unused):
        (dx,) = ctx.saved_tensors
        return (dx * grad_loss).to(ctx.x_dtype), None, None, None, None


def fused_linear_ce(x, w16, target, ce_weight, need_grad=None, chunk_rows=CHUNK_ROWS):
    """loss = sum_i ce_weight_i * CE(x_i @ w16^T, target_i), plus per-row stats (reference
    op.py:151-175). need_grad=None: grad mode is on and x requires grad; without a gradient the
    g pass and the g @ W GEMM are skipped."""
    if not (x.dim() == 2 and w16.dim() == 2 and x.shape[1] == w16.shape[1]):
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, w16 {tuple(w16.shape)}")
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("x must be fp16, bf16 or fp32")
    if w16.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("w16 must be fp16 or bf16")
    if target.shape != (x.shape[0],) or ce_weight.shape != (x.shape[0],):
        raise ValueError("target and ce_weight must be [N]")
    if not (x.is_cuda and w16.is_cuda):
        raise ValueError("fused_linear_ce runs on the GPU (HIP tensors)")
    if need_grad is None:
        need_grad = torch.is_grad_enabled() and x.requires_grad
    w16 = w16.contiguous()
    target = target.to(torch.int64)
    if not x.shape[0]:
        z = torch.zeros(0, device=x.device, dtype=torch.float32)
        loss = x.float().sum() * 0.0 if need_grad else z.sum()
        return loss, dict(zip(_KEYS, (z, z, z, z, z.long())))
    if need_grad:
        loss, *stats = FusedLinearCE.apply(x, w16, target, ce_weight, chunk_rows)
    else:
        with torch.no_grad():
            loss, stats, _ = _forward(x, w16, target, ce_weight, False, chunk_rows)
    return loss, dict(zip(_KEYS, stats))
