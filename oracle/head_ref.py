"""CPU oracle for the fused LM head (test infrastructure only: imported by tests/, never by the
product path).

Restates, in float64 numpy, what the reference computes:

* row_softmax: the row kernel (solution/head/kernels.py:38-93, head_row_softmax_kernel) on a
  logits chunk z [rows, V] given as the float values of its fp16 / bf16 elements:
    lse    = log sum_v exp(z_v)
    ent    = -sum_v p_v log p_v                      (p = softmax(z))
    amax   = first v with z_v = max z                (kernels.py:48-50, 72: strict '>' per lane,
                                                      ties to the smallest index)
    tlogit = z[target] if 0 <= target < V else 0     (kernels.py:62, op.py:125)
    g      = (p - onehot(target)) * g_scale          (kernels.py:80-93), written only on rows
                                                      with cew != 0; other rows keep z
  The kernel's one-pass form (running max, S = sum exp(z - M), T = sum exp(z - M)(z - M),
  entropy = log S - T / S) is algebraically the same; here everything is evaluated two-pass in
  float64, so the oracle carries no summation-order error of its own.

* linear_ce: the op (solution/head/op.py:88-128, 151-175) for given logits
  z = fp16(x16 @ w16^T):  rows with a target outside [0, V) get weight 0 and target -1;
    loss = sum_i cew_i (lse_i - z_i[target_i]),   ce_i = lse_i - tlogit_i (0 for ignored rows)
    dX_i = cew_i * (p_i - onehot_i) @ W           (op.py:90-91: g @ W, then * cew / G_SCALE)
  dX is returned unrounded (float64) so a test can state its own tolerance.

Pinned in tests/test_oracle_head.py against torch.log_softmax / autograd in float64, closed
forms (uniform rows, a single dominant logit) and hand-made ties.
"""

import numpy as np

G_SCALE = 1024.0  # solution/head/op.py:37


def _valid_target(target, V):
    t = np.asarray(target, dtype=np.int64)
    ok = (t >= 0) & (t < V)
    return ok, np.where(ok, t, 0)


def row_softmax(z, target, cew=None, write_g=False, g_scale=G_SCALE, g_dtype=np.float16):
    """(lse, tlogit, ent, amax, zout) for a chunk z [rows, V]. zout is z in g_dtype with the
    weighted rows replaced by g when write_g (unweighted rows are z, unchanged)."""
    z = np.asarray(z, dtype=np.float64)
    rows, V = z.shape
    ok, safe = _valid_target(target, V)
    m = z.max(axis=1, keepdims=True)
    e = np.exp(z - m)
    s = e.sum(axis=1, keepdims=True)
    lse = (m + np.log(s))[:, 0]
    logp = z - lse[:, None]
    p = np.exp(logp)
    ent = -(p * logp).sum(axis=1)
    amax = z.argmax(axis=1).astype(np.int64)  # numpy returns the first maximal index
    tlogit = np.where(ok, z[np.arange(rows), safe], 0.0)
    zout = z.astype(g_dtype)
    if write_g:
        cew = np.asarray(cew, dtype=np.float32)
        g = p.copy()
        r = np.nonzero(ok)[0]
        g[r, safe[r]] -= 1.0
        g *= g_scale
        live = cew != 0
        zout[live] = g[live].astype(g_dtype)
    return lse, tlogit, ent, amax, zout


def linear_ce(z, w, target, ce_weight):
    """(loss, stats, dx) of fused_linear_ce for logits z [N, V] (the values the op's GEMM gives),
    weight w [V, H]; stats = dict(lse, target_logit, ce, entropy, argmax)."""
    z = np.asarray(z, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    n, V = z.shape
    ok, safe = _valid_target(target, V)
    cew = np.where(ok, np.asarray(ce_weight, dtype=np.float64), 0.0)
    lse, tlogit, ent, amax, _ = row_softmax(z, np.where(ok, target, -1))
    ce = np.where(ok, lse - tlogit, 0.0)
    loss = float((cew * ce).sum())
    p = np.exp(z - lse[:, None])
    r = np.nonzero(ok)[0]
    p[r, safe[r]] -= 1.0
    dx = (cew[:, None] * p) @ w
    stats = dict(lse=lse, target_logit=tlogit, ce=ce, entropy=ent, argmax=amax)
    return loss, stats, dx
