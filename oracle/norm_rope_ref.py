"""CPU oracle of the decoder-body RMSNorm / RoPE path: a numpy restatement of the reference's
kernel math (gojosatorukz/esep-soup-kernels, solution/body/norm_rope.py and packed.py).

TEST INFRASTRUCTURE ONLY. Nothing in the product (the solution package, libesep_body.so)
imports or calls this module; only tests/, __graft_entry__.smoke() and bench.py's CPU
baseline leg use it, and only as the checker. Each function names the reference lines it
follows. Arithmetic runs in `acc` precision (np.float64 by default, np.float32 to mimic the
kernels' fp32 accumulation); 16-bit outputs are rounded to nearest even like the kernels'
stores.

How each function is pinned (tests/test_oracle_*.py):
  rmsnorm_fwd / add_rmsnorm_fwd  HF Qwen2RMSNorm golden vectors (tests/golden), the constant-row
                                 closed form, scale invariance, brute-force sums
  rmsnorm_bwd / add_rmsnorm_bwd  torch autograd of HF Qwen2RMSNorm (golden vectors), central
                                 finite differences, the sum(dr * xhat) = 0 identity, the
                                 dr_out pass-through and fan-in identities
  dgamma                         HF module weight gradient (golden), finite differences
  special_channels               the reference tests' designed weights (K = 0 / 8 / 3)
  rope_fwd                       HF apply_rotary_pos_emb + Qwen2RotaryEmbedding golden vectors,
                                 unit-vector known answers, pos = 0 identity, norm preservation,
                                 forward-then-backward identity
  default_inv_freq               HF Qwen2RotaryEmbedding.inv_freq (exact)
  positions_from_cu_seqlens      brute-force per-sequence aranges
  packed_positions               brute-force of the reference's idx % L / gather rule
"""

import numpy as np

# ----------------------------------------------------------------------------------------
# rounding helpers
# ----------------------------------------------------------------------------------------


def round_bf16(x):
    """fp32 -> bf16 -> fp32, round to nearest even (NaN kept quiet)."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    nan = np.isnan(a)
    out[nan] = np.nan
    return out


def round_to(x, dtype):
    """Round fp values to the storage dtype ('f32', 'f16', 'bf16'; 'f64' keeps them),
    returned as float64."""
    x = np.asarray(x)
    if dtype == "f64":
        return x.astype(np.float64)
    if dtype == "f32":
        return x.astype(np.float32).astype(np.float64)
    if dtype == "f16":
        return x.astype(np.float32).astype(np.float16).astype(np.float64)
    if dtype == "bf16":
        return round_bf16(x.astype(np.float32)).astype(np.float64)
    raise ValueError(dtype)


# ----------------------------------------------------------------------------------------
# K1: RMSNorm (+ residual add)
# ----------------------------------------------------------------------------------------


def add_rmsnorm_fwd(r_in, delta, w, eps, out_dtype="f32", acc=np.float64, slots=None,
                    r_dtype="f32"):
    """Forward of reference _add_rmsnorm_fwd (norm_rope.py:83-109) on rows [T, n]:
    r = r_in (+ delta), rounded to the residual dtype r_dtype; ms = sum(r^2)/n;
    inv = 1/sqrt(ms + eps); xhat = r * inv; y = w * xhat (rounded to out_dtype).
    Returns (r_out, y, rstd, xs) with xs[t, slots[j]] = xhat[t, j] for slots[j] >= 0."""
    r = np.asarray(r_in, dtype=acc)
    if delta is not None:
        # the residual add rounds once, to the residual's dtype (fp32 for the reference)
        r = round_to(r + np.asarray(delta, dtype=acc), r_dtype).astype(acc)
    n = r.shape[-1]
    ms = (r * r).sum(-1) / n
    inv = 1.0 / np.sqrt(ms + eps)
    xhat = r * inv[:, None]
    y = round_to(np.asarray(w, dtype=acc)[None, :] * xhat, out_dtype)
    xs = None
    if slots is not None:
        slots = np.asarray(slots)
        k = int((slots >= 0).sum())
        xs = np.zeros((r.shape[0], k), dtype=acc)
        for j in np.nonzero(slots >= 0)[0]:
            xs[:, slots[j]] = xhat[:, j]
    return r, y, inv, xs


def rmsnorm_fwd(x, w, eps, out_dtype="f32", acc=np.float64):
    """Plain RMSNorm (HF Qwen2RMSNorm.forward, modeling_qwen2.py:247-252, with one rounding at
    the end as the reference kernel does, norm_rope.py:103-105). Returns (y, rstd)."""
    _, y, inv, _ = add_rmsnorm_fwd(x, None, w, eps, out_dtype, acc)
    return y, inv


def add_rmsnorm_bwd(dys, dr_out, x, w, eps, rstd=None, from_y=False, slots=None, xs=None,
                    acc=np.float64):
    """Backward of reference _add_rmsnorm_bwd (norm_rope.py:116-162):
    dy = sum dys; xhat = x * rstd (x the residual) or y / w with exact channels from xs
    (from_y); g = dy * w; proj = sum(g * xhat) / n; dr = rstd * (g - xhat * proj) + dr_out.
    rstd None: recomputed from x (x the residual). Returns (dr, dw) with the weight gradient
    dw_j = sum_t dy_tj * xhat_tj (no reference counterpart: the reference freezes w)."""
    x = np.asarray(x, dtype=acc)
    n = x.shape[-1]
    w = np.asarray(w, dtype=acc)
    if not dys:
        dr = np.zeros_like(x) if dr_out is None else np.asarray(dr_out, dtype=acc).copy()
        return dr, np.zeros(n, dtype=acc)
    dy = np.zeros_like(x)
    for d in dys:
        dy = dy + np.asarray(d, dtype=acc)
    if rstd is None:
        assert not from_y
        rstd = 1.0 / np.sqrt((x * x).sum(-1) / n + eps)
    rstd = np.asarray(rstd, dtype=acc)
    if from_y:
        with np.errstate(divide="ignore", invalid="ignore"):
            xhat = x / w[None, :]
        if slots is not None:
            slots = np.asarray(slots)
            for j in np.nonzero(slots >= 0)[0]:
                xhat[:, j] = np.asarray(xs, dtype=acc)[:, slots[j]]
    else:
        xhat = x * rstd[:, None]
    g = dy * w[None, :]
    proj = (g * xhat).sum(-1) / n
    dr = rstd[:, None] * (g - xhat * proj[:, None])
    if dr_out is not None:
        dr = dr + np.asarray(dr_out, dtype=acc)
    dw = (dy * xhat).sum(0)
    return dr, dw


def rmsnorm_bwd(dy, x, w, eps, rstd=None, acc=np.float64):
    """Plain RMSNorm backward: (dx, dw) of y = w * x * rsqrt(mean(x^2) + eps)."""
    return add_rmsnorm_bwd([dy], None, x, w, eps, rstd=rstd, acc=acc)


def special_channels(w, special_w_min=2.0 ** -10):
    """Reference special_channels (norm_rope.py:183-205): slots[j] = 0..K-1 in ascending channel
    order where |w| < special_w_min, |w| > 65504 / sqrt(H) or w is not finite, else -1."""
    a = np.abs(np.asarray(w, dtype=np.float32))
    big = 65504.0 / float(a.shape[0]) ** 0.5
    with np.errstate(invalid="ignore"):
        special = (a < special_w_min) | (a > big) | ~np.isfinite(a)
    slots = np.full(a.shape, -1, dtype=np.int32)
    idx = np.nonzero(special)[0]
    slots[idx] = np.arange(idx.size, dtype=np.int32)
    return slots, int(idx.size)


# ----------------------------------------------------------------------------------------
# K2: rotary embedding
# ----------------------------------------------------------------------------------------


def default_inv_freq(head_dim=128, theta=1e6):
    """Reference default_inv_freq (norm_rope.py:423-426) = HF compute_default_rope_parameters:
    1 / theta ** (arange(0, D, 2) / D) in fp32 on the CPU. torch's CPU pow is what HF runs, so
    torch computes it here too (float32 numpy pow can differ in the last bit)."""
    import torch

    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    return inv.numpy()


def rope_angles(pos, inv_freq):
    """angle[t, j] = float32(pos[t]) * inv_freq[j], one fp32 multiply (norm_rope.py:361-363,
    the same product as HF's K=1 matmul in Qwen2RotaryEmbedding.forward)."""
    p = np.asarray(pos).astype(np.float32)
    return (p[:, None] * np.asarray(inv_freq, dtype=np.float32)[None, :]).astype(np.float32)


def rope_fwd(x, pos, inv_freq, sign=1.0, delta=None, store="f32", acc=np.float64):
    """Reference _rope_kernel / _rotate_heads (norm_rope.py:330-369) on x [T, H, D]:
    x (+ delta, added and rounded in the storage dtype), c = cos(angle), s = sign * sin(angle),
    out[:D/2] = x1 c - x2 s, out[D/2:] = x2 c + x1 s, rounded to the storage dtype."""
    x = np.asarray(x, dtype=np.float64)
    if delta is not None:
        x = round_to(x + np.asarray(delta, dtype=np.float64).reshape(x.shape), store)
    x = x.astype(acc)
    ang = rope_angles(pos, inv_freq).astype(np.float64)
    c = np.cos(ang).astype(acc)[:, None, :]
    s = (sign * np.sin(ang)).astype(acc)[:, None, :]
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    o = np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)
    return round_to(o, store)


def positions_from_cu_seqlens(cu_seqlens):
    """Packed positions restarting at every sequence: pos[t] = t - cu[i] for cu[i] <= t <
    cu[i+1] (the varlen counterpart of the reference's per-row arange, packed.py:808-814)."""
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    out = np.empty(int(cu[-1]), dtype=np.int64)
    for i in range(cu.size - 1):
        out[cu[i]:cu[i + 1]] = np.arange(cu[i + 1] - cu[i])
    return out


def packed_positions(mask, position_ids=None):
    """Reference packed_forward positions (packed.py:800-814): the real tokens of a [B, L]
    attention mask in row-major order; position = column index (HF's arange(L) per row, also
    for left padding) or position_ids gathered at those tokens."""
    mask = np.asarray(mask).astype(bool)
    B, L = mask.shape
    idx = np.nonzero(mask.reshape(-1))[0]
    if position_ids is None:
        return idx % L
    pid = np.broadcast_to(np.asarray(position_ids), (B, L)).reshape(-1)
    return pid[idx].astype(np.int64)
