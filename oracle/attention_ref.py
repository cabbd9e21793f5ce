"""CPU oracle for the varlen causal attention (test infrastructure only: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product path).

Restates the reference decoder's attention, solution/body/packed.py:404-436 (_attention): per
original row (a sequence of the packed tokens), causal softmax attention with
scale = attn.scaling, query head h reading kv head h // (HQ // HK) (HF repeat_kv order,
packed.py:425-427), dropout 0. The backward is the closed form of that function's gradient,
as torch's scaled_dot_product_attention backward computes it:
    P = softmax(scale * Q K^T + causal mask),  O = P V
    dV = P^T dO,  dP = dO V^T,  dS = P * (dP - rowsum(dO * O)),  dQ = scale * dS K,
    dK = scale * dS^T Q     (dK, dV of a kv head summed over the query heads that read it)
Everything in float64 numpy. Pinned in tests/test_oracle_attention.py against torch's SDPA
(math path, float64, CPU), closed forms and finite differences.
"""

import numpy as np


def _bounds(cu):
    cu = np.asarray(cu, dtype=np.int64)
    return [(int(cu[i]), int(cu[i + 1])) for i in range(len(cu) - 1)]


def attn_fwd(q, k, v, cu, scale):
    """q [T, HQ, D], k, v [T, HK, D] (any float) -> (o [T, HQ, D], lse [HQ, T]) in float64.
    Tokens outside every sequence keep o = 0, lse = -inf."""
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    T, HQ, D = q.shape
    HK = k.shape[1]
    G = HQ // HK
    o = np.zeros((T, HQ, D))
    lse = np.full((HQ, T), -np.inf)
    for s0, s1 in _bounds(cu):
        n = s1 - s0
        if n <= 0:
            continue
        mask = np.tril(np.ones((n, n), dtype=bool))
        for h in range(HQ):
            kh = h // G
            sc = scale * q[s0:s1, h] @ k[s0:s1, kh].T
            sc = np.where(mask, sc, -np.inf)
            mx = sc.max(axis=1, keepdims=True)
            e = np.exp(sc - mx)
            den = e.sum(axis=1, keepdims=True)
            o[s0:s1, h] = (e / den) @ v[s0:s1, kh]
            lse[h, s0:s1] = (mx + np.log(den))[:, 0]
    return o, lse


def attn_bwd(q, k, v, do, cu, scale):
    """Gradients of sum(o * do) for o = attn_fwd(q, k, v, cu, scale)[0]: (dq, dk, dv) float64."""
    q, k, v, do = (np.asarray(t, dtype=np.float64) for t in (q, k, v, do))
    T, HQ, D = q.shape
    HK = k.shape[1]
    G = HQ // HK
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    for s0, s1 in _bounds(cu):
        n = s1 - s0
        if n <= 0:
            continue
        mask = np.tril(np.ones((n, n), dtype=bool))
        for h in range(HQ):
            kh = h // G
            qs, ks, vs, dos = q[s0:s1, h], k[s0:s1, kh], v[s0:s1, kh], do[s0:s1, h]
            sc = np.where(mask, scale * qs @ ks.T, -np.inf)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            os_ = p @ vs
            dv[s0:s1, kh] += p.T @ dos
            dp = dos @ vs.T
            ds = p * (dp - (dos * os_).sum(axis=1, keepdims=True))
            dq[s0:s1, h] = scale * ds @ ks
            dk[s0:s1, kh] += scale * ds.T @ qs
    return dq, dk, dv


def cu_from_lengths(lengths):
    return np.concatenate([[0], np.cumsum(np.asarray(lengths, dtype=np.int64))]).astype(np.int32)
