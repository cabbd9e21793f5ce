"""Pins of the attention oracle (oracle/attention_ref.py) on the CPU.

* torch's scaled_dot_product_attention (math path, float64, CPU) per sequence with the kv heads
  repeated as HF's repeat_kv does, forward and autograd backward: the library routine the
  reference calls (packed.py:428-429);
* closed forms: a one-token sequence returns its v; q = 0 gives the running mean of v and
  lse = ln(count); a sequence never sees another sequence's tokens;
* central finite differences of sum(o * do) on a tiny case;
* mutation tests: a planted mistake (no causal mask, wrong kv-head order, scale left out of dK)
  must fail the checks above.
"""

import types

import numpy as np
import pytest
import torch

from oracle import attention_ref as ref


def _case(lengths, HQ, HK, D, seed=0):
    rng = np.random.default_rng(seed)
    T = int(sum(lengths))
    q = rng.standard_normal((T, HQ, D))
    k = rng.standard_normal((T, HK, D))
    v = rng.standard_normal((T, HK, D))
    return q, k, v, ref.cu_from_lengths(lengths)


def _torch_sdpa(q, k, v, cu, scale):
    """Per-sequence SDPA in float64 on the CPU; kv heads repeated (HF repeat_kv order)."""
    qt, kt, vt = (torch.tensor(t, dtype=torch.float64, requires_grad=True) for t in (q, k, v))
    HQ, HK = q.shape[1], k.shape[1]
    outs = []
    for i in range(len(cu) - 1):
        s0, s1 = int(cu[i]), int(cu[i + 1])
        qs = qt[s0:s1].transpose(0, 1)                                   # [HQ, n, D]
        ks = kt[s0:s1].transpose(0, 1).repeat_interleave(HQ // HK, 0)   # [HQ, n, D]
        vs = vt[s0:s1].transpose(0, 1).repeat_interleave(HQ // HK, 0)
        o = torch.nn.functional.scaled_dot_product_attention(qs, ks, vs, is_causal=True, scale=scale)
        outs.append(o.transpose(0, 1))
    return torch.cat(outs, 0), (qt, kt, vt)


def _check_vs_torch(fwd, bwd, lengths, HQ, HK, D, seed=0):
    q, k, v, cu = _case(lengths, HQ, HK, D, seed)
    scale = D ** -0.5
    o_t, leaves = _torch_sdpa(q, k, v, cu, scale)
    o, lse = fwd(q, k, v, cu, scale)
    np.testing.assert_allclose(o, o_t.detach().numpy(), atol=1e-12, rtol=1e-10)
    do = np.random.default_rng(seed + 1).standard_normal(o.shape)
    o_t.backward(torch.tensor(do))
    got = bwd(q, k, v, do, cu, scale)
    for g, leaf in zip(got, leaves):
        np.testing.assert_allclose(g, leaf.grad.numpy(), atol=1e-10, rtol=1e-9)
    return o, lse


@pytest.mark.parametrize("lengths,HQ,HK,D", [([5, 1, 7], 4, 2, 8), ([33, 2], 6, 3, 16),
                                            ([17], 2, 2, 4), ([9, 12, 3], 12, 2, 8)])
def test_matches_torch_sdpa(lengths, HQ, HK, D):
    _check_vs_torch(ref.attn_fwd, ref.attn_bwd, lengths, HQ, HK, D)


def test_closed_forms():
    lengths = [1, 6, 4]
    q, k, v, cu = _case(lengths, 4, 2, 8, seed=3)
    o, lse = ref.attn_fwd(q, k, v, cu, 0.3)
    # a one-token sequence returns its v (query head h reads kv head h // 2)
    np.testing.assert_allclose(o[0], np.stack([v[0, h // 2] for h in range(4)]), atol=1e-14)
    # q = 0: uniform weights over the visible keys -> running mean, lse = ln(count)
    z = np.zeros_like(q)
    o0, lse0 = ref.attn_fwd(z, k, v, cu, 0.3)
    for s0, s1 in zip(cu[:-1], cu[1:]):
        for t in range(s0, s1):
            for h in range(4):
                np.testing.assert_allclose(o0[t, h], v[s0:t + 1, h // 2].mean(0), atol=1e-14)
                assert abs(lse0[h, t] - np.log(t - s0 + 1)) < 1e-14
    # sequences are isolated: changing another sequence leaves this one's output bitwise equal
    k2 = k.copy()
    k2[cu[2]:] += 5.0
    o2, _ = ref.attn_fwd(q, k2, v, cu, 0.3)
    assert np.array_equal(o2[:cu[2]], o[:cu[2]])


def test_finite_differences():
    q, k, v, cu = _case([4, 3], 2, 1, 4, seed=5)
    scale = 0.7
    do = np.random.default_rng(9).standard_normal((7, 2, 4))
    dq, dk, dv = ref.attn_bwd(q, k, v, do, cu, scale)
    f = lambda q_, k_, v_: float((ref.attn_fwd(q_, k_, v_, cu, scale)[0] * do).sum())
    eps = 1e-6
    for x, g, which in ((q, dq, 0), (k, dk, 1), (v, dv, 2)):
        for idx in [(0, 0, 0), (3, 0, 2), (5, 0, 1), (6, x.shape[1] - 1, 3)]:
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[which], args_m[which] = xp, xm
            num = (f(*args_p) - f(*args_m)) / (2 * eps)
            assert abs(num - g[idx]) < 1e-7, (which, idx, num, g[idx])


def _planted_fwd(causal, kv_head):
    """The oracle's forward with the causal mask optional and a given query -> kv head map."""
    def fwd(q, k, v, cu, scale):
        q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
        T, HQ, D = q.shape
        HK = k.shape[1]
        o = np.zeros((T, HQ, D))
        for s0, s1 in ref._bounds(cu):
            n = s1 - s0
            for h in range(HQ):
                kh = kv_head(h, HQ, HK)
                sc = scale * q[s0:s1, h] @ k[s0:s1, kh].T
                if causal:
                    sc = np.where(np.tril(np.ones((n, n), dtype=bool)), sc, -np.inf)
                e = np.exp(sc - sc.max(1, keepdims=True))
                o[s0:s1, h] = e / e.sum(1, keepdims=True) @ v[s0:s1, kh]
        return o, None
    return fwd


def _mutant(name):
    """A copy of the oracle with one planted mistake."""
    m = types.SimpleNamespace(attn_fwd=ref.attn_fwd, attn_bwd=ref.attn_bwd)
    if name == "no_causal":
        m.attn_fwd = _planted_fwd(False, lambda h, HQ, HK: h // (HQ // HK))
    elif name == "kv_order":  # kv head h % HK instead of h // (HQ / HK)
        m.attn_fwd = _planted_fwd(True, lambda h, HQ, HK: h % HK)
    elif name == "dk_no_scale":
        def bwd(q, k, v, do, cu, scale):
            dq, dk, dv = ref.attn_bwd(q, k, v, do, cu, scale)
            return dq, dk / scale, dv
        m.attn_bwd = bwd
    return m


@pytest.mark.parametrize("name", ["no_causal", "kv_order", "dk_no_scale"])
def test_mutants_are_caught(name):
    m = _mutant(name)
    with pytest.raises(AssertionError):
        _check_vs_torch(m.attn_fwd, m.attn_bwd, [9, 12, 3], 4, 2, 8)
