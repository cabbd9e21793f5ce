"""Pins of the fused LM head oracle (oracle/head_ref.py) on the CPU.

* torch in float64 as the independent routine: lse = logsumexp, entropy from log_softmax, and
  dX = autograd of sum_i cew_i * cross_entropy(x_i @ W^T, target_i) (ignored rows: weight 0).
* Closed forms: a constant row (lse = c + log V, entropy = log V, argmax 0, g = 1/V - onehot) and a
  row with one dominant logit (entropy and lse in closed form).
* argmax is the first maximal index (ties built by hand), and target logit / CE are 0 for targets
  outside [0, V) (-100 and V).
* Rows with zero CE weight keep their logits when g is written.
* Planted mistakes (onehot dropped, last-index argmax) fail these checks.
"""

import math

import numpy as np
import pytest
import torch

from oracle import head_ref as ref


def _case(n=37, h=24, V=301, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, h))
    w = rng.standard_normal((V, h)) * 0.5
    target = rng.integers(0, V, n)
    target[::5] = -100
    target[3] = V  # out of range counts as ignored
    cew = rng.random(n)
    cew[2::7] = 0.0
    return x, w, target, cew


def _torch_ref(x, w, target, cew):
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64)
    t = torch.tensor(target)
    V = w.shape[0]
    ok = (t >= 0) & (t < V)
    z = xt @ wt.T
    logp = torch.log_softmax(z, dim=-1)
    nll = -logp.gather(1, torch.where(ok, t, 0)[:, None])[:, 0]
    c = torch.where(ok, torch.tensor(cew, dtype=torch.float64), 0.0)
    loss = (c * nll).sum()
    (dx,) = torch.autograd.grad(loss, xt)
    with torch.no_grad():
        return dict(z=z.numpy(), loss=loss.item(), dx=dx.numpy(),
                    lse=torch.logsumexp(z, -1).numpy(),
                    ent=(-(logp.exp() * logp).sum(-1)).numpy(),
                    ce=torch.where(ok, nll, 0.0).numpy())


def test_linear_ce_matches_torch_autograd():
    x, w, target, cew = _case()
    want = _torch_ref(x, w, target, cew)
    loss, st, dx = ref.linear_ce(want["z"], w, target, cew)
    np.testing.assert_allclose(loss, want["loss"], rtol=1e-12)
    np.testing.assert_allclose(dx, want["dx"], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(st["lse"], want["lse"], rtol=1e-12)
    np.testing.assert_allclose(st["entropy"], want["ent"], rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(st["ce"], want["ce"], rtol=1e-10, atol=1e-12)
    ign = (target < 0) | (target >= w.shape[0])
    assert np.all(st["target_logit"][ign] == 0) and np.all(st["ce"][ign] == 0)
    assert np.all(dx[ign | (cew == 0)] == 0)
    assert np.array_equal(st["argmax"], want["z"].argmax(axis=1))


def test_closed_forms():
    V = 1000
    z = np.full((1, V), 3.25)
    lse, tl, ent, amax, g = ref.row_softmax(z, [17], cew=[1.0], write_g=True, g_dtype=np.float64)
    assert math.isclose(lse[0], 3.25 + math.log(V), rel_tol=1e-14)
    assert math.isclose(ent[0], math.log(V), rel_tol=1e-12)
    assert amax[0] == 0 and tl[0] == 3.25
    want = np.full(V, 1024.0 / V)
    want[17] -= 1024.0
    np.testing.assert_allclose(g[0], want, rtol=1e-12)
    L, k = 20.0, 123
    z = np.zeros((1, V))
    z[0, k] = L
    lse, tl, ent, amax, _ = ref.row_softmax(z, [-100])
    S = math.exp(L) + V - 1
    pk = math.exp(L) / S
    assert math.isclose(lse[0], math.log(S), rel_tol=1e-14)
    assert math.isclose(ent[0], -pk * math.log(pk) + (V - 1) / S * math.log(S), rel_tol=1e-10)
    assert amax[0] == k and tl[0] == 0.0


def test_first_index_ties_and_unweighted_rows_kept():
    z = np.array([[0.0, 1.0, 5.0, 2.0, 5.0, 5.0], [7.0, 7.0, 7.0, 7.0, 7.0, 7.0]])
    _, _, _, amax, out = ref.row_softmax(z, [1, 2], cew=[0.0, 2.0], write_g=True)
    assert list(amax) == [2, 0]
    assert np.array_equal(out[0], z[0].astype(np.float16))  # weight 0: logits kept
    assert out.dtype == np.float16 and np.all(out[1, [0, 1, 3, 4, 5]] == np.float16(1024 / 6))
    assert out[1, 2] == np.float16(1024 / 6 - 1024)


def test_planted_mistakes_are_caught():
    x, w, target, cew = _case(seed=1)
    want = _torch_ref(x, w, target, cew)

    def no_onehot(z, w, target, cew):
        z = np.asarray(z, dtype=np.float64)
        ok = (target >= 0) & (target < w.shape[0])
        c = np.where(ok, cew, 0.0)
        p = np.exp(z - ref.row_softmax(z, target)[0][:, None])
        return (c[:, None] * p) @ w

    with pytest.raises(AssertionError):
        np.testing.assert_allclose(no_onehot(want["z"], w, target, cew), want["dx"], rtol=1e-6)
    z = np.array([[1.0, 9.0, 9.0]])
    last = z.shape[1] - 1 - z[:, ::-1].argmax(axis=1)
    with pytest.raises(AssertionError):
        assert np.array_equal(last, ref.row_softmax(z, [0])[3])
