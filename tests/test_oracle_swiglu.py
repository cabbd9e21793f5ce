"""Pins of the SwiGLU oracle (oracle/swiglu_ref.py): torch autograd of F.silu(g) * u in float64
on the CPU, central finite differences, closed-form special cases, and a planted mistake (the
derivative of sigmoid left out of dg) that the autograd check must catch."""

import numpy as np
import pytest
import torch

from oracle import swiglu_ref as ref


def _torch(g, u, dh):
    gt = torch.tensor(g, requires_grad=True)
    ut = torch.tensor(u, requires_grad=True)
    h = torch.nn.functional.silu(gt) * ut
    h.backward(torch.tensor(dh))
    return h.detach().numpy(), gt.grad.numpy(), ut.grad.numpy()


def _check(fwd, bwd, seed=0):
    rng = np.random.default_rng(seed)
    g, u, dh = (rng.standard_normal(1000) * 4 for _ in range(3))
    h_t, dg_t, du_t = _torch(g, u, dh)
    np.testing.assert_allclose(fwd(g, u), h_t, rtol=1e-13, atol=1e-13)
    dg, du = bwd(dh, g, u)
    np.testing.assert_allclose(dg, dg_t, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(du, du_t, rtol=1e-12, atol=1e-12)


def test_matches_torch_autograd():
    _check(ref.swiglu_fwd, ref.swiglu_bwd)


def test_finite_differences():
    rng = np.random.default_rng(3)
    g, u, dh = rng.standard_normal(16), rng.standard_normal(16), rng.standard_normal(16)
    dg, du = ref.swiglu_bwd(dh, g, u)
    eps = 1e-6
    num_g = ((ref.swiglu_fwd(g + eps, u) - ref.swiglu_fwd(g - eps, u)) / (2 * eps)) * dh
    num_u = ((ref.swiglu_fwd(g, u + eps) - ref.swiglu_fwd(g, u - eps)) / (2 * eps)) * dh
    np.testing.assert_allclose(dg, num_g, atol=1e-8)
    np.testing.assert_allclose(du, num_u, atol=1e-8)


def test_special_cases():
    u = np.array([1.5, -2.0, 3.0])
    assert np.all(ref.swiglu_fwd(np.zeros(3), u) == 0)               # silu(0) = 0
    dg, du = ref.swiglu_bwd(np.ones(3), np.zeros(3), u)
    np.testing.assert_allclose(dg, 0.5 * u)                           # silu'(0) = 1/2
    assert np.all(du == 0)
    big = np.array([40.0, -40.0])
    np.testing.assert_allclose(ref.swiglu_fwd(big, np.ones(2)), [40.0, 0.0], atol=1e-15)
    assert np.all(np.isfinite(ref.swiglu_fwd(np.array([1e4, -1e4]), np.ones(2))))


def test_planted_mistake_is_caught():
    def bad_bwd(dh, g, u):
        s = ref.sigmoid(g)
        return dh * u * s, dh * g * s  # d sigmoid / dg dropped

    with pytest.raises(AssertionError):
        _check(ref.swiglu_fwd, bad_bwd)
