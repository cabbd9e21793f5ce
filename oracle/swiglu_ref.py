"""CPU oracle for SwiGLU (test infrastructure only: imported by tests/, never by the product
path). Restates the reference's example kernels, solution/swiglu.py:15-37:
    s = sigmoid(g),  h = g * s * u,  du = dh * g * s,  dg = dh * u * s * (1 + g * (1 - s))
in float64 numpy. Pinned in tests/test_oracle_swiglu.py against torch autograd of
F.silu(g) * u (float64, CPU), finite differences and closed-form special cases.
"""

import numpy as np


def sigmoid(g):
    g = np.asarray(g, dtype=np.float64)
    return 0.5 * (1.0 + np.tanh(0.5 * g))  # overflow-free form of 1 / (1 + exp(-g))


def swiglu_fwd(g, u):
    g = np.asarray(g, dtype=np.float64)
    return g * sigmoid(g) * np.asarray(u, dtype=np.float64)


def swiglu_bwd(dh, g, u):
    """(dg, du) of h = silu(g) * u for upstream gradient dh."""
    dh, g, u = (np.asarray(t, dtype=np.float64) for t in (dh, g, u))
    s = sigmoid(g)
    return dh * u * s * (1.0 + g * (1.0 - s)), dh * g * s
