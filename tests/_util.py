"""Shared helpers of the test suite (seeded inputs, comparisons)."""

import numpy as np
import torch

DEV = "cuda"


def gen(seed):
    return torch.Generator().manual_seed(seed)


def randn(shape, g, scale=1.0, dtype=torch.float32, dev=DEV):
    """N(0, scale^2) drawn on the CPU generator (so CPU and GPU see the same values)."""
    return (torch.randn(shape, generator=g) * scale).to(dtype).to(dev)


def np64(t):
    return t.detach().to("cpu", torch.float64).numpy()


def err(a, b):
    """(max abs error, max abs error relative to max |b|), as the reference's tests' _err."""
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    ae = float(np.abs(a - b).max()) if a.size else 0.0
    return ae, ae / max(float(np.abs(b).max()) if b.size else 0.0, 1e-30)


def assert_close(a, b, atol, rtol, what=""):
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    bad = np.abs(a - b) > atol + rtol * np.abs(b)
    if bad.any():
        i = np.unravel_index(np.argmax(np.abs(a - b) - rtol * np.abs(b)), a.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {a.size} outside atol={atol} "
                             f"rtol={rtol}; worst at {i}: got {a[i]!r} want {b[i]!r}")


STORE = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}
