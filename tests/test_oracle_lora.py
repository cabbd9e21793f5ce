"""Pins of the LoRA-dropout oracle (oracle/lora_ref.py) on the CPU.

* Philox4x32-10 against the known-answer vectors published with the generator (Salmon et al.,
  SC 2011; the Random123 distribution's kat_vectors): all-zero counter and key, all-ones counter
  and key, and the pi-digits counter / key.
* The mask: keep rate within 5 standard deviations of 1 - p, independent of position (first and
  second halves), different keys give different masks, and the mask is a pure function of
  (key, element).
* The LoRA math against torch autograd in float64 (base + scaling * (x_d A^T) B^T), and a
  planted mistake (the dropout scale left out of dx) that the check must catch.
"""

import numpy as np
import pytest
import torch

from oracle import lora_ref as ref

KAT = [  # (counter words, key words, output words), philox4x32 with 10 rounds
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    got = ref.philox4x32_10(np.array(ctr, dtype=np.uint32), np.array(key, dtype=np.uint32))
    assert tuple(int(w) for w in got) == want


def test_mask_statistics():
    n, p = 1 << 20, 0.05
    keep = ref.dropout_mask(12345, n, p)
    sd = np.sqrt(n * p * (1 - p))
    assert abs((~keep).sum() - n * p) < 5 * sd
    for half in (keep[: n // 2], keep[n // 2:]):
        assert abs((~half).sum() - n / 2 * p) < 5 * np.sqrt(n / 2 * p * (1 - p))
    other = ref.dropout_mask(12346, n, p)
    assert (keep != other).sum() > 0.05 * n  # a different key is a different mask
    assert np.array_equal(ref.dropout_mask(12345, 1000, p), keep[:1000])  # pure in (key, e)
    u = ref.uniforms(7, 4096)
    assert u.min() >= 0.0 and u.max() < 1.0


def _check(fwd, bwd, seed=0):
    rng = np.random.default_rng(seed)
    T, IN, R, N, p, s = 9, 12, 4, 7, 0.2, 2.0
    x, base = rng.standard_normal((T, IN)), rng.standard_normal((T, N))
    a, b, dout = rng.standard_normal((R, IN)), rng.standard_normal((N, R)), rng.standard_normal((T, N))
    keep = rng.random((T, IN)) >= p
    xt, bt, at, btt = (torch.tensor(v, requires_grad=True) for v in (x, base, a, b))
    out = bt + s * ((xt * torch.tensor(keep) / (1 - p)) @ at.T) @ btt.T
    out.backward(torch.tensor(dout))
    np.testing.assert_allclose(fwd(x, base, a, b, keep, p, s), out.detach().numpy(), atol=1e-12)
    for g, leaf in zip(bwd(x, a, b, dout, keep, p, s), (xt, bt, at, btt)):
        np.testing.assert_allclose(g, leaf.grad.numpy(), atol=1e-12)


def test_lora_math_matches_torch():
    _check(ref.lora_fwd, ref.lora_bwd)


def test_planted_mistake_is_caught():
    def bad_bwd(x, a, b, dout, keep, p, s):
        dx, db_, da, db = ref.lora_bwd(x, a, b, dout, keep, p, s)
        return dx * (1 - p), db_, da, db  # dropout scale left out of dx

    with pytest.raises(AssertionError):
        _check(ref.lora_fwd, bad_bwd)
