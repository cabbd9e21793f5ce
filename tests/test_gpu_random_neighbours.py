"""Seeded random sizes for the path's neighbours (SwiGLU, the LoRA dropout, NF4 dequant, the LM
head's row kernel) against their CPU oracles at the bars of their fixed-size tests:

  swiglu     h, dg, du within one rounding (rtol 2^-8 bf16 / 2^-11 fp16 / 1e-6 fp32); in place
             the same bits
  dropout    the keep mask bit for bit (oracle Philox), kept values x / (1 - p) exactly, dropped 0;
             the backward regenerates the same bits
  nf4        bit-exact against the format's reference decoder
  head rows  lse, target logit, entropy, argmax and (optionally) g as test_gpu_head's checks

Each case's sizes come from numpy's default_rng(seed); ESEP_RANDOM_SHAPES_SCALE=k runs k times as
many seeds (1 by default)."""

import os

import numpy as np
import pytest
import torch

from _util import DEV, np64
from oracle import lora_ref
from oracle import nf4_ref
from oracle import swiglu_ref

pytestmark = pytest.mark.gpu

SCALE = max(1, int(os.environ.get("ESEP_RANDOM_SHAPES_SCALE", "1")))
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _seeds(first, count):
    return list(range(first, first + count)) + [first + 10000 + i for i in range(count * (SCALE - 1))]


def _size(rng, hi):
    """A size from 1 to hi, log-uniform, sometimes a multiple of 8 and sometimes one past it."""
    n = int(np.exp(rng.uniform(0, np.log(hi))))
    return max(1, [n, n - n % 8, n - n % 8 + 1][int(rng.integers(3))])


@pytest.mark.parametrize("seed", _seeds(600, 10))
def test_random_swiglu(seed):
    from solution.body import _hip

    rng = np.random.default_rng(seed)
    n = _size(rng, 3_000_000)
    dtype = DTYPES[int(rng.integers(3))]
    print(f"seed {seed}: n={n} {dtype}")
    g = torch.from_numpy(rng.standard_normal(n) * 3).float().to(dtype).to(DEV)
    u = torch.from_numpy(rng.standard_normal(n)).float().to(dtype).to(DEV)
    dh = torch.from_numpy(rng.standard_normal(n)).float().to(dtype).to(DEV)
    h = torch.full_like(g, float("nan"))
    _hip.swiglu_fwd(g, u, h)
    dg, du = torch.full_like(g, float("nan")), torch.full_like(g, float("nan"))
    _hip.swiglu_bwd(dh, g, u, dg, du)
    rt = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 1e-6}[dtype]
    np.testing.assert_allclose(np64(h), swiglu_ref.swiglu_fwd(np64(g), np64(u)), rtol=rt, atol=1e-6)
    dg64, du64 = swiglu_ref.swiglu_bwd(np64(dh), np64(g), np64(u))
    np.testing.assert_allclose(np64(dg), dg64, rtol=rt, atol=1e-6)
    np.testing.assert_allclose(np64(du), du64, rtol=rt, atol=1e-6)
    g2, u2 = g.clone(), u.clone()
    _hip.swiglu_bwd(dh, g2, u2, g2, u2)
    assert torch.equal(g2, dg) and torch.equal(u2, du)


@pytest.mark.parametrize("seed", _seeds(700, 10))
def test_random_lora_dropout(seed):
    from solution.body import _hip

    rng = np.random.default_rng(seed)
    n = _size(rng, 3_000_000)
    dtype = DTYPES[int(rng.integers(3))]
    p = float(np.float32(rng.uniform(0.01, 0.9)))
    key_v = int(rng.integers(-(1 << 62), 1 << 62))
    print(f"seed {seed}: n={n} {dtype} p={p} key={key_v}")
    key = torch.tensor([key_v], dtype=torch.int64, device=DEV)
    x = torch.from_numpy(rng.standard_normal(n)).float().to(dtype).to(DEV)
    xd = torch.full_like(x, float("nan"))
    _hip.lora_dropout_fwd(x, key, xd, p)
    keep = torch.from_numpy(lora_ref.dropout_mask(key_v, n, p)).to(DEV)
    inv = float(np.float32(1.0) / (np.float32(1.0) - np.float32(p)))
    want = torch.where(keep, (x.float() * inv).to(dtype), torch.zeros_like(x))
    assert torch.equal(xd, want)
    g = torch.from_numpy(rng.standard_normal(n)).float().to(dtype).to(DEV)
    xd2, dx = torch.empty_like(x), torch.empty_like(x)
    _hip.lora_dropout_bwd(x, g, key, xd2, dx, p)
    assert torch.equal(xd2, xd)
    assert torch.equal(dx, torch.where(keep, (g.float() * inv).to(dtype), torch.zeros_like(g)))


@pytest.mark.parametrize("seed", _seeds(800, 10))
def test_random_nf4_dequant(seed):
    from solution.body import _hip

    rng = np.random.default_rng(seed)
    n, k = _size(rng, 9000), 64 * _size(rng, 140)
    dtype = DTYPES[int(rng.integers(3))]
    print(f"seed {seed}: [{n}, {k}] {dtype}")
    nb = n * k // 64
    packed = rng.integers(0, 256, nb * 32, dtype=np.uint8)
    absmax = rng.integers(0, 256, nb, dtype=np.uint8)
    absmax2 = (rng.random((nb + 255) // 256) * 0.1 + 0.01).astype(np.float32)
    code2 = np.sort(rng.standard_normal(256)).astype(np.float32)
    offset = np.float32(rng.random() * 0.05)

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)

    out = torch.full((n, k), float("nan"), device=DEV, dtype=dtype)
    _hip.nf4_dequant(dev(packed), dev(absmax), dev(absmax2), dev(code2),
                     dev(np.array([offset], dtype=np.float32)), dev(nf4_ref.NF4), out)
    want32 = nf4_ref.dequantize_nf4(packed, absmax, absmax2, code2, offset, out_dtype=np.float32)
    assert torch.equal(out.cpu(), torch.from_numpy(want32.reshape(n, k)).to(dtype))


@pytest.mark.parametrize("seed", _seeds(900, 10))
def test_random_head_rows(seed):
    from solution.body import _hip
    from test_gpu_head import _check_row_kernel, _chunk, _outs

    rng = np.random.default_rng(seed)
    V = _size(rng, 160_000)
    rows = int(rng.integers(1, max(2, min(64, 2_000_000 // V))))
    dtype = [torch.float16, torch.bfloat16][int(rng.integers(2))]
    write_g = bool(rng.integers(2))
    print(f"seed {seed}: rows={rows} V={V} {dtype} write_g={write_g}")
    z, target, cew = _chunk(rows, V, dtype, seed=seed)
    zd = z.to(DEV)
    outs = _outs(rows)
    _hip.head_row_softmax(zd, target.to(DEV), cew.to(DEV), *outs, write_g, 1024.0)
    _check_row_kernel(zd, z, target, cew, write_g, dtype, outs)
