"""The LoRA path (solution/body/lora.py) on the GPU, restating the reference's
solution/test_body_lora.py (:66-254) where peft is not needed, plus bit-level parity of the
dropout mask with the oracle.

* The HIP dropout mask equals oracle.lora_ref.dropout_mask(key, n, p) bit for bit (integer
  work: bit-exact), kept values are x / (1 - p) rounded once, the backward regenerates the
  forward's xd bit for bit, and dx = [dx +] g * keep / (1 - p).
* LoRAFunction / LoRADeltaFunction against an fp32 torch reference with the same mask (relative
  error of the largest magnitude < 1e-2, as the reference's _check), dtypes of the outputs and
  weight gradients, a fresh key per forward call, keys following torch.manual_seed, and the
  keep rate.
"""

import numpy as np
import pytest
import torch

from _util import DEV, gen, np64
from oracle import lora_ref as ref

pytestmark = pytest.mark.gpu

IN, R, SCALING, P = 1536, 16, 2.0, 0.05


def _key(v):
    return torch.tensor([v], dtype=torch.int64, device=DEV)


def _mask64(key, n, p):
    return ref.dropout_mask(key, n, float(np.float32(p)))  # the kernel compares in fp32


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("n", [1, 7, 8, 1000, (1 << 20) + 3])
def test_mask_matches_oracle_and_backward_regenerates(n, dtype):
    from solution.body import _hip

    key_v, p = 0x1234_5678_9ABC_DEF, 0.3
    key = _key(key_v)
    g_ = gen(n)
    x = torch.randn(n, generator=g_).to(dtype).to(DEV)
    xd = torch.full_like(x, float("nan"))
    _hip.lora_dropout_fwd(x, key, xd, p)
    keep = _mask64(key_v, n, p)
    got_keep = (np64(xd) != 0) | (np64(x) == 0)
    assert np.array_equal(got_keep | (np64(x) == 0), keep | (np64(x) == 0))
    inv = np.float32(1.0) / (np.float32(1.0) - np.float32(p))
    want = (x.float() * float(inv)).to(dtype)
    assert torch.equal(xd[torch.from_numpy(keep).to(DEV)], want[torch.from_numpy(keep).to(DEV)])
    assert torch.all(xd[torch.from_numpy(~keep).to(DEV)] == 0)
    # backward: same mask (xd regenerated bit for bit), dx = g * keep / (1 - p), accumulate
    g = torch.randn(n, generator=g_).to(dtype).to(DEV)
    xd2, dx = torch.empty_like(x), torch.empty_like(x)
    _hip.lora_dropout_bwd(x, g, key, xd2, dx, p)
    assert torch.equal(xd2, xd)
    km = torch.from_numpy(keep).to(DEV)
    assert torch.equal(dx, torch.where(km, (g.float() * float(inv)).to(dtype), torch.zeros_like(g)))
    acc = torch.randn(n, generator=g_).to(dtype).to(DEV)
    dx2 = acc.clone()
    _hip.lora_dropout_bwd(x, g, key, xd2, dx2, p, accumulate=True)
    want_acc = (acc.float() + torch.where(km, g.float() * float(inv), torch.zeros_like(g.float()))).to(dtype)
    assert torch.equal(dx2, want_acc)
    g2 = g.clone()  # dx may be g itself
    _hip.lora_dropout_bwd(x, g2, key, xd2, g2, p)
    assert torch.equal(g2, dx)


def test_dropout_distribution_and_scaling():
    from solution.body import lora as L

    x = torch.ones(1 << 22, device=DEV, dtype=torch.float16)
    xd = L.lora_dropout(x, L.new_dropout_key(DEV), P)
    dropped = (xd == 0).float().mean().item()
    sd = (P * (1 - P) / x.numel()) ** 0.5
    assert abs(dropped - P) < 6 * sd, dropped
    assert torch.all(xd[xd != 0] == torch.tensor(1 / (1 - P), dtype=torch.float16, device=DEV))


def _inputs(T, N, dtype, seed=0):
    g = gen(seed)
    x = torch.randn(T, IN, generator=g).to(dtype).to(DEV)
    base = torch.randn(T, N, generator=g).to(dtype).to(DEV)
    a = (torch.randn(R, IN, generator=g) * 0.02).to(DEV)
    b = (torch.randn(N, R, generator=g) * 0.02).to(DEV)
    dout = torch.randn(T, N, generator=g).to(dtype).to(DEV)
    return x, base, a, b, dout


def _reference(x, base, a, b, dout, keep=None, p=0.0, delta=False):
    """fp32 torch reference (reference test_body_lora.py:47-57); keep: bool mask or None."""
    xr = x.float().requires_grad_(True)
    br = base.float().requires_grad_(True)
    ar, bb = a.clone().requires_grad_(True), b.clone().requires_grad_(True)
    xd = xr * keep / (1.0 - p) if keep is not None else xr
    term = SCALING * (xd @ ar.t()) @ bb.t()
    out = term if delta else br + term
    out.backward(dout.float())
    return out, xr.grad, br.grad, ar.grad, bb.grad


def _check(got, want, tol=1e-2):
    d = (got.float() - want.float()).abs().max().item()
    assert d / max(want.float().abs().max().item(), 1e-12) < tol, d


def _capture_keys(monkeypatch):
    from solution.body import lora as L

    keys, orig = [], L.new_dropout_key

    def rec(device):
        k = orig(device)
        keys.append(int(k.item()))
        return k

    monkeypatch.setattr(L, "new_dropout_key", rec)
    return keys


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("p", [0.0, P])
@pytest.mark.parametrize("T,N", [(1, 1536), (37, 256), (1000, 1536)])
def test_lora_function_vs_reference(T, N, p, dtype, monkeypatch):
    from solution.body import lora as L

    keys = _capture_keys(monkeypatch)
    x, base, a, b, dout = _inputs(T, N, dtype, seed=T + N)
    xo, bo = x.clone().requires_grad_(True), base.clone().requires_grad_(True)
    ao, bbo = a.clone().requires_grad_(True), b.clone().requires_grad_(True)
    out = L.LoRAFunction.apply(xo, bo * 1, ao, bbo, p, SCALING)  # bo * 1: a fresh non-leaf
    out.backward(dout)
    keep = None
    if p > 0:
        assert len(keys) == 1
        keep = torch.from_numpy(_mask64(keys[0], T * IN, p).reshape(T, IN)).to(DEV)
    r_out, r_dx, r_dbase, r_da, r_db = _reference(x, base, a, b, dout, keep, p)
    assert out.dtype == dtype and xo.grad.dtype == dtype
    assert ao.grad.dtype == torch.float32 and bbo.grad.dtype == torch.float32
    _check(out, r_out)
    _check(xo.grad, r_dx)
    _check(bo.grad, r_dbase, tol=1e-6)
    _check(ao.grad, r_da)
    _check(bbo.grad, r_db)
    # the delta form (q_proj): the same term alone
    xo2, ao2, bbo2 = (t.clone().requires_grad_(True) for t in (x, a, b))
    keys.clear()
    delta = L.LoRADeltaFunction.apply(xo2, ao2, bbo2, p, SCALING)
    delta.backward(dout)
    keep2 = None
    if p > 0:
        keep2 = torch.from_numpy(_mask64(keys[0], T * IN, p).reshape(T, IN)).to(DEV)
    d_out, d_dx, _, d_da, d_db = _reference(x, base, a, b, dout, keep2, p, delta=True)
    _check(delta, d_out)
    _check(xo2.grad, d_dx)
    _check(ao2.grad, d_da)
    _check(bbo2.grad, d_db)


def test_fresh_mask_per_call_and_seeded_keys(monkeypatch):
    from solution.body import lora as L

    keys = _capture_keys(monkeypatch)
    x, base, a, b, _ = _inputs(64, 256, torch.float16)
    o1 = L.LoRAFunction.apply(x, base.clone(), a, b, P, SCALING)
    o2 = L.LoRAFunction.apply(x, base.clone(), a, b, P, SCALING)
    assert len(keys) == 2 and keys[0] != keys[1] and not torch.equal(o1, o2)
    torch.manual_seed(7)
    k1 = L.new_dropout_key(DEV).item()
    torch.manual_seed(7)
    k2 = L.new_dropout_key(DEV).item()
    assert k1 == k2


def test_dx_accumulate_into_buffer():
    """lora_down_bwd adds the LoRA part of dx into a given buffer (reference :159-175)."""
    from solution.body import lora as L

    T = 100
    x, _, a, _, _ = _inputs(T, 256, torch.float16, seed=3)
    a16 = a.to(torch.float16)
    dxa = torch.randn(T, R, generator=gen(4)).to(torch.float16).to(DEV)
    key = L.new_dropout_key(DEV)
    plain, da1 = L.lora_down_bwd(x, a16, dxa, key, P)
    acc = torch.randn(T, IN, generator=gen(5)).to(torch.float16).to(DEV)
    summed, da2 = L.lora_down_bwd(x, a16, dxa, key, P, dx_accum=acc.clone())
    assert torch.equal(da1, da2)
    _check(summed, acc.float() + plain.float(), tol=2e-3)


def test_dropout_bench_shape():
    """The bench's dropout workload (config 4's q_proj LoRA input, 8192 x 1536 bf16, p = 0.05:
    several grid-strided passes per thread): the whole mask bit for bit against the oracle, and
    the backward's regenerated x_d equal to the forward's."""
    from solution.body import _hip

    key_v, p = 0x0BAD_5EED_1234_5678, 0.05
    key = _key(key_v)
    n = 8192 * 1536
    x = torch.randn(n, generator=gen(1536)).to(torch.bfloat16).to(DEV)
    xd = torch.full_like(x, float("nan"))
    _hip.lora_dropout_fwd(x, key, xd, p)
    keep = _mask64(key_v, n, p)
    km = torch.from_numpy(keep).to(DEV)
    nz = x != 0
    assert torch.equal((xd != 0) & nz, km & nz)
    inv = np.float32(1.0) / (np.float32(1.0) - np.float32(p))
    assert torch.equal(xd[km], (x[km].float() * float(inv)).to(torch.bfloat16))
    g = torch.randn(n, generator=gen(1537)).to(torch.bfloat16).to(DEV)
    xd2, dx = torch.empty_like(x), torch.empty_like(x)
    _hip.lora_dropout_bwd(x, g, key, xd2, dx, p)
    assert torch.equal(xd2, xd)
    assert abs(float(keep.mean()) - (1 - p)) < 1e-3
