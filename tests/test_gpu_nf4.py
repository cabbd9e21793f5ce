"""NF4 dequantization (esep_nf4_dequant, solution.nf4) on the GPU against the oracle
(oracle/nf4_ref.py), which restates the format the reference's kernel decodes
(solution/nf4/dequant.py:1-57).

Integer and rounding work, so the bar is bit-exact: random packed bytes, random uint8 scale
indices, random second-level scales, code tables and offset, at the four weight shapes of
Qwen2.5-1.5B (reference test_nf4.py:16) and ragged block counts; fp16 out (the reference's) plus
bf16 and fp32. A weight quantized by the oracle's QLoRA-style quantizer goes through
dequantize_nf4 with a bitsandbytes-shaped quant state, the multi-weight form writes bit-identical
slices, and NF4Linear matches a dense linear on the dequantized weight in both directions. The
one-launch multi-weight entry (esep_nf4_dequant_multi) decodes 8 weights of ragged sizes, each
with its own tables, bit-identically to the oracle and to one single-weight launch per weight.
"""

import types

import numpy as np
import pytest
import torch

from _util import DEV
from oracle import nf4_ref as ref

pytestmark = pytest.mark.gpu

SHAPES = [(1536, 1536), (256, 1536), (8960, 1536), (1536, 8960), (3, 64), (5, 192)]


def _random_state(nb, seed):
    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, nb * 32, dtype=np.uint8)
    absmax = rng.integers(0, 256, nb, dtype=np.uint8)
    absmax2 = (rng.random((nb + 255) // 256) * 0.1 + 0.01).astype(np.float32)
    code2 = np.sort(rng.standard_normal(256)).astype(np.float32)
    offset = np.float32(rng.random() * 0.05)
    return packed, absmax, absmax2, code2, offset


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("n,k", SHAPES)
def test_dequant_bit_exact(n, k, dtype):
    from solution.body import _hip

    nb = n * k // 64
    packed, absmax, absmax2, code2, offset = _random_state(nb, seed=n + k)
    out = torch.full((n, k), float("nan"), device=DEV, dtype=dtype)
    _hip.nf4_dequant(_dev(packed), _dev(absmax), _dev(absmax2), _dev(code2),
                     _dev(np.array([offset], dtype=np.float32)), _dev(ref.NF4), out)
    want32 = ref.dequantize_nf4(packed, absmax, absmax2, code2, offset, out_dtype=np.float32)
    want = torch.from_numpy(want32.reshape(n, k)).to(dtype)  # one rounding of the fp32 value
    assert torch.equal(out.cpu(), want)


def _quant_state(w):
    packed, absmax, absmax2, code2, offset = ref.quantize_nf4(w)
    qs = types.SimpleNamespace(
        quant_type="nf4", blocksize=64, nested=True, shape=w.shape,
        absmax=_dev(absmax), code=_dev(ref.NF4), offset=_dev(np.array(offset, dtype=np.float32)),
        state2=types.SimpleNamespace(absmax=_dev(absmax2), code=_dev(code2), blocksize=256))
    return _dev(packed).reshape(-1, 1), qs, (packed, absmax, absmax2, code2, offset)


def test_dequantize_nf4_api_multi_and_linear():
    from solution import nf4

    rng = np.random.default_rng(1)
    ws = [(rng.standard_normal(shape) * 0.02).astype(np.float32) for shape in ((96, 128), (32, 128))]
    ws[0][0, :64] *= 50
    states = [_quant_state(w) for w in ws]
    for (packed, qs, raw), w in zip(states, ws):
        assert nf4.supported(qs)
        got = nf4.dequantize_nf4(packed, qs)
        want = ref.dequantize_nf4(*raw).reshape(w.shape)
        assert got.dtype == torch.float16 and np.array_equal(got.cpu().numpy(), want)
        assert torch.equal(nf4.dequantize_nf4(packed.t(), qs), got)  # any view of the bytes
    cat = nf4.dequantize_nf4_multi([s[0] for s in states], [s[1] for s in states])
    assert torch.equal(cat[:96], nf4.dequantize_nf4(states[0][0], states[0][1]))
    assert torch.equal(cat[96:], nf4.dequantize_nf4(states[1][0], states[1][1]))
    packed, qs, _ = states[0]
    x = torch.randn(4, 7, 128, device=DEV, dtype=torch.float16, requires_grad=True)
    bias = torch.randn(96, device=DEV, dtype=torch.float16)
    y = nf4.nf4_linear(x, packed, bias, qs)
    dy = torch.randn_like(y)
    (dx,) = torch.autograd.grad(y, [x], dy)
    w16 = nf4.dequantize_nf4(packed, qs)
    xr = x.detach().clone().requires_grad_()
    yr = torch.nn.functional.linear(xr, w16, bias)
    (dxr,) = torch.autograd.grad(yr, [xr], dy)
    assert torch.equal(y, yr) and torch.equal(dx, dxr)
    bad = types.SimpleNamespace(**{**vars(qs), "quant_type": "fp4"})
    assert not nf4.supported(bad)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32],
                         ids=["fp16", "bf16", "fp32"])
def test_multi_launch_bit_exact(dtype):
    """esep_nf4_dequant_multi: 8 weights of ragged block counts (some not a multiple of the
    256-thread block, so blocks straddle weights) in one launch, each with its own tables, equal
    bit for bit to the oracle and to one esep_nf4_dequant per weight; a single weight too."""
    from solution.body import _hip

    sizes = [1, 3, 255, 256, 257, 1000, 6144, 4097]
    items, wants, singles = [], [], []
    for k, nb in enumerate(sizes):
        packed, absmax, absmax2, code2, offset = _random_state(nb, seed=100 + k)
        nf4 = np.sort(np.random.default_rng(k).standard_normal(16)).astype(np.float32)
        t = (_dev(packed), _dev(absmax), _dev(absmax2), _dev(code2),
             _dev(np.array([offset], dtype=np.float32)), _dev(nf4))
        out = torch.full((nb * 64,), float("nan"), device=DEV, dtype=dtype)
        items.append(t + (out,))
        want32 = ref.dequantize_nf4(packed, absmax, absmax2, code2, offset, nf4=nf4,
                                    out_dtype=np.float32)
        wants.append(torch.from_numpy(want32).to(dtype))
        single = torch.empty_like(out)
        _hip.nf4_dequant(*t, single)
        singles.append(single)
    with _hip.count_launches() as names:
        _hip.nf4_dequant_multi(items)
    assert names == ["_nf4_dequant_multi"]
    for it, want, single in zip(items, wants, singles):
        assert torch.equal(it[-1].cpu(), want)
        assert torch.equal(it[-1], single)
    one = torch.empty_like(items[5][-1])
    _hip.nf4_dequant_multi([items[5][:-1] + (one,)])
    assert torch.equal(one, singles[5])


def test_dequantize_nf4_multi_one_launch_per_eight():
    from solution import nf4
    from solution.body import _hip

    rng = np.random.default_rng(2)
    ws = [(rng.standard_normal((n, 128)) * 0.02).astype(np.float32) for n in (96, 32, 64) * 3]
    states = [_quant_state(w) for w in ws]
    with _hip.count_launches() as names:
        cat = nf4.dequantize_nf4_multi([s[0] for s in states], [s[1] for s in states])
    assert names == ["_nf4_dequant_multi"] * 2  # 9 weights: 8 + 1
    r = 0
    for packed, qs, _ in states:
        assert torch.equal(cat[r:r + qs.shape[0]], nf4.dequantize_nf4(packed, qs))
        r += qs.shape[0]
