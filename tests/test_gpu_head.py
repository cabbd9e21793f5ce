"""The fused LM head on the GPU: the row kernel (esep_head_row_softmax) against the oracle
(oracle/head_ref.py), and fused_linear_ce (solution.head) restating the reference's
solution/test_head.py (:11-209) against a plain torch fp32 reference.

Row kernel, on logits chunks with V in {1, 7, 8, 1001, 5003, 151936}, fp16 and bf16, rows that are
flat, peaked or carry hand-made ties, targets in range / -100 / V, CE weights with zeros:
* argmax (first maximal index) and target logit: bit-exact (index and copy work);
* lse: |err| <= 1e-5 + 1e-6 |lse|; entropy: |err| <= 5e-5 (fp32 one-pass sums over up to 151936
  terms against the float64 two-pass oracle);
* g on weighted rows: within one unit in the last place of the logits dtype of the exact
  (p - onehot) * 1024, plus 2^-20 * 1024 p for the fp32 evaluation of p (one v_exp_f32 and the
  rounding of log2 S in its argument; the reference's fp32 p - 1 carries the same kind of error);
  unweighted rows, and every row without write_g, keep their logits bit for bit; strided and
  unaligned chunks take the element-wise path with the same results.
fused_linear_ce: the reference's tolerances (loss rtol 1e-3, stats vs fp16-logit statistics
1e-4 .. 1e-6, dX relative norm error < 1e-2, zero dX on unweighted rows) at 77 x 64 x 1001 (chunks
of 32 and 256 rows), 2048 x 1536 x 151936 (the Qwen2.5 head), a no-grad call that launches the
row kernel without g, fp32 input with a contiguous ignored prefix, and a bf16 head weight.
"""

import numpy as np
import pytest
import torch

from _util import DEV, gen, np64
from oracle import head_ref as ref

pytestmark = pytest.mark.gpu

MANT = {torch.float16: (10, -14), torch.bfloat16: (7, -126)}


def _ulp(x, dtype):
    mant, emin = MANT[dtype]
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** emin)))
    return 2.0 ** (e - mant)


def _chunk(rows, V, dtype, seed):
    g = gen(seed)
    temp = torch.rand(rows, 1, generator=g) * 4 + 0.1
    z = torch.randn(rows, V, generator=g) * temp
    if V > 1:
        hot = torch.randint(0, V, (rows,), generator=g)
        z[torch.arange(rows), hot] += torch.rand(rows, generator=g) * 30  # peaked rows
    if V > 9:
        z[0, [5, 9, V - 1]] = z[0].max() + 10  # ties: first index wins
    z[1 % rows] = 0.5  # a flat row
    target = torch.randint(0, V, (rows,), generator=g)
    target[::5] = -100
    target[3 % rows] = V
    cew = torch.rand(rows, generator=g)
    cew[2::7] = 0.0
    return z.to(dtype), target, cew


def _outs(rows):
    f = [torch.full((rows,), float("nan"), device=DEV) for _ in range(3)]
    return f + [torch.full((rows,), -7, device=DEV, dtype=torch.int32)]


def _check_row_kernel(zd, z_in, target, cew, write_g, dtype, outs):
    lse, tl, ent, amax = outs
    want = ref.row_softmax(np64(z_in), target.numpy(), cew.numpy(), write_g=write_g,
                           g_dtype=np.float64)
    assert np.array_equal(amax.cpu().numpy(), want[3])
    assert np.array_equal(np64(tl), want[1])
    d = np.abs(np64(lse) - want[0])
    assert np.all(d <= 1e-5 + 1e-6 * np.abs(want[0])), d.max()
    assert np.all(np.abs(np64(ent) - want[2]) <= 5e-5), np.abs(np64(ent) - want[2]).max()
    got = np64(zd)
    live = (cew.numpy() != 0) if write_g else np.zeros(len(cew), dtype=bool)
    assert np.array_equal(got[~live], np64(z_in)[~live])
    if live.any():
        gw, gg = want[4][live], got[live]
        p = np.exp(np64(z_in)[live] - want[0][live][:, None])
        bad = np.abs(gg - gw) > _ulp(gw, dtype) + 1024.0 * p * 2.0 ** -20
        assert not bad.any(), (int(bad.sum()), gg[bad][:4], gw[bad][:4])


@pytest.mark.parametrize("write_g", [False, True], ids=["stats", "g"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("V", [1, 7, 8, 1001, 5003, 151936])
def test_row_kernel_vs_oracle(V, dtype, write_g):
    from solution.body import _hip

    rows = 9 if V > 10000 else 37
    z, target, cew = _chunk(rows, V, dtype, seed=V)
    zd = z.to(DEV)
    outs = _outs(rows)
    _hip.head_row_softmax(zd, target.to(DEV), cew.to(DEV), *outs, write_g, 1024.0)
    _check_row_kernel(zd, z, target, cew, write_g, dtype, outs)


@pytest.mark.parametrize("pad,offset", [(8, 0), (3, 0), (0, 1)], ids=["ld+8", "ld+3", "unaligned"])
def test_row_kernel_strided_and_unaligned(pad, offset):
    from solution.body import _hip

    rows, V, dtype = 13, 4096, torch.float16
    z, target, cew = _chunk(rows, V, dtype, seed=11)
    ld = V + pad
    base = torch.zeros(rows * ld + offset + 8, device=DEV, dtype=dtype)
    zd = base[offset:offset + rows * ld].view(rows, ld)[:, :V]
    zd.copy_(z.to(DEV))
    outs = _outs(rows)
    _hip.head_row_softmax(zd, target.to(DEV), cew.to(DEV), *outs, True, 1024.0)
    _check_row_kernel(zd, z, target, cew, True, dtype, outs)
    assert torch.all(base[offset:offset + rows * ld].view(rows, ld)[:, V:] == 0)  # padding kept


# ---------------------------------------------------------------------------------------------
# fused_linear_ce, after the reference's solution/test_head.py
# ---------------------------------------------------------------------------------------------
def _reference(x, w, target, ce_weight, rows_per_step=256):
    """fp32 logits x.float() @ w.float().T, log_softmax in fp32, dX by autograd (reference
    test_head.py:11-52); the *16 statistics come from logits rounded to the weight's dtype."""
    w32 = w.float()
    v = w.shape[0]
    outs = {k: [] for k in ("lse", "tlogit", "ent", "maxlogit", "dx", "lse16", "tlogit16", "ent16")}
    loss = torch.zeros((), device=x.device, dtype=torch.float64)
    for r0 in range(0, x.shape[0], rows_per_step):
        xs = x[r0:r0 + rows_per_step].float().requires_grad_(True)
        ts = target[r0:r0 + rows_per_step]
        cs = ce_weight[r0:r0 + rows_per_step].float()
        logits = xs @ w32.T
        logp = torch.log_softmax(logits, dim=-1)
        valid = (ts >= 0) & (ts < v)
        safe_t = torch.where(valid, ts, torch.zeros_like(ts))
        nll = -logp.gather(1, safe_t[:, None])[:, 0]
        part = (torch.where(valid, cs, torch.zeros_like(cs)) * nll).sum()
        (dxs,) = torch.autograd.grad(part, xs)
        with torch.no_grad():
            lse = torch.logsumexp(logits, dim=-1)
            zero = torch.zeros_like(lse)
            outs["lse"].append(lse)
            outs["tlogit"].append(torch.where(valid, logits.gather(1, safe_t[:, None])[:, 0], zero))
            outs["ent"].append(-(logp.exp() * logp).sum(-1))
            outs["maxlogit"].append(logits.max(-1).values)
            outs["dx"].append(dxs)
            z16 = (x[r0:r0 + rows_per_step].to(w.dtype) @ w.T).float()
            lp16 = torch.log_softmax(z16, dim=-1)
            outs["lse16"].append(torch.logsumexp(z16, dim=-1))
            outs["tlogit16"].append(torch.where(valid, z16.gather(1, safe_t[:, None])[:, 0], zero))
            outs["ent16"].append(-(lp16.exp() * lp16).sum(-1))
            del z16, lp16
        loss += part.detach().double()
        del logits, logp
    res = {k: torch.cat(vs) for k, vs in outs.items()}
    res["loss"] = loss
    return res, w32


def _make(n, h, v, scale_w, peak, seed=0, wdtype=torch.float16):
    """Reference test_head.py:59-77: rows pushed towards their target embedding with a random
    strength (flat to very peaked logits), every 7th row ignored, some zero-weight rows."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    w = (torch.randn(v, h, device=DEV, generator=g) * scale_w).to(wdtype)
    target = torch.randint(0, v, (n,), device=DEV, generator=g)
    x = torch.randn(n, h, device=DEV, generator=g)
    if peak:
        wt = w[target].float()
        strength = torch.rand(n, 1, device=DEV, generator=g) * peak
        x = x + strength * wt / wt.pow(2).sum(-1, keepdim=True)
    x = x.to(wdtype)
    ce_weight = torch.rand(n, device=DEV, generator=g) / n
    target[::7] = -100
    ce_weight[::7] = 0.0
    ce_weight[3::11] = 0.0
    return x, w, target, ce_weight


def _check_all(x, w, target, ce_weight, chunk_rows, dx_rtol, half_ulp=1.6e-2):
    """Reference test_head.py:80-116, tolerances as there (half_ulp: half an ulp of the largest
    logits in the weight's dtype, the bound of the rounded-logit statistics vs fp32 ones)."""
    from solution.head import fused_linear_ce

    ref_, w32 = _reference(x, w, target, ce_weight)
    xg = x.clone().requires_grad_(True)
    loss, pt = fused_linear_ce(xg, w, target, ce_weight, chunk_rows=chunk_rows)
    loss.backward()
    dx = xg.grad
    assert torch.isfinite(loss)
    tc = torch.testing.assert_close
    tc(loss.double(), ref_["loss"], rtol=1e-3, atol=1e-4)
    tc(pt["lse"], ref_["lse"], rtol=0, atol=half_ulp)
    tc(pt["target_logit"], ref_["tlogit"], rtol=0, atol=half_ulp)
    tc(pt["entropy"], ref_["ent"], rtol=0, atol=2 * half_ulp)
    tc(pt["lse"], ref_["lse16"], rtol=1e-6, atol=1e-4)
    tc(pt["target_logit"], ref_["tlogit16"], rtol=0, atol=1e-6)
    tc(pt["entropy"], ref_["ent16"], rtol=1e-4, atol=1e-4)
    ours_at = (x.float() * w32[pt["argmax"]]).sum(-1)
    tc(ours_at, ref_["maxlogit"], rtol=0, atol=half_ulp)
    assert pt["argmax"].dtype == torch.int64
    zero = torch.zeros_like(ref_["lse"])
    tc(pt["ce"], torch.where(target >= 0, ref_["lse"] - ref_["tlogit"], zero), rtol=0,
       atol=2 * half_ulp)
    tc(pt["ce"], torch.where(target >= 0, ref_["lse16"] - ref_["tlogit16"], zero), rtol=1e-5,
       atol=1e-4)
    assert dx.dtype == x.dtype and dx.shape == x.shape
    zero_rows = (ce_weight == 0) | (target < 0)
    assert torch.all(dx[zero_rows] == 0)
    err = (dx.float() - ref_["dx"]).norm() / ref_["dx"].norm()
    assert err.item() < dx_rtol, f"dx relative error {err.item():.3e}"
    assert ((dx.float() - ref_["dx"]).abs().max() / ref_["dx"].abs().max()).item() < 2 * dx_rtol
    return err.item()


@pytest.mark.parametrize("chunk_rows", [32, 256])
def test_small_odd_shapes(chunk_rows):
    x, w, target, ce_weight = _make(77, 64, 1001, scale_w=0.3, peak=20.0)
    _check_all(x, w, target, ce_weight, chunk_rows, dx_rtol=1e-2)


def test_realistic_lm_head():
    x, w, target, ce_weight = _make(2048, 1536, 151936, scale_w=0.02, peak=30.0, seed=1)
    _check_all(x, w, target, ce_weight, chunk_rows=1024, dx_rtol=1e-2)
    del x, w
    torch.cuda.empty_cache()


def test_bf16_head_weight():
    x, w, target, ce_weight = _make(300, 128, 5003, scale_w=0.2, peak=25.0, seed=4,
                                    wdtype=torch.bfloat16)
    # bf16 logits: half an ulp at |z| < 64 is 0.125
    _check_all(x, w, target, ce_weight, chunk_rows=128, dx_rtol=2e-2, half_ulp=0.125)


def test_no_grad_path_skips_dx(monkeypatch):
    from solution.head import fused_linear_ce
    import solution.head.op as op

    x, w, target, ce_weight = _make(77, 64, 1001, scale_w=0.3, peak=20.0)
    ref_, _ = _reference(x, w, target, ce_weight)
    calls = []
    orig = op._hip.head_row_softmax

    def spy(*args, **kw):
        calls.append(bool(args[7]))
        return orig(*args, **kw)

    monkeypatch.setattr(op._hip, "head_row_softmax", spy)
    xg = x.clone().requires_grad_(True)
    with torch.no_grad():
        loss, pt = fused_linear_ce(xg, w, target, ce_weight)
    assert calls == [False]
    assert not loss.requires_grad
    torch.testing.assert_close(loss.double(), ref_["loss"], rtol=1e-3, atol=1e-4)
    torch.testing.assert_close(pt["lse"], ref_["lse16"], rtol=1e-6, atol=1e-4)
    torch.testing.assert_close(pt["entropy"], ref_["ent16"], rtol=1e-4, atol=1e-4)
    loss2, _ = fused_linear_ce(xg, w, target, ce_weight)
    assert calls == [False, True] and loss2.requires_grad
    torch.testing.assert_close(loss2.detach(), loss, rtol=1e-6, atol=1e-6)


def test_fp32_input_and_half_ignored():
    """fp32 x is cast inside, dX comes back in fp32; a contiguous ignored prefix (reference
    test_head.py:163-180). Also the empty batch."""
    from solution.head import fused_linear_ce

    x, w, target, ce_weight = _make(300, 128, 5003, scale_w=0.2, peak=25.0, seed=3)
    target[:150] = -100
    ce_weight[:150] = 0.0
    ref_, _ = _reference(x, w, target, ce_weight)
    xg = x.float().requires_grad_(True)
    loss, st = fused_linear_ce(xg, w, target, ce_weight, chunk_rows=128)
    loss.backward()
    assert xg.grad.dtype == torch.float32 and loss.dtype == torch.float32 and loss.dim() == 0
    torch.testing.assert_close(loss.double(), ref_["loss"], rtol=1e-3, atol=1e-4)
    torch.testing.assert_close(st["entropy"], ref_["ent16"], rtol=1e-4, atol=1e-4)
    assert (st["target_logit"][:150] == 0).all() and (st["ce"][:150] == 0).all()
    err = (xg.grad - ref_["dx"]).norm() / ref_["dx"].norm()
    assert err.item() < 1e-2
    xe = torch.zeros(0, 128, device=DEV, dtype=torch.float16, requires_grad=True)
    le, se = fused_linear_ce(xe, w, target[:0], ce_weight[:0])
    le.backward()
    assert le.item() == 0.0 and se["argmax"].dtype == torch.int64 and se["lse"].numel() == 0


def test_edge_cases():
    """All rows ignored (no weighted row: no g pass, dX all zero, loss 0), a single row, a chunk
    larger than N and an N that is not a multiple of the chunk, against the torch fp32 reference."""
    from solution.head import fused_linear_ce

    x, w, target, ce_weight = _make(50, 64, 777, scale_w=0.3, peak=10.0, seed=5)
    ign = torch.full_like(target, -100)
    xg = x.clone().requires_grad_(True)
    loss, st = fused_linear_ce(xg, w, ign, ce_weight, chunk_rows=16)
    loss.backward()
    assert loss.item() == 0.0 and torch.all(xg.grad == 0)
    assert torch.all(st["ce"] == 0) and torch.all(st["target_logit"] == 0)
    ref_, _ = _reference(x, w, ign, ce_weight)
    torch.testing.assert_close(st["lse"], ref_["lse16"], rtol=1e-6, atol=1e-4)
    for n, chunk in ((1, 256), (50, 7), (50, 1000)):
        xs, ts, cs = x[:n], target[:n].clone(), ce_weight[:n].clone()
        if n == 1:
            ts[0], cs[0] = 3, 1.0
        _check_all(xs, w, ts, cs, chunk_rows=chunk, dx_rtol=1e-2)
