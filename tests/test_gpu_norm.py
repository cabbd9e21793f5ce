"""RMSNorm (K1) on the GPU: the reference's own unit tests restated (reference
solution/test_body_norm_rope.py:22-77, :178-430), plus parity of every variant with the CPU
oracle (oracle/norm_rope_ref.py) on seeded inputs.

Tolerances: 16-bit outputs atol 2e-3 / rtol 1e-2 against the fp64 oracle (the north-star
bar), fp32 outputs 1e-5; the reference's own tests keep their own tolerances (quoted)."""

import ctypes
import numpy as np
import pytest
import torch

from _util import DEV, STORE, assert_close, err, gen, np64, randn
from oracle import norm_rope_ref as ref

pytestmark = pytest.mark.gpu

H, EPS = 1536, 1e-6
TS = [1, 37, 1000, 2048]


def _nr():
    from solution.body import norm_rope

    return norm_rope


# ------------------------------------------------------------------ reference tests, restated

def ref_add_rmsnorm(r_in, delta, w, out_dtype):
    """Eager HF math (reference test_body_norm_rope.py:24-29)."""
    r = r_in + delta if delta is not None else r_in
    h = r.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + EPS)
    return r, (w * h.to(torch.float32)).to(out_dtype)


@pytest.mark.parametrize("T", TS)
@pytest.mark.parametrize("case", ["fp16_delta", "fp32_delta", "no_delta", "fp32_out",
                                  "bf16_delta", "bf16_out"])
def test_add_rmsnorm(T, case):
    """Reference test_add_rmsnorm (:32-62): r_out exact, y within 2e-3 (16-bit) / 1e-5, grads
    within 5e-3 / 1e-5 relative; the weight is an nn.Parameter as there (:41) and
    torch.autograd.grad leaves its .grad None (:62). bf16 cases added. This build's deliberate
    difference: a backward() through a trainable weight fills w.grad with
    dw_j = sum_t dy_tj * xhat_tj (the reference detaches the weight), checked last."""
    nr = _nr()
    g = gen(T)
    delta_dtype = {"fp16_delta": torch.float16, "fp32_delta": torch.float32, "no_delta": None,
                   "fp32_out": torch.float16, "bf16_delta": torch.bfloat16,
                   "bf16_out": torch.bfloat16}[case]
    out_dtype = {"fp32_out": torch.float32, "bf16_out": torch.bfloat16,
                 "bf16_delta": torch.bfloat16}.get(case, torch.float16)
    r_in = randn((1, T, H), g, 3.0).requires_grad_()
    delta = None
    if delta_dtype is not None:
        delta = randn((1, T, H), g, dtype=delta_dtype).requires_grad_()
    w = torch.nn.Parameter((1 + 0.1 * torch.randn(H, generator=g)).to(DEV))

    r_out, y = nr.add_rmsnorm(r_in, delta, w, EPS, out_dtype)
    rr, yr = ref_add_rmsnorm(r_in, delta, w.detach(), out_dtype)
    assert r_out.dtype == torch.float32 and y.dtype == out_dtype
    assert r_out.shape == r_in.shape and y.shape == r_in.shape
    torch.testing.assert_close(r_out, rr, rtol=0, atol=0)
    tol = {torch.float16: 2e-3, torch.bfloat16: 1e-2, torch.float32: 1e-5}[out_dtype]
    torch.testing.assert_close(y.float(), yr.float(), rtol=tol, atol=tol)

    # against the fp64 oracle (the kernel's own contract: one rounding of the exact value)
    d_np = None if delta is None else np64(delta)
    _, y64, rstd64, _ = ref.add_rmsnorm_fwd(np64(r_in)[0], None if d_np is None else d_np[0],
                                            np64(w.detach()), EPS, STORE[out_dtype])
    assert_close(np64(y)[0], y64, 2e-3 if out_dtype != torch.float32 else 1e-5, 1e-2, "y")

    gy = torch.randn(y.shape, generator=g).to(out_dtype).to(DEV)
    gr = torch.randn(r_out.shape, generator=g).to(DEV)
    ins = [r_in] + ([delta] if delta is not None else [])
    gk = torch.autograd.grad([r_out, y], ins, [gr, gy], retain_graph=True)
    gref = torch.autograd.grad([rr, yr], ins, [gr, gy])
    for a, b in zip(gk, gref):
        assert a.dtype == b.dtype
        ae, re = err(np64(a), np64(b))
        lim = 5e-3 if a.dtype != torch.float32 else 1e-5
        assert re < lim, (ae, re)
    dr64, dw64 = ref.add_rmsnorm_bwd([np64(gy)[0]], np64(gr)[0], np64(rr)[0], np64(w.detach()),
                                     EPS)
    assert_close(np64(gk[0])[0], dr64, 1e-4, 1e-4, "d_r_in vs fp64")
    assert w.grad is None  # autograd.grad does not accumulate (reference :62)

    # backward() with the trainable Parameter: its gradient is the kernel's dw
    torch.autograd.backward([r_out, y], [gr, gy])
    assert w.grad is not None and w.grad.dtype == torch.float32
    assert_close(np64(w.grad), dw64, 1e-4 * np.abs(dw64).max(), 1e-4, "w.grad")


def test_add_rmsnorm_dy_only():
    """Reference :65-77. Final norm: r_out unused (dr_out None), y fp32."""
    nr = _nr()
    T = 37
    g = gen(0)
    r_in = randn((T, H), g).requires_grad_()
    delta = randn((T, H), g, dtype=torch.float16).requires_grad_()
    w = (torch.rand(H, generator=g) + 0.5).to(DEV)
    _, y = nr.add_rmsnorm(r_in, delta, w, EPS, torch.float32)
    _, yr = ref_add_rmsnorm(r_in, delta, w, torch.float32)
    gy = torch.randn(y.shape, generator=g).to(DEV)
    a = torch.autograd.grad(y, [r_in, delta], gy)
    b = torch.autograd.grad(yr, [r_in, delta], gy)
    torch.testing.assert_close(a[0], b[0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(a[1], b[1], rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("n_out", [1, 2, 3, 5])
@pytest.mark.parametrize("unused", [False, True], ids=["all_used", "some_unused"])
def test_add_rmsnorm_fanout(n_out, unused):
    """Reference :178-220: n_out views of one y; backward sums their grads in ONE launch."""
    from solution.body import _hip

    nr = _nr()
    T = 300
    g = gen(n_out)
    r_in = randn((1, T, H), g, 3.0).requires_grad_()
    delta = randn((1, T, H), g, dtype=torch.float16).requires_grad_()
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(DEV)
    r_out, ys = nr.add_rmsnorm(r_in, delta, w, EPS, torch.float16, n_out=n_out)
    if n_out == 1:
        ys = (ys,)
    assert len(ys) == n_out and all(y.data_ptr() == ys[0].data_ptr() for y in ys)
    used = [i for i in range(n_out) if not (unused and i % 2 == 1)]
    gys = [torch.randn((1, T, H), generator=g).half().to(DEV) for _ in used]
    gr = torch.randn((1, T, H), generator=g).to(DEV)
    with _hip.count_launches() as runs:
        gk = torch.autograd.grad([r_out] + [ys[i] for i in used], [r_in, delta], [gr] + gys)
    assert runs == ["_add_rmsnorm_bwd"], runs
    rr, yr32 = ref_add_rmsnorm(r_in, delta, w, torch.float32)
    gsum = torch.stack([gy.float() for gy in gys]).sum(0)
    g_ref = torch.autograd.grad([rr, yr32], [r_in, delta], [gr, gsum])
    for a, b in zip(gk, g_ref):
        assert a.dtype == b.dtype
        ae, re = err(np64(a), np64(b))
        assert re < (5e-3 if a.dtype == torch.float16 else 1e-5), (ae, re)


def test_add_rmsnorm_fanout_no_grad_outputs():
    """Reference :223-232: only r_out used -> d_r_in == dr_out and d_delta == dr_out.half()."""
    nr = _nr()
    g = gen(1)
    r_in = randn((1, 8, H), g).requires_grad_()
    delta = randn((1, 8, H), g, dtype=torch.float16).requires_grad_()
    w = torch.ones(H, device=DEV)
    r_out, ys = nr.add_rmsnorm(r_in, delta, w, EPS, torch.float16, n_out=3)
    gr = torch.randn((1, 8, H), generator=g).to(DEV)
    a, b = torch.autograd.grad(r_out, [r_in, delta], gr)
    torch.testing.assert_close(a, gr, rtol=0, atol=0)
    torch.testing.assert_close(b, gr.half(), rtol=0, atol=0)


def test_add_rmsnorm_fanout_fp32_sum_no_overflow():
    """Reference :235-253: two fp16 grads of 40000 sum in fp32 (an fp16 sum overflows)."""
    nr = _nr()
    T = 16
    g = gen(0)
    r_in = randn((1, T, H), g).requires_grad_()
    delta = randn((1, T, H), g, dtype=torch.float16).requires_grad_()
    w = torch.ones(H, device=DEV)
    r_out, (y1, y2) = nr.add_rmsnorm(r_in, delta, w, EPS, torch.float16, n_out=2)
    big = torch.full((1, T, H), 40000.0, device=DEV)
    big[..., ::2] = -40000.0
    big[..., 0] = 40000.0
    g1, g2 = big.half(), big.half()
    assert torch.isinf(g1 + g2).any()
    d_rin, _ = torch.autograd.grad([y1, y2], [r_in, delta], [g1, g2])
    rr, yr = ref_add_rmsnorm(r_in, delta, w, torch.float32)
    want, = torch.autograd.grad(yr, [r_in], [g1.float() + g2.float()])
    assert torch.isfinite(d_rin).all()
    torch.testing.assert_close(d_rin, want, rtol=1e-4, atol=1e-2)


# ------------------------------------------------------------------ save_output mode

def _weight(kind, g):
    """Reference _weight (:258-273): K = 0 / 8 / 3 exact channels."""
    w = 1 + 0.1 * torch.randn(H, generator=g)
    if kind == "zeros_tiny":
        w[[0, 7, 100]] = 0.0
        w[[1, 2]] = torch.tensor([1e-6, -3e-5])
        w[[3, 4]] = torch.tensor([2.0 ** -10 * 0.999, -2.0 ** -10 * 0.5])
        w[5] = 2.0 ** -10 * 1.001
        w[H - 1] = 2000.0
    elif kind == "qwen_like":
        w = (0.3 + 2.7 * torch.rand(H, generator=g)) * torch.sign(torch.randn(H, generator=g))
        w[[11, 500, 1400]] = torch.tensor([2e-5, 6.5e-6, 9e-4])
        w[[12, 501]] = torch.tensor([2e-3, 4e-3])
    return w.to(DEV)


def _rows(T, outliers, g):
    r = torch.randn(T, H, generator=g) * 3
    if outliers:
        r[:, [0, 11, 500, 3, 12]] *= 300.0
        r[: T // 2] *= 50.0
        r.clamp_(-1e3, 1e3)
    return r.to(DEV)


def _norm_grads(r_in, delta, w, gys, gr, save_output, out_dtype=torch.float16):
    nr = _nr()
    r_in = r_in.clone().requires_grad_()
    delta = delta.clone().requires_grad_()
    r_out, ys = nr.add_rmsnorm(r_in, delta, w, EPS, out_dtype, n_out=len(gys),
                               save_output=save_output)
    ys = ys if isinstance(ys, tuple) else (ys,)
    gk = torch.autograd.grad([r_out, *ys], [r_in, delta], [gr, *gys])
    return r_out.detach(), ys[0].detach(), gk


def _ref_grads_f64(r_in, delta, w, gys, gr):
    """Reference _ref_grads_f64 (:297-302)."""
    r = (r_in.double() + delta.double()).requires_grad_()
    y = w.double() * (r * torch.rsqrt(r.pow(2).mean(-1, keepdim=True) + EPS))
    gsum = torch.stack([x.double() for x in gys]).sum(0)
    (dr,) = torch.autograd.grad(y, [r], [gsum])
    return dr + gr.double()


@pytest.mark.parametrize("T", TS)
@pytest.mark.parametrize("kind", ["regular", "zeros_tiny", "qwen_like"])
def test_add_rmsnorm_save_output(T, kind):
    """Reference :305-351: saved tensors, forward bit-identical to the r_out mode, grads vs fp64."""
    nr = _nr()
    g = gen(T)
    w = _weight(kind, g)
    slots, k = nr.special_channels(w)
    assert k == {"regular": 0, "zeros_tiny": 8, "qwen_like": 3}[kind]
    assert int((slots >= 0).sum()) == k
    if k:
        assert sorted(slots[slots >= 0].tolist()) == list(range(k))
    assert nr.special_channels(w)[0] is slots
    s_np, k_np = ref.special_channels(np64(w))
    assert k_np == k and (s_np == slots.cpu().numpy()).all()
    r_in = _rows(T, False, g).view(1, T, H)
    delta = torch.randn(1, T, H, generator=g).half().to(DEV)
    gys = [torch.randn(1, T, H, generator=g).half().to(DEV) for _ in range(2)]
    gr = torch.randn(1, T, H, generator=g).to(DEV)

    saved = []

    def pack(x):
        saved.append((x.dtype, tuple(x.shape)))
        return x

    with torch.autograd.graph.saved_tensors_hooks(pack, lambda x: x):
        nr.add_rmsnorm(r_in.clone().requires_grad_(), delta.clone().requires_grad_(), w, EPS,
                       torch.float16, n_out=2, save_output=True)
    expect = [(torch.float16, (T, H)), (torch.float32, (T,)), (torch.float32, (H,)),
              (torch.int32, (H,))] + ([(torch.float32, (T, k))] if k else [])
    assert saved == expect, saved

    r0, y0, g_old = _norm_grads(r_in, delta, w, gys, gr, False)
    r1, y1, g_new = _norm_grads(r_in, delta, w, gys, gr, True)
    assert torch.equal(r0, r1) and torch.equal(y0, y1)
    want = _ref_grads_f64(r_in, delta, w, gys, gr)
    for x in g_new:
        assert torch.isfinite(x).all()
    assert err(np64(g_new[0]), np64(want))[1] < 2e-3
    assert err(np64(g_new[1]), np64(want))[1] < 5e-3


@pytest.mark.parametrize("delta_dt,out_dt", [(torch.float16, torch.bfloat16),
                                              (torch.bfloat16, torch.float16)],
                         ids=["fp16_delta_bf16_y", "bf16_delta_fp16_y"])
@pytest.mark.parametrize("kind", ["regular", "qwen_like"])
def test_add_rmsnorm_save_output_mixed_16bit(delta_dt, out_dt, kind):
    """save_output with a delta of the other 16-bit type than y: the backward reads the saved y
    (one 16-bit type) and writes the delta's gradient in the other. The forward is bitwise that
    of the r_out mode; the gradients are within the saved-y bars of the fp64 closed form (2e-3 /
    5e-3 of their largest magnitude for an fp16 y, 8 times that for a bf16 y)."""
    g = gen(77)
    T = 300
    w = _weight(kind, g)
    r_in = _rows(T, False, g).view(1, T, H)
    delta = torch.randn(1, T, H, generator=g).to(delta_dt).to(DEV)
    gys = [torch.randn(1, T, H, generator=g).to(out_dt).to(DEV) for _ in range(2)]
    gr = torch.randn(1, T, H, generator=g).to(DEV)
    r0, y0, _ = _norm_grads(r_in, delta, w, gys, gr, False, out_dt)
    r1, y1, (d_rin, d_delta) = _norm_grads(r_in, delta, w, gys, gr, True, out_dt)
    assert torch.equal(r0, r1) and torch.equal(y0, y1)
    assert d_rin.dtype == torch.float32 and d_delta.dtype == delta_dt
    want = _ref_grads_f64(r_in, delta, w, gys, gr)
    k = 8 if out_dt == torch.bfloat16 else 1
    assert err(np64(d_rin), np64(want))[1] < 2e-3 * k
    assert err(np64(d_delta), np64(want))[1] < 5e-3 * k


def test_add_rmsnorm_save_output_precision():
    """Reference :354-379: realistic magnitudes and outliers, y-based backward error bounds."""
    T = 1000
    g = gen(1)
    w = _weight("qwen_like", g)
    for outliers in (False, True):
        r_in = _rows(T, outliers, g).view(1, T, H)
        delta = (torch.randn(1, T, H, generator=g) * 0.5).half().to(DEV)
        gys = [torch.randn(1, T, H, generator=g).half().to(DEV) * 1e-2 for _ in range(5)]
        gr = torch.zeros(1, T, H, device=DEV)
        want = _ref_grads_f64(r_in, delta, w, gys, gr)[0]
        gk = _norm_grads(r_in, delta, w, gys, gr, True)[2][0][0].double()
        row_rel = ((gk - want).abs().amax(1) / want.abs().amax(1)).max().item()
        assert err(np64(gk), np64(want))[1] < 2e-3 and row_rel < 5e-3


def test_add_rmsnorm_save_output_ignored():
    """Reference :382-391: no delta or an fp32 y -> r_out is saved."""
    nr = _nr()
    for delta, dt in ((None, torch.float16), (torch.randn(4, H, device=DEV).half(), torch.float32)):
        saved = []
        r_in = torch.randn(4, H, device=DEV, requires_grad=True)
        with torch.autograd.graph.saved_tensors_hooks(
                lambda x: (saved.append((x.dtype, tuple(x.shape))), x)[1], lambda x: x):
            nr.add_rmsnorm(r_in, delta, torch.ones(H, device=DEV), EPS, dt, save_output=True)
        assert saved == [(torch.float32, (4, H)), (torch.float32, (4,)), (torch.float32, (H,))]


def test_special_channels_cache_invalidation():
    """Reference :394-401."""
    nr = _nr()
    w = torch.ones(H, device=DEV)
    assert nr.special_channels(w)[1] == 0
    w[3] = 0.0
    slots, k = nr.special_channels(w)
    assert k == 1 and slots[3].item() == 0


def test_add_rmsnorm_save_output_needs_exact_channels(monkeypatch):
    """Reference :404-430 (negative control): without exact channels a w == 0 channel gives a
    non-finite gradient and tiny |w| a >10x larger error."""
    nr = _nr()
    g = gen(5)
    T = 64
    r_in = _rows(T, False, g).view(1, T, H)
    delta = torch.randn(1, T, H, generator=g).half().to(DEV)
    gys = [torch.randn(1, T, H, generator=g).half().to(DEV)]
    gr = torch.zeros(1, T, H, device=DEV)
    for tiny in (0.0, 1e-6):
        w = _weight("regular", g)
        w[[9, 99]] = tiny
        want = _ref_grads_f64(r_in, delta, w, gys, gr)
        monkeypatch.setattr(nr, "SPECIAL_W_MIN", 0.0)
        bad = _norm_grads(r_in, delta, w.clone(), gys, gr, True)[2][0]
        monkeypatch.setattr(nr, "SPECIAL_W_MIN", 2.0 ** -10)
        good = _norm_grads(r_in, delta, w.clone(), gys, gr, True)[2][0]
        assert torch.isfinite(good).all() and err(np64(good), np64(want))[1] < 2e-3
        if tiny == 0.0:
            assert not torch.isfinite(bad).all()
        else:
            assert err(np64(bad), np64(want))[1] > 10 * err(np64(good), np64(want))[1]


def test_rmsnorm_recompute_bitwise():
    """Reference rmsnorm_recompute contract (norm_rope.py:309-323): y from the saved fp32
    residual is bit-identical to add_rmsnorm's y."""
    nr = _nr()
    g = gen(3)
    T = 513
    r_in = randn((T, H), g, 3.0)
    delta = randn((T, H), g, dtype=torch.float16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(DEV)
    r_out, y = nr.add_rmsnorm(r_in, delta, w, EPS, torch.float16)
    y2 = nr.rmsnorm_recompute(r_out.detach(), w, EPS, torch.float16)
    assert torch.equal(y, y2)


# ------------------------------------------------------------------ plain RMSNorm (north star)

WIDTHS = [1536, 3584, 896, 2048, 4096, 8192, 16384, 1000, 1001, 24]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("n", WIDTHS)
@pytest.mark.parametrize("recompute", [False, True], ids=["saved_rstd", "recomputed_rstd"])
def test_rmsnorm_vs_oracle(dtype, n, recompute):
    """y, dx, dw of the plain norm against the fp64 oracle; every row width class (one to
    eleven wavefronts per row, ragged n % 8 != 0 on the element-wise kernel)."""
    nr = _nr()
    g = gen(n)
    T = 67
    x = randn((T, n), g, dtype=dtype).requires_grad_()
    w = (1 + 0.02 * torch.randn(n, generator=g)).to(DEV).requires_grad_()
    y = nr.rmsnorm(x, w, EPS, recompute_rstd=recompute)
    assert y.dtype == dtype and y.shape == x.shape
    dy = randn((T, n), g, dtype=dtype)
    dx, dw = torch.autograd.grad(y, [x, w], dy)
    assert dx.dtype == dtype and dw.dtype == torch.float32
    y64, _ = ref.rmsnorm_fwd(np64(x), np64(w), EPS, STORE[dtype])
    dx64, dw64 = ref.rmsnorm_bwd(np64(dy), np64(x), np64(w), EPS)
    lp = dtype != torch.float32
    assert_close(np64(y), y64, 2e-3 if lp else 1e-5, 1e-2 if lp else 1e-5, "y")
    assert_close(np64(dx), ref.round_to(dx64, STORE[dtype]), 2e-3 if lp else 1e-5,
                 1e-2 if lp else 1e-5, "dx")
    assert_close(np64(dw), dw64, 1e-4 * np.abs(dw64).max(), 1e-4, "dw")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [1536, 896, 1000])
@pytest.mark.parametrize("recompute", [False, True], ids=["saved_rstd", "recomputed_rstd"])
def test_rmsnorm_dx_independent_of_weight_grad(dtype, n, recompute):
    """The backward runs a form of its kernel fixed to the call (saved rstd, dx only, with or
    without the weight gradient): dx is the same bits whether or not the weight gradient is
    taken, and within the bar of the fp64 oracle."""
    nr = _nr()
    g = gen(900 + n)
    T = 300
    x = randn((T, n), g, dtype=dtype).requires_grad_()
    wv = 1 + 0.02 * torch.randn(n, generator=g)
    w1 = wv.to(DEV).requires_grad_()
    w0 = wv.to(DEV)
    dy = randn((T, n), g, dtype=dtype)
    y1 = nr.rmsnorm(x, w1, EPS, recompute_rstd=recompute)
    dx1, dw1 = torch.autograd.grad(y1, [x, w1], dy)
    y0 = nr.rmsnorm(x, w0, EPS, recompute_rstd=recompute)
    (dx0,) = torch.autograd.grad(y0, [x], dy)
    assert torch.equal(y0, y1)
    assert torch.equal(dx0, dx1)
    dx64, dw64 = ref.rmsnorm_bwd(np64(dy), np64(x), np64(wv), EPS)
    assert_close(np64(dx0), ref.round_to(dx64, STORE[dtype]), 2e-3, 1e-2, "dx")
    assert_close(np64(dw1), dw64, 1e-4 * np.abs(dw64).max(), 1e-4, "dw")


@pytest.mark.parametrize("n", [64, 1536])
def test_rmsnorm_bwd_many_rows_per_wavefront(n):
    """Past 64 rows per wavefront (one vector load of saved rstd values) the entry point sends the
    call from the pipelined backward to the wide one: 150000 rows of 64 columns give ~147 rows
    per wavefront on 256 blocks, with and without the weight gradient; 40000 rows of 1536 give
    ~39 (the pipelined kernel). dx on rows spread over the input and dw against the fp64 oracle,
    and dx the same bits with and without the weight gradient."""
    nr = _nr()
    g = gen(77 + n)
    T = 150000 if n == 64 else 40000
    x = randn((T, n), g, dtype=torch.bfloat16).requires_grad_()
    wv = 1 + 0.02 * torch.randn(n, generator=g)
    w1 = wv.to(DEV).requires_grad_()
    dy = randn((T, n), g, dtype=torch.bfloat16)
    y = nr.rmsnorm(x, w1, EPS)
    dx1, dw1 = torch.autograd.grad(y, [x, w1], dy)
    y0 = nr.rmsnorm(x, wv.to(DEV), EPS)
    (dx0,) = torch.autograd.grad(y0, [x], dy)
    assert torch.equal(dx0, dx1)
    rows = sorted(set([0, 1, T - 1] + torch.randint(0, T, (509,), generator=gen(5)).tolist()))
    dx64, _ = ref.rmsnorm_bwd(np64(dy[rows]), np64(x[rows]), np64(wv), EPS)
    assert_close(np64(dx1[rows]), ref.round_to(dx64, "bf16"), 2e-3, 1e-2, "dx")
    _, dw64 = ref.rmsnorm_bwd(np64(dy), np64(x), np64(wv), EPS)
    assert_close(np64(dw1), dw64, 1e-5 * np.abs(dw64).max(), 1e-5, "dw")


def test_rmsnorm_recompute_matches_saved_bitwise():
    """The rstd-recompute backward computes rstd with the forward's own arithmetic: its dx and
    dw equal the saved-rstd backward's bit for bit."""
    nr = _nr()
    g = gen(11)
    x = randn((1024, H), g, dtype=torch.bfloat16).requires_grad_()
    w = (1 + 0.02 * torch.randn(H, generator=g)).to(DEV).requires_grad_()
    dy = randn((1024, H), g, dtype=torch.bfloat16)
    a = torch.autograd.grad(nr.rmsnorm(x, w, EPS), [x, w], dy)
    b = torch.autograd.grad(nr.rmsnorm(x, w, EPS, recompute_rstd=True), [x, w], dy)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("T", [1, 16, 17, 1000, 4097, 8192])
def test_dgamma_deterministic(T):
    """dw is reduced in two fixed-order stages: repeated runs are bitwise equal, and the
    residual-stream API gives the same bits as the plain API for the same fp32 input."""
    nr = _nr()
    g = gen(T)
    x = randn((T, H), g)
    w = (1 + 0.02 * torch.randn(H, generator=g)).to(DEV).requires_grad_()
    dy = randn((T, H), g)
    runs = []
    for _ in range(3):
        xr = x.clone().requires_grad_()
        runs.append(torch.autograd.grad(nr.rmsnorm(xr, w, EPS), [w], dy)[0])
    assert all(torch.equal(runs[0], r) for r in runs[1:])
    xr = x.clone().requires_grad_()
    _, y = nr.add_rmsnorm(xr, None, w, EPS, torch.float32)
    dw2 = torch.autograd.grad(y, [w], dy)[0]
    assert torch.equal(runs[0], dw2)
    _, dw64 = ref.rmsnorm_bwd(np64(dy), np64(x), np64(w), EPS)
    assert_close(np64(runs[0]), dw64, 1e-5 * np.abs(dw64).max(), 1e-5, "dw")


@pytest.mark.parametrize("T,n", [(1, 1536), (4097, 1536), (300, 3584), (65, 1001)])
def test_dgamma_partials_then_reduce(T, n):
    """Stage 1 alone (partials into the caller's buffer) and esep_dgamma_reduce later give the
    fused call's dw bit for bit, with dx unchanged; no rows and no partials give dw = 0."""
    from solution.body import _hip

    g = gen(T + n)
    x = randn((T, n), g, dtype=torch.bfloat16)
    dy = randn((T, n), g, dtype=torch.bfloat16)
    w = (1 + 0.02 * torch.randn(n, generator=g)).to(DEV)
    dx1, dx2 = torch.empty_like(x), torch.empty_like(x)
    dw1, dw2 = torch.empty(n, device=DEV), torch.full((n,), float("nan"), device=DEV)
    _hip.rmsnorm_bwd([dy], x, w, EPS, dx=dx1, dw=dw1)
    part = torch.full((_hip.rmsnorm_partials(T, n), n), float("nan"), device=DEV)
    _hip.rmsnorm_bwd([dy], x, w, EPS, dx=dx2, partials=part)
    _hip.dgamma_reduce(part, dw2)
    assert torch.equal(dx1, dx2) and torch.equal(dw1, dw2)
    _, dw64 = ref.rmsnorm_bwd(np64(dy), np64(x), np64(w), EPS)
    assert_close(np64(dw2), dw64, 1e-4 * np.abs(dw64).max(), 1e-4, "dw")
    # rows = 0 through the C ABI (torch gives empty views a NULL data pointer, which the ABI
    # rejects even for empty inputs, so the full tensors' pointers stand in)
    z = torch.full((n,), float("nan"), device=DEV, dtype=torch.bfloat16)
    lib = _hip.lib()
    rc = lib.esep_rmsnorm_bwd((ctypes.c_void_p * 5)(dy.data_ptr()), 1, 2, n, None, x.data_ptr(),
                              2, n, 0, None, w.data_ptr(), None, None, 0, None, dx1.data_ptr(), 2,
                              n, part.data_ptr(), 0, z.data_ptr(), 2, 0, n, EPS,
                              torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.esep_last_error()
    assert torch.equal(z, torch.zeros_like(z))
    z.fill_(float("nan"))
    _hip.dgamma_reduce(torch.empty((0, n), device=DEV), z)
    assert torch.equal(z, torch.zeros_like(z))


def test_dgamma_reduce_batch_matches_per_norm():
    """One batched stage-2 launch over several norms' partials (different row counts, so different
    partial counts, plus an empty one) writes each dw bit for bit as its own esep_dgamma_reduce;
    fp32 and bf16 dw."""
    from solution.body import _hip

    n = 1536
    g = gen(11)
    w = (1 + 0.02 * torch.randn(n, generator=g)).to(DEV)
    parts = []
    for T in (8192, 300, 1, 4097):
        x = randn((T, n), g, dtype=torch.bfloat16)
        dy = randn((T, n), g, dtype=torch.bfloat16)
        part = torch.empty((_hip.rmsnorm_partials(T, n), n), device=DEV)
        _hip.rmsnorm_bwd([dy], x, w, EPS, dx=torch.empty_like(x), partials=part)
        parts.append(part)
    parts.append(torch.empty((0, n), device=DEV))
    for dt in (torch.float32, torch.bfloat16):
        one = [torch.full((n,), float("nan"), device=DEV, dtype=dt) for _ in parts]
        batch = [torch.full((n,), float("nan"), device=DEV, dtype=dt) for _ in parts]
        for p, d in zip(parts, one):
            _hip.dgamma_reduce(p, d)
        _hip.dgamma_reduce_batch(parts, batch)
        for a, b in zip(one, batch):
            assert torch.equal(a, b)
        assert torch.equal(batch[-1], torch.zeros_like(batch[-1]))
    # the first norm's dw against the float64 oracle sum of its partials
    ref64 = parts[0].double().sum(0)
    got = torch.empty(n, device=DEV)
    _hip.dgamma_reduce_batch(parts[:1], [got])
    assert (got.double() - ref64).abs().max() <= 1e-5 * ref64.abs().max()


def test_add_rmsnorm_weight_grad():
    """A trainable weight gets dw in its own dtype (bf16 weight -> bf16 grad) = sum dy * xhat."""
    nr = _nr()
    g = gen(21)
    T = 300
    r_in = randn((T, H), g, 3.0).requires_grad_()
    delta = randn((T, H), g, dtype=torch.bfloat16).requires_grad_()
    w = (1 + 0.02 * torch.randn(H, generator=g)).to(torch.bfloat16).to(DEV).requires_grad_()
    r_out, (y1, y2) = nr.add_rmsnorm(r_in, delta, w, EPS, torch.bfloat16, n_out=2)
    gy1, gy2 = randn((T, H), g, dtype=torch.bfloat16), randn((T, H), g, dtype=torch.bfloat16)
    (dw,) = torch.autograd.grad([y1, y2], [w], [gy1, gy2])
    assert dw.dtype == torch.bfloat16
    r64 = np64(r_in) + np64(delta)
    _, dw64 = ref.add_rmsnorm_bwd([np64(gy1), np64(gy2)], None, r64, np64(w), EPS)
    assert_close(np64(dw), dw64, 1e-3 * np.abs(dw64).max(), 1e-2, "dw")


def test_bf16_residual_stream():
    """x and delta bf16 (HF's bf16 residual stream): r_out = bf16(x + delta), normalized as
    rounded, as HF computes norm(residual + delta) in bf16."""
    from solution.body import _hip

    g = gen(31)
    T = 129
    x = randn((T, H), g, dtype=torch.bfloat16)
    d = randn((T, H), g, dtype=torch.bfloat16)
    w = (1 + 0.02 * torch.randn(H, generator=g)).to(DEV)
    r = torch.empty_like(x)
    y = torch.empty_like(x)
    rstd = torch.empty(T, device=DEV)
    _hip.rmsnorm_fwd(x, w, y, EPS, delta=d, r_out=r, rstd=rstd)
    assert torch.equal(r, x + d)  # torch's bf16 add rounds once, to nearest even
    r64, y64, rstd64, _ = ref.add_rmsnorm_fwd(np64(x), np64(d), np64(w), EPS, "bf16",
                                              r_dtype="bf16")
    assert_close(np64(y), y64, 2e-3, 1e-2, "y")
    assert_close(np64(rstd), rstd64, 0, 1e-6, "rstd")


def test_rows_zero_and_errors():
    """Empty inputs launch nothing; bad arguments raise (no silent fallback)."""
    from solution.body import _hip

    nr = _nr()
    x = torch.empty((0, H), device=DEV, requires_grad=True)
    w = torch.ones(H, device=DEV, requires_grad=True)
    y = nr.rmsnorm(x, w, EPS)
    dx, dw = torch.autograd.grad(y, [x, w], torch.empty_like(y))
    assert dx.shape == (0, H) and torch.equal(dw, torch.zeros_like(dw))
    with pytest.raises(_hip.EsepError):
        _hip.rmsnorm_fwd(torch.ones(4, H, device=DEV), torch.ones(H + 1, device=DEV),
                         torch.empty(4, H, device=DEV), EPS)
    with pytest.raises(_hip.EsepError):
        nr.rmsnorm(torch.ones(4, H), torch.ones(H), EPS)  # CPU tensors: no CPU path


def _norm_case_vs_oracle(shape, g):
    """rmsnorm fwd + bwd of x ~ N(0, 1) fp16 with w = 1 + 0.02 N(0, 1) (eps 1e-6) against the
    fp64 oracle: y and dx at the 16-bit bar, dw within 1e-4 of max |dw|."""
    nr = _nr()
    x = randn(shape, g, dtype=torch.float16).requires_grad_()
    w = (1 + 0.02 * torch.randn(H, generator=g)).to(DEV).requires_grad_()
    dy = randn(shape, g, dtype=torch.float16)
    y = nr.rmsnorm(x, w, EPS)
    dx, dw = torch.autograd.grad(y, [x, w], dy)
    assert y.shape == x.shape and dx.dtype == torch.float16
    x2, dy2 = np64(x).reshape(-1, H), np64(dy).reshape(-1, H)
    y64, _ = ref.rmsnorm_fwd(x2, np64(w), EPS, "f16")
    dx64, dw64 = ref.rmsnorm_bwd(dy2, x2, np64(w), EPS)
    assert_close(np64(y).reshape(-1, H), y64, 2e-3, 1e-2, "y")
    assert_close(np64(dx).reshape(-1, H), dx64, 2e-3, 1e-2, "dx")
    assert_close(np64(dw), dw64, 1e-4 * np.abs(dw64).max(), 1e-4, "dw")


def test_config1_shape():
    """Config 1 at its own size: x [4, 512, 1536] fp16 (2048 rows), w = 1 + 0.02 N(0, 1),
    eps 1e-6, seeded; y, dx and dw against the oracle."""
    _norm_case_vs_oracle((4, 512, H), gen(0))


def test_single_row():
    """One row (the smallest input, a one-row grid)."""
    _norm_case_vs_oracle((1, H), gen(1))


def test_config3_norm_varlen_tokens():
    """Config 3's norm half at its own size: the 8 sequences of lengths U[64, 1024] (seed 0)
    packed to T = 4557 tokens, x [T, 1536] fp16."""
    lens = torch.randint(64, 1025, (8,), generator=gen(0)).tolist()
    assert lens == [113, 962, 544, 574, 556, 614, 422, 772] and sum(lens) == 4557
    _norm_case_vs_oracle((sum(lens), H), gen(3))


def test_one_row_views():
    """A one-row input with a non-unit column stride, or an expanded row, is copied to
    contiguous rows first (the kernels read unit-stride rows): the result equals the
    contiguous input's bit for bit."""
    nr = _nr()
    g = gen(5)
    base = randn((1, 2 * H), g, dtype=torch.bfloat16)
    w = (1 + 0.02 * torch.randn(H, generator=g)).to(DEV)
    strided = base[:, ::2]
    assert torch.equal(nr.rmsnorm(strided, w, EPS), nr.rmsnorm(strided.contiguous(), w, EPS))
    row = randn((H,), g, dtype=torch.bfloat16)
    expanded = row.expand(3, H)
    assert torch.equal(nr.rmsnorm(expanded, w, EPS), nr.rmsnorm(expanded.contiguous(), w, EPS))
