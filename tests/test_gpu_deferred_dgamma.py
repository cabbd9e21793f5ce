"""The deferred weight-gradient stage 2 (norm_rope.DEFER_WEIGHT_GRAD): a loss.backward() pass
keeps every trainable norm's [P, n] partials and reduces all of them in one
esep_dgamma_reduce_batch launch at the end of the pass, then accumulates into .grad. The
gradients must be the bits of the per-call reduction (the batched reduce sums each norm's
partials in the same order), and every case where deferral cannot see the gradient's consumer
(autograd.grad, backward(inputs=...), hooks, create_graph) must take the per-call path."""

import numpy as np
import pytest
import torch

from _util import DEV, assert_close, gen, np64, randn
from oracle import norm_rope_ref as ref

pytestmark = pytest.mark.gpu

H, EPS = 1536, 1e-6


def _nr():
    from solution.body import norm_rope

    return norm_rope


def _stack(seed, T=300, bf16_weight=False):
    """Three norms in a chain (plain bf16 norm, residual-add norm, final norm) with trainable
    weights, like a decoder layer's input / post-attention / final norms."""
    g = gen(seed)
    wdt = torch.bfloat16 if bf16_weight else torch.float32
    ws = [torch.nn.Parameter((1 + 0.02 * torch.randn(H, generator=g)).to(wdt).to(DEV))
          for _ in range(3)]
    x = randn((T, H), g, dtype=torch.bfloat16).requires_grad_()
    r = randn((T, H), g, 2.0).requires_grad_()
    gy = [randn((T, H), g, dtype=dt) for dt in (torch.bfloat16, torch.bfloat16, torch.float32)]
    return ws, x, r, gy


def _run(ws, x, r, gy, defer, backward=None):
    nr = _nr()
    old = nr.DEFER_WEIGHT_GRAD
    nr.DEFER_WEIGHT_GRAD = defer
    try:
        y0 = nr.rmsnorm(x, ws[0], EPS)
        r1, y1 = nr.add_rmsnorm(r, y0, ws[1], EPS, torch.bfloat16)
        _, y2 = nr.add_rmsnorm(r1, y1, ws[2], EPS, torch.float32)
        loss = (y0.float() * gy[0].float()).sum() + (y1.float() * gy[1].float()).sum() \
            + (y2 * gy[2]).sum()
        if backward is None:
            loss.backward()
        else:
            return backward(loss)
    finally:
        nr.DEFER_WEIGHT_GRAD = old


@pytest.mark.parametrize("bf16_weight", [False, True], ids=["fp32_weight", "bf16_weight"])
def test_deferred_equals_per_call_bitwise(bf16_weight):
    from solution.body import _hip

    ws_a, x, r, gy = _stack(1, bf16_weight=bf16_weight)
    ws_b = [torch.nn.Parameter(w.detach().clone()) for w in ws_a]
    xa, ra = x.detach().clone().requires_grad_(), r.detach().clone().requires_grad_()
    with _hip.count_launches() as names:
        _run(ws_a, xa, ra, gy, defer=True)
        torch.cuda.synchronize()
    assert names.count("_dgamma_reduce_batch") == 1 and names.count("_add_rmsnorm_bwd") == 3
    xb, rb = x.detach().clone().requires_grad_(), r.detach().clone().requires_grad_()
    with _hip.count_launches() as names_b:
        _run(ws_b, xb, rb, gy, defer=False)
        torch.cuda.synchronize()
    assert names_b.count("_dgamma_reduce_batch") == 0
    for wa, wb in zip(ws_a, ws_b):
        assert wa.grad is not None and wa.grad.dtype == wa.dtype
        assert torch.equal(wa.grad, wb.grad)
    assert torch.equal(xa.grad, xb.grad) and torch.equal(ra.grad, rb.grad)


def test_deferred_matches_oracle():
    """The first norm's weight gradient against the fp64 closed form sum_t dy_tj * xhat_tj."""
    ws, x, r, gy = _stack(2)
    nr = _nr()
    old = nr.DEFER_WEIGHT_GRAD
    nr.DEFER_WEIGHT_GRAD = True
    try:
        y0 = nr.rmsnorm(x, ws[0], EPS)
        (y0.float() * gy[0].float()).sum().backward()
    finally:
        nr.DEFER_WEIGHT_GRAD = old
    _, dw64 = ref.rmsnorm_bwd(np64(gy[0]), np64(x), np64(ws[0]), EPS)
    assert_close(np64(ws[0].grad), dw64, 1e-5 * np.abs(dw64).max(), 1e-5, "dw")


def test_deferred_accumulates_over_passes():
    """Two backward passes (gradient accumulation) give the per-call path's .grad."""
    ws_a, x, r, gy = _stack(3)
    ws_b = [torch.nn.Parameter(w.detach().clone()) for w in ws_a]
    for _ in range(2):
        _run(ws_a, x.detach().requires_grad_(), r.detach().requires_grad_(), gy, defer=True)
        _run(ws_b, x.detach().requires_grad_(), r.detach().requires_grad_(), gy, defer=False)
    for wa, wb in zip(ws_a, ws_b):
        assert torch.equal(wa.grad, wb.grad)


def test_not_deferred_when_the_engine_does_not_accumulate():
    """autograd.grad and backward(inputs=...) without the weight: the per-call path (the weight
    gradient is returned, or not computed into .grad at all)."""
    from solution.body import _hip

    ws, x, r, gy = _stack(4)
    ref_ws = [torch.nn.Parameter(w.detach().clone()) for w in ws]
    _run(ref_ws, x.detach().requires_grad_(), r.detach().requires_grad_(), gy, defer=False)
    with _hip.count_launches() as names:
        grads = _run(ws, x, r, gy, defer=True,
                     backward=lambda loss: torch.autograd.grad(loss, ws))
    assert names.count("_dgamma_reduce_batch") == 0
    for gw, wb in zip(grads, ref_ws):
        assert torch.equal(gw, wb.grad)
    assert all(w.grad is None for w in ws)
    _run(ws, x, r, gy, defer=True, backward=lambda loss: loss.backward(inputs=[x]))
    torch.cuda.synchronize()
    assert all(w.grad is None for w in ws) and x.grad is not None


def test_not_deferred_with_hooks():
    """A hook on the weight sees its gradient through autograd (no deferral for that weight)."""
    ws, x, r, gy = _stack(5)
    ref_ws = [torch.nn.Parameter(w.detach().clone()) for w in ws]
    _run(ref_ws, x.detach().requires_grad_(), r.detach().requires_grad_(), gy, defer=False)
    seen = {}
    ws[1].register_hook(lambda g: seen.setdefault("grad", g.clone()))
    _run(ws, x, r, gy, defer=True)
    assert torch.equal(seen["grad"], ref_ws[1].grad)
    for wa, wb in zip(ws, ref_ws):
        assert torch.equal(wa.grad, wb.grad)


def test_deferred_inside_graph_capture_replays():
    """A whole forward + backward captured in a HIP graph with deferral on: every replay
    rewrites the same .grad bits as the eager pass."""
    nr = _nr()
    g = gen(6)
    w = torch.nn.Parameter((1 + 0.02 * torch.randn(H, generator=g)).to(DEV))
    x = randn((512, H), g, dtype=torch.bfloat16).requires_grad_()
    gy = randn((512, H), g, dtype=torch.bfloat16)

    def step():
        w.grad = None
        y = nr.rmsnorm(x, w, EPS)
        (y.float() * gy.float()).sum().backward()

    step()
    torch.cuda.synchronize()
    eager = w.grad.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    w.grad = None
    with torch.cuda.graph(graph):
        y = nr.rmsnorm(x, w, EPS)
        (y.float() * gy.float()).sum().backward()
    captured = w.grad
    for _ in range(3):
        captured.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager)


@pytest.mark.parametrize("kind", ["scaled", "stacked_row", "exp"])
def test_derived_weight_gets_the_chain_rule(kind):
    """A weight computed from a parameter (p * 0.5, a row of a stacked [3, H] parameter, exp(p))
    is not the parameter or its cast: its gradient goes through autograd per call, so .grad is the
    same with deferral on and off, and equals the chain rule of the fp64 oracle's dw."""
    nr = _nr()
    g = gen(21)
    x = randn((300, H), g, dtype=torch.bfloat16)
    gy = randn((300, H), g, dtype=torch.bfloat16)
    base = (1 + 0.02 * torch.randn(3, H, generator=g)) if kind == "stacked_row" else \
        (1 + 0.02 * torch.randn(H, generator=g))
    grads, w_eff = [], None
    for defer in (True, False):
        p = torch.nn.Parameter(base.clone().to(DEV))
        w_eff = {"scaled": lambda: p * 0.5, "stacked_row": lambda: p[1],
                 "exp": lambda: p.exp()}[kind]()
        old = nr.DEFER_WEIGHT_GRAD
        nr.DEFER_WEIGHT_GRAD = defer
        try:
            (nr.rmsnorm(x, w_eff, EPS).float() * gy.float()).sum().backward()
        finally:
            nr.DEFER_WEIGHT_GRAD = old
        torch.cuda.synchronize()
        grads.append(p.grad.clone())
    assert torch.equal(grads[0], grads[1])
    _, dw64 = ref.rmsnorm_bwd(np64(gy), np64(x), np64(w_eff.detach()), EPS)
    if kind == "scaled":
        want = 0.5 * dw64
    elif kind == "exp":
        want = dw64 * np64(w_eff.detach())
    else:
        want = np.zeros((3, H))
        want[1] = dw64
    assert_close(np64(grads[0]), want, 1e-4 * np.abs(want).max(), 1e-4, "grad")


def test_pass_that_raises_drops_its_partials():
    """A backward pass that raises after a norm deferred its partials (the failing node is
    upstream of the norm) leaves nothing queued once the pass is gone, and the next pass gives
    the per-call gradient."""
    import gc
    import time

    nr = _nr()

    class Boom(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x):
            return x.clone()

        @staticmethod
        def backward(ctx, g):
            raise RuntimeError("planted failure upstream of the norm")

    g = gen(22)
    w = torch.nn.Parameter((1 + 0.02 * torch.randn(H, generator=g)).to(DEV))
    x = randn((256, H), g, dtype=torch.bfloat16).requires_grad_()
    gy = randn((256, H), g, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="planted failure"):
        (nr.rmsnorm(Boom.apply(x), w, EPS).float() * gy.float()).sum().backward()
    for _ in range(100):  # the engine releases the failed pass (and its callbacks) on its own
        gc.collect()
        if not nr._deferred:
            break
        time.sleep(0.01)
    assert not nr._deferred
    assert w.grad is None
    (nr.rmsnorm(x, w, EPS).float() * gy.float()).sum().backward()
    torch.cuda.synchronize()
    assert not nr._deferred
    wr = torch.nn.Parameter(w.detach().clone())
    old = nr.DEFER_WEIGHT_GRAD
    nr.DEFER_WEIGHT_GRAD = False
    try:
        (nr.rmsnorm(x, wr, EPS).float() * gy.float()).sum().backward()
    finally:
        nr.DEFER_WEIGHT_GRAD = old
    assert torch.equal(w.grad, wr.grad)


def test_deferral_falls_back_when_the_engine_callback_fails(monkeypatch):
    """If queueing the end-of-pass callback fails, the norm reduces its own partials and returns
    dw through autograd: the same bits as the per-call path."""
    nr = _nr()

    real = torch.autograd.Variable._execution_engine

    class Engine:
        """The real engine, except that it refuses end-of-pass callbacks."""

        def __getattr__(self, name):
            return getattr(real, name)

        def queue_callback(self, cb):
            raise RuntimeError("no callbacks here")

    g = gen(23)
    w = torch.nn.Parameter((1 + 0.02 * torch.randn(H, generator=g)).to(DEV))
    x = randn((256, H), g, dtype=torch.bfloat16)
    gy = randn((256, H), g, dtype=torch.bfloat16)
    wr = torch.nn.Parameter(w.detach().clone())
    old = nr.DEFER_WEIGHT_GRAD
    nr.DEFER_WEIGHT_GRAD = False
    try:
        (nr.rmsnorm(x, wr, EPS).float() * gy.float()).sum().backward()
    finally:
        nr.DEFER_WEIGHT_GRAD = old
    monkeypatch.setattr(torch.autograd.Variable, "_execution_engine", Engine())
    (nr.rmsnorm(x, w, EPS).float() * gy.float()).sum().backward()
    torch.cuda.synchronize()
    assert not nr._deferred
    assert torch.equal(w.grad, wr.grad)
