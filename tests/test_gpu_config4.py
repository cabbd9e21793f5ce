"""Config 4 (the graded workload: Qwen2.5-1.5B training-step shape, bf16, T = 8192 tokens,
hidden 1536, 12 / 2 heads of 128, padded [8, 1024] layout with implicit positions) at full size,
launched exactly as bench.py launches it: bench.Body's tensors and C-ABI calls.

Checked against the CPU oracle (oracle/norm_rope_ref.py):
  y, dx   64 sampled rows (the first and the last among them), atol 2e-3 / rtol 1e-2 against
          the fp64 oracle (the north-star bar for 16-bit outputs)
  dw      all 8192 rows against the fp64 sum, relative 1e-5 of max |dw| (fp32 accumulation)
  RoPE    64 sampled tokens of q / k forward (sign +1) and dq / dk backward (sign -1), positions
          s = 0..1023 of each padded row, atol 2e-3 / rtol 1e-2
"""

import numpy as np
import pytest
import torch

from _util import DEV, assert_close, gen, np64
from oracle import norm_rope_ref as ref

pytestmark = pytest.mark.gpu

TOL_A, TOL_R = 2e-3, 1e-2


def _bench():
    import bench

    return bench


def _sample_rows(T, k=64, seed=4):
    rows = torch.randint(0, T, (k - 2,), generator=gen(seed)).tolist()
    return sorted(set([0, T - 1] + rows))


def _check_norm(body, i, rows, eps):
    x, w, y, dy, dx, dw = (body.x[i], body.w[i], body.y[i], body.dy[i], body.dx[i], body.dw[i])
    xs, dys, wn = np64(x[rows]), np64(dy[rows]), np64(w)
    y64, rstd64 = ref.rmsnorm_fwd(xs, wn, eps, "bf16")
    assert_close(np64(y[rows]), y64, TOL_A, TOL_R, f"norm {i}: y")
    if body.rstd[i] is not None:
        assert_close(np64(body.rstd[i][rows]), rstd64, 0, 1e-6, f"norm {i}: rstd")
    dx64, _ = ref.rmsnorm_bwd(dys, xs, wn, eps)
    assert_close(np64(dx[rows]), ref.round_to(dx64, "bf16"), TOL_A, TOL_R, f"norm {i}: dx")
    _, dw64 = ref.rmsnorm_bwd(np64(dy), np64(x), wn, eps)
    assert_close(np64(dw), dw64, 1e-5 * np.abs(dw64).max(), 1e-5, f"norm {i}: dw")


def _check_rope(body, l, tokens, inv_freq):
    B, S = body.cfg["B"], body.cfg["S"]
    b_idx = [t // S for t in tokens]
    s_idx = [t % S for t in tokens]
    pos = np.asarray(s_idx)
    f = inv_freq.cpu().numpy()
    for src, out, sign, what in ((body.q[l], body.qo[l], 1.0, "q"), (body.k[l], body.ko[l], 1.0, "k"),
                                 (body.dqo[l], body.dq[l], -1.0, "dq"),
                                 (body.dko[l], body.dk[l], -1.0, "dk")):
        xin = np64(src[b_idx, s_idx])            # [tokens, H, D]
        want = ref.rope_fwd(xin, pos, f, sign, store="bf16")
        assert_close(np64(out[b_idx, s_idx]), want, TOL_A, TOL_R, f"rope layer {l}: {what}")


@pytest.mark.parametrize("rstd", ["saved", "recomputed"])
def test_config4_two_layers_through_bench_body(rstd):
    """Two decoder layers of config 4 through bench.Body.step (input norm, q/k RoPE and
    post-attention norm per layer, then the final norm; forward then backward with dx, dw,
    dq, dk), every output checked against the oracle."""
    bench = _bench()
    cfg = dict(bench.CFG4, layers=2)
    torch.cuda.synchronize()
    body = bench.Body(cfg, rstd == "saved", torch.device(DEV))
    body.step()
    torch.cuda.synchronize()
    T = body.T
    assert T == 8192 and body.x[0].dtype == torch.bfloat16
    rows = _sample_rows(T)
    for i in range(2 * cfg["layers"] + 1):
        _check_norm(body, i, rows, cfg["eps"])
    for l in range(cfg["layers"]):
        _check_rope(body, l, rows, body.inv_freq)


def test_config4_deferred_dgamma_equals_per_call():
    """The bench's deferred weight-gradient schedule (every norm backward keeps its partials,
    one esep_dgamma_reduce_batch after the sweep) gives the per-call dw bit for bit, and the
    same dx."""
    bench = _bench()
    cfg = dict(bench.CFG4, layers=1)
    dev = torch.device(DEV)
    fused = bench.Body(cfg, True, dev, deferred_dgamma=False)
    batched = bench.Body(cfg, True, dev, deferred_dgamma=True)
    fused.step()
    batched.step()
    torch.cuda.synchronize()
    for i in range(2 * cfg["layers"] + 1):
        assert torch.equal(fused.x[i], batched.x[i])  # same seeded inputs
        assert torch.equal(fused.dw[i], batched.dw[i]), i
        assert torch.equal(fused.dx[i], batched.dx[i]), i


def test_config4_recomputed_rstd_equals_saved():
    """The bench's two rstd legs at config 4 (one layer, deferred weight gradient): the
    backward's form for rstd recomputed from x (dx only, with the weight gradient) gives the
    saved-rstd form's dx and dw bit for bit, since it recomputes rstd with the forward's own
    arithmetic."""
    bench = _bench()
    cfg = dict(bench.CFG4, layers=1)
    dev = torch.device(DEV)
    saved = bench.Body(cfg, True, dev)
    recomputed = bench.Body(cfg, False, dev)
    saved.step()
    recomputed.step()
    torch.cuda.synchronize()
    for i in range(2 * cfg["layers"] + 1):
        assert recomputed.rstd[i] is None and saved.rstd[i] is not None
        assert torch.equal(saved.x[i], recomputed.x[i])  # same seeded inputs
        assert torch.equal(saved.y[i], recomputed.y[i]), i
        assert torch.equal(saved.dx[i], recomputed.dx[i]), i
        assert torch.equal(saved.dw[i], recomputed.dw[i]), i


def test_config4_norm_api_full_size():
    """The public rmsnorm() API at config 4's norm shape ([8, 1024, 1536] bf16, trainable fp32
    weight 1 + 0.02 N(0, 1)): y and dx on sampled rows, dw over all rows."""
    from solution.body import norm_rope

    g = torch.Generator(device=DEV).manual_seed(40)
    x = torch.randn(8, 1024, 1536, generator=g, device=DEV).to(torch.bfloat16).requires_grad_()
    w = (1 + 0.02 * torch.randn(1536, generator=g, device=DEV)).requires_grad_()
    dy = torch.randn(8, 1024, 1536, generator=g, device=DEV).to(torch.bfloat16)
    y = norm_rope.rmsnorm(x, w, 1e-6)
    dx, dw = torch.autograd.grad(y, [x, w], dy)
    x2, y2, dy2, dx2 = (t.reshape(-1, 1536) for t in (x, y, dy, dx))
    rows = _sample_rows(8192, seed=41)
    y64, _ = ref.rmsnorm_fwd(np64(x2[rows]), np64(w), 1e-6, "bf16")
    assert_close(np64(y2[rows]), y64, TOL_A, TOL_R, "y")
    dx64, _ = ref.rmsnorm_bwd(np64(dy2[rows]), np64(x2[rows]), np64(w), 1e-6)
    assert_close(np64(dx2[rows]), ref.round_to(dx64, "bf16"), TOL_A, TOL_R, "dx")
    _, dw64 = ref.rmsnorm_bwd(np64(dy2), np64(x2), np64(w), 1e-6)
    assert_close(np64(dw), dw64, 1e-5 * np.abs(dw64).max(), 1e-5, "dw")
