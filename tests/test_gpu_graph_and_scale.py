"""HIP-graph capture of the C-ABI launches, and the config-5 stress shape at full size.

Graphs: the norm forward, the norm backward with its weight-gradient reduction (per call, and
two calls' partials reduced by one batched launch) and both RoPE directions, captured once and replayed several times with other GPU work and host syncs in
between; every replay must equal the eager launches bit for bit (the library records no
memset and allocates nothing, so replays are self-contained).

Config 5 (T = 65536 packed tokens, H = 3584, 28 / 4 heads, varlen U[128, 4096]): too large for
the fp64 oracle as a whole, so it is checked through properties that do not depend on size:
sampled rows against the oracle, the weight gradient on sampled columns against its closed form
summed over all rows in fp64 and as the sum of its halves (linearity over rows), cu_seqlens
positions equal to explicit positions bitwise, and RoPE forward-then-backward returning the
input."""

import numpy as np
import pytest
import torch

from _util import DEV, assert_close, gen, np64
from oracle import norm_rope_ref as ref

pytestmark = pytest.mark.gpu

EPS = 1e-6


def test_graph_replays_match_eager():
    from solution.body import _hip

    T, H, HQ, HK, D = 4096, 1536, 12, 2, 128
    g = torch.Generator(device=DEV).manual_seed(3)

    def rn(*s):
        return torch.randn(s, generator=g, device=DEV).to(torch.bfloat16)

    x, dy = rn(T, H), rn(T, H)
    w = 1 + 0.02 * torch.randn(H, generator=g, device=DEV)
    q, k, dq_in, dk_in = rn(1, T, HQ, D), rn(1, T, HK, D), rn(1, T, HQ, D), rn(1, T, HK, D)
    inv = (1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float) / D))).to(DEV)
    cu = torch.tensor([0, 1000, 1001, 3000, T], dtype=torch.int32, device=DEV)
    ws = torch.empty(_hip.rmsnorm_partials(T, H), H, device=DEV)
    # two norm backwards keeping their partials, reduced by one batched launch
    dy2 = rn(T, H)
    parts = [torch.empty(_hip.rmsnorm_partials(T, H), H, device=DEV) for _ in range(2)]

    def outputs():
        return dict(y=torch.empty_like(x), rstd=torch.empty(T, device=DEV),
                    dx=torch.empty_like(x), dw=torch.empty(H, device=DEV),
                    qo=torch.empty_like(q), ko=torch.empty_like(k),
                    dq=torch.empty_like(q), dk=torch.empty_like(k),
                    dx2=torch.empty_like(x), dwb0=torch.empty(H, device=DEV),
                    dwb1=torch.empty(H, device=DEV))

    def run(o):
        _hip.rmsnorm_fwd(x, w, o["y"], EPS, rstd=o["rstd"])
        _hip.rmsnorm_bwd([dy], x, w, EPS, rstd=o["rstd"], dx=o["dx"], dw=o["dw"], workspace=ws)
        _hip.rope(q, k, o["qo"], o["ko"], inv, 1.0, cu_seqlens=cu)
        _hip.rope(dq_in, dk_in, o["dq"], o["dk"], inv, -1.0, cu_seqlens=cu)
        _hip.rmsnorm_bwd([dy], x, w, EPS, rstd=o["rstd"], dx=o["dx"], partials=parts[0])
        _hip.rmsnorm_bwd([dy2], x, w, EPS, rstd=o["rstd"], dx=o["dx2"], partials=parts[1])
        _hip.dgamma_reduce_batch(parts, [o["dwb0"], o["dwb1"]])

    eager = outputs()
    run(eager)
    torch.cuda.synchronize()
    assert torch.equal(eager["dwb0"], eager["dw"])  # batched stage 2 == the fused call's
    graphed = outputs()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(graphed)  # warm-up on a side stream, as torch recommends before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(graphed)
    for rep in range(4):
        for t in graphed.values():
            t.fill_(float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name in eager:
            assert torch.equal(graphed[name], eager[name]), (rep, name)


def _config5():
    import bench

    return bench.CFG5, bench.config5_lengths(bench.CFG5)


def _dw_columns_fp64(x, dy, w, cols, chunk=8192):
    """The weight gradient's closed form on columns `cols`, over every row, in fp64 on the CPU:
    dw_j = sum_t dy_tj * x_tj * rstd_t with each row's rstd from the oracle's forward on the
    whole row (chunks of rows), and the column sums from the oracle's backward given that rstd."""
    T = x.shape[0]
    wn = np64(w)
    out = np.zeros(len(cols))
    for t0 in range(0, T, chunk):
        xc = np64(x[t0:t0 + chunk])
        _, rstd = ref.rmsnorm_fwd(xc, wn, EPS)
        _, dw = ref.rmsnorm_bwd(np64(dy[t0:t0 + chunk, cols]), xc[:, cols], wn[cols], EPS, rstd=rstd)
        out += dw
    return out


def test_config5_rmsnorm_full_size():
    from solution.body import norm_rope

    cfg, _ = _config5()
    T, H = cfg["T"], cfg["H"]
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(T, H, generator=g, device=DEV).to(torch.bfloat16).requires_grad_()
    w = (1 + 0.02 * torch.randn(H, generator=g, device=DEV)).requires_grad_()
    dy = torch.randn(T, H, generator=g, device=DEV).to(torch.bfloat16)
    y = norm_rope.rmsnorm(x, w, EPS)
    dx, dw = torch.autograd.grad(y, [x, w], dy)
    rows = torch.randint(0, T, (48,), generator=gen(1)).tolist() + [0, T - 1]
    xs, dys, wn = np64(x[rows]), np64(dy[rows]), np64(w)
    y64, _ = ref.rmsnorm_fwd(xs, wn, EPS, "bf16")
    dx64, _ = ref.rmsnorm_bwd(dys, xs, wn, EPS)
    assert_close(np64(y[rows]), y64, 2e-3, 1e-2, "sampled y")
    assert_close(np64(dx[rows]), dx64, 2e-3, 1e-2, "sampled dx")
    # linearity over rows: dw(all) = dw(first half) + dw(second half), up to fp32 summation
    h = T // 2
    parts = []
    for sl in (slice(0, h), slice(h, T)):
        xh = x.detach()[sl].clone().requires_grad_()
        parts.append(torch.autograd.grad(norm_rope.rmsnorm(xh, w, EPS), [w], dy[sl])[0])
    both = (parts[0].double() + parts[1].double()).cpu().numpy()
    assert_close(np64(dw), both, 1e-4 * np.abs(both).max(), 1e-4, "dw halves")
    # and the same call twice gives the same bits
    dw2 = torch.autograd.grad(norm_rope.rmsnorm(x, w, EPS), [w], dy)[0]
    assert torch.equal(dw, dw2)
    # 64 sampled columns against the closed form summed over all 65536 rows in fp64
    cols = sorted(set([0, H - 1] + torch.randint(0, H, (62,), generator=gen(3)).tolist()))
    want = _dw_columns_fp64(x.detach(), dy, w.detach(), cols)
    assert_close(np64(dw)[cols], want, 1e-5 * np.abs(want).max(), 1e-5, "dw columns vs fp64")


def test_config5_bench_norm_backward_weight_gradient():
    """The bench's own config-5 launch (bench.Stress: the C ABI with a workspace, 512 partial
    rows, the wide kernel) against the weight gradient's closed form in fp64 on 64 columns over
    all rows, and its dx on sampled rows against the oracle."""
    import bench

    cfg = bench.CFG5
    st = bench.Stress(cfg, torch.device(DEV))
    from solution.body import _hip

    assert st.ws.shape[0] == _hip.rmsnorm_partials(cfg["T"], cfg["H"]) == 512
    st.norm_fwd()
    st.norm_bwd()
    torch.cuda.synchronize()
    T, H = cfg["T"], cfg["H"]
    cols = sorted(set([0, H - 1] + torch.randint(0, H, (62,), generator=gen(4)).tolist()))
    want = _dw_columns_fp64(st.x, st.dy, st.w, cols)
    assert_close(np64(st.dw)[cols], want, 1e-5 * np.abs(want).max(), 1e-5, "bench dw vs fp64")
    rows = torch.randint(0, T, (32,), generator=gen(6)).tolist() + [0, T - 1]
    dx64, _ = ref.rmsnorm_bwd(np64(st.dy[rows]), np64(st.x[rows]), np64(st.w), EPS)
    assert_close(np64(st.dx[rows]), ref.round_to(dx64, "bf16"), 2e-3, 1e-2, "bench dx")
    del st
    torch.cuda.empty_cache()


def test_config5_rope_full_size():
    from solution.body import norm_rope

    cfg, lens = _config5()
    assert len(lens) == 29 and lens[-1] == 249 and sum(lens) == cfg["T"]
    T, HQ, HK, D = cfg["T"], cfg["HQ"], cfg["HK"], cfg["D"]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    pos = torch.from_numpy(ref.positions_from_cu_seqlens(cu.cpu().numpy())).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(6)
    q = torch.randn(T, HQ, D, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(T, HK, D, generator=g, device=DEV).to(torch.bfloat16)
    inv = norm_rope.default_inv_freq(D, cfg["theta"], DEV)
    a = norm_rope.rope(q, k, None, inv, cu_seqlens=cu)
    b = norm_rope.rope(q, k, pos, inv)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    rows = torch.randint(0, T, (64,), generator=gen(2)).tolist() + [0, T - 1]
    f = inv.cpu().numpy()
    p = pos.cpu().numpy()[rows]
    assert_close(np64(a[0][rows]), ref.rope_fwd(np64(q[rows]), p, f, store="bf16"), 2e-3, 1e-2, "q")
    assert_close(np64(a[1][rows]), ref.rope_fwd(np64(k[rows]), p, f, store="bf16"), 2e-3, 1e-2, "k")
    qf = q.float().requires_grad_()
    kf = k.float().requires_grad_()
    qo, ko = norm_rope.rope(qf, kf, None, inv, cu_seqlens=cu)
    back = torch.autograd.grad([qo, ko], [qf, kf], [qo.detach(), ko.detach()])
    assert_close(np64(back[0][rows]), np64(qf[rows]), 1e-5, 1e-5, "roundtrip q")
    assert_close(np64(back[1][rows]), np64(kf[rows]), 1e-5, 1e-5, "roundtrip k")
