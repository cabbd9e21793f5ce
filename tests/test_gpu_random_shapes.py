"""Seeded random shapes through the public API of the three operations (norm, RoPE, varlen
attention), each case against the fp64 CPU oracle at the bars of the fixed-shape tests:

  rmsnorm   y, dx atol 2e-3 / rtol 1e-2 (16-bit) or 1e-5 (fp32); dw 1e-4 of max |dw|
  rope      q, k forward (sign +1) and dq, dk backward (sign -1), the same bars as rmsnorm's y
  attention o within atol 1e-2 (bf16) / 2e-3 (fp16) + rtol 1e-2; dq, dk, dv within that atol
            times the gradient's largest magnitude + rtol 1e-2 + 1e-5

The shapes are drawn per case from numpy's default_rng(seed) (the case id is the seed), so a
failure names a reproducible case: ragged widths and lengths, empty sequences, a max_seqlen
larger than the longest sequence, odd query-head groups. ESEP_RANDOM_SHAPES_SCALE=k runs k times
as many seeds per operation (a wider sweep by hand; 1 by default)."""

import os

import numpy as np
import pytest
import torch

from _util import DEV, STORE, assert_close, err, np64
from oracle import attention_ref as aref
from oracle import norm_rope_ref as ref

pytestmark = pytest.mark.gpu

SCALE = max(1, int(os.environ.get("ESEP_RANDOM_SHAPES_SCALE", "1")))


def _seeds(first, count):
    """Case seeds: count per operation, scaled; the scaled ones continue past the defaults'
    range of every operation (10000 apart)."""
    return list(range(first, first + count)) + [first + 10000 + i for i in range(count * (SCALE - 1))]


EPS = 1e-6
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def _nr():
    from solution.body import norm_rope

    return norm_rope


def _tensor(rng, shape, dtype, scale=1.0):
    return torch.from_numpy(rng.standard_normal(shape) * scale).to(torch.float32).to(dtype).to(DEV)


def _norm_case(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.choice([int(rng.integers(1, 200)), int(rng.integers(200, 4097)),
                        int(rng.integers(4097, 16385)), 1536, 3584]))
    rows = int(rng.integers(1, max(2, min(2500, 4_000_000 // n))))
    dtype = DTYPES[int(rng.integers(3))]
    recompute = bool(rng.integers(2))
    return rng, rows, n, dtype, recompute


@pytest.mark.parametrize("seed", _seeds(100, 16))
def test_random_rmsnorm(seed):
    nr = _nr()
    rng, rows, n, dtype, recompute = _norm_case(seed)
    # half the cases read x as a column slice of a wider buffer: a row stride above n, and an
    # offset that may leave the rows without 16-byte alignment (the element-wise kernels)
    pad, off = (int(rng.integers(0, 40)), int(rng.integers(0, 9))) if rng.integers(2) else (0, 0)
    print(f"seed {seed}: rows={rows} n={n} {dtype} recompute_rstd={recompute} "
          f"row pad={pad} offset={off}")
    if pad or off:
        buf = _tensor(rng, (rows, n + pad + off), dtype).requires_grad_()
        x = buf[:, off:off + n]
    else:
        x = _tensor(rng, (rows, n), dtype).requires_grad_()
    w = (1 + 0.02 * _tensor(rng, (n,), torch.float32)).requires_grad_()
    dy = _tensor(rng, (rows, n), dtype)
    y = nr.rmsnorm(x, w, EPS, recompute_rstd=recompute)
    dx, dw = torch.autograd.grad(y, [x, w], dy)
    y64, _ = ref.rmsnorm_fwd(np64(x), np64(w), EPS, STORE[dtype])
    dx64, dw64 = ref.rmsnorm_bwd(np64(dy), np64(x), np64(w), EPS)
    lp = dtype != torch.float32
    atol, rtol = (2e-3, 1e-2) if lp else (1e-5, 1e-5)
    assert_close(np64(y), y64, atol, rtol, "y")
    assert_close(np64(dx), ref.round_to(dx64, STORE[dtype]), atol, rtol, "dx")
    assert_close(np64(dw), dw64, 1e-4 * np.abs(dw64).max(), 1e-4, "dw")


@pytest.mark.parametrize("seed", _seeds(400, 12))
def test_random_add_rmsnorm(seed):
    """The reference API's add_rmsnorm (residual add, fan-out, save_output) on random shapes:
    r_out exact, y at the bar above; d_r_in, d_delta and the weight's gradient against the fp64
    closed form (relative 2e-3 / 5e-3 of their largest magnitude on the saved-y backward, as its
    fixed-shape tests, 8 times that for a bf16 y). A delta of the other 16-bit type than y's
    exercises the backward kernel's mixed forms (x and dy fp16, dx bf16 and the reverse)."""
    nr = _nr()
    rng = np.random.default_rng(seed)
    n = int(rng.choice([int(rng.integers(1, 300)), int(rng.integers(300, 16385)), 1536, 3584]))
    T = int(rng.integers(1, max(2, min(2000, 3_000_000 // n))))
    delta_dt = [None, torch.float16, torch.bfloat16, torch.float32][int(rng.integers(4))]
    out_dt = DTYPES[int(rng.integers(3))]
    n_out = int(rng.integers(1, 4))
    save_output = bool(rng.integers(2))
    print(f"seed {seed}: T={T} n={n} delta {delta_dt} y {out_dt} n_out={n_out} "
          f"save_output={save_output}")
    r_in = _tensor(rng, (T, n), torch.float32, 3.0).requires_grad_()
    delta = None if delta_dt is None else _tensor(rng, (T, n), delta_dt).requires_grad_()
    w = torch.nn.Parameter(1 + 0.1 * _tensor(rng, (n,), torch.float32))
    r_out, ys = nr.add_rmsnorm(r_in, delta, w, EPS, out_dt, n_out=n_out, save_output=save_output)
    ys = (ys,) if n_out == 1 else ys
    d_np = None if delta is None else np64(delta)
    r64, y64, _, _ = ref.add_rmsnorm_fwd(np64(r_in), d_np, np64(w.detach()), EPS, STORE[out_dt])
    assert_close(np64(r_out), r64, 0, 0, "r_out")
    lp = out_dt != torch.float32
    assert_close(np64(ys[0]), y64, 2e-3 if lp else 1e-5, 1e-2 if lp else 1e-5, "y")
    gys = [_tensor(rng, (T, n), out_dt) for _ in range(n_out)]
    gr = _tensor(rng, (T, n), torch.float32)
    torch.autograd.backward([r_out, *ys], [gr, *gys])
    dr64, dw64 = ref.add_rmsnorm_bwd([np64(g) for g in gys], np64(gr), r64, np64(w.detach()), EPS)
    from_y = save_output and delta is not None and lp  # the backward from the saved y
    # xhat = y / w there: the bars of the fp16 tests, 8x for a bf16 y (3 fewer mantissa bits)
    yk = 8 if out_dt == torch.bfloat16 else 1
    if from_y:
        assert err(np64(r_in.grad), dr64)[1] < 2e-3 * yk
        assert err(np64(delta.grad), dr64)[1] < 5e-3 * yk
    else:
        assert_close(np64(r_in.grad), dr64, 1e-4 * np.abs(dr64).max(), 1e-4, "d_r_in")
        if delta is not None:
            assert_close(np64(delta.grad), ref.round_to(dr64, STORE[delta_dt]),
                         2e-3 * np.abs(dr64).max() if delta_dt != torch.float32 else 1e-5,
                         1e-2 if delta_dt != torch.float32 else 1e-4, "d_delta")
    assert_close(np64(w.grad), dw64, 2e-3 * yk * np.abs(dw64).max() if from_y else
                 1e-4 * np.abs(dw64).max(), 1e-4, "w.grad")


@pytest.mark.parametrize("seed", _seeds(450, 10))
def test_random_deferred_weight_grad_graphs(seed):
    """Random chains of rmsnorm / add_rmsnorm calls over a small pool of trainable weights (so
    that a weight is shared by several norms of one pass), fp32 or bf16 parameters, some calls
    on a derived weight (p * 0.5: autograd's chain rule, per call), one loss.backward(): the
    inputs' gradients bit for bit, a weight used by one norm bit for bit, and a shared weight's
    .grad within the rounding of summing its contributions in another order (autograd fixes no
    order: the deferred ones are added at the end of the pass, the engine adds the per-call
    ones as they arrive): |deferred - per call| <= uses * eps(dtype) * sum |contribution|, the
    contributions measured in a third run with each use on a weight tensor of its own."""
    nr = _nr()
    rng = np.random.default_rng(seed)
    n = [64, 1000, 1536, 3584][int(rng.integers(4))]
    T = int(rng.integers(1, 400))
    n_params = int(rng.integers(1, 4))
    p_dt = [torch.float32, torch.bfloat16][int(rng.integers(2))]
    calls = [(int(rng.integers(2)), int(rng.integers(n_params)), bool(rng.random() < 0.2),
              bool(rng.integers(2))) for _ in range(int(rng.integers(2, 7)))]
    print(f"seed {seed}: n={n} T={T} params={n_params} {p_dt} calls (add, param, derived, chain) "
          f"{calls}")
    w0 = [1 + 0.02 * _tensor(rng, (n,), torch.float32) for _ in range(n_params)]
    x0 = _tensor(rng, (T, n), torch.bfloat16)
    r0 = _tensor(rng, (T, n), torch.float32, 2.0)
    proj = [_tensor(rng, (T, n), torch.float32) for _ in calls]

    def run(defer, separate=False):
        old = nr.DEFER_WEIGHT_GRAD
        nr.DEFER_WEIGHT_GRAD = defer
        try:
            ps = [torch.nn.Parameter(w.to(p_dt)) for w in w0]
            x, r = x0.clone().requires_grad_(), r0.clone().requires_grad_()
            h, res, loss, uses = x, r, 0.0, []
            for (add, pi, derived, chain), pj in zip(calls, proj):
                base = ps[pi] * 1.0 if separate else ps[pi]  # a tensor of its own per use
                uses.append((pi, base))
                w = base * 0.5 if derived else base
                inp = h if chain else x
                if add:
                    res, y = nr.add_rmsnorm(res, inp, w, EPS, torch.bfloat16)
                else:
                    y = nr.rmsnorm(inp, w, EPS)
                h = y.to(torch.bfloat16)
                loss = loss + (y.float() * pj).sum()
            if separate:
                return uses, torch.autograd.grad(loss, [b for _, b in uses])
            loss.backward()
            torch.cuda.synchronize()
            return [p.grad for p in ps], x.grad, r.grad
        finally:
            nr.DEFER_WEIGHT_GRAD = old

    gd, xd, rd = run(True)
    gp, xp, rp = run(False)
    uses, contrib = run(False, separate=True)
    eps = {torch.float32: 2.0 ** -23, torch.bfloat16: 2.0 ** -8}[p_dt]
    for i, (a, b) in enumerate(zip(gd, gp)):
        mine = [c.float() for (pi, _), c in zip(uses, contrib) if pi == i]
        assert (a is None) == (b is None) == (not mine)
        if a is None:
            continue
        assert a.dtype == p_dt
        if len(mine) == 1:
            assert torch.equal(a, b)
        else:
            bound = len(mine) * eps * torch.stack(mine).abs().sum(0)
            assert torch.all((a.float() - b.float()).abs() <= bound), \
                ((a.float() - b.float()).abs() - bound).max().item()
    for a, b in ((xd, xp), (rd, rp)):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(a, b)


def _lengths(rng, n_seq, hi, p_empty=0.15):
    lens = [0 if rng.random() < p_empty else int(rng.integers(1, hi)) for _ in range(n_seq)]
    if max(lens) == 0:
        lens[0] = int(rng.integers(1, hi))
    return lens


@pytest.mark.parametrize("seed", _seeds(200, 12))
def test_random_rope(seed):
    nr = _nr()
    rng = np.random.default_rng(seed)
    hq, hk = [(12, 2), (28, 4), (4, 4), (6, 1), (16, 8)][int(rng.integers(5))]
    d = [64, 128, 256][int(rng.integers(3))]
    dtype = DTYPES[int(rng.integers(3))]
    kind = ["positions", "cu_seqlens", "large_positions"][int(rng.integers(3))]
    inv_freq = nr.default_inv_freq(d, 1e6, DEV)
    if kind == "cu_seqlens":
        lens = _lengths(rng, int(rng.integers(1, 12)), 600)
        cu = torch.tensor(aref.cu_from_lengths(lens), dtype=torch.int32)
        pos_np = ref.positions_from_cu_seqlens(cu.numpy())
        T = int(cu[-1])
    else:
        T = int(rng.integers(1, 3000))
        top = 32768 if kind == "large_positions" else 1024
        pos_np = rng.integers(0, top, T).astype(np.int64)
    print(f"seed {seed}: T={T} heads {hq}/{hk} D={d} {dtype} {kind}")
    q = _tensor(rng, (T, hq, d), dtype).requires_grad_()
    k = _tensor(rng, (T, hk, d), dtype).requires_grad_()
    if kind == "cu_seqlens":
        qo, ko = nr.rope(q, k, None, inv_freq, cu_seqlens=cu.to(DEV))
    else:
        qo, ko = nr.rope(q, k, torch.from_numpy(pos_np).to(DEV), inv_freq)
    f = inv_freq.cpu().numpy()
    lp = dtype != torch.float32
    atol, rtol = (2e-3, 1e-2) if lp else (1e-5, 1e-5)
    assert_close(np64(qo), ref.rope_fwd(np64(q), pos_np, f, store=STORE[dtype]), atol, rtol, "q")
    assert_close(np64(ko), ref.rope_fwd(np64(k), pos_np, f, store=STORE[dtype]), atol, rtol, "k")
    gq, gk = _tensor(rng, qo.shape, dtype), _tensor(rng, ko.shape, dtype)
    dq, dk = torch.autograd.grad([qo, ko], [q, k], [gq, gk])
    assert_close(np64(dq), ref.rope_fwd(np64(gq), pos_np, f, -1.0, store=STORE[dtype]), atol, rtol,
                 "dq")
    assert_close(np64(dk), ref.rope_fwd(np64(gk), pos_np, f, -1.0, store=STORE[dtype]), atol, rtol,
                 "dk")


@pytest.mark.parametrize("seed", _seeds(500, 12))
def test_random_rope_layouts(seed):
    """rope on q / k sliced from one fused [T, (HQ + 2 HK) D] projection buffer, with or without
    the LoRA term q_delta (its gradient bitwise q's), and rope_bhsd on the padded [B, H, S, D]
    layout (contiguous or HF's transposed view; positions implicit, per row or one broadcast
    row), forward and backward against the oracle."""
    nr = _nr()
    rng = np.random.default_rng(seed)
    hq, hk = [(12, 2), (28, 4), (4, 4), (6, 1)][int(rng.integers(4))]
    d = [64, 128, 256][int(rng.integers(3))]
    dtype = DTYPES[int(rng.integers(3))]
    inv_freq = nr.default_inv_freq(d, 1e6, DEV)
    f = inv_freq.cpu().numpy()
    atol, rtol = (2e-3, 1e-2) if dtype != torch.float32 else (1e-5, 1e-5)
    st = STORE[dtype]
    if rng.integers(2):
        T = int(rng.integers(1, 2500))
        with_delta = bool(rng.integers(2))
        print(f"seed {seed}: fused qkv T={T} heads {hq}/{hk} D={d} {dtype} q_delta={with_delta}")
        qkv = _tensor(rng, (T, (hq + 2 * hk) * d), dtype).requires_grad_()
        qv = qkv[:, : hq * d].view(T, hq, d)
        kv = qkv[:, hq * d:(hq + hk) * d].view(T, hk, d)
        qd = _tensor(rng, (T, hq * d), dtype, 0.3).requires_grad_() if with_delta else None
        pos = rng.integers(0, 4096, T).astype(np.int64)
        qo, ko = nr.rope(qv, kv, torch.from_numpy(pos).to(DEV), inv_freq, qd)
        dq_np = None if qd is None else np64(qd)
        assert_close(np64(qo), ref.rope_fwd(np64(qv), pos, f, delta=dq_np, store=st), atol, rtol, "q")
        assert_close(np64(ko), ref.rope_fwd(np64(kv), pos, f, store=st), atol, rtol, "k")
        gq, gk = _tensor(rng, qo.shape, dtype), _tensor(rng, ko.shape, dtype)
        leaves = [qkv] + ([qd] if qd is not None else [])
        grads = torch.autograd.grad([qo, ko], leaves, [gq, gk])
        gqkv = grads[0]
        assert_close(np64(gqkv[:, : hq * d]).reshape(T, hq, d),
                     ref.rope_fwd(np64(gq), pos, f, -1.0, store=st), atol, rtol, "dq")
        assert_close(np64(gqkv[:, hq * d:(hq + hk) * d]).reshape(T, hk, d),
                     ref.rope_fwd(np64(gk), pos, f, -1.0, store=st), atol, rtol, "dk")
        assert not gqkv[:, (hq + hk) * d:].any()  # v's columns get no gradient
        if qd is not None:
            assert torch.equal(grads[1], gqkv[:, : hq * d])
        return
    B, S = int(rng.integers(1, 5)), int(rng.integers(1, 700))
    view = bool(rng.integers(2))
    pos_kind = ["implicit", "per_row", "broadcast"][int(rng.integers(3))]
    print(f"seed {seed}: bhsd B={B} S={S} heads {hq}/{hk} D={d} {dtype} hf_view={view} {pos_kind}")
    if view:
        q = _tensor(rng, (B, S, hq * d), dtype).requires_grad_()
        k = _tensor(rng, (B, S, hk * d), dtype).requires_grad_()
        qv, kv = q.view(B, S, hq, d).transpose(1, 2), k.view(B, S, hk, d).transpose(1, 2)
    else:
        q = _tensor(rng, (B, hq, S, d), dtype).requires_grad_()
        k = _tensor(rng, (B, hk, S, d), dtype).requires_grad_()
        qv, kv = q, k
    if pos_kind == "implicit":
        pid, posr = None, np.tile(np.arange(S), B)
    elif pos_kind == "per_row":
        p = rng.integers(0, 8192, (B, S)).astype(np.int64)
        pid, posr = torch.from_numpy(p).to(DEV), p.reshape(-1)
    else:
        p = rng.integers(0, 8192, (1, S)).astype(np.int64)
        pid, posr = torch.from_numpy(p).to(DEV), np.tile(p[0], B)
    qo, ko = nr.rope_bhsd(qv, kv, inv_freq, pid)

    def tok(t, h):  # [B, H, S, D] -> token-major [B S, H, D]
        return np64(t.transpose(1, 2)).reshape(B * S, h, d)

    def bhsd(a, h):
        return a.reshape(B, S, h, d).transpose(0, 2, 1, 3)

    assert_close(np64(qo), bhsd(ref.rope_fwd(tok(qv, hq), posr, f, store=st), hq), atol, rtol, "q")
    assert_close(np64(ko), bhsd(ref.rope_fwd(tok(kv, hk), posr, f, store=st), hk), atol, rtol, "k")
    gq, gk = _tensor(rng, tuple(qo.shape), dtype), _tensor(rng, tuple(ko.shape), dtype)
    dq, dk = torch.autograd.grad([qo, ko], [qv, kv], [gq, gk])
    assert_close(np64(dq), bhsd(ref.rope_fwd(tok(gq, hq), posr, f, -1.0, store=st), hq), atol, rtol,
                 "dq")
    assert_close(np64(dk), bhsd(ref.rope_fwd(tok(gk, hk), posr, f, -1.0, store=st), hk), atol, rtol,
                 "dk")


@pytest.mark.parametrize("seed", _seeds(300, 12))
def test_random_attention(seed):
    from solution.body import _hip

    rng = np.random.default_rng(seed)
    lens = _lengths(rng, int(rng.integers(1, 7)), 330)
    HQ, HK = [(2, 1), (4, 2), (6, 2), (8, 8), (12, 2), (7, 1)][int(rng.integers(6))]
    D = [64, 128][int(rng.integers(2))]
    dtype = [torch.bfloat16, torch.float16][int(rng.integers(2))]
    max_seqlen = max(lens) + int(rng.integers(0, 40))  # any bound >= the longest sequence
    print(f"seed {seed}: lengths {lens} heads {HQ}/{HK} D={D} {dtype} max_seqlen={max_seqlen}")
    T = sum(lens)
    q, do = _tensor(rng, (T, HQ, D), dtype), _tensor(rng, (T, HQ, D), dtype)
    k, v = _tensor(rng, (T, HK, D), dtype), _tensor(rng, (T, HK, D), dtype)
    cu = torch.tensor(aref.cu_from_lengths(lens), dtype=torch.int32)
    scale = D ** -0.5
    o = torch.full_like(q, float("nan"))
    lse = torch.full((HQ, T), float("nan"), device=DEV)
    _hip.attn_fwd(q, k, v, o, cu.to(DEV), max_seqlen, scale, lse=lse)
    dq, dk, dv = (torch.full_like(t, float("nan")) for t in (q, k, v))
    _hip.attn_bwd(q, k, v, o, do, lse, dq, dk, dv, cu.to(DEV), max_seqlen, scale)
    cu_np = cu.numpy()
    o64, lse64 = aref.attn_fwd(np64(q), np64(k), np64(v), cu_np, scale)
    atol = 1e-2 if dtype == torch.bfloat16 else 2e-3
    assert_close(np64(o), o64, atol, 1e-2, "o")
    np.testing.assert_allclose(np64(lse), lse64, atol=1e-4, rtol=1e-5)
    want = aref.attn_bwd(np64(q), np64(k), np64(v), np64(do), cu_np, scale)
    for name, got, w64 in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
        assert_close(np64(got), w64, atol * np.abs(w64).max() + 1e-5, 1e-2, name)
