"""Varlen causal attention on the GPU (esep_attn_fwd) against the float64 oracle
(oracle/attention_ref.py), which restates the reference decoder's per-row SDPA loop
(packed.py:404-436).

Tolerance against the float64 result computed from the same (rounded) inputs: fp16 outputs
within atol 2e-3 + rtol 1e-2; bf16 outputs within atol 1e-2 + rtol 1e-2 (the probabilities enter
the P V product in bf16, as in every bf16 flash kernel, so outputs near zero carry ~2^-9 of the
magnitude of v: torch's own bf16 SDPA misses 2e-3 there too); lse (fp32) within 1e-4. The error
is also compared with torch's SDPA on the GPU in the same dtype (the reference's kernel): our
largest error at most twice torch's largest, our mean error at most 1.5 times torch's mean."""

import numpy as np
import pytest
import torch

from _util import DEV, gen, np64
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

CASES = [
    ([1], 2, 2, 64),
    ([31, 33, 64, 65, 127, 128, 129, 200], 12, 2, 128),
    ([513, 7], 4, 2, 64),
    ([300, 1, 257], 28, 4, 128),
    ([96, 160], 8, 8, 128),
]


def _inputs(lengths, HQ, HK, D, dtype, seed):
    g = gen(seed)
    T = int(sum(lengths))
    q = torch.randn(T, HQ, D, generator=g).to(dtype)
    k = torch.randn(T, HK, D, generator=g).to(dtype)
    v = torch.randn(T, HK, D, generator=g).to(dtype)
    cu = torch.tensor(ref.cu_from_lengths(lengths), dtype=torch.int32)
    return q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV)


def _torch_sdpa(q, k, v, lengths, scale):
    HQ, HK = q.shape[1], k.shape[1]
    outs = []
    for qs, ks, vs in zip(q.split(lengths), k.split(lengths), v.split(lengths)):
        n, D = qs.shape[0], qs.shape[2]
        qh = qs.reshape(n, HK, HQ // HK, D).permute(1, 2, 0, 3)
        kh = ks.permute(1, 0, 2).unsqueeze(1).expand(HK, HQ // HK, n, D)
        vh = vs.permute(1, 0, 2).unsqueeze(1).expand(HK, HQ // HK, n, D)
        o = torch.nn.functional.scaled_dot_product_attention(qh, kh, vh, is_causal=True, scale=scale)
        outs.append(o.permute(2, 0, 1, 3).reshape(n, HQ, D))
    return torch.cat(outs, 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_attn_fwd_vs_oracle(case, dtype):
    from solution.body import _hip

    lengths, HQ, HK, D = CASES[case]
    q, k, v, cu = _inputs(lengths, HQ, HK, D, dtype, seed=case)
    T = q.shape[0]
    scale = D ** -0.5
    o = torch.full_like(q, float("nan"))
    lse = torch.full((HQ, T), float("nan"), device=DEV)
    _hip.attn_fwd(q, k, v, o, cu, max(lengths), scale, lse=lse)
    o64, lse64 = ref.attn_fwd(np64(q), np64(k), np64(v), cu.cpu().numpy(), scale)
    err = np.abs(np64(o) - o64)
    err_t = np.abs(np64(_torch_sdpa(q, k, v, lengths, scale)) - o64)
    print(f"case {case} {dtype}: max err {err.max():.2e} (torch {err_t.max():.2e}), mean "
          f"{err.mean():.2e} (torch {err_t.mean():.2e}), lse err {np.abs(np64(lse) - lse64).max():.2e}")
    atol = 1e-2 if dtype == torch.bfloat16 else 2e-3
    assert np.all(err <= atol + 1e-2 * np.abs(o64)), err.max()
    assert err.max() <= 2 * err_t.max() + 1e-6 and err.mean() <= 1.5 * err_t.mean() + 1e-7
    np.testing.assert_allclose(np64(lse), lse64, atol=1e-4, rtol=1e-5)


def test_attn_fwd_sequences_isolated_and_deterministic():
    """Changing one sequence's keys leaves every other sequence's output bitwise equal; repeated
    runs are bitwise equal."""
    from solution.body import _hip

    lengths = [70, 130, 33]
    q, k, v, cu = _inputs(lengths, 4, 2, 128, torch.bfloat16, seed=11)
    outs = []
    for kk in (k, k.clone().index_fill_(0, torch.arange(70, 200, device=DEV), 3.0)):
        o = torch.empty_like(q)
        _hip.attn_fwd(q, kk, v, o, cu, 130, 128 ** -0.5)
        outs.append(o)
    assert torch.equal(outs[0][:70], outs[1][:70]) and torch.equal(outs[0][200:], outs[1][200:])
    o2 = torch.empty_like(q)
    _hip.attn_fwd(q, k, v, o2, cu, 130, 128 ** -0.5)
    assert torch.equal(outs[0], o2)


def _torch_grads(q, k, v, do, lengths, scale):
    qq, kk, vv = (t.detach().clone().requires_grad_() for t in (q, k, v))
    o = _torch_sdpa(qq, kk, vv, lengths, scale)
    return torch.autograd.grad(o, [qq, kk, vv], do)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_attn_bwd_vs_oracle(case, dtype):
    """dq, dk, dv against the float64 closed form (oracle.attn_bwd) and torch's autograd SDPA in
    the same dtype: each gradient's error is within 1e-2 (bf16) / 2e-3 (fp16) of its largest
    magnitude plus 1e-2 relative (plus 1e-5 absolute), its largest error at most twice
    torch's, its mean error at most 1.5 times torch's."""
    from solution.body import _hip

    lengths, HQ, HK, D = CASES[case]
    q, k, v, cu = _inputs(lengths, HQ, HK, D, dtype, seed=100 + case)
    do = torch.randn(q.shape, generator=gen(200 + case)).to(dtype).to(DEV)
    scale = D ** -0.5
    o = torch.empty_like(q)
    lse = torch.empty((HQ, q.shape[0]), device=DEV)
    _hip.attn_fwd(q, k, v, o, cu, max(lengths), scale, lse=lse)
    dq, dk, dv = (torch.full_like(t, float("nan")) for t in (q, k, v))
    _hip.attn_bwd(q, k, v, o, do, lse, dq, dk, dv, cu, max(lengths), scale)
    want = ref.attn_bwd(np64(q), np64(k), np64(v), np64(do), cu.cpu().numpy(), scale)
    tg = _torch_grads(q, k, v, do, lengths, scale)
    atol = 1e-2 if dtype == torch.bfloat16 else 2e-3
    for name, got, w64, t in zip(("dq", "dk", "dv"), (dq, dk, dv), want, tg):
        err = np.abs(np64(got) - w64)
        err_t = np.abs(np64(t) - w64)
        print(f"case {case} {dtype} {name}: max err {err.max():.2e} (torch {err_t.max():.2e}), "
              f"mean {err.mean():.2e} (torch {err_t.mean():.2e}), max |g| {np.abs(w64).max():.2e}")
        # (+1e-5: a one-token sequence's exact dq is 0, and both kernels leave rounding there)
        assert np.all(err <= atol * np.abs(w64).max() + 1e-2 * np.abs(w64) + 1e-5), (name, err.max())
        assert err.max() <= 2 * err_t.max() + 1e-6, (name, err.max(), err_t.max())
        assert err.mean() <= 1.5 * err_t.mean() + 1e-7, (name, err.mean(), err_t.mean())


def test_attn_bwd_deterministic():
    from solution.body import _hip

    lengths = [300, 45]
    q, k, v, cu = _inputs(lengths, 12, 2, 128, torch.bfloat16, seed=21)
    do = torch.randn(q.shape, generator=gen(22)).to(torch.bfloat16).to(DEV)
    o = torch.empty_like(q)
    lse = torch.empty((12, q.shape[0]), device=DEV)
    _hip.attn_fwd(q, k, v, o, cu, 300, 128 ** -0.5, lse=lse)
    runs = []
    for _ in range(2):
        g = [torch.empty_like(t) for t in (q, k, v)]
        _hip.attn_bwd(q, k, v, o, do, lse, *g, cu, 300, 128 ** -0.5)
        runs.append(g)
    assert all(torch.equal(a, b) for a, b in zip(*runs))


@pytest.mark.parametrize("lengths", [[4096] * 4, [4000, 4097, 3999, 4100],
                                     [3000, 4100, 2500, 4096, 3900, 1800, 4000, 3500, 2900]],
                         ids=["even", "ragged", "ragged9"])
def test_attn_bwd_long_sequences_sampled_keys(lengths):
    """A config-5-like shape (4 or 9 sequences of up to ~4096, 28 / 4 heads, D = 128: enough key
    blocks that the kernel does not split the query heads, so the 4-wavefront dK / dV kernel
    runs) checked on sampled keys against float64 sums restated from the formulas
    (dV_j = sum_q P_qj dO_q, dK_j = scale sum_q P_qj (dP_qj - delta_q) Q_q over the causal
    queries of every query head of the kv head), with the kernel's own lse and O for P and delta,
    and on sampled queries (O_q = sum_j P_qj V_j / l_q, dQ_q = scale sum_j P_qj (dP_qj - delta_q)
    K_j over the causal keys). The ragged lengths put the end of every sequence inside a query
    tile (rows past the end staged and masked); the sample takes keys from the last 40 tokens of
    each sequence as well as from anywhere. These grids are too large for the longest-first
    block order, so the forward and dQ kernels (and, with 9 sequences, the dK / dV kernel) run
    the length-sorted XCD order (kOrderSorted), equal-length sequences ranked by index."""
    from solution.body import _hip

    HQ, HK, D = 28, 4, 128
    q, k, v, cu = _inputs(lengths, HQ, HK, D, torch.bfloat16, seed=31)
    T = q.shape[0]
    assert ((T + 255) // 256) * HK >= 256  # no split: the 4-wavefront kernel
    do = torch.randn(q.shape, generator=gen(32)).to(torch.bfloat16).to(DEV)
    scale = D ** -0.5
    o = torch.empty_like(q)
    lse = torch.empty((HQ, T), device=DEV)
    L_max = max(lengths)
    _hip.attn_fwd(q, k, v, o, cu, L_max, scale, lse=lse)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    _hip.attn_bwd(q, k, v, o, do, lse, dq, dk, dv, cu, L_max, scale)
    Q, K, V, DO, O, L = (np64(t) for t in (q, k, v, do, o, lse))
    DK, DV = np64(dk), np64(dv)
    G = HQ // HK
    bounds = np.concatenate([[0], np.cumsum(lengths)])
    rng = np.random.default_rng(33)
    tails = [int(rng.integers(e - 40, e)) for e in bounds[1:]]
    for j in sorted(set(rng.choice(T, 20, replace=False).tolist() + tails)):
        s_end = bounds[np.searchsorted(bounds, j, side="right")]
        t = np.arange(j, s_end)  # causal queries of key j
        for hk in range(HK):
            gdk = np.zeros(D)
            gdv = np.zeros(D)
            for h in range(hk * G, (hk + 1) * G):
                p = np.exp(scale * (Q[t, h] @ K[j, hk]) - L[h, t])
                dp = DO[t, h] @ V[j, hk]
                delta = np.sum(DO[t, h] * O[t, h], axis=1)
                gdv += p @ DO[t, h]
                gdk += scale * ((p * (dp - delta)) @ Q[t, h])
            for name, got, want in (("dk", DK[j, hk], gdk), ("dv", DV[j, hk], gdv)):
                err = np.abs(got - want)
                assert np.all(err <= 1e-2 * np.abs(want).max() + 1e-2 * np.abs(want) + 1e-5), \
                    (name, j, hk, err.max(), np.abs(want).max())
    DQ = np64(dq)
    for i in sorted(set(rng.choice(T, 12, replace=False).tolist() + tails)):
        s_start = bounds[np.searchsorted(bounds, i, side="right") - 1]
        kk = np.arange(s_start, i + 1)  # causal keys of query i
        for h in range(HQ):
            hk = h // G
            s_ = scale * (K[kk, hk] @ Q[i, h])
            p = np.exp(s_ - s_.max())
            p /= p.sum()
            want_o = p @ V[kk, hk]
            pk = np.exp(scale * (K[kk, hk] @ Q[i, h]) - L[h, i])
            dp = V[kk, hk] @ DO[i, h]
            delta = np.sum(DO[i, h] * O[i, h])
            want_dq = scale * ((pk * (dp - delta)) @ K[kk, hk])
            for name, got, want in (("o", O[i, h], want_o), ("dq", DQ[i, h], want_dq)):
                err = np.abs(got - want)
                assert np.all(err <= 1e-2 * np.abs(want).max() + 1e-2 * np.abs(want) + 1e-5), \
                    (name, i, h, err.max(), np.abs(want).max())


@pytest.mark.parametrize("n_seq", [60, 70], ids=["sorted_order", "group_order"])
def test_attn_many_sequences_block_orders(n_seq):
    """Many packed sequences (lengths 0 .. 640 with empty ones, 28 / 4 heads, D = 128): grids past
    two rounds of residency, so the kernels run the length-sorted XCD order (kOrderSorted: up to
    64 sequences, ranked by length with ties and empty sequences) or, past 64 sequences, the
    group-by-group order. Output and gradients against torch's SDPA computed in float32 from the
    same bf16 inputs, within 1e-2 of the largest magnitude plus 1e-2 relative."""
    from solution.body import _hip

    g = gen(40 + n_seq)
    lengths = torch.randint(0, 641, (n_seq,), generator=g).tolist()
    lengths[3] = lengths[17] = 0
    lengths[5] = lengths[30] = 640
    HQ, HK, D = 28, 4, 128
    q, k, v, cu = _inputs(lengths, HQ, HK, D, torch.bfloat16, seed=50 + n_seq)
    do = torch.randn(q.shape, generator=gen(60 + n_seq)).to(torch.bfloat16).to(DEV)
    T, scale, L = q.shape[0], D ** -0.5, max(lengths)
    o = torch.full_like(q, float("nan"))
    lse = torch.empty((HQ, T), device=DEV)
    _hip.attn_fwd(q, k, v, o, cu, L, scale, lse=lse)
    dq, dk, dv = (torch.full_like(t, float("nan")) for t in (q, k, v))
    _hip.attn_bwd(q, k, v, o, do, lse, dq, dk, dv, cu, L, scale)
    live = [n for n in lengths if n > 0]
    keep = torch.cat([torch.ones(n, dtype=torch.bool) for n in live]).to(DEV)
    assert keep.numel() == T
    q32, k32, v32, do32 = (t.float() for t in (q, k, v, do))
    want_o = _torch_sdpa(q32, k32, v32, live, scale)
    want = _torch_grads(q32, k32, v32, do32, live, scale)
    for name, got, w in (("o", o, want_o), ("dq", dq, want[0]), ("dk", dk, want[1]),
                         ("dv", dv, want[2])):
        g64, w64 = np64(got), np64(w)
        err = np.abs(g64 - w64)
        assert np.all(err <= 1e-2 * np.abs(w64).max() + 1e-2 * np.abs(w64) + 1e-5), \
            (name, float(err.max()), float(np.abs(w64).max()))


def test_attn_config4_shape():
    """Config 4's attention as bench.py times it: 8 rows of 1024 tokens, 12 / 2 heads, D = 128,
    bf16 (a grid of one residency round: the longest-first block order; the dK / dV kernel with
    the query heads of a kv head split six ways and the partials' reduce). Output and gradients
    against torch's SDPA in float32 from the same bf16 inputs, within 1e-2 of the largest
    magnitude plus 1e-2 relative."""
    from solution.body import _hip

    lengths = [1024] * 8
    HQ, HK, D = 12, 2, 128
    q, k, v, cu = _inputs(lengths, HQ, HK, D, torch.bfloat16, seed=404)
    do = torch.randn(q.shape, generator=gen(405)).to(torch.bfloat16).to(DEV)
    T, scale = q.shape[0], D ** -0.5
    o = torch.full_like(q, float("nan"))
    lse = torch.empty((HQ, T), device=DEV)
    _hip.attn_fwd(q, k, v, o, cu, 1024, scale, lse=lse)
    dq, dk, dv = (torch.full_like(t, float("nan")) for t in (q, k, v))
    _hip.attn_bwd(q, k, v, o, do, lse, dq, dk, dv, cu, 1024, scale)
    q32, k32, v32, do32 = (t.float() for t in (q, k, v, do))
    want_o = _torch_sdpa(q32, k32, v32, lengths, scale)
    want = _torch_grads(q32, k32, v32, do32, lengths, scale)
    for name, got, w in (("o", o, want_o), ("dq", dq, want[0]), ("dk", dk, want[1]),
                         ("dv", dv, want[2])):
        g64, w64 = np64(got), np64(w)
        err = np.abs(g64 - w64)
        assert np.all(err <= 1e-2 * np.abs(w64).max() + 1e-2 * np.abs(w64) + 1e-5), \
            (name, float(err.max()), float(np.abs(w64).max()))


@pytest.mark.parametrize("D", [128, 64])
def test_attn_strided_fused_qkv(D):
    """q, k and v as column slices of one fused [T, (HQ + 2 HK) * D] bf16 projection output (token
    stride (HQ + 2 HK) * D, not HQ * D), and dq, dk, dv written into column slices of one fused
    gradient buffer, with ragged lengths so partial last tiles occur: the LDS-DMA fills address
    rows with the token stride. Output and gradients against float32 SDPA on the same values
    (1e-2 of the largest magnitude plus 1e-2 relative), and bitwise the dense layout's results."""
    from solution.body import _hip

    lengths, HQ, HK = [37, 300, 1, 129, 64], 12, 2
    T, W = sum(lengths), (HQ + 2 * HK) * D
    g = gen(500 + D)
    fused = torch.randn(T, W, generator=g).to(torch.bfloat16).to(DEV)
    q = fused[:, :HQ * D].view(T, HQ, D)
    k = fused[:, HQ * D:(HQ + HK) * D].view(T, HK, D)
    v = fused[:, (HQ + HK) * D:].view(T, HK, D)
    assert q.stride(0) == W and not q.is_contiguous()
    cu = torch.tensor(ref.cu_from_lengths(lengths), dtype=torch.int32, device=DEV)
    do = torch.randn(T, HQ, D, generator=gen(600 + D)).to(torch.bfloat16).to(DEV)
    scale = D ** -0.5
    o = torch.full((T, HQ, D), float("nan"), device=DEV, dtype=torch.bfloat16)
    lse = torch.empty((HQ, T), device=DEV)
    _hip.attn_fwd(q, k, v, o, cu, max(lengths), scale, lse=lse)
    gfused = torch.full((T, W), float("nan"), device=DEV, dtype=torch.bfloat16)
    dq = gfused[:, :HQ * D].view(T, HQ, D)
    dk = gfused[:, HQ * D:(HQ + HK) * D].view(T, HK, D)
    dv = gfused[:, (HQ + HK) * D:].view(T, HK, D)
    _hip.attn_bwd(q, k, v, o, do, lse, dq, dk, dv, cu, max(lengths), scale)
    q32, k32, v32, do32 = (t.float().contiguous() for t in (q, k, v, do))
    want_o = _torch_sdpa(q32, k32, v32, lengths, scale)
    want = _torch_grads(q32, k32, v32, do32, lengths, scale)
    for name, got, w in (("o", o, want_o), ("dq", dq, want[0]), ("dk", dk, want[1]),
                         ("dv", dv, want[2])):
        g64, w64 = np64(got), np64(w)
        err = np.abs(g64 - w64)
        assert np.all(err <= 1e-2 * np.abs(w64).max() + 1e-2 * np.abs(w64) + 1e-5), \
            (name, float(err.max()), float(np.abs(w64).max()))
    # the dense layout gives the same bits
    qd, kd, vd = (t.contiguous() for t in (q, k, v))
    od = torch.empty_like(qd)
    lsed = torch.empty_like(lse)
    _hip.attn_fwd(qd, kd, vd, od, cu, max(lengths), scale, lse=lsed)
    dqd, dkd, dvd = (torch.empty_like(t) for t in (qd, kd, vd))
    _hip.attn_bwd(qd, kd, vd, od, do, lsed, dqd, dkd, dvd, cu, max(lengths), scale)
    assert torch.equal(od, o) and torch.equal(lsed, lse)
    assert torch.equal(dqd, dq) and torch.equal(dkd, dk) and torch.equal(dvd, dv)
