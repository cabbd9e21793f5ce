"""Rotary embedding (K2) on the GPU: the reference's unit tests restated (reference
solution/test_body_norm_rope.py:80-166) plus parity with the CPU oracle for the packed
[T, H, D], varlen (cu_seqlens) and padded [B, H, S, D] layouts.

Tolerances: the reference's abs 4e-3 for fp16 (|x| up to ~6); against the fp64 oracle
16-bit outputs atol 2e-3 / rtol 1e-2, fp32 1e-5."""

import numpy as np
import pytest
import torch

from _util import DEV, STORE, assert_close, err, gen, np64, randn
from oracle import norm_rope_ref as ref

pytestmark = pytest.mark.gpu

HQ, HK, D, THETA = 12, 2, 128, 1e6
TS = [1, 37, 1000, 2048]


def _nr():
    from solution.body import norm_rope

    return norm_rope


def _rotate_half(x):
    x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def ref_rope(q, k, pos, inv_freq, q_delta=None):
    """Reference test's eager HF math (:87-95), fp32 cos/sin."""
    if q_delta is not None:
        q = q + q_delta.view(q.shape)
    freqs = (inv_freq[None, :, None].float() @ pos[None, None, :].float()).transpose(1, 2)[0]
    emb = torch.cat((freqs, freqs), dim=-1)
    cos, sin = emb.cos()[:, None, :], emb.sin()[:, None, :]
    return ((q * cos) + (_rotate_half(q) * sin)).to(q.dtype), \
        ((k * cos) + (_rotate_half(k) * sin)).to(k.dtype)


def _packed_positions(T, g):
    out, left = [], T
    while left > 0:
        n = min(left, int(torch.randint(1, 600, (1,), generator=g)))
        out.append(torch.arange(n))
        left -= n
    return torch.cat(out)


def _tol(dt):
    return (2e-3, 1e-2) if dt != torch.float32 else (1e-5, 1e-5)


@pytest.mark.parametrize("T", TS)
@pytest.mark.parametrize("layout", ["contiguous", "strided_qkv"])
@pytest.mark.parametrize("with_delta", [False, True])
@pytest.mark.parametrize("pos_dtype", [torch.int64, torch.int32])
def test_rope(T, layout, with_delta, pos_dtype):
    """Reference test_rope (:107-150): outputs and grads within 4e-3 abs of the eager HF math;
    d(q_delta) == dq bitwise. Plus the fp64 oracle."""
    nr = _nr()
    g = gen(T)
    pos = _packed_positions(T, g).to(DEV, pos_dtype)
    inv_freq = nr.default_inv_freq(D, THETA, DEV)
    if layout == "contiguous":
        q = randn((T, HQ * D), g, dtype=torch.float16).requires_grad_()
        k = randn((T, HK * D), g, dtype=torch.float16).requires_grad_()
        qv, kv = q.view(T, HQ, D), k.view(T, HK, D)
        leaves = [q, k]
    else:
        qkv = randn((T, (HQ + 2 * HK) * D), g, dtype=torch.float16).requires_grad_()
        qv = qkv[:, : HQ * D].view(T, HQ, D)
        kv = qkv[:, HQ * D:(HQ + HK) * D].view(T, HK, D)
        assert T == 1 or not qv.is_contiguous()
        leaves = [qkv]
    qd = None
    if with_delta:
        qd = randn((T, HQ * D), g, 0.3, dtype=torch.float16).requires_grad_()
        leaves.append(qd)

    qo, ko = nr.rope(qv, kv, pos, inv_freq, qd)
    qr, kr = ref_rope(qv, kv, pos, inv_freq, qd)
    assert qo.shape == (T, HQ, D) and ko.shape == (T, HK, D) and qo.is_contiguous()
    assert qo.dtype == torch.float16 and ko.dtype == torch.float16
    for a, b in ((qo, qr), (ko, kr)):
        ae, _ = err(np64(a), np64(b))
        assert ae <= 4e-3, ae

    q64 = ref.rope_fwd(np64(qv), pos.cpu().numpy(), inv_freq.cpu().numpy(),
                       delta=None if qd is None else np64(qd), store="f16")
    k64 = ref.rope_fwd(np64(kv), pos.cpu().numpy(), inv_freq.cpu().numpy(), store="f16")
    assert_close(np64(qo), q64, 2e-3, 1e-2, "q")
    assert_close(np64(ko), k64, 2e-3, 1e-2, "k")

    gq = torch.randn(qo.shape, generator=g).half().to(DEV)
    gk = torch.randn(ko.shape, generator=g).half().to(DEV)
    gg = torch.autograd.grad([qo, ko], leaves, [gq, gk])
    gr = torch.autograd.grad([qr, kr], leaves, [gq, gk])
    for a, b in zip(gg, gr):
        ae, _ = err(np64(a), np64(b))
        assert ae <= 4e-3, ae
    if with_delta:
        dq_view = gg[0][:, : HQ * D] if layout == "strided_qkv" else gg[0]
        torch.testing.assert_close(gg[-1].view(T, HQ * D), dq_view.reshape(T, HQ * D),
                                   rtol=0, atol=0)


def test_rope_cos_sin_match_torch():
    """Reference :153-166: unit vectors at positions up to 32760 give (cos, sin) of the fp32
    angle within 1e-3 of torch's fp32 cos/sin."""
    nr = _nr()
    T = 2048
    pos = torch.arange(T, device=DEV) * 16
    inv_freq = nr.default_inv_freq(D, THETA, DEV)
    q = torch.zeros(T, 1, D, device=DEV, dtype=torch.float16)
    q[..., : D // 2] = 1.0
    k = q.clone()
    qo, _ = nr.rope(q, k, pos, inv_freq)
    ang = pos.float()[:, None] * inv_freq[None, :]
    torch.testing.assert_close(qo[:, 0, : D // 2].float(), ang.cos().half().float(),
                               rtol=0, atol=1e-3)
    torch.testing.assert_close(qo[:, 0, D // 2:].float(), ang.sin().half().float(),
                               rtol=0, atol=1e-3)


def test_rope_cos_sin_fp32_accuracy():
    """fp32 unit vectors (no 16-bit rounding): in-kernel cos/sin of the fp32 angle within 2e-6
    of the exact cos/sin of that same fp32 angle, positions to 32760 (accurate reduction)."""
    nr = _nr()
    T = 2048
    pos = torch.arange(T, device=DEV) * 16
    inv_freq = nr.default_inv_freq(D, THETA, DEV)
    q = torch.zeros(T, 1, D, device=DEV, dtype=torch.float32)
    q[..., : D // 2] = 1.0
    qo, _ = nr.rope(q, q.clone(), pos, inv_freq)
    ang = ref.rope_angles(pos.cpu().numpy(), inv_freq.cpu().numpy()).astype(np.float64)
    assert_close(np64(qo)[:, 0, : D // 2], np.cos(ang), 2e-6, 0, "cos")
    assert_close(np64(qo)[:, 0, D // 2:], np.sin(ang), 2e-6, 0, "sin")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_rope_dtypes_head_dims(dtype, d):
    """Every dtype and head dim against the oracle, forward and backward (sign -1)."""
    nr = _nr()
    g = gen(d)
    T, hq, hk = 333, 28, 4
    pos = _packed_positions(T, g).to(DEV)
    inv_freq = nr.default_inv_freq(d, THETA, DEV)
    q = randn((T, hq, d), g, dtype=dtype).requires_grad_()
    k = randn((T, hk, d), g, dtype=dtype).requires_grad_()
    qo, ko = nr.rope(q, k, pos, inv_freq)
    p, f = pos.cpu().numpy(), inv_freq.cpu().numpy()
    atol, rtol = _tol(dtype)
    assert_close(np64(qo), ref.rope_fwd(np64(q), p, f, store=STORE[dtype]), atol, rtol, "q")
    assert_close(np64(ko), ref.rope_fwd(np64(k), p, f, store=STORE[dtype]), atol, rtol, "k")
    gq, gk = randn(qo.shape, g, dtype=dtype), randn(ko.shape, g, dtype=dtype)
    dq, dk = torch.autograd.grad([qo, ko], [q, k], [gq, gk])
    assert_close(np64(dq), ref.rope_fwd(np64(gq), p, f, -1.0, store=STORE[dtype]), atol, rtol, "dq")
    assert_close(np64(dk), ref.rope_fwd(np64(gk), p, f, -1.0, store=STORE[dtype]), atol, rtol, "dk")


def _varlen_lengths(seed, n, lo, hi, total=None):
    g = gen(seed)
    lens = torch.randint(lo, hi + 1, (n,), generator=g).tolist()
    if total is not None:
        out, acc = [], 0
        while acc < total:
            ln = int(torch.randint(lo, hi + 1, (1,), generator=g))
            ln = min(ln, total - acc)
            out.append(ln)
            acc += ln
        lens = out
    return lens


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rope_cu_seqlens_equals_positions(dtype):
    """cu_seqlens positions (reset per sequence) give the same bits as the explicit-positions
    path with positions built by the oracle; includes an empty sequence and a 1-token one."""
    nr = _nr()
    lens = [113, 962, 0, 544, 1, 574, 556, 614, 422, 772]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    T = int(cu[-1])
    pos = torch.from_numpy(ref.positions_from_cu_seqlens(cu.numpy())).to(DEV)
    g = gen(3)
    inv_freq = nr.default_inv_freq(D, THETA, DEV)
    q = randn((T, HQ, D), g, dtype=dtype)
    k = randn((T, HK, D), g, dtype=dtype)
    a = nr.rope(q, k, None, inv_freq, cu_seqlens=cu.to(DEV))
    b = nr.rope(q, k, pos, inv_freq)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_rope_cu_seqlens_many_sequences():
    """More than 64 sequences (several ballot rounds of the in-kernel sequence search)."""
    nr = _nr()
    lens = _varlen_lengths(7, 300, 1, 40)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    T = int(cu[-1])
    pos = torch.from_numpy(ref.positions_from_cu_seqlens(cu.numpy())).to(DEV)
    g = gen(8)
    inv_freq = nr.default_inv_freq(D, THETA, DEV)
    q, k = randn((T, HQ, D), g, dtype=torch.bfloat16), randn((T, HK, D), g, dtype=torch.bfloat16)
    a = nr.rope(q, k, None, inv_freq, cu_seqlens=cu.to(DEV))
    b = nr.rope(q, k, pos, inv_freq)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_config3_varlen():
    """Config 3: 8 sequences, lengths U[64, 1024] (seed 0) packed with cu_seqlens; fp16
    forward + backward against the oracle."""
    nr = _nr()
    lens = torch.randint(64, 1025, (8,), generator=gen(0)).tolist()
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    T = int(cu[-1])
    g = gen(0)
    inv_freq = nr.default_inv_freq(D, THETA, DEV)
    q = randn((T, HQ, D), g, dtype=torch.float16).requires_grad_()
    k = randn((T, HK, D), g, dtype=torch.float16).requires_grad_()
    qo, ko = nr.rope(q, k, None, inv_freq, cu_seqlens=cu.to(DEV))
    pos = ref.positions_from_cu_seqlens(cu.numpy())
    f = inv_freq.cpu().numpy()
    assert_close(np64(qo), ref.rope_fwd(np64(q), pos, f, store="f16"), 2e-3, 1e-2, "q")
    assert_close(np64(ko), ref.rope_fwd(np64(k), pos, f, store="f16"), 2e-3, 1e-2, "k")
    gq, gk = randn(qo.shape, g, dtype=torch.float16), randn(ko.shape, g, dtype=torch.float16)
    dq, dk = torch.autograd.grad([qo, ko], [q, k], [gq, gk])
    assert_close(np64(dq), ref.rope_fwd(np64(gq), pos, f, -1.0, store="f16"), 2e-3, 1e-2, "dq")
    assert_close(np64(dk), ref.rope_fwd(np64(gk), pos, f, -1.0, store="f16"), 2e-3, 1e-2, "dk")


@pytest.mark.parametrize("layout", ["contiguous_bhsd", "hf_transposed_view"])
@pytest.mark.parametrize("pos_kind", ["arange", "position_ids", "broadcast_row"])
def test_config2_padded_bhsd(layout, pos_kind):
    """Config 2: q [4, 12, 512, 128], k [4, 2, 512, 128] fp16 in HF's padded layout (a
    contiguous [B, H, S, D] tensor or HF's view(B, S, H, D).transpose(1, 2)); positions 0..511
    implicit, explicit [B, S], or [1, S] broadcast. Against the oracle and HF's eager math."""
    from oracle import hf_eager

    nr = _nr()
    B, S = 4, 512
    g = gen(0)
    if layout == "contiguous_bhsd":
        q = randn((B, HQ, S, D), g, dtype=torch.float16).requires_grad_()
        k = randn((B, HK, S, D), g, dtype=torch.float16).requires_grad_()
        qv, kv = q, k
    else:
        q = randn((B, S, HQ * D), g, dtype=torch.float16).requires_grad_()
        k = randn((B, S, HK * D), g, dtype=torch.float16).requires_grad_()
        qv, kv = q.view(B, S, HQ, D).transpose(1, 2), k.view(B, S, HK, D).transpose(1, 2)
    inv_freq = nr.default_inv_freq(D, THETA, DEV)
    pid = torch.arange(S, device=DEV).expand(B, S)
    arg = {"arange": None, "position_ids": pid.contiguous(), "broadcast_row": pid[:1]}[pos_kind]
    qo, ko = nr.rope_bhsd(qv, kv, inv_freq, arg)
    assert qo.shape == qv.shape and ko.shape == kv.shape and qo.stride() == qv.stride()
    f = inv_freq.cpu().numpy()
    posr = np.tile(np.arange(S), B)
    q_tok = np64(qv.transpose(1, 2)).reshape(B * S, HQ, D)
    k_tok = np64(kv.transpose(1, 2)).reshape(B * S, HK, D)
    q64 = ref.rope_fwd(q_tok, posr, f, store="f16").reshape(B, S, HQ, D).transpose(0, 2, 1, 3)
    k64 = ref.rope_fwd(k_tok, posr, f, store="f16").reshape(B, S, HK, D).transpose(0, 2, 1, 3)
    assert_close(np64(qo), q64, 2e-3, 1e-2, "q")
    assert_close(np64(ko), k64, 2e-3, 1e-2, "k")
    cos, sin = hf_eager.rotary_cos_sin(inv_freq, pid, torch.float32)
    qh, kh = hf_eager.apply_rotary_pos_emb(qv.float(), kv.float(), cos, sin, unsqueeze_dim=1)
    assert err(np64(qo), np64(qh))[0] <= 4e-3 and err(np64(ko), np64(kh))[0] <= 4e-3
    gq, gk = randn(qo.shape, g, dtype=torch.float16), randn(ko.shape, g, dtype=torch.float16)
    dq, dk = torch.autograd.grad([qo, ko], [q, k], [gq, gk])
    dqh, dkh = torch.autograd.grad([qh, kh], [q, k], [gq.float(), gk.float()])
    assert err(np64(dq), np64(dqh))[0] <= 4e-3 and err(np64(dk), np64(dkh))[0] <= 4e-3


def test_rope_invariants():
    """pos = 0 is the identity (bitwise, fp32); forward then backward returns the input
    (fp32, 1e-6); the rotation keeps every pair's norm."""
    nr = _nr()
    g = gen(4)
    T = 500
    inv_freq = nr.default_inv_freq(D, THETA, DEV)
    q = randn((T, HQ, D), g)
    k = randn((T, HK, D), g)
    zero = torch.zeros(T, dtype=torch.int64, device=DEV)
    qo, ko = nr.rope(q, k, zero, inv_freq)
    assert torch.equal(qo, q) and torch.equal(ko, k)
    pos = torch.randint(0, 32768, (T,), generator=g).to(DEV)
    qo, ko = nr.rope(q, k, pos, inv_freq)
    # the backward kernel (rotation by -angle) applied to the output recovers the input
    from solution.body import _hip

    q4, k4 = qo.unsqueeze(0), ko.unsqueeze(0)
    rq, rk = torch.empty_like(q4), torch.empty_like(k4)
    _hip.rope(q4, k4, rq, rk, inv_freq, -1.0, positions=pos.view(1, -1))
    assert_close(np64(rq)[0], np64(q), 1e-5, 1e-5, "roundtrip q")
    assert_close(np64(rk)[0], np64(k), 1e-5, 1e-5, "roundtrip k")
    h = D // 2
    n_in = np64(q)[..., :h] ** 2 + np64(q)[..., h:] ** 2
    n_out = np64(qo)[..., :h] ** 2 + np64(qo)[..., h:] ** 2
    assert_close(n_out, n_in, 1e-5, 1e-5, "pair norms")


def test_rope_empty_and_errors():
    nr = _nr()
    from solution.body import _hip

    inv_freq = nr.default_inv_freq(D, THETA, DEV)
    q = torch.empty((0, HQ, D), device=DEV, dtype=torch.float16)
    k = torch.empty((0, HK, D), device=DEV, dtype=torch.float16)
    qo, ko = nr.rope(q, k, torch.empty(0, dtype=torch.int64, device=DEV), inv_freq)
    assert qo.shape == (0, HQ, D) and ko.shape == (0, HK, D)
    with pytest.raises(_hip.EsepError):
        q = torch.zeros((4, HQ, 96), device=DEV, dtype=torch.float16)  # D/2 = 48 unsupported
        k = torch.zeros((4, HK, 96), device=DEV, dtype=torch.float16)
        _hip.rope(q.unsqueeze(0), k.unsqueeze(0), q.unsqueeze(0).clone(), k.unsqueeze(0).clone(),
                  torch.ones(48, device=DEV), 1.0)
