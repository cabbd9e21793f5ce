"""The CPU oracle against what the mathematics fixes: closed forms, known answers, invariants,
central finite differences on tiny inputs, brute-force position rules; and mutation tests
that plant plausible mistakes in copies of the oracle and check that the golden comparisons
(tests/test_oracle_golden.py) catch every one."""

import types

import numpy as np
import pytest
import torch

import test_oracle_golden as golden
from oracle import norm_rope_ref as ref

EPS = 1e-6


def rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------------- RMSNorm

def test_constant_row_closed_form():
    """x = c everywhere, w = 1: y = c / sqrt(c^2 + eps)."""
    for c in (3.0, -0.25, 1e-3):
        x = np.full((2, 64), c)
        y, rstd = ref.rmsnorm_fwd(x, np.ones(64), EPS, "f64")
        assert np.allclose(y, c / np.sqrt(c * c + EPS), rtol=1e-14, atol=0)
        assert np.allclose(rstd, 1 / np.sqrt(c * c + EPS), rtol=1e-14)


def test_scale_invariance_and_weight_linearity():
    r = rng(1)
    x, w = r.normal(size=(5, 96)), r.normal(size=96)
    y1, _ = ref.rmsnorm_fwd(x, w, 0.0, "f64")
    y2, _ = ref.rmsnorm_fwd(1e3 * x, w, 0.0, "f64")
    assert np.allclose(y1, y2, rtol=1e-12, atol=1e-12)
    y3, _ = ref.rmsnorm_fwd(x, 2.5 * w, 0.0, "f64")
    assert np.allclose(y3, 2.5 * y1, rtol=1e-12, atol=1e-12)
    assert np.allclose((ref.rmsnorm_fwd(x, np.ones(96), 0.0, "f64")[0] ** 2).mean(-1), 1.0, rtol=1e-12)


def _fd_grads(x, w, dy, eps, h=1e-6):
    def loss(xx, ww):
        return float((dy * ref.rmsnorm_fwd(xx, ww, eps, "f64")[0]).sum())
    gx = np.zeros_like(x)
    for idx in np.ndindex(*x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        gx[idx] = (loss(xp, w) - loss(xm, w)) / (2 * h)
    gw = np.zeros_like(w)
    for j in range(w.size):
        wp, wm = w.copy(), w.copy()
        wp[j] += h
        wm[j] -= h
        gw[j] = (loss(x, wp) - loss(x, wm)) / (2 * h)
    return gx, gw


@pytest.mark.parametrize("eps", [1e-6, 0.5])
def test_rmsnorm_bwd_finite_differences(eps):
    """dx and dw of the oracle equal central differences of sum(dy * y) (brute force)."""
    r = rng(2)
    x, w, dy = r.normal(size=(3, 8)), 1 + 0.3 * r.normal(size=8), r.normal(size=(3, 8))
    dx, dw = ref.rmsnorm_bwd(dy, x, w, eps)
    gx, gw = _fd_grads(x, w, dy, eps)
    assert np.allclose(dx, gx, rtol=1e-6, atol=1e-8)
    assert np.allclose(dw, gw, rtol=1e-6, atol=1e-8)


def test_dr_orthogonal_to_xhat_without_eps():
    """With eps = 0 the norm's input gradient is orthogonal to xhat (the norm is scale
    invariant): sum_j dr_j * xhat_j = 0."""
    r = rng(3)
    x, w, dy = r.normal(size=(7, 200)), r.normal(size=200), r.normal(size=(7, 200))
    dr, _ = ref.rmsnorm_bwd(dy, x, w, 0.0)
    xhat = x / np.sqrt((x * x).mean(-1, keepdims=True))
    assert np.abs((dr * xhat).sum(-1)).max() < 1e-10 * np.abs(dr).max() * 200


def test_fan_in_and_pass_through():
    r = rng(4)
    x, w = r.normal(size=(6, 40)), r.normal(size=40)
    d1, d2, d3, dro = (r.normal(size=(6, 40)) for _ in range(4))
    a, aw = ref.add_rmsnorm_bwd([d1, d2, d3], dro, x, w, EPS)
    b, bw = ref.add_rmsnorm_bwd([d1 + d2 + d3], None, x, w, EPS)
    assert np.allclose(a, b + dro, rtol=1e-12, atol=1e-12) and np.allclose(aw, bw, rtol=1e-12)
    c, cw = ref.add_rmsnorm_bwd([], dro, x, w, EPS)
    assert np.array_equal(c, dro) and not cw.any()


def test_from_y_recovery_and_exact_channels():
    """xhat from y / w equals xhat from the residual (fp64 y); channels with w == 0 come
    from xs and keep the gradient finite; without them the gradient is not finite."""
    r = rng(5)
    x, dy = r.normal(size=(4, 32)) * 3, r.normal(size=(4, 32))
    w = 1 + 0.1 * r.normal(size=32)
    w[[3, 17]] = 0.0
    slots, k = ref.special_channels(w)
    assert k == 2 and list(np.nonzero(slots >= 0)[0]) == [3, 17]
    _, y, rstd, xs = ref.add_rmsnorm_fwd(x, None, w, EPS, "f64", slots=slots)
    want, _ = ref.add_rmsnorm_bwd([dy], None, x, w, EPS)
    y64 = w[None, :] * x * rstd[:, None]
    got, _ = ref.add_rmsnorm_bwd([dy], None, y64, w, EPS, rstd=rstd, from_y=True, slots=slots, xs=xs)
    assert np.allclose(got, want, rtol=1e-10, atol=1e-12)
    bad, _ = ref.add_rmsnorm_bwd([dy], None, y64, w, EPS, rstd=rstd, from_y=True)
    assert not np.isfinite(bad).all()


def test_special_channels_designed_weights():
    """The reference tests' weight constructions (test_body_norm_rope.py:258-273) give
    K = 0 / 8 / 3 exact channels."""
    H = 1536
    g = torch.Generator().manual_seed(0)
    w = 1 + 0.1 * torch.randn(H, generator=g)
    assert ref.special_channels(w.numpy())[1] == 0
    wz = w.clone()
    wz[[0, 7, 100]] = 0.0
    wz[[1, 2]] = torch.tensor([1e-6, -3e-5])
    wz[[3, 4]] = torch.tensor([2.0 ** -10 * 0.999, -2.0 ** -10 * 0.5])
    wz[5] = 2.0 ** -10 * 1.001
    wz[H - 1] = 2000.0
    slots, k = ref.special_channels(wz.numpy())
    assert k == 8 and slots[5] == -1 and slots[H - 1] == 7 and slots[0] == 0
    wq = (0.3 + 2.7 * torch.rand(H, generator=g)) * torch.sign(torch.randn(H, generator=g))
    wq[[11, 500, 1400]] = torch.tensor([2e-5, 6.5e-6, 9e-4])
    wq[[12, 501]] = torch.tensor([2e-3, 4e-3])
    assert ref.special_channels(wq.numpy())[1] == 3
    wn = w.clone()
    wn[9] = float("nan")
    assert ref.special_channels(wn.numpy())[0][9] == 0


def test_round_bf16_matches_torch():
    r = rng(6)
    v = np.concatenate([r.normal(size=5000).astype(np.float32) * 10 ** r.uniform(-8, 8, 5000),
                        np.array([0.0, -0.0, 1.0, 65504.0, 3.3895314e38, 1e-40, -1e-40],
                                 dtype=np.float32)]).astype(np.float32)
    want = torch.from_numpy(v).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(ref.round_bf16(v), want)


# ------------------------------------------------------------------------- RoPE

def test_rope_is_complex_rotation():
    """out = (x1 + i x2) * exp(i * angle), written as complex arithmetic (an independent form
    of the rotate_half convention)."""
    r = rng(7)
    x = r.normal(size=(50, 3, 16))
    pos = r.integers(0, 40000, size=50)
    inv = ref.default_inv_freq(16, 1e4)
    out = ref.rope_fwd(x, pos, inv, store="f64")
    ang = ref.rope_angles(pos, inv).astype(np.float64)[:, None, :]
    z = (x[..., :8] + 1j * x[..., 8:]) * np.exp(1j * ang)
    assert np.allclose(out, np.concatenate([z.real, z.imag], -1), rtol=1e-12, atol=1e-12)


def test_rope_invariants():
    r = rng(8)
    x = r.normal(size=(30, 4, 128))
    inv = ref.default_inv_freq(128, 1e6)
    assert np.array_equal(ref.rope_fwd(x, np.zeros(30, int), inv, store="f64"), x)
    pos = r.integers(0, 32768, size=30)
    y = ref.rope_fwd(x, pos, inv, store="f64")
    assert np.allclose(ref.rope_fwd(y, pos, inv, sign=-1.0, store="f64"), x, rtol=1e-12, atol=1e-12)
    n_in = x[..., :64] ** 2 + x[..., 64:] ** 2
    n_out = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert np.allclose(n_in, n_out, rtol=1e-12)


def test_rope_unit_vector_known_answer():
    inv = ref.default_inv_freq(128, 1e6)
    pos = np.arange(0, 32768, 16)
    x = np.zeros((pos.size, 1, 128))
    x[..., :64] = 1.0
    out = ref.rope_fwd(x, pos, inv, store="f64")
    ang = (pos.astype(np.float32)[:, None] * inv[None, :]).astype(np.float64)
    assert np.array_equal(out[:, 0, :64], np.cos(ang)) and np.array_equal(out[:, 0, 64:], np.sin(ang))


def test_rope_delta_rounds_in_storage_dtype():
    """q + q_delta is formed in the storage dtype first (reference norm_rope.py:341-346)."""
    x = np.array([[[1.0, 2.0 ** -11, 0.0, 0.0]]])
    d = np.array([[[2.0 ** -11, 2.0 ** -11, 0.0, 0.0]]])
    out = ref.rope_fwd(x, np.array([0]), np.array([1.0, 0.5], np.float32), delta=d, store="f16")
    assert out[0, 0, 0] == 1.0 and out[0, 0, 1] == 2.0 ** -10  # 1 + 2^-11 rounds to 1 in fp16


# ------------------------------------------------------------------------- positions

def test_positions_from_cu_seqlens_brute_force():
    r = rng(9)
    lens = list(r.integers(0, 50, size=40)) + [0, 1]
    cu = np.concatenate([[0], np.cumsum(lens)])
    want = []
    for n in lens:
        for t in range(n):
            want.append(t)
    assert np.array_equal(ref.positions_from_cu_seqlens(cu), np.array(want))


def test_packed_positions_reference_rule():
    """Reference packed_forward (packed.py:808-814): real tokens in row-major order; position
    = column index (left padding keeps HF's arange, no reset) or position_ids gathered."""
    mask = np.array([[1, 1, 1, 0, 0], [0, 0, 1, 1, 1], [1, 1, 1, 1, 1]])
    got = ref.packed_positions(mask)
    assert list(got) == [0, 1, 2, 2, 3, 4, 0, 1, 2, 3, 4]
    pid = np.arange(5)[None, :] + 100
    assert list(ref.packed_positions(mask, pid)) == [100, 101, 102, 102, 103, 104, 100, 101, 102, 103, 104]


# ------------------------------------------------------------------------- mutation tests

def _rebind(fn, module):
    """fn with its globals taken from `module` (so it calls the module's mutated helpers)."""
    return types.FunctionType(fn.__code__, module.__dict__, fn.__name__, fn.__defaults__,
                              fn.__closure__)


def _mutant(**overrides):
    m = types.ModuleType("mutant_oracle")
    m.__dict__.update({k: v for k, v in vars(ref).items() if not k.startswith("__")})
    m.__dict__.update(overrides)
    return m


def _rope_wrong_sign(x, pos, inv_freq, sign=1.0, delta=None, store="f32", acc=np.float64):
    return ref.rope_fwd(x, pos, inv_freq, -sign, delta, store, acc)


def _rope_swapped_halves(x, pos, inv_freq, sign=1.0, delta=None, store="f32", acc=np.float64):
    o = ref.rope_fwd(x, pos, inv_freq, sign, delta, store, acc)
    h = o.shape[-1] // 2
    return np.concatenate([o[..., h:], o[..., :h]], -1)


def _angles_fp64(pos, inv_freq):
    return np.asarray(pos, np.float64)[:, None] * np.asarray(inv_freq, np.float64)[None, :]


def _bwd_no_proj_mean(dys, dr_out, x, w, eps, rstd=None, from_y=False, slots=None, xs=None,
                      acc=np.float64):
    dr, dw = ref.add_rmsnorm_bwd(dys, dr_out, x, w, eps, rstd, from_y, slots, xs, acc)
    # forgets the 1/n of proj: dr = rstd (g - xhat * sum(g xhat))
    dy = sum(np.asarray(d, np.float64) for d in dys)
    r = 1 / np.sqrt((x * x).mean(-1) + eps)
    xhat = x * r[:, None]
    g = dy * w
    return r[:, None] * (g - xhat * (g * xhat).sum(-1, keepdims=True)), dw


def _bwd_dw_from_g(dys, dr_out, x, w, eps, rstd=None, from_y=False, slots=None, xs=None,
                   acc=np.float64):
    dr, _ = ref.add_rmsnorm_bwd(dys, dr_out, x, w, eps, rstd, from_y, slots, xs, acc)
    dy = sum(np.asarray(d, np.float64) for d in dys)
    xhat = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return dr, (dy * w * xhat).sum(0)  # multiplies by w once too often


def _fwd_sum_not_mean(r_in, delta, w, eps, out_dtype="f32", acc=np.float64, slots=None, r_dtype="f32"):
    r = np.asarray(r_in, np.float64)
    inv = 1 / np.sqrt((r * r).sum(-1) + eps)  # sum instead of mean
    return r, ref.round_to(w * r * inv[:, None], out_dtype), inv, None


def _inv_freq_fp64(head_dim=128, theta=1e6):
    return (1.0 / (theta ** (np.arange(0, head_dim, 2) / head_dim))).astype(np.float32)


@pytest.mark.parametrize("check,overrides", [
    (golden.check_rope, dict(rope_fwd=_rope_wrong_sign)),
    (golden.check_rope, dict(rope_fwd=_rope_swapped_halves)),
    (golden.check_rope, dict(rope_angles=_angles_fp64)),
    (golden.check_rmsnorm_f32, dict(add_rmsnorm_bwd=_bwd_no_proj_mean)),
    (golden.check_rmsnorm_f32, dict(add_rmsnorm_bwd=_bwd_dw_from_g)),
    (golden.check_rmsnorm_f32, dict(add_rmsnorm_fwd=_fwd_sum_not_mean)),
    (golden.check_inv_freq, dict(default_inv_freq=_inv_freq_fp64)),
], ids=["rope_sign", "rope_halves", "rope_fp64_angle", "norm_proj_mean", "norm_dw_times_w",
        "norm_sum_not_mean", "inv_freq_numpy_pow"])
def test_golden_checks_catch_planted_mistakes(check, overrides):
    mutant = _mutant(**overrides)
    if "add_rmsnorm_fwd" in overrides:  # rmsnorm_fwd calls it through module globals
        mutant.rmsnorm_fwd = _rebind(ref.rmsnorm_fwd, mutant)
    if "add_rmsnorm_bwd" in overrides:
        mutant.rmsnorm_bwd = _rebind(ref.rmsnorm_bwd, mutant)
    if "rope_angles" in overrides:
        mutant.rope_fwd = _rebind(ref.rope_fwd, mutant)
    with pytest.raises(AssertionError):
        check(mutant)
    check(ref)  # and the real oracle passes the same check
