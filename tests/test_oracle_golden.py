"""The CPU oracle against HF transformers' own outputs (tests/golden/*.npz, written by
tests/golden/make_golden.py from Qwen2RMSNorm, Qwen2RotaryEmbedding and
apply_rotary_pos_emb with torch autograd). HF computes in fp32, the oracle in fp64: the
tolerances are fp32-level, far below what a wrong term, sign, index or operand would give
(tests/test_oracle_math.py plants such mistakes and checks these comparisons catch them)."""

from pathlib import Path

import numpy as np
import pytest

from oracle import norm_rope_ref as ref

GOLD = Path(__file__).resolve().parent / "golden"
EPS = 1e-6


def load(name):
    return dict(np.load(GOLD / name))


def close(a, b, rel, what):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    scale = max(float(np.abs(b).max()), 1e-30)
    err = float(np.abs(a - b).max()) / scale
    assert err <= rel, f"{what}: max error {err:.3g} of max |ref| (limit {rel})"


# ------------------------------------------------------------------------- checks (reused by
# the mutation tests in test_oracle_math.py, which swap in a broken oracle function)

def check_rmsnorm_f32(o=ref):
    g = load("rmsnorm_f32.npz")
    for c in ("a", "b"):
        x, w, dy = g[f"{c}_x"], g[f"{c}_w"], g[f"{c}_dy"]
        y, rstd = o.rmsnorm_fwd(x, w, EPS)
        close(y, g[f"{c}_y"], 2e-6, f"{c} y")
        dx, dw = o.rmsnorm_bwd(dy, x, w, EPS)
        close(dx, g[f"{c}_dx"], 2e-5, f"{c} dx")
        close(dw, g[f"{c}_dw"], 2e-5, f"{c} dw")
        dx2, dw2 = o.rmsnorm_bwd(dy, x, w, EPS, rstd=rstd)
        close(dx2, g[f"{c}_dx"], 2e-5, f"{c} dx (saved rstd)")


def check_rope(o=ref):
    g = load("rope.npz")
    B, HQ, S, D = g["q"].shape
    HK = g["k"].shape[1]
    pos = g["pos"].reshape(-1)
    ang = o.rope_angles(pos, g["inv_freq"]).astype(np.float64)
    cos_hf = g["cos"].reshape(B * S, D)[:, : D // 2]
    sin_hf = g["sin"].reshape(B * S, D)[:, : D // 2]
    close(np.cos(ang), cos_hf, 5e-7, "cos")
    close(np.sin(ang), sin_hf, 5e-7, "sin")

    def tok(x, h):  # [B, H, S, D] -> [B*S, H, D]
        return x.transpose(0, 2, 1, 3).reshape(B * S, h, D)

    for name, x, h, out, dout, grad in (("q", g["q"], HQ, g["q_embed"], g["dq"], g["q_grad"]),
                                        ("k", g["k"], HK, g["k_embed"], g["dk"], g["k_grad"])):
        close(o.rope_fwd(tok(x, h), pos, g["inv_freq"]), tok(out, h), 2e-6, f"{name} embed")
        close(o.rope_fwd(tok(dout, h), pos, g["inv_freq"], sign=-1.0), tok(grad, h), 2e-6,
              f"{name} grad")


def check_inv_freq(o=ref):
    g = load("inv_freq.npz")
    for key, want in g.items():
        d, theta = key.split("_")
        got = o.default_inv_freq(int(d[1:]), float(theta[5:]))
        assert got.dtype == np.float32 and np.array_equal(got, want), key


# ------------------------------------------------------------------------- tests

def test_rmsnorm_matches_hf():
    check_rmsnorm_f32()


def test_rmsnorm_bf16_semantics():
    """HF's bf16 Qwen2RMSNorm rounds xhat to bf16 before * w and rounds again; the kernels
    round once. Restating HF's double rounding reproduces HF bit for bit (except where HF's
    fp32 xhat and the fp64 one straddle a bf16 rounding boundary); the single-rounding oracle
    differs from HF by at most one bf16 ulp."""
    g = load("rmsnorm_bf16.npz")
    x, w, y_hf = g["x"], g["w"], g["y"]
    _, _, rstd, _ = ref.add_rmsnorm_fwd(x, None, np.ones_like(w), EPS)
    xhat = x * rstd[:, None]
    double = ref.round_to(w[None, :] * ref.round_to(xhat, "bf16"), "bf16")
    assert (double == y_hf).mean() > 0.999
    single, _ = ref.rmsnorm_fwd(x, w, EPS, "bf16")
    ulp = np.abs(y_hf) * 2.0 ** -7
    assert (np.abs(single - y_hf) <= ulp + 1e-30).all()


def test_rope_matches_hf():
    check_rope()


def test_inv_freq_matches_hf_exactly():
    check_inv_freq()


@pytest.mark.parametrize("name", ["rmsnorm_f32.npz", "rmsnorm_bf16.npz", "rope.npz", "inv_freq.npz"])
def test_fixture_is_data_only(name):
    """Fixtures load without pickle (plain arrays)."""
    with np.load(GOLD / name, allow_pickle=False) as f:
        assert len(f.files) > 0
