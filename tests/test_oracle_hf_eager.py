"""Pins oracle/hf_eager.py (the PyTorch-eager restatement of HF's Qwen2RMSNorm / rotary path
that bench.py times as the CPU baseline) against HF transformers' own outputs: the golden
vectors of tests/golden/*.npz, written by tests/golden/make_golden.py from Qwen2RMSNorm,
Qwen2RotaryEmbedding and apply_rotary_pos_emb with torch autograd.

Both sides run the same fp32 torch arithmetic, so the comparisons are tight (1e-6 relative, bf16
bit-exact). Planted mistakes (sum instead of mean, the rotate_half sign, the weight applied
before the bf16 rounding, a dropped weight gradient) must each fail them."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import hf_eager

GOLD = Path(__file__).resolve().parent / "golden"
EPS = 1e-6


def load(name):
    return dict(np.load(GOLD / name))


def close(a, b, rel, what):
    a = a.detach().double().numpy() if isinstance(a, torch.Tensor) else np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    err = float(np.abs(a - b).max()) / max(float(np.abs(b).max()), 1e-30)
    assert err <= rel, f"{what}: max error {err:.3g} of max |ref| (limit {rel})"


def t32(a):
    return torch.from_numpy(np.asarray(a)).to(torch.float32)


def check_rms_norm():
    """rms_norm forward and its autograd gradients against HF's fp32 module (two shapes), and
    HF's bf16 module bit for bit (xhat rounded to bf16 before the weight)."""
    g = load("rmsnorm_f32.npz")
    for c in ("a", "b"):
        x = t32(g[f"{c}_x"]).requires_grad_()
        w = t32(g[f"{c}_w"]).requires_grad_()
        y = hf_eager.rms_norm(x, w, EPS)
        close(y, g[f"{c}_y"], 1e-6, f"{c} y")
        dx, dw = torch.autograd.grad(y, [x, w], t32(g[f"{c}_dy"]))
        close(dx, g[f"{c}_dx"], 1e-6, f"{c} dx")
        close(dw, g[f"{c}_dw"], 1e-6, f"{c} dw")
    b = load("rmsnorm_bf16.npz")
    y = hf_eager.rms_norm(t32(b["x"]).to(torch.bfloat16), t32(b["w"]).to(torch.bfloat16), EPS)
    assert y.dtype == torch.bfloat16
    assert np.array_equal(y.double().numpy(), b["y"]), "bf16 y differs from HF's bits"


def check_rope():
    """rotary_cos_sin and apply_rotary_pos_emb against HF's Qwen2RotaryEmbedding +
    apply_rotary_pos_emb, forward and gradients, positions up to 32752."""
    g = load("rope.npz")
    inv = torch.from_numpy(g["inv_freq"])
    pos = torch.from_numpy(g["pos"])
    cos, sin = hf_eager.rotary_cos_sin(inv, pos, torch.float32)
    close(cos, g["cos"], 1e-6, "cos")
    close(sin, g["sin"], 1e-6, "sin")
    q, k = t32(g["q"]).requires_grad_(), t32(g["k"]).requires_grad_()
    qe, ke = hf_eager.apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=1)
    close(qe, g["q_embed"], 1e-6, "q_embed")
    close(ke, g["k_embed"], 1e-6, "k_embed")
    dq, dk = torch.autograd.grad([qe, ke], [q, k], [t32(g["dq"]), t32(g["dk"])])
    close(dq, g["q_grad"], 1e-6, "q grad")
    close(dk, g["k_grad"], 1e-6, "k grad")


def check_body_step():
    """body_step (the timed CPU leg: norms with their weight gradients, then one RoPE) returns
    HF's gradients: [dx, dw] per norm, then dq, dk."""
    n, r = load("rmsnorm_f32.npz"), load("rope.npz")
    xs = [t32(n["a_x"]), t32(n["b_x"])]
    ws = [t32(n["a_w"]), t32(n["b_w"])]
    dys = [t32(n["a_dy"]), t32(n["b_dy"])]
    out = hf_eager.body_step(xs, ws, t32(r["q"]), t32(r["k"]), dys, t32(r["dq"]), t32(r["dk"]),
                             torch.from_numpy(r["inv_freq"]), torch.from_numpy(r["pos"]), EPS)
    assert len(out) == 6
    for i, c in enumerate(("a", "b")):
        close(out[2 * i], n[f"{c}_dx"], 1e-6, f"{c} dx")
        close(out[2 * i + 1], n[f"{c}_dw"], 1e-6, f"{c} dw")
    close(out[4], r["q_grad"], 1e-6, "dq")
    close(out[5], r["k_grad"], 1e-6, "dk")


def test_rms_norm_matches_hf():
    check_rms_norm()


def test_rope_matches_hf():
    check_rope()


def test_body_step_matches_hf():
    check_body_step()


# ----------------------------------------------------------------------- planted mistakes

def _rms_norm_sum(x, weight, eps):
    h = x.to(torch.float32)
    var = h.pow(2).sum(-1, keepdim=True)  # sum instead of mean
    return weight * (h * torch.rsqrt(var + eps)).to(x.dtype)


def _rms_norm_weight_first(x, weight, eps):
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    return (weight.to(torch.float32) * h * torch.rsqrt(var + eps)).to(x.dtype)


def _rms_norm_frozen_weight(x, weight, eps):
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    return weight.detach() * (h * torch.rsqrt(var + eps)).to(x.dtype) + 0 * weight


def _rotate_half_sign(x):
    x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
    return torch.cat((x2, -x1), dim=-1)


@pytest.mark.parametrize("name,fn,check", [
    ("rms_norm", _rms_norm_sum, check_rms_norm),
    ("rms_norm", _rms_norm_weight_first, check_rms_norm),
    ("rms_norm", _rms_norm_sum, check_body_step),
    ("rms_norm", _rms_norm_frozen_weight, check_body_step),
    ("rotate_half", _rotate_half_sign, check_rope),
    ("rotate_half", _rotate_half_sign, check_body_step),
], ids=["sum_not_mean", "weight_before_rounding", "body_sum_not_mean", "body_no_dw",
        "rotate_half_sign", "body_rotate_half_sign"])
def test_planted_mistake_is_caught(monkeypatch, name, fn, check):
    monkeypatch.setattr(hf_eager, name, fn)
    with pytest.raises(AssertionError):
        check()
