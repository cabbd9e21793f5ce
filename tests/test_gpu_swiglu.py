"""SwiGLU kernels (esep_swiglu_fwd / esep_swiglu_bwd) and the recompute MLP on the GPU.

Kernels against the float64 oracle (oracle/swiglu_ref.py, which restates the reference's example
kernels, solution/swiglu.py:15-37) computed from the same rounded inputs: fp32 math and one
rounding at the store, so the error is at most half an output ulp plus fp32 rounding
(rtol 2^-8 bf16, 2^-11 fp16, 1e-6 fp32, plus atol 1e-6). Sizes cover the 8-element vector body
and the ragged tail; the in-place forms (out = gate, dgate = gate, dup = up) that the recompute
MLP uses must give the same bits as separate outputs.

The recompute MLP (packed._RecomputeMLP) against HF's Qwen2MLP under autograd: same output and
input gradients (fp16 tolerance), and no saved tensor of size [T, intermediate]
(reference test_body_recompute.py:145-189 checks the same for its NF4 version).
"""

import numpy as np
import pytest
import torch

from _util import DEV, gen, np64
from oracle import swiglu_ref as ref

pytestmark = pytest.mark.gpu

RTOL = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 1e-6}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32],
                         ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("n", [1, 7, 8, 1000, 8 * 1000 + 5, (1 << 20) + 3])
def test_swiglu_kernels_vs_oracle(n, dtype):
    from solution.body import _hip

    g_ = gen(n)
    g = (torch.randn(n, generator=g_) * 3).to(dtype).to(DEV)
    u = torch.randn(n, generator=g_).to(dtype).to(DEV)
    dh = torch.randn(n, generator=g_).to(dtype).to(DEV)
    h = torch.full_like(g, float("nan"))
    _hip.swiglu_fwd(g, u, h)
    dg, du = torch.full_like(g, float("nan")), torch.full_like(g, float("nan"))
    _hip.swiglu_bwd(dh, g, u, dg, du)
    rt = RTOL[dtype]
    np.testing.assert_allclose(np64(h), ref.swiglu_fwd(np64(g), np64(u)), rtol=rt, atol=1e-6)
    dg64, du64 = ref.swiglu_bwd(np64(dh), np64(g), np64(u))
    np.testing.assert_allclose(np64(dg), dg64, rtol=rt, atol=1e-6)
    np.testing.assert_allclose(np64(du), du64, rtol=rt, atol=1e-6)
    # in place: h into g, (dg, du) into (g, u) -- the same bits
    g2, u2 = g.clone(), u.clone()
    _hip.swiglu_fwd(g2, u2, g2)
    assert torch.equal(g2, h)
    g3, u3 = g.clone(), u.clone()
    _hip.swiglu_bwd(dh, g3, u3, g3, u3)
    assert torch.equal(g3, dg) and torch.equal(u3, du)


def test_swiglu_function_and_patch():
    """solution.swiglu (the reference's example API) on the HIP kernels: autograd against
    F.silu(g) * u in fp32, and patch_qwen2_mlp routes Qwen2MLP through it."""
    from transformers import Qwen2Config
    from transformers.models.qwen2 import modeling_qwen2

    from solution import swiglu as sw
    from solution.body import _hip

    g_ = gen(5)
    gate = torch.randn(64, 300, generator=g_).to(torch.float16).to(DEV).requires_grad_()
    up = torch.randn(64, 300, generator=g_).to(torch.float16).to(DEV).requires_grad_()
    dout = torch.randn(64, 300, generator=g_).to(torch.float16).to(DEV)
    out = sw.swiglu(gate, up)
    dg, du = torch.autograd.grad(out, [gate, up], dout)
    gf, uf = gate.detach().float().requires_grad_(), up.detach().float().requires_grad_()
    of = torch.nn.functional.silu(gf) * uf
    dgf, duf = torch.autograd.grad(of, [gf, uf], dout.float())
    for a, b in ((out, of), (dg, dgf), (du, duf)):
        torch.testing.assert_close(a.float(), b, atol=2e-3, rtol=1e-2)
    cfg = Qwen2Config(hidden_size=64, intermediate_size=160)
    mlp = modeling_qwen2.Qwen2MLP(cfg).to(DEV).half()
    x = torch.randn(3, 5, 64, generator=g_).to(torch.float16).to(DEV)
    want = mlp(x)
    original = modeling_qwen2.Qwen2MLP.forward
    try:
        sw.patch_qwen2_mlp()
        with _hip.count_launches() as names:
            got = mlp(x)
        assert names.count("_swiglu_fwd") == 1
    finally:
        modeling_qwen2.Qwen2MLP.forward = original
    torch.testing.assert_close(got, want, atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_recompute_mlp_matches_and_saves_no_intermediate(dtype):
    from transformers import Qwen2Config
    from transformers.models.qwen2 import modeling_qwen2

    from solution.body import packed

    T, H, I = 200, 128, 352
    cfg = Qwen2Config(hidden_size=H, intermediate_size=I)
    mlp = modeling_qwen2.Qwen2MLP(cfg).to(DEV).to(dtype)
    for prm in mlp.parameters():
        prm.requires_grad_(False)
    g_ = gen(9)
    x = torch.randn(1, T, H, generator=g_).to(dtype).to(DEV).requires_grad_()
    dout = torch.randn(1, T, H, generator=g_).to(dtype).to(DEV)
    want = mlp(x)
    (dx_want,) = torch.autograd.grad(want, [x], dout)

    saved = []

    def pack(t):
        saved.append((tuple(t.shape), t.data_ptr()))
        return t

    assert packed._mlp_layers(mlp, x) is not None
    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        got = packed._mlp(mlp, (x, x))
    (dx,) = torch.autograd.grad(got, [x], dout)
    tol = dict(atol=2e-3, rtol=1e-2) if dtype == torch.float16 else dict(atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(got, want, **tol)
    torch.testing.assert_close(dx, dx_want, **tol)
    # nothing [T, I] saved; the only I-sized tensors kept are the weights themselves (already
    # in the compute dtype, so kept without a copy)
    weights = {p.data_ptr() for p in mlp.parameters()}
    assert saved and all(T not in shp for shp, ptr in saved if I in shp), saved
    assert all(ptr in weights for shp, ptr in saved if I in shp), saved
    # a trainable projection sends the block to the non-recompute path
    mlp.up_proj.weight.requires_grad_(True)
    assert packed._mlp_layers(mlp, x) is None


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_recompute_mlp_autocast_casts_each_weight_once(dtype):
    """fp32 frozen weights under autocast (a LoRA run's fp32 master copy): the recompute MLP
    matches HF's Qwen2MLP under the same autocast, its forward casts each of the three weights
    once, and its backward (g and u recomputed, dh and dx products) casts none: it uses the
    forward's casts. Autocast caches only casts of leaves that require grad, so reading the
    frozen weights again in backward would cast them five more times."""
    from torch.utils._python_dispatch import TorchDispatchMode
    from transformers import Qwen2Config
    from transformers.models.qwen2 import modeling_qwen2

    from solution.body import packed

    T, H, I = 200, 128, 352
    mlp = modeling_qwen2.Qwen2MLP(Qwen2Config(hidden_size=H, intermediate_size=I)).to(DEV)
    for prm in mlp.parameters():
        prm.requires_grad_(False)
    g_ = gen(10)
    x = torch.randn(1, T, H, generator=g_).to(dtype).to(DEV).requires_grad_()
    dout = torch.randn(1, T, H, generator=g_).to(dtype).to(DEV)

    class Casts(TorchDispatchMode):
        """Records casts of [I, H] / [H, I] fp32 tensors (the weights) and counts products."""

        def __init__(self):
            super().__init__()
            self.casts, self.products = [], 0

        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            a = args[0] if args else None
            if (func == torch.ops.aten._to_copy.default and a.dtype == torch.float32
                    and I in a.shape and a.dim() == 2):
                self.casts.append(tuple(a.shape))
            if func in (torch.ops.aten.mm.default, torch.ops.aten.addmm.default):
                self.products += 1
            return func(*args, **(kwargs or {}))

    with torch.autocast("cuda", dtype=dtype):
        want = mlp(x)
        assert packed._mlp_layers(mlp, x) is not None
        fwd = Casts()
        with fwd:
            got = packed._mlp(mlp, (x, x))
    (dx_want,) = torch.autograd.grad(want, [x], dout)
    bwd = Casts()
    with bwd:
        (dx,) = torch.autograd.grad(got, [x], dout)
    assert sorted(fwd.casts) == sorted([(I, H), (I, H), (H, I)]), fwd.casts
    assert bwd.products >= 5 and bwd.casts == [], (bwd.products, bwd.casts)  # 3 recomputed + 2 dx
    tol = dict(atol=2e-3, rtol=1e-2) if dtype == torch.float16 else dict(atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(got, want, **tol)
    torch.testing.assert_close(dx, dx_want, **tol)


def test_swiglu_bench_shape():
    """The bench's SwiGLU workload (T = 8192 tokens x intermediate 8960, bf16: 73.4M elements,
    many grid-strided passes per thread): forward and backward on 2^20 sampled elements against
    the float64 oracle, at the same bar as the small sizes."""
    from solution.body import _hip

    n = 8192 * 8960
    g_ = gen(8960)
    g = (torch.randn(n, generator=g_) * 3).to(torch.bfloat16).to(DEV)
    u = torch.randn(n, generator=g_).to(torch.bfloat16).to(DEV)
    dh = torch.randn(n, generator=g_).to(torch.bfloat16).to(DEV)
    h = torch.full_like(g, float("nan"))
    _hip.swiglu_fwd(g, u, h)
    dg, du = torch.full_like(g, float("nan")), torch.full_like(g, float("nan"))
    _hip.swiglu_bwd(dh, g, u, dg, du)
    idx = torch.cat([torch.tensor([0, n - 1]), torch.randint(0, n, (1 << 20,), generator=gen(3))]).to(DEV)
    gs, us, dhs = np64(g[idx]), np64(u[idx]), np64(dh[idx])
    rt = RTOL[torch.bfloat16]
    np.testing.assert_allclose(np64(h[idx]), ref.swiglu_fwd(gs, us), rtol=rt, atol=1e-6)
    dg64, du64 = ref.swiglu_bwd(dhs, gs, us)
    np.testing.assert_allclose(np64(dg[idx]), dg64, rtol=rt, atol=1e-6)
    np.testing.assert_allclose(np64(du[idx]), du64, rtol=rt, atol=1e-6)
    assert not torch.isnan(h).any() and not torch.isnan(dg).any() and not torch.isnan(du).any()
