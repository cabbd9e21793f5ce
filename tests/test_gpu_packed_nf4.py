"""NF4 base projections through the patch point, restating the reference's tests of that route
(solution/test_body_packed.py:388-475: every q/k/v/o base through nf4.linear4bit, q/k/v fused
into one nf4.linear4bit_multi call; test_body_recompute.py:103-143, :222-247: the recompute MLP
on NF4 projections with gate and up dequantized in one launch, and its guards).

bitsandbytes and peft are not installed, so the tiny Qwen2 of test_gpu_packed gets stand-ins:
every decoder projection becomes `Linear4bit` below (bitsandbytes' Linear4bit interface: an NF4
double-quant weight with its quant_state, compute dtype fp16, a frozen fp32 bias; forward as
bitsandbytes 0.50's), q_proj and v_proj are then wrapped in test_gpu_packed_lora's LoRA
stand-in, and only the LoRA weights train (with a gradient into the embedding output, as peft's
k-bit preparation arranges). The stand-in's weight is quantized and dequantized by the CPU
oracle (oracle/nf4_ref.py), not by the kernel under test, so HF's original forward on it is an
independent reference. fp16 autocast, as the reference's QLoRA runs."""

import types

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import test_gpu_packed as tp
import test_gpu_packed_lora as tl
from oracle import nf4_ref as nref

pytestmark = pytest.mark.gpu


class Linear4bit(torch.nn.Module):
    """bitsandbytes' Linear4bit as the patch point and HF's forward see it (class name and
    attributes): weight = the packed NF4 bytes with a bitsandbytes-shaped quant_state,
    compute_dtype fp16, compute_type_is_set, a frozen bias; forward as bitsandbytes 0.50's
    (x to the compute dtype, the bias cast in place to it, F.linear on the dequantized weight,
    the output back in x's dtype), the weight dequantized once by the CPU oracle."""

    def __init__(self, lin):
        super().__init__()
        dev = lin.weight.device
        N, K = lin.weight.shape
        w = lin.weight.detach().to(torch.float16).float().cpu().numpy()
        packed, absmax, absmax2, code2, offset = nref.quantize_nf4(w)

        def to_dev(a):
            return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

        self.in_features, self.out_features = K, N
        self.weight = torch.nn.Parameter(to_dev(packed).reshape(-1, 1), requires_grad=False)
        self.weight.quant_state = types.SimpleNamespace(
            quant_type="nf4", blocksize=64, nested=True, shape=torch.Size((N, K)),
            absmax=to_dev(absmax), code=to_dev(nref.NF4),
            offset=to_dev(np.array(offset, dtype=np.float32)),
            state2=types.SimpleNamespace(absmax=to_dev(absmax2), code=to_dev(code2),
                                         blocksize=256))
        w16 = nref.dequantize_nf4(packed, absmax, absmax2, code2, offset).reshape(N, K)
        self.register_buffer("w16", to_dev(w16), persistent=False)
        self.bias = None if lin.bias is None else \
            torch.nn.Parameter(lin.bias.detach().float().clone(), requires_grad=False)
        self.compute_dtype = torch.float16
        self.compute_type_is_set = True

    def forward(self, x):
        inp = x.dtype
        x = x.to(self.compute_dtype)
        if self.bias is not None and self.bias.dtype != self.compute_dtype:
            self.bias.data = self.bias.data.to(self.compute_dtype)
        return F.linear(x, self.w16.to(x.dtype), self.bias).to(inp)


def _build_nf4():
    model = tp._build("frozen")
    for p in model.parameters():
        p.requires_grad_(False)
    for layer in model.model.layers:
        for parent in (layer.self_attn, layer.mlp):
            for name, lin in list(parent.named_children()):
                if isinstance(lin, torch.nn.Linear):
                    setattr(parent, name, Linear4bit(lin))
        attn = layer.self_attn
        attn.q_proj = tl.LoraLinear(attn.q_proj)
        attn.v_proj = tl.LoraLinear(attn.v_proj)
    model.model.embed_tokens.register_forward_hook(lambda m, i, o: o.requires_grad_(True))
    model.train()
    return model


def _patched():
    from solution.body import patch

    patch()


def _nf4_counts(names):
    return {k: names.count(k) for k in ("_nf4_dequant", "_nf4_dequant_multi", "_rope_kernel",
                                        "_add_rmsnorm_bwd", "_swiglu_fwd", "_swiglu_bwd")}


def test_nf4_api_matches_the_module_forward():
    """nf4.linear4bit / linear4bit_multi / dequant_multi on Linear4bit modules: the forward's
    values are the module's own forward's bits (bit-exact dequant, the same fp16 GEMM), dx and
    the bias gradient those of the dense fp16 linear."""
    from solution import nf4

    torch.manual_seed(3)
    lins = [torch.nn.Linear(256, n, bias=True, device="cuda") for n in (256, 128, 128)]
    mods = [Linear4bit(lin) for lin in lins]
    assert all(nf4.is_linear4bit(m) for m in mods)
    assert not nf4.is_linear4bit(lins[0])
    x = torch.randn(50, 256, device="cuda", dtype=torch.float16)
    for m in mods:
        assert torch.equal(nf4.linear4bit(x, m, keep_fp16=True), m(x))
    w_cat = nf4.dequant_multi(mods)
    assert torch.equal(w_cat, torch.cat([m.w16 for m in mods]))
    for m in mods:
        m.bias.requires_grad_(True)
    xg = x.clone().requires_grad_()
    ys = nf4.linear4bit_multi(xg, mods)
    dys = [torch.randn_like(y) for y in ys]
    grads = torch.autograd.grad(ys, [xg] + [m.bias for m in mods], dys)
    xr = x.clone().requires_grad_()
    refs = [F.linear(xr, m.w16, m.bias.to(torch.float16)) for m in mods]
    for y, r in zip(ys, refs):
        assert (y - r).abs().max() <= 1e-2 * r.abs().max()
    rgrads = torch.autograd.grad(refs, [xr] + [m.bias for m in mods], dys)
    for g, r in zip(grads, rgrads):
        assert (g.float() - r.float()).abs().max() <= 1e-2 * r.float().abs().max()
    # fewer than MIN_ROWS rows, or an fp32 compute dtype without fp16 autocast: the module
    mods[0].compute_dtype = torch.float32
    assert torch.equal(nf4.linear4bit(x, mods[0]), mods[0](x))
    mods[0].compute_dtype = torch.float16
    assert torch.equal(nf4.linear4bit(x[:3], mods[0]), mods[0](x[:3]))
    assert nf4.patch() is False  # no bitsandbytes class to patch in this environment


@pytest.mark.parametrize("left", [False, True], ids=["right_pad", "left_pad"])
def test_nf4_lora_matches_original(left):
    """The NF4 + LoRA model through the patch point against HF's original forward (reference
    test_body_packed.py's nf4_lora variant): q/k/v as one fused call per layer and forward,
    o / gate / up / down through linear4bit, the recompute MLP's gate and up in one dequant."""
    from solution.body import _hip

    _patched()
    model = _build_nf4()
    ids, mask, labels = tp._batch(left)
    with tp._original_forward():
        ref = tp._run(model, ids, mask, labels)
    with _hip.count_launches() as names:
        new = tp._run(model, ids, mask, labels)
    tp._compare(ref, new, mask)
    c = _nf4_counts(names)
    n = model.config.num_hidden_layers
    # per layer: forward (x2: the loss pass and the hidden pass) one multi (q/k/v) + o, gate,
    # up, down; backward one multi (q/k/v) + o + down + one multi (gate/up)
    assert c["_nf4_dequant_multi"] == n * (2 * 1 + 2), c
    assert c["_nf4_dequant"] == n * (2 * 4 + 2), c
    assert c["_rope_kernel"] == 3 * n, c
    assert c["_add_rmsnorm_bwd"] > 0 and c["_swiglu_bwd"] == n, c


def test_nf4_linear4bit_route(monkeypatch):
    """With the fused q/k/v call off, every NF4 base projection (q, k, v, o and the recompute
    MLP's gate, up, down) runs as nf4.linear4bit(x16 [T, in], module, keep_fp16=True)
    (reference test_nf4_linear4bit_hook); results match the original."""
    from solution import nf4
    from solution.body import packed

    _patched()
    calls = []
    real = nf4.linear4bit

    def recording(x, module, keep_fp16=False):
        assert keep_fp16 and x.dtype == torch.float16 and x.dim() == 2
        calls.append(type(module).__name__)
        return real(x, module, keep_fp16=keep_fp16)

    monkeypatch.setattr(nf4, "linear4bit", recording)
    monkeypatch.setattr(packed, "_qkv", lambda *a: None)
    model = _build_nf4()
    ids, mask, labels = tp._batch()
    with tp._original_forward():
        ref = tp._run(model, ids, mask, labels)
    new = tp._run(model, ids, mask, labels)
    tp._compare(ref, new, mask)
    per_layer = 7 if packed.RECOMPUTE_MLP else 4
    assert len(calls) == per_layer * model.config.num_hidden_layers * 2, len(calls)
    assert set(calls) == {"Linear4bit"}


@pytest.mark.parametrize("left", [False, True], ids=["right_pad", "left_pad"])
def test_nf4_qkv_fused_matches_separate(left, monkeypatch):
    """q/k/v fused into one linear4bit_multi call per layer and forward against the separate
    calls and the original (reference test_nf4_qkv_multi_hook): q's LoRA term still goes to
    RoPE, v's is added out of place, and the norm backward sums the q / v LoRA gradients and the
    one base gradient itself."""
    from solution import nf4
    from solution.body import _hip, packed

    _patched()
    model = _build_nf4()
    ids, mask, labels = tp._batch(left)
    with tp._original_forward():
        ref = tp._run(model, ids, mask, labels)
    with monkeypatch.context() as m:
        m.setattr(packed, "_qkv", lambda *a: None)
        sep = tp._run(model, ids, mask, labels)
    calls = []
    real = nf4.linear4bit_multi

    def recording(x, modules, split=True):
        calls.append(tuple(type(md).__name__ for md in modules))
        return real(x, modules, split)

    monkeypatch.setattr(nf4, "linear4bit_multi", recording)
    with _hip.count_launches() as names:
        new = tp._run(model, ids, mask, labels)
    tp._compare(ref, new, mask)
    tp._compare(sep, new, mask)
    n = model.config.num_hidden_layers
    assert calls == [("Linear4bit",) * 3] * (2 * n), calls
    assert names.count("_rope_kernel") == 3 * n


def test_recompute_mlp_nf4(monkeypatch):
    """RECOMPUTE_MLP on NF4 projections against the same model without it: the forward is the
    same computation (bitwise the same hidden states and loss), the gradients within fp16
    noise (gate and up dequantized in one launch, dx as one mm + addmm), and both against the
    original (reference test_recompute_dequant_multi)."""
    from solution import nf4
    from solution.body import packed

    _patched()
    model = _build_nf4()
    ids, mask, labels = tp._batch()
    with tp._original_forward():
        ref = tp._run(model, ids, mask, labels)
    monkeypatch.setattr(packed, "RECOMPUTE_MLP", False)
    off = tp._run(model, ids, mask, labels)
    monkeypatch.setattr(packed, "RECOMPUTE_MLP", True)
    calls = []
    real = nf4.dequant_multi

    def recording(modules):
        calls.append(len(modules))
        return real(modules)

    monkeypatch.setattr(nf4, "dequant_multi", recording)
    on = tp._run(model, ids, mask, labels)
    assert calls == [2] * model.config.num_hidden_layers, calls
    assert torch.equal(on["hidden"], off["hidden"]) and torch.equal(on["loss"], off["loss"])
    worst = max(tp._rel(on["grads"][k], off["grads"][k]) for k in off["grads"])
    assert worst < 1e-2, worst
    tp._compare(ref, on, mask)


def test_recompute_mlp_nf4_guards(monkeypatch):
    """_mlp_layers on the NF4 MLP: taken under fp16 autocast with grad mode on; not with
    RECOMPUTE_MLP off, under no_grad, for an fp32 x, without autocast, for a non-silu config
    (reference test_recompute_guards)."""
    from solution.body import packed

    model = _build_nf4()
    mlp = model.model.layers[0].mlp
    x = torch.randn(1, 8, 256, device="cuda", dtype=torch.float16)
    with torch.autocast("cuda", dtype=torch.float16):
        assert packed._mlp_layers(mlp, x) is not None
        with torch.no_grad():
            assert packed._mlp_layers(mlp, x) is None
        assert packed._mlp_layers(mlp, x.float()) is None
        old = mlp.config.hidden_act
        mlp.config.hidden_act = "gelu"
        try:
            assert packed._mlp_layers(mlp, x) is None
        finally:
            mlp.config.hidden_act = old
        monkeypatch.setattr(packed, "RECOMPUTE_MLP", False)
        assert packed._mlp_layers(mlp, x) is None
        monkeypatch.setattr(packed, "RECOMPUTE_MLP", True)
    assert packed._mlp_layers(mlp, x) is None  # no autocast
