"""The packed decoder's LoRA route and the reference's remaining patch-point tests, on the GPU.

peft is not installed, so q_proj / v_proj become a stand-in LoRA wrapper with peft's LoRA layer
attributes and forward (base_layer(x) + lora_B(lora_A(dropout(x))) * scaling, one "default"
adapter): the packed path routes it through lora.py (q's term into the RoPE kernel as q_delta,
v's added into its base output, the input norm fanning out to 5 consumers; reference
packed.py:240-352, :705), and HF's original forward runs the wrapper's own forward.

Restated from the reference (solution/test_body_packed.py, test_body_norm_save.py):
  test_lora_route_matches_original      the tiny model vs the original forward (:216-268)
  test_no_16bit_grad_adds               no 16-bit add / fill kernels in a fwd + bwd (:497-536)
  test_partial_fallback_warnings        warn once per (piece, reason), in training (:621-670)
  test_norm_save_output_saved_tensors   no fp32 [T, H] residual saved with NORM_SAVE_OUTPUT
                                        (test_body_norm_save.py:115-145)
  test_norm_save_output_matches         on / off: the same forward, close gradients (:51-78)
  test_scatter_in_place_grads           the scatter back to [B, L, H] (:148-171)
"""

import contextlib
import logging

import pytest
import torch

import test_gpu_packed as tp

pytestmark = pytest.mark.gpu

HID = 256
R, ALPHA = 8, 16


class LoraLinear(torch.nn.Module):
    """peft's LoRA Linear layer as far as the packed route and HF's forward see it."""

    def __init__(self, base, r=R, alpha=ALPHA, dropout=0.0):
        super().__init__()
        self.base_layer = base
        dev = base.weight.device
        self.lora_A = torch.nn.ModuleDict(
            {"default": torch.nn.Linear(base.in_features, r, bias=False, device=dev)})
        self.lora_B = torch.nn.ModuleDict(
            {"default": torch.nn.Linear(r, base.out_features, bias=False, device=dev)})
        self.lora_dropout = torch.nn.ModuleDict({"default": torch.nn.Dropout(dropout)})
        self.scaling = {"default": alpha / r}
        self.active_adapters = ["default"]
        self.disable_adapters = False
        self.merged = False
        with torch.no_grad():  # B is zero at peft's init; a nonzero B makes the term visible
            self.lora_B["default"].weight.normal_(0, 0.05)

    def forward(self, x):
        out = self.base_layer(x)
        a, b = self.lora_A["default"], self.lora_B["default"]
        return out + b(a(self.lora_dropout["default"](x))) * self.scaling["default"]


def _build_lora(dropout=0.0, weights="regular", input_grads=False):
    """The tiny Qwen2 with LoRA wrappers on q_proj / v_proj (only their A and B train).
    input_grads: the embedding output requires a gradient, as peft's k-bit preparation
    (enable_input_require_grads) arranges in the reference's runs."""
    model = tp._build("frozen")
    if input_grads:
        model.model.embed_tokens.register_forward_hook(lambda m, i, o: o.requires_grad_(True))
    for p in model.parameters():
        p.requires_grad_(False)
    for layer in model.model.layers:
        attn = layer.self_attn
        attn.q_proj = LoraLinear(attn.q_proj, dropout=dropout)
        attn.v_proj = LoraLinear(attn.v_proj, dropout=dropout)
        if weights == "zeros_tiny":  # exact channels in save-output mode (K > 0)
            with torch.no_grad():
                for i, norm in enumerate((layer.input_layernorm, layer.post_attention_layernorm)):
                    w = norm.weight
                    w[[0, 17 + i]] = 0.0
                    w[[5, 99]] = torch.tensor([1e-5, -3e-4], device=w.device)
                    w[200] = 2e-3  # above the threshold: recovered from y
    model.train()
    return model


@contextlib.contextmanager
def _lora_forwards():
    """Counts LoRA-term forwards of lora.py (each casts its A and B once)."""
    from solution.body import lora

    calls, orig = [], lora.cast_lora_weights

    def counting(*a, **k):
        calls.append(1)
        return orig(*a, **k)

    lora.cast_lora_weights = counting
    try:
        yield calls
    finally:
        lora.cast_lora_weights = orig


@pytest.mark.parametrize("left", [False, True], ids=["right_pad", "left_pad"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_lora_route_matches_original(left, dtype):
    from solution.body import _hip, patch

    patch()
    model = _build_lora()
    ids, mask, labels = tp._batch(left)
    with tp._original_forward():
        ref = tp._run(model, ids, mask, labels, dtype=dtype)
    with _hip.count_launches() as names, _lora_forwards() as lora_calls:
        new = tp._run(model, ids, mask, labels, dtype=dtype)
    tol = dict(tol_h=5e-3, tol_loss=1e-3, tol_g=2e-2) if dtype == torch.float16 else \
        dict(tol_h=3e-2, tol_loss=5e-3, tol_g=6e-2)
    tp._compare(ref, new, mask, **tol)
    assert len(ref["grads"]) == 4 * model.config.num_hidden_layers  # A and B of q and v
    n_layers = model.config.num_hidden_layers
    # q and v LoRA terms per layer in both forwards (loss and hidden states)
    assert len(lora_calls) == 2 * 2 * n_layers, len(lora_calls)
    c = tp._counts(names)
    assert c["_rope_kernel"] == 3 * n_layers, c
    # one backward per norm except the first input norm (neither its input, the frozen
    # embedding's output, nor its weight needs a gradient); each sums its consumers' grads,
    # the LoRA inputs' among them
    assert c["_add_rmsnorm_bwd"] == 2 * n_layers, c


def test_lora_route_with_dropout():
    """p = 0.05: the dropout kernels run in both directions (mask regenerated in backward) and
    the LoRA gradients are finite and nonzero."""
    from solution.body import _hip, patch

    patch()
    model = _build_lora(dropout=0.05)
    ids, mask, labels = tp._batch()
    with _hip.count_launches() as names:
        new = tp._run(model, ids, mask, labels)
    n_layers = model.config.num_hidden_layers
    # forward: q and v terms per layer in both forwards; backward: the mask applied to dx
    # (one pass with the regenerated input) in every layer whose LoRA input needs a gradient,
    # and in layer 0 (whose input does not) only the input regenerated for dA
    assert names.count("_lora_dropout_bwd") == 2 * (n_layers - 1), names
    assert names.count("_lora_dropout_fwd") == 2 * 2 * n_layers + 2, names
    for g in new["grads"].values():
        assert torch.isfinite(g).all() and g.abs().max() > 0


@pytest.mark.parametrize("recompute", [False, True], ids=["mlp", "recompute_mlp"])
def test_no_16bit_grad_adds(recompute, monkeypatch):
    """Reference test_no_fp16_grad_adds: with the LoRA route (dropout 0.05) the gradients of the
    normed x from its consumers (q / k / v, q / v LoRA; gate / up) are summed inside the norm
    backward kernel, so one fp16 forward + backward launches no 16-bit element-wise add and no
    16-bit zero fill."""
    from torch.profiler import ProfilerActivity, profile

    from solution.body import packed, patch

    patch()
    model = _build_lora(dropout=0.05)
    ids, mask, labels = tp._batch()
    monkeypatch.setattr(packed, "RECOMPUTE_MLP", recompute)
    tp._run(model, ids, mask, labels)  # warm
    model.zero_grad(set_to_none=True)
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        with torch.autocast("cuda", dtype=torch.float16):
            out = model(input_ids=ids, attention_mask=mask, labels=labels, use_cache=False)
        out.loss.backward()
        torch.cuda.synchronize()
    names = [e.name for e in prof.events() if e.device_type.name == "CUDA"]
    assert any("k_rmsnorm_bwd" in n for n in names), sorted(set(names))[:40]
    bad = [n for n in names for t in ("Half", "BFloat16")
           if f"CUDAFunctor_add<c10::{t}>" in n or f"FillFunctor<c10::{t}>" in n]
    assert not bad, bad[:5]


def _fallback_messages(caplog):
    return [r.getMessage() for r in caplog.records if " not used (" in r.getMessage()]


def test_partial_fallback_warnings(monkeypatch, caplog):
    """A guard that sends one decoder piece to HF / torch warns once per (piece, reason) while
    training, naming the first layer; the normal path warns nothing; eval forwards warn
    nothing; a 16-bit embedding output under an fp32 embedding weight is named too."""
    from solution.body import packed, patch

    patch()
    caplog.set_level(logging.WARNING, logger="solution.body.packed")
    monkeypatch.setattr(packed, "_warned", set())
    model = _build_lora()
    ids, mask, labels = tp._batch()
    tp._run(model, ids, mask, labels)
    assert _fallback_messages(caplog) == []

    base = model.model
    layer = base.layers[1]
    hooks = [layer.post_attention_layernorm.register_forward_hook(lambda m, a, o: None),
             layer.mlp.register_forward_hook(lambda m, a, o: None),
             layer.self_attn.q_proj.register_forward_hook(lambda m, a, o: None)]
    try:
        tp._run(model, ids, mask, labels)
        msgs = _fallback_messages(caplog)
        assert len(msgs) == 3, msgs
        assert all("first at layer 1" in m for m in msgs), msgs
        assert {m.split(" not used")[0].split(": ")[-1] for m in msgs} == \
            {"norm kernel", "recompute MLP", "LoRA path"}, msgs
        tp._run(model, ids, mask, labels)  # once per process
        assert len(_fallback_messages(caplog)) == 3
        monkeypatch.setattr(packed, "_warned", set())
        model.eval()
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
            base(input_ids=ids, attention_mask=mask, use_cache=False)
        assert len(_fallback_messages(caplog)) == 3
        model.train()
    finally:
        for h in hooks:
            h.remove()
    monkeypatch.setattr(packed, "_warned", set())
    h = base.embed_tokens.register_forward_hook(lambda m, a, o: o.half())
    try:
        tp._run(model, ids, mask, labels)
    finally:
        h.remove()
    assert any("fp32 residual stream not used (embedding output is torch.float16; first at "
               "layer embedding)" in m for m in _fallback_messages(caplog)), caplog.text


def _saved_per_layer(model, ids, mask):
    """{layer: {storage ptr: (nbytes, dtype, shape)}} of one fp16 forward, parameters
    excluded (reference test_body_norm_save.py:81-112)."""
    from solution.body import packed

    params = {p.untyped_storage().data_ptr() for p in model.parameters()}
    per, cur = {}, [None]
    orig = packed._layer

    def wrap(*a, **k):
        cur[0] = len(per)
        per[cur[0]] = {}
        try:
            return orig(*a, **k)
        finally:
            cur[0] = None

    def pack(x):
        if cur[0] is not None and x.is_cuda:
            st = x.untyped_storage()
            if st.data_ptr() not in params:
                per[cur[0]][st.data_ptr()] = (st.nbytes(), x.dtype, tuple(x.shape))
        return x

    packed._layer = wrap
    try:
        with torch.autograd.graph.saved_tensors_hooks(pack, lambda x: x), \
                torch.autocast("cuda", dtype=torch.float16):
            out = model(input_ids=ids, attention_mask=mask, use_cache=False)
        del out
    finally:
        packed._layer = orig
    return per


@pytest.mark.parametrize("recompute", [False, True], ids=["mlp", "recompute_mlp"])
def test_norm_save_output_saved_tensors(recompute, monkeypatch):
    """Per decoder layer: two fp32 [T, H] residuals are saved with NORM_SAVE_OUTPUT off and
    none with it on (layer 0 keeps the embedding output: its input norm has no delta)."""
    from solution.body import packed

    model = _build_lora(weights="zeros_tiny", input_grads=True)
    ids, mask, _ = tp._batch()
    T = int(mask.sum())
    monkeypatch.setattr(packed, "RECOMPUTE_MLP", recompute)
    res = {}
    for save in (False, True):
        monkeypatch.setattr(packed, "NORM_SAVE_OUTPUT", save)
        res[save] = _saved_per_layer(model, ids, mask)
    for save, per in res.items():
        assert per, "no decoder layer ran through the packed path"
        for layer, st in per.items():
            fp32 = [v for v in st.values() if v[1] == torch.float32 and v[0] >= T * HID * 4]
            want = (1 if layer == 0 else 0) if save else 2
            assert len(fp32) == want, (save, layer, fp32)
    for layer in res[False]:
        if layer > 0:
            b_off = sum(v[0] for v in res[False][layer].values())
            b_on = sum(v[0] for v in res[True][layer].values())
            assert b_off - b_on >= T * HID * 4, (b_off, b_on)


@pytest.mark.parametrize("weights", ["regular", "zeros_tiny"])
def test_norm_save_output_matches(weights, monkeypatch):
    """NORM_SAVE_OUTPUT on and off: the same forward bit for bit, LoRA gradients within fp16
    noise of each other, both against the original forward; zeros_tiny weights give exact
    channels (K > 0) and regular ones none."""
    from solution.body import norm_rope, packed, patch

    patch()
    model = _build_lora(weights=weights)
    ids, mask, labels = tp._batch()
    with tp._original_forward():
        ref = tp._run(model, ids, mask, labels)
    monkeypatch.setattr(packed, "NORM_SAVE_OUTPUT", False)
    off = tp._run(model, ids, mask, labels)
    monkeypatch.setattr(packed, "NORM_SAVE_OUTPUT", True)
    on = tp._run(model, ids, mask, labels)
    tp._compare(ref, off, mask)
    tp._compare(ref, on, mask)
    assert torch.equal(on["hidden"], off["hidden"]) and torch.equal(on["loss"], off["loss"])
    assert max(tp._rel(on["grads"][n], off["grads"][n]) for n in off["grads"]) < 1e-2
    ks = [norm_rope.special_channels(n.weight)[1] for layer in model.model.layers
          for n in (layer.input_layernorm, layer.post_attention_layernorm)]
    assert (sum(ks) > 0) == (weights == "zeros_tiny"), ks


def test_scatter_in_place_grads():
    """The scatter back to [B, L, H] (index_copy_ into fresh zeros): the hidden-state gradient
    reaches the packed tokens' embedding outputs as in the original forward."""
    from solution.body import patch

    patch()
    model = _build_lora()
    ids, mask, _ = tp._batch()
    base = model.model
    w = torch.randn(*ids.shape, HID, device="cuda") * mask[..., None]  # pads weigh 0
    grads = []
    for original in (True, False):
        ctx = tp._original_forward() if original else contextlib.nullcontext()
        emb = []
        # the frozen embedding's output made to require a gradient (what peft's input-grad
        # hook does), so that it collects one
        hook = base.embed_tokens.register_forward_hook(
            lambda m, i, o: (o.requires_grad_(), emb.append(o))[1])
        try:
            with ctx, torch.autocast("cuda", dtype=torch.float16):
                h = base(input_ids=ids, attention_mask=mask, use_cache=False).last_hidden_state
            (h.float() * w).sum().backward()
        finally:
            hook.remove()
        g = emb[0].grad
        grads.append(g.reshape(-1, HID)[mask.reshape(-1).bool()] if original else g.reshape(-1, HID))
        model.zero_grad(set_to_none=True)
    assert tp._rel(grads[1], grads[0]) < 2e-2
