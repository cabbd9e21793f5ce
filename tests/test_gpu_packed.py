"""The packed-decoder patch point on the GPU: a tiny random Qwen2 through the patched
Qwen2Model.forward (HIP norms, RoPE and varlen attention) against HF's original forward, restating the reference's
solution/test_body_packed.py (:20-338): hidden states, loss and every gradient within the
reference's tolerances, pad positions exactly zero, launch counts by kernel name, and the
guarded fallbacks. peft / bitsandbytes are not installed, so the reference's "lora" and
"nf4_lora" variants are replaced by "frozen" (only q/v projections train, as a LoRA run
freezes the base model: frozen norm weights, no gradient into the embedding)."""

import contextlib

import pytest
import torch

pytestmark = pytest.mark.gpu

LENS = [37, 20, 9, 30]
L = 40
VOCAB = 1000


def _config():
    from transformers import Qwen2Config

    cfg = Qwen2Config(vocab_size=VOCAB, hidden_size=256, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                      head_dim=64, max_position_embeddings=1024, rms_norm_eps=1e-6,
                      rope_theta=1e6, tie_word_embeddings=True, use_cache=False)
    cfg._attn_implementation = "sdpa"
    return cfg


def _build(variant):
    from transformers import Qwen2ForCausalLM

    torch.manual_seed(0)
    model = Qwen2ForCausalLM(_config())
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name:
                p.add_(0.1 * torch.randn_like(p))
            elif name.endswith("bias"):
                p.normal_(0, 0.1)
    model = model.cuda().float()
    if variant == "frozen":
        for name, p in model.named_parameters():
            p.requires_grad_(name.endswith(("q_proj.weight", "v_proj.weight")))
    model.train()
    return model


def _batch(left=False):
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, VOCAB, (len(LENS), L), generator=g)
    mask = torch.zeros(len(LENS), L, dtype=torch.long)
    for b, n in enumerate(LENS):
        if left:
            mask[b, L - n:] = 1
        else:
            mask[b, :n] = 1
    ids[mask == 0] = 0
    labels = ids.clone()
    labels[mask == 0] = -100
    labels[:, :3] = -100
    if left:
        for b, n in enumerate(LENS):
            labels[b, L - n] = -100
    return ids.cuda(), mask.cuda(), labels.cuda()


@contextlib.contextmanager
def _original_forward():
    from transformers.models.qwen2 import modeling_qwen2

    cls = modeling_qwen2.Qwen2Model
    patched = cls.forward
    cls.forward = patched.__wrapped__
    try:
        yield
    finally:
        cls.forward = patched


def _run(model, ids, mask, labels, autocast=True, dtype=torch.float16):
    model.zero_grad(set_to_none=True)
    with torch.autocast("cuda", dtype=dtype, enabled=autocast):
        out = model(input_ids=ids, attention_mask=mask, labels=labels, use_cache=False)
        hidden = model.model(input_ids=ids, attention_mask=mask, use_cache=False).last_hidden_state
    out.loss.backward()
    grads = {n: p.grad.detach().float().clone() for n, p in model.named_parameters()
             if p.requires_grad and p.grad is not None}
    return {"hidden": hidden.detach().float(), "loss": out.loss.detach().float(), "grads": grads}


def _rel(a, b):
    return ((a - b).abs().max() / b.abs().max().clamp(min=1e-12)).item()


def _compare(ref, new, mask, tol_h=5e-3, tol_loss=1e-3, tol_g=2e-2):
    """Reference _compare (test_body_packed.py:216-232)."""
    real = mask.bool()
    assert set(new["grads"]) == set(ref["grads"]) and new["grads"]
    assert torch.all(new["hidden"][~real] == 0)
    assert _rel(new["hidden"][real], ref["hidden"][real]) < tol_h
    assert abs((new["loss"] - ref["loss"]).item()) / abs(ref["loss"].item()) < tol_loss
    worst = max(_rel(new["grads"][n], ref["grads"][n]) for n in ref["grads"])
    assert worst < tol_g, worst


def _counts(names):
    return {k: names.count(k) for k in ("_add_rmsnorm_fwd", "_add_rmsnorm_bwd", "_rope_kernel",
                                        "_attn_fwd", "_attn_bwd", "_swiglu_fwd", "_swiglu_bwd")}


@pytest.mark.parametrize("kernels", [True, False], ids=["kernels", "torch"])
@pytest.mark.parametrize("left", [False, True], ids=["right_pad", "left_pad"])
@pytest.mark.parametrize("variant", ["plain", "frozen"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_packed_matches_original(variant, left, kernels, dtype):
    from solution.body import _hip, packed, patch

    patch()
    model = _build(variant)
    ids, mask, labels = _batch(left)
    with _original_forward():
        ref = _run(model, ids, mask, labels, dtype=dtype)
    with packed.kernels_enabled(kernels), _hip.count_launches() as names:
        new = _run(model, ids, mask, labels, dtype=dtype)
    tol = dict(tol_h=5e-3, tol_loss=1e-3, tol_g=2e-2) if dtype == torch.float16 else \
        dict(tol_h=3e-2, tol_loss=5e-3, tol_g=6e-2)
    _compare(ref, new, mask, **tol)
    n_layers = model.config.num_hidden_layers
    c = _counts(names)
    if kernels:
        norms = 2 * n_layers + 1
        # a frozen model gives the first norm no backward (its input needs no gradient)
        norm_bwd = norms - (1 if variant == "frozen" else 0)
        assert c["_add_rmsnorm_fwd"] == 2 * norms, c  # loss forward + hidden forward
        assert c["_add_rmsnorm_bwd"] == norm_bwd, c
        assert c["_rope_kernel"] == 3 * n_layers, c
        # one varlen attention launch per layer and direction (loss forward + hidden forward)
        assert c["_attn_fwd"] == 2 * n_layers and c["_attn_bwd"] == n_layers, c
        # SwiGLU on the HIP kernel: through the recompute MLP when the MLP is frozen
        assert c["_swiglu_fwd"] == 2 * n_layers and c["_swiglu_bwd"] == n_layers, c
    else:
        assert not any(c.values()), c


def test_packed_kernels_pure_fp32():
    """No autocast, fp32 model (reference :279-292): only summation order differs."""
    from solution.body import _hip, patch

    patch()
    model = _build("plain")
    ids, mask, labels = _batch()
    with _original_forward():
        ref = _run(model, ids, mask, labels, autocast=False)
    with _hip.count_launches() as names:
        new = _run(model, ids, mask, labels, autocast=False)
    _compare(ref, new, mask, tol_h=1e-4, tol_loss=1e-5, tol_g=1e-3)
    c = _counts(names)
    assert c["_add_rmsnorm_fwd"] > 0 and c["_rope_kernel"] > 0, c


def test_packed_fp16_residual_falls_back():
    """A pure fp16 model keeps HF's norm rounding (reference :295-309): the norm kernel is not
    used, RoPE still is; outputs match the original."""
    from solution.body import _hip, patch

    patch()
    model = _build("frozen").half()
    ids, mask, labels = _batch()
    with _original_forward():
        ref = _run(model, ids, mask, labels, autocast=False)
    with _hip.count_launches() as names:
        new = _run(model, ids, mask, labels, autocast=False)
    _compare(ref, new, mask)
    c = _counts(names)
    assert c["_add_rmsnorm_fwd"] == 0 and c["_add_rmsnorm_bwd"] == 0, c
    assert c["_rope_kernel"] > 0, c


def test_fallbacks_match_original():
    """No mask, a row without tokens, output_hidden_states and return_dict=False (reference
    :312-338)."""
    from solution.body import patch

    patch()
    model = _build("plain")
    ids, mask, _ = _batch()
    base = model.model
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
        with _original_forward():
            want = base(input_ids=ids, use_cache=False).last_hidden_state
        got = base(input_ids=ids, use_cache=False).last_hidden_state
        assert torch.equal(want, got)
        empty = mask.clone()
        empty[2] = 0
        with _original_forward():
            want = base(input_ids=ids, attention_mask=empty, use_cache=False).last_hidden_state
        got = base(input_ids=ids, attention_mask=empty, use_cache=False).last_hidden_state
        assert torch.equal(want, got)
        out = base(input_ids=ids, attention_mask=mask, use_cache=False, output_hidden_states=True)
        assert out.hidden_states is not None and len(out.hidden_states) == 3
        tup = base(input_ids=ids, attention_mask=mask, use_cache=False, return_dict=False)
        assert isinstance(tup, tuple) and tup[0].shape == (len(LENS), L, 256)


def test_patch_is_idempotent():
    from transformers.models.qwen2 import modeling_qwen2

    from solution.body import patch

    patch()
    fwd = modeling_qwen2.Qwen2Model.forward
    patch()
    assert modeling_qwen2.Qwen2Model.forward is fwd and hasattr(fwd, "__wrapped__")


@pytest.mark.parametrize("save_output", [True, False], ids=["norm_saves_y", "recompute_norm"])
def test_packed_recompute_mlp(save_output, monkeypatch):
    """Frozen MLP through the recompute MLP, with the post-attention norm saving its output (x
    saved as is) or not (x recomputed from the fp32 residual by the norm kernel in backward,
    reference test_body_recompute.py:192-219); against HF's original forward and with the
    recompute MLP switched off."""
    from solution.body import _hip, packed, patch

    patch()
    model = _build("frozen")
    ids, mask, labels = _batch()
    with _original_forward():
        ref = _run(model, ids, mask, labels)
    monkeypatch.setattr(packed, "NORM_SAVE_OUTPUT", save_output)
    with _hip.count_launches() as names:
        new = _run(model, ids, mask, labels)
    _compare(ref, new, mask)
    n_layers = model.config.num_hidden_layers
    c = _counts(names)
    assert c["_swiglu_fwd"] == 2 * n_layers and c["_swiglu_bwd"] == n_layers, c
    # recompute from the residual: one more norm forward per layer in the backward
    extra = 0 if save_output else n_layers
    assert c["_add_rmsnorm_fwd"] == 2 * (2 * n_layers + 1) + extra, c
    monkeypatch.setattr(packed, "RECOMPUTE_MLP", False)
    off = _run(model, ids, mask, labels)
    _compare(ref, off, mask)


@pytest.mark.parametrize("variant", ["plain", "frozen"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_fused_qkv(variant, dtype, monkeypatch):
    """Plain nn.Linear q / k / v run as one GEMM against their concatenated weights (FUSE_QKV):
    one fused call per layer and forward, against HF's original forward at the usual
    tolerances and against the three separate projections (FUSE_QKV off) at the same ones;
    the trainable q / v weights get their gradients through the concatenation (k's is
    never formed: frozen), and the norm's k and v copies get none."""
    from solution.body import packed, patch

    patch()
    model = _build(variant)
    ids, mask, labels = _batch()
    with _original_forward():
        ref = _run(model, ids, mask, labels, dtype=dtype)
    calls = []
    orig = packed._linear_multi

    def counting(x2, bases):
        out = orig(x2, bases)
        calls.append(out is not None)
        return out

    monkeypatch.setattr(packed, "_linear_multi", counting)
    fused = _run(model, ids, mask, labels, dtype=dtype)
    n_layers = model.config.num_hidden_layers
    assert calls == [True] * (2 * n_layers), calls  # loss forward + hidden forward
    monkeypatch.setattr(packed, "FUSE_QKV", False)
    calls.clear()
    separate = _run(model, ids, mask, labels, dtype=dtype)
    assert calls == []
    tol = dict(tol_h=5e-3, tol_loss=1e-3, tol_g=2e-2) if dtype == torch.float16 else \
        dict(tol_h=3e-2, tol_loss=5e-3, tol_g=6e-2)
    _compare(ref, fused, mask, **tol)
    _compare(separate, fused, mask, **tol)
    if variant == "frozen":
        assert set(fused["grads"]) == {n for n, p in model.named_parameters() if p.requires_grad}
        assert all("k_proj" not in n for n in fused["grads"])


@pytest.mark.parametrize("with_delta", [False, True], ids=["no_delta", "q_delta"])
@pytest.mark.parametrize("v_grad", [True, False], ids=["dv", "no_dv"])
def test_qkv_rope_matches_split(with_delta, v_grad):
    """_QKVRope (RoPE on the fused q / k / v output's columns, the backward writing the
    gradient of all three column blocks into one tensor) against the column views it replaces:
    y.split, norm_rope.rope on the q / k views (q_delta added inside) and a copy of v. The same
    kernels on the same data: outputs and gradients (y's, q_delta's) bit for bit, with and
    without v's gradient (its columns zero)."""
    from solution.body import packed
    from solution.body.norm_rope import default_inv_freq, rope

    T, HQ, HK, D = 301, 4, 2, 64
    nq, nk = HQ * D, HK * D
    g = torch.Generator().manual_seed(3)
    y0 = torch.randn(T, nq + 2 * nk, generator=g).to(torch.bfloat16).cuda()
    qd0 = torch.randn(T, nq, generator=g).to(torch.bfloat16).cuda() if with_delta else None
    pos = torch.randint(0, 900, (T,), generator=g).cuda()
    inv = default_inv_freq(D, 1e6, "cuda")
    dq_o = torch.randn(1, T, HQ, D, generator=g).to(torch.bfloat16).cuda()
    dk_o = torch.randn(1, T, HK, D, generator=g).to(torch.bfloat16).cuda()
    dv_o = torch.randn(T, nk, generator=g).to(torch.bfloat16).cuda()

    def run(fused):
        y = y0.clone().requires_grad_()
        qd = None if qd0 is None else qd0.clone().requires_grad_()
        if fused:
            qo, ko, v = packed._QKVRope.apply(y, nq, nk, D, pos, inv, qd)
        else:
            q, k, v = y.split([nq, nk, nk], dim=-1)
            qo, ko = rope(q.view(T, HQ, D), k.view(T, HK, D), pos, inv,
                          q_delta=None if qd is None else qd.view(T, HQ, D))
            qo, ko, v = qo.unsqueeze(0), ko.unsqueeze(0), v.contiguous()
        outs, grads = [qo, ko] + ([v] if v_grad else []), [dq_o, dk_o] + ([dv_o] if v_grad else [])
        got = torch.autograd.grad(outs, [y] + ([qd] if qd is not None else []), grads)
        return [t.detach() for t in (qo, ko, v)] + list(got)

    for a, b in zip(run(True), run(False)):
        assert torch.equal(a, b)


def test_frozen_bias_cat_cache():
    """The fused projection's concatenation of frozen biases is built once and reused, rebuilt
    after an in-place change of a bias (its version), a replaced bias Parameter or another
    dtype, and never used for a bias that trains (the concatenation is then differentiable)."""
    from solution.body import packed

    lins = [torch.nn.Linear(16, n).cuda() for n in (32, 8, 8)]
    for lin in lins:
        lin.requires_grad_(False)
    bs = [lin.bias for lin in lins]
    first = packed._frozen_bias_cat(lins, bs, torch.bfloat16)
    assert torch.equal(first, torch.cat(bs).to(torch.bfloat16))
    assert packed._frozen_bias_cat(lins, bs, torch.bfloat16) is first
    with torch.no_grad():
        lins[1].bias.add_(1.0)
    second = packed._frozen_bias_cat(lins, [lin.bias for lin in lins], torch.bfloat16)
    assert second is not first and torch.equal(second, torch.cat(
        [lin.bias for lin in lins]).to(torch.bfloat16))
    lins[2].bias = torch.nn.Parameter(torch.full((8,), 3.0, device="cuda"), requires_grad=False)
    third = packed._frozen_bias_cat(lins, [lin.bias for lin in lins], torch.bfloat16)
    assert third is not second and torch.equal(third[-8:], torch.full((8,), 3.0, device="cuda",
                                                                       dtype=torch.bfloat16))
    assert packed._frozen_bias_cat(lins, [lin.bias for lin in lins], torch.float16).dtype \
        == torch.float16
    # a trainable bias: _linear_multi concatenates per call, with gradients to each bias
    lins[0].bias.requires_grad_(True)
    x = torch.randn(5, 16, device="cuda")
    y = packed._linear_multi(x, lins)
    y.sum().backward()
    assert torch.equal(lins[0].bias.grad, torch.full((32,), 5.0, device="cuda"))
