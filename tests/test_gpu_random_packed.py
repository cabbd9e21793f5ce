"""Seeded random batches and model shapes through the packed-decoder patch point: a tiny random
Qwen2 (query / kv heads, head dim, layers drawn per case) on a random batch (rows, padded
length, per-row lengths down to one token and up to the full row, left or right padding),
plain or frozen (only q / v projections train), fp16 or bf16 autocast, against HF's original
forward at test_gpu_packed's tolerances: hidden states, loss, every gradient; pad positions
exactly zero. ESEP_RANDOM_SHAPES_SCALE=k runs k times as many seeds (1 by default)."""

import os

import numpy as np
import pytest
import torch

from test_gpu_packed import _compare, _original_forward, _run

pytestmark = pytest.mark.gpu

SCALE = max(1, int(os.environ.get("ESEP_RANDOM_SHAPES_SCALE", "1")))
SEEDS = list(range(1000, 1008)) + [11000 + i for i in range(8 * (SCALE - 1))]


def _model(rng, variant):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    heads, kv = [(4, 2), (4, 4), (6, 2), (8, 1), (12, 2)][int(rng.integers(5))]
    head_dim = [64, 128][int(rng.integers(2))]
    layers = int(rng.integers(1, 4))
    cfg = Qwen2Config(vocab_size=500, hidden_size=256, intermediate_size=int(rng.choice([384, 512])),
                      num_hidden_layers=layers, num_attention_heads=heads,
                      num_key_value_heads=kv, head_dim=head_dim, max_position_embeddings=1024,
                      rms_norm_eps=1e-6, rope_theta=1e6, tie_word_embeddings=True, use_cache=False)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(int(rng.integers(1 << 30)))
    model = Qwen2ForCausalLM(cfg)
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
    return model, (heads, kv, head_dim, layers)


def _batch(rng, vocab):
    B, L = int(rng.integers(1, 6)), int(rng.integers(2, 90))
    lens = [int(rng.integers(1, L + 1)) for _ in range(B)]
    if rng.integers(2):
        lens[int(rng.integers(B))] = L  # a row without padding
    if max(lens) < 2:
        lens[0] = 2  # at least one label the loss can use
    left = bool(rng.integers(2))
    ids = torch.from_numpy(rng.integers(0, vocab, (B, L))).long()
    mask = torch.zeros(B, L, dtype=torch.long)
    for b, n in enumerate(lens):
        if left:
            mask[b, L - n:] = 1
        else:
            mask[b, :n] = 1
    ids[mask == 0] = 0
    labels = ids.clone()
    labels[mask == 0] = -100
    for b, n in enumerate(lens):  # the first real token of a row has no previous one
        labels[b, L - n if left else 0] = -100
    return ids.cuda(), mask.cuda(), labels.cuda(), lens, left


@pytest.mark.parametrize("seed", SEEDS)
def test_random_packed_matches_original(seed):
    from solution.body import patch

    patch()
    rng = np.random.default_rng(seed)
    variant = ["plain", "frozen"][int(rng.integers(2))]
    dtype = [torch.float16, torch.bfloat16][int(rng.integers(2))]
    model, shape = _model(rng, variant)
    ids, mask, labels, lens, left = _batch(rng, 500)
    print(f"seed {seed}: {variant} {dtype} heads/kv/head_dim/layers {shape} lens {lens} "
          f"L={ids.shape[1]} left={left}")
    with _original_forward():
        ref = _run(model, ids, mask, labels, dtype=dtype)
    new = _run(model, ids, mask, labels, dtype=dtype)
    tol = dict(tol_h=5e-3, tol_loss=1e-3, tol_g=2e-2) if dtype == torch.float16 else \
        dict(tol_h=3e-2, tol_loss=5e-3, tol_g=6e-2)
    # Every gradient relative to its own largest magnitude, as _compare, but with a floor of
    # 1e-3 of the largest gradient of the model: in short batches some gradients are zero in
    # exact arithmetic (a one-token sequence's softmax is 1 whatever its q and k), and both
    # implementations leave rounding noise there whose ratio means nothing.
    g_ref, g_new = ref["grads"], new["grads"]
    assert set(g_new) == set(g_ref) and g_new
    top = max(g.abs().max().item() for g in g_ref.values())
    worst = max(((g_new[n] - g).abs().max() / max(g.abs().max().item(), 1e-3 * top)).item()
                for n, g in g_ref.items())
    assert worst < tol["tol_g"], worst
    _compare(ref, new, mask, tol_h=tol["tol_h"], tol_loss=tol["tol_loss"], tol_g=float("inf"))
