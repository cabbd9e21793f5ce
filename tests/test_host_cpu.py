"""Host-side logic of the drop-in API without a GPU: exact-channel selection and its cache,
the HF-exact inverse frequencies, and the rule that the kernels never fall back to a CPU
path (CPU tensors are an error)."""

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import norm_rope_ref as ref
from solution.body import _hip, norm_rope

ROOT = Path(__file__).resolve().parents[1]


def test_reference_constants():
    """Names the reference's module exports (norm_rope.py:73, :113, :170)."""
    assert norm_rope.MAX_DY == 5 and norm_rope.SPECIAL_W_MIN == 2.0 ** -10
    assert norm_rope.NORM_BLOCK >= 3584  # the reference caps at 2048; config 5 needs 3584


def test_inv_freq_matches_hf():
    """Reference test_inv_freq_matches_hf (test_body_norm_rope.py:169-175): exact."""
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding

    cfg = Qwen2Config(hidden_size=1536, num_attention_heads=12, num_key_value_heads=2,
                      rope_theta=1e6, max_position_embeddings=32768)
    emb = Qwen2RotaryEmbedding(cfg)
    torch.testing.assert_close(emb.inv_freq, norm_rope.default_inv_freq(128, 1e6), rtol=0, atol=0)


def test_special_channels_matches_oracle_and_caches():
    g = torch.Generator().manual_seed(0)
    w = 1 + 0.1 * torch.randn(1536, generator=g)
    w[[4, 90]] = 0.0
    w[700] = 1e-5
    slots, k = norm_rope.special_channels(w)
    want, kk = ref.special_channels(w.numpy())
    assert k == kk == 3 and np.array_equal(slots.numpy(), want)
    assert norm_rope.special_channels(w)[0] is slots  # cached
    w[5] = 0.0  # in-place edit bumps the version counter: recomputed
    slots2, k2 = norm_rope.special_channels(w)
    assert k2 == 4 and slots2[5].item() == 1


def test_special_channels_threshold_read_at_call_time(monkeypatch):
    w = torch.ones(64)
    w[3] = 1e-4
    assert norm_rope.special_channels(w)[1] == 1
    monkeypatch.setattr(norm_rope, "SPECIAL_W_MIN", 0.0)
    assert norm_rope.special_channels(w)[1] == 0


def test_no_cpu_fallback():
    """The kernels run on the device or not at all: CPU tensors raise EsepError."""
    x = torch.randn(4, 64)
    w = torch.ones(64)
    with pytest.raises(_hip.EsepError):
        norm_rope.rmsnorm(x, w)
    with pytest.raises(_hip.EsepError):
        norm_rope.add_rmsnorm(x, None, w, 1e-6, torch.float32)
    q, k = torch.randn(4, 2, 64), torch.randn(4, 1, 64)
    with pytest.raises(_hip.EsepError):
        norm_rope.rope(q, k, torch.arange(4), norm_rope.default_inv_freq(64))


def test_bench_refuses_several_gpus():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2 and "one GPU" in res.stderr


def test_bench_byte_model_matches_baseline():
    """Config 4's algorithmic bytes per step: 28 * (2 * 125.90 + 117.44) + 125.90 MB."""
    import bench

    c = bench.CFG4
    T = c["B"] * c["S"]
    norm = bench.norm_fwd_bytes(T, c["H"], 2, True) + bench.norm_bwd_bytes(T, c["H"], 2, True)
    rope = 2 * bench.rope_bytes(T, c["HQ"], c["HK"], c["D"], 2)
    assert round(norm / 1e6, 2) == 125.90 and round(rope / 1e6, 2) == 117.44
    total = (2 * c["layers"] + 1) * norm + c["layers"] * rope
    assert abs(total / 1e9 - 10.465) < 1e-3


def test_rows_ld_rejects_strided_and_expanded_rows():
    """A one-row view with a non-unit column stride, an expanded row and overlapping rows are
    refused instead of read as if contiguous (the kernels take unit-stride, non-overlapping
    rows)."""
    n = 1536
    assert _hip._rows_ld(torch.zeros(3, n), n) == n
    assert _hip._rows_ld(torch.zeros(1, n), n) == n
    assert _hip._rows_ld(torch.zeros(4, 2 * n)[:, :n], n) == 2 * n
    for bad in (torch.zeros(1, 2 * n)[:, ::2], torch.zeros(1).expand(1, n),
                torch.zeros(n).expand(4, n), torch.zeros(1, 1).expand(3, n)):
        with pytest.raises(_hip.EsepError):
            _hip._rows_ld(bad, n)


def test_warmup_in_a_fresh_interpreter():
    """Reference test_warmup.py:21-54 runs the warmup in a fresh interpreter. Here the kernels are
    compiled ahead of time, so warmup() only loads the library: after it, the binding holds the
    loaded handle (no load at the first step). With the library missing it does not raise (best
    effort, as the reference's), and the first real use raises EsepError naming the build step."""
    import os

    root = Path(__file__).resolve().parent.parent
    env = dict(os.environ, PYTHONPATH=f"{root / 'esep-soup-kernels_amd'}{os.pathsep}{root}")
    ok = ("from solution.body import warmup, _hip\n"
          "assert _hip._lib is None\n"
          "warmup()\n"
          "assert _hip._lib is not None and _hip.lib() is _hip._lib\n"
          "print('loaded')\n")
    r = subprocess.run([sys.executable, "-c", ok], env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and "loaded" in r.stdout, r.stderr[-2000:]
    missing = ("from pathlib import Path\n"
               "from solution.body import warmup, _hip\n"
               "_hip.LIB_PATH = Path('/nonexistent/libesep_body.so')\n"
               "warmup()\n"
               "assert _hip._lib is None\n"
               "try:\n"
               "    _hip.lib()\n"
               "except _hip.EsepError as e:\n"
               "    assert 'build' in str(e)\n"
               "    print('raised')\n")
    r = subprocess.run([sys.executable, "-c", missing], env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and "raised" in r.stdout, r.stderr[-2000:]


def test_weight_leaf_only_through_the_casts():
    """The deferred weight gradient is written straight into a leaf's .grad, so the leaf is taken
    only where the kernel weight is the parameter itself or _weight_f32's cast / copy of it."""
    from solution.body import norm_rope as nr

    p = torch.nn.Parameter(torch.ones(8))
    pb = torch.nn.Parameter(torch.ones(8, dtype=torch.bfloat16))
    stacked = torch.nn.Parameter(torch.ones(3, 8))
    assert nr._weight_leaf(nr._weight_f32(p, True)) is p
    assert nr._weight_leaf(nr._weight_f32(pb, True)) is pb
    for w in (nr._weight_f32(p * 0.5, True), nr._weight_f32(p.exp(), True),
              nr._weight_f32(stacked[1], True), nr._weight_f32(p.view(2, 4).view(8), True),
              nr._weight_f32(stacked.to(torch.float64)[1], True)):
        assert nr._weight_leaf(w) is None
    assert nr._weight_leaf(torch.ones(8)) is None  # no gradient wanted


def _can_defer_inside_backward(nr):
    """_can_defer for a parameter whose AccumulateGrad runs in the pass, evaluated inside a CPU
    backward (what the norm backward sees)."""
    leaf = torch.nn.Parameter(torch.ones(4))
    seen = []

    class Probe(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x, w):
            return x.clone()

        @staticmethod
        def backward(ctx, g):
            seen.append(nr._can_defer(leaf))
            return g, torch.zeros_like(leaf)

    Probe.apply(torch.ones(4, requires_grad=True), leaf).sum().backward()
    return seen[0]


def test_can_defer_without_engine_internals(monkeypatch):
    """The deferral rests on private autograd entry points: with one of them gone (a torch
    without it) _can_defer answers False instead of raising, and _defer declines."""
    from solution.body import norm_rope as nr

    assert _can_defer_inside_backward(nr) is True
    monkeypatch.delattr(torch._C, "_will_engine_execute_node")
    assert _can_defer_inside_backward(nr) is False
    assert nr._defer(None, torch.empty(1, 8)) is False
    assert not nr._deferred


def test_bitsandbytes_looked_up_once(monkeypatch):
    """is_linear4bit, which the packed decoder asks ten times per layer, looks bitsandbytes up
    once per process: Python remembers no failed import, and a search of sys.path per call
    made the patched forward launch-bound."""
    import builtins

    from solution import nf4

    tries = []
    real_import = builtins.__import__

    def counting(name, *args, **kwargs):
        if name.startswith("bitsandbytes"):
            tries.append(name)
        return real_import(name, *args, **kwargs)

    nf4._bnb_class.cache_clear()
    monkeypatch.setattr(builtins, "__import__", counting)
    try:
        for _ in range(5):
            assert nf4.is_linear4bit(torch.nn.Linear(4, 4)) is False
    finally:
        monkeypatch.undo()
        nf4._bnb_class.cache_clear()
    assert len(tries) <= 1, tries
