#!/usr/bin/env python3
"""Benchmark of the decoder-body RMSNorm + RoPE path (forward + backward) on one MI355X.

Workload (the Qwen2.5-1.5B training-step shape): a full 28-layer
body sweep, B = 8, S = 1024 (T = 8192 tokens), hidden 1536, 12 q / 2 kv heads, head_dim 128,
bf16 activations ~ N(0, 1), weights 1 + 0.02 N(0, 1), theta 1e6, eps 1e-6. One step =
forward (per layer: input RMSNorm, q/k RoPE, post-attention RMSNorm; then the final norm)
followed by backward in reverse order (every norm: dx and the weight gradient; RoPE: dq, dk).
Every layer owns its own tensors (as in training), ~9 GB resident in HBM before timing.
The step is captured once in a HIP graph (the launches go through the C ABI of
libesep_body.so, ordered on one stream) and replayed.

The norm-weight gradients follow the Python API's schedule in a loss.backward() pass
(norm_rope.DEFER_WEIGHT_GRAD): every norm backward writes its fixed-order partials and one
batched launch after the sweep reduces all 57 (the per-call schedule, a reduce launch inside
every norm backward, is timed too: config4_per_call_dgamma).

value = algorithmic bytes of one step / measured seconds per step. Algorithmic bytes count
each required tensor once (e = 2 bytes):
  RMSNorm fwd 2eTH + 4T (rstd)   RMSNorm bwd 3eTH + 4T (rstd) + 4H (dw)   RoPE 2eT(HQ+HK)D
With --rstd recomputed the 4T terms go away (rstd is recomputed from x in backward).

Also printed: the roofline of the dominant kernel (per-launch HIP-event timing of graphs of
that kernel alone, on the stream it runs on); the streaming ceiling (the fastest of the bench's
streaming probes, benchlib/probe.hip, at each kernel's bytes and launch pattern, and the step
built of those probes, timed); configs 1-3
(cache-resident and with the Infinity Cache flushed); config 5; the neighbours' kernels; and
the CPU baseline: the PyTorch-eager fp32 restatement of HF's Qwen2RMSNorm / rotary path
(oracle/hf_eager.py) timed on this host's cores on one layer of the same workload.

    python bench.py [--steps K] [--warmup W] [--rstd saved|recomputed] [--no-cpu]
    python bench.py --pmc-kernel rmsnorm_bwd   # counter run for rocprofv3 --pmc (no timing)
    python bench.py --packed-only              # the end-to-end packed decoder leg alone
"""

import argparse
import itertools
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "esep-soup-kernels_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

PEAK_GBS = 8000.0  # MI355X HBM3E, published
CFG4 = dict(layers=28, B=8, S=1024, H=1536, HQ=12, HK=2, D=128, theta=1e6, eps=1e-6)
# Config 5: large-token stress at Qwen2.5-7B-like width, varlen lengths U[128, 4096] (seed 0)
CFG5 = dict(T=65536, H=3584, HQ=28, HK=4, D=128, theta=1e6, eps=1e-6, lo=128, hi=4096)


def log(msg):
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def norm_fwd_bytes(T, H, e, rstd):
    return 2 * e * T * H + (4 * T if rstd else 0)


def norm_bwd_bytes(T, H, e, rstd):
    return 3 * e * T * H + (4 * T if rstd else 0) + 4 * H


def rope_bytes(T, HQ, HK, D, e):
    return 2 * e * T * (HQ + HK) * D


class Body:
    """Resident tensors of the whole sweep and the launch sequence of one step."""

    def __init__(self, cfg, save_rstd, dev, deferred_dgamma=True):
        import torch

        from solution.body import _hip

        self.hip, self.cfg, self.save_rstd = _hip, cfg, save_rstd
        self.deferred = deferred_dgamma
        L, B, S, H, HQ, HK, D = (cfg[k] for k in ("layers", "B", "S", "H", "HQ", "HK", "D"))
        T = B * S
        self.T = T
        bf = torch.bfloat16
        g = torch.Generator(device=dev).manual_seed(0)

        def rn(*shape):
            return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(bf)

        def wt():
            return 1 + 0.02 * torch.randn(H, generator=g, device=dev)

        n_norms = 2 * L + 1
        self.x = [rn(T, H) for _ in range(n_norms)]
        self.w = [wt() for _ in range(n_norms)]
        self.y = [torch.empty(T, H, device=dev, dtype=bf) for _ in range(n_norms)]
        self.rstd = [torch.empty(T, device=dev) if save_rstd else None for _ in range(n_norms)]
        self.dy = [rn(T, H) for _ in range(n_norms)]
        self.dx = [torch.empty(T, H, device=dev, dtype=bf) for _ in range(n_norms)]
        self.dw = [torch.empty(H, device=dev) for _ in range(n_norms)]
        self.ws = torch.empty(max(_hip.rmsnorm_partials(T, H), 1), H, device=dev)
        # deferred stage 2 (the Python API's schedule in a loss.backward() pass,
        # norm_rope.DEFER_WEIGHT_GRAD): every norm backward of the sweep keeps its own partials
        # and one launch after the sweep reduces all of them (esep_dgamma_reduce_batch)
        self.parts = ([torch.empty(_hip.rmsnorm_partials(T, H), H, device=dev) for _ in range(n_norms)]
                      if deferred_dgamma else None)
        self.q = [rn(B, S, HQ, D) for _ in range(L)]
        self.k = [rn(B, S, HK, D) for _ in range(L)]
        self.qo = [torch.empty_like(t) for t in self.q]
        self.ko = [torch.empty_like(t) for t in self.k]
        self.dqo = [rn(B, S, HQ, D) for _ in range(L)]
        self.dko = [rn(B, S, HK, D) for _ in range(L)]
        self.dq = [torch.empty_like(t) for t in self.q]
        self.dk = [torch.empty_like(t) for t in self.k]
        self.inv_freq = (1.0 / (cfg["theta"] ** (torch.arange(0, D, 2, dtype=torch.float) / D))).to(dev)

    # single launches ---------------------------------------------------------------
    def norm_fwd(self, i):
        self.hip.rmsnorm_fwd(self.x[i], self.w[i], self.y[i], self.cfg["eps"], rstd=self.rstd[i])

    def norm_bwd(self, i):
        if self.deferred:
            self.hip.rmsnorm_bwd([self.dy[i]], self.x[i], self.w[i], self.cfg["eps"],
                                 rstd=self.rstd[i], dx=self.dx[i], partials=self.parts[i])
            return
        self.hip.rmsnorm_bwd([self.dy[i]], self.x[i], self.w[i], self.cfg["eps"],
                             rstd=self.rstd[i], dx=self.dx[i], dw=self.dw[i], workspace=self.ws)

    def rope_fwd(self, l):
        # padded [B, S, H, D] projections, positions 0..S-1 per row (implicit)
        self.hip.rope(self.q[l], self.k[l], self.qo[l], self.ko[l], self.inv_freq, 1.0)

    def rope_bwd(self, l):
        self.hip.rope(self.dqo[l], self.dko[l], self.dq[l], self.dk[l], self.inv_freq, -1.0)

    # one step ------------------------------------------------------------------------
    def step(self):
        L = self.cfg["layers"]
        for l in range(L):
            self.norm_fwd(2 * l)
            self.rope_fwd(l)
            self.norm_fwd(2 * l + 1)
        self.norm_fwd(2 * L)
        self.norm_bwd(2 * L)
        for l in reversed(range(L)):
            self.norm_bwd(2 * l + 1)
            self.rope_bwd(l)
            self.norm_bwd(2 * l)
        if self.deferred:
            self.dgamma_stage2()

    def dgamma_stage2(self):
        self.hip.dgamma_reduce_batch(self.parts, self.dw)

    def step_bytes(self):
        c, T, e = self.cfg, self.T, 2
        L = c["layers"]
        norm = norm_fwd_bytes(T, c["H"], e, self.save_rstd) + norm_bwd_bytes(T, c["H"], e, self.save_rstd)
        rope = 2 * rope_bytes(T, c["HQ"], c["HK"], c["D"], e)
        return (2 * L + 1) * norm + L * rope


def config5_lengths(cfg):
    """Sequence lengths U[lo, hi] drawn from seed 0 until T tokens (the last one truncated)."""
    import torch

    g = torch.Generator().manual_seed(0)
    lens, total = [], 0
    while total < cfg["T"]:
        n = min(int(torch.randint(cfg["lo"], cfg["hi"] + 1, (1,), generator=g)), cfg["T"] - total)
        lens.append(n)
        total += n
    return lens


class Stress:
    """Config 5: one RMSNorm (x [T, H] -> y, rstd; backward dx, dw) and one q/k RoPE on the
    packed varlen layout with cu_seqlens (positions restart per sequence), forward + backward."""

    def __init__(self, cfg, dev):
        import torch

        from solution.body import _hip

        self.hip, self.cfg = _hip, cfg
        T, H, HQ, HK, D = (cfg[k] for k in ("T", "H", "HQ", "HK", "D"))
        bf = torch.bfloat16
        g = torch.Generator(device=dev).manual_seed(5)

        def rn(*shape):
            return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(bf)

        self.lens = config5_lengths(cfg)
        cu = [0]
        for n in self.lens:
            cu.append(cu[-1] + n)
        self.cu = torch.tensor(cu, dtype=torch.int32, device=dev)
        self.x, self.dy = rn(T, H), rn(T, H)
        self.w = 1 + 0.02 * torch.randn(H, generator=g, device=dev)
        self.y, self.dx = torch.empty(T, H, device=dev, dtype=bf), torch.empty(T, H, device=dev, dtype=bf)
        self.rstd, self.dw = torch.empty(T, device=dev), torch.empty(H, device=dev)
        self.ws = torch.empty(_hip.rmsnorm_partials(T, H), H, device=dev)
        self.q, self.k = rn(1, T, HQ, D), rn(1, T, HK, D)
        self.dqo, self.dko = rn(1, T, HQ, D), rn(1, T, HK, D)
        self.qo, self.ko = torch.empty_like(self.q), torch.empty_like(self.k)
        self.dq, self.dk = torch.empty_like(self.q), torch.empty_like(self.k)
        self.inv_freq = (1.0 / (cfg["theta"] ** (torch.arange(0, D, 2, dtype=torch.float) / D))).to(dev)

    def norm_fwd(self):
        self.hip.rmsnorm_fwd(self.x, self.w, self.y, self.cfg["eps"], rstd=self.rstd)

    def norm_bwd(self):
        self.hip.rmsnorm_bwd([self.dy], self.x, self.w, self.cfg["eps"], rstd=self.rstd,
                             dx=self.dx, dw=self.dw, workspace=self.ws)

    def rope_fwd(self):
        self.hip.rope(self.q, self.k, self.qo, self.ko, self.inv_freq, 1.0, cu_seqlens=self.cu)

    def rope_bwd(self):
        self.hip.rope(self.dqo, self.dko, self.dq, self.dk, self.inv_freq, -1.0, cu_seqlens=self.cu)

    def step(self):
        self.norm_fwd()
        self.rope_fwd()
        self.norm_bwd()
        self.rope_bwd()

    def kernel_bytes(self):
        c = self.cfg
        return {"rmsnorm_fwd": norm_fwd_bytes(c["T"], c["H"], 2, True),
                "rmsnorm_bwd": norm_bwd_bytes(c["T"], c["H"], 2, True),
                "rope_fwd": rope_bytes(c["T"], c["HQ"], c["HK"], c["D"], 2),
                "rope_bwd": rope_bytes(c["T"], c["HQ"], c["HK"], c["D"], 2)}


def run_config5(dev, steps):
    """Times config 5 (graph replay) and each of its kernels; returns the JSON object."""
    import torch

    st = Stress(CFG5, dev)
    torch.cuda.synchronize()
    g = capture(st.step)
    time_graph(g, 2)
    ev_ms, wall_ms = time_graph(g, steps)
    ms = max(ev_ms, wall_ms)
    kb = st.kernel_bytes()
    total = sum(kb.values())
    kernels = {}
    methods = {"rmsnorm_fwd": st.norm_fwd, "rmsnorm_bwd": st.norm_bwd, "rope_fwd": st.rope_fwd,
               "rope_bwd": st.rope_bwd}
    for name in kb:
        kg = capture(methods[name])
        time_graph(kg, 2)
        kms, _ = time_graph(kg, steps)
        kernels[name] = {"us": round(kms * 1e3, 2), "GB/s": round(kb[name] / (kms * 1e-3) / 1e9, 1)}
    gbs = total / (ms * 1e-3) / 1e9
    log(f"config 5: {ms:.3f} ms per fwd+bwd, {gbs:.0f} GB/s = {gbs / PEAK_GBS:.1%} of peak")
    del st, g
    torch.cuda.empty_cache()
    return {"workload": "config5: T=65536 packed (29 sequences, lengths U[128,4096] seed 0, "
                        "cu_seqlens), H=3584, HQ=28, HK=4, D=128, bf16; RMSNorm + q/k RoPE "
                        "forward + backward (dx, dw, dq, dk)",
            "ms_per_step": round(ms, 4), "GB/s": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_GBS, 4),
            "tokens_per_s": round(CFG5["T"] / (ms * 1e-3), 1), "bytes_per_step": total,
            "kernels": kernels}


def run_config4_per_call_dgamma(dev, steps, save_rstd):
    """Config 4's step with the weight-gradient stage 2 inside every norm backward call (what a
    backward pass gets that cannot defer it: autograd.grad, hooks on the weight, create_graph):
    one reduce launch per norm. Same bytes; 56 launches more per step."""
    import torch

    body = Body(CFG4, save_rstd, dev, deferred_dgamma=False)
    torch.cuda.synchronize()
    g = capture(body.step)
    time_graph(g, 2)
    ev_ms, wall_ms = time_graph(g, steps)
    ms = max(ev_ms, wall_ms)
    nbytes = body.step_bytes()
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"config 4, weight-gradient stage 2 per call: {ms:.3f} ms per step, {gbs:.0f} GB/s = "
        f"{gbs / PEAK_GBS:.1%} of peak")
    del g, body
    torch.cuda.empty_cache()
    return {"schedule": "every norm backward reduces its own weight gradient (2 launches per norm)",
            "ms_per_step": round(ms, 4), "GB/s": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_GBS, 4),
            "launches_per_step": 4 * CFG4["layers"] + 2 + 2 * CFG4["layers"] + 1 + 2 * CFG4["layers"] + 1 - 1}


# Streaming probes (benchlib/libesep_probe.so): one-shot grids with U = 1, 2, 4, 8 chunks of 16
# bytes per stream per lane, and fixed strided grids with the next step's U chunks issued before
# this step's stores (2U in flight), over 256 to 2048 blocks.
PROBE_VARIANTS = ([("oneshot", u, t, 1) for u in (1, 2, 4, 8) for t in (256, 512)]
                  + [("strided", u, t, b) for u, t in ((1, 512), (2, 512), (4, 256), (4, 512), (8, 256))
                     for b in (256, 512, 1024, 2048)])


def _probe_launch(variant, bufs, n_src):
    import benchlib

    mode, u, t, blocks = variant
    m = benchlib.ONESHOT if mode == "oneshot" else benchlib.STRIDED
    benchlib.stream(bufs[0], bufs[-1], bufs[1] if n_src == 2 else None, mode=m, u=u, threads=t,
                    blocks=blocks)


def _probe_sweep(bufsets, n_src, reps):
    """Per-launch microseconds of every probe variant over the launches of bufsets (one graph of
    one launch per buffer set), fastest first."""
    res = []
    for v in PROBE_VARIANTS:
        def fn(v=v):
            for bs in bufsets:
                _probe_launch(v, bs, n_src)
        gr = capture(fn)
        time_graph(gr, 2)
        ms, _ = time_graph(gr, reps)
        res.append((ms * 1e3 / len(bufsets), v))
        del gr
    return sorted(res)


def _vname(v):
    mode, u, t, b = v
    return f"{mode} U{u} x {t} threads" + ("" if mode == "oneshot" else f", {b} blocks")


def stream_ceiling(dev, cfg, kernel_us, reps, step_ms):
    """The streaming ceiling of each path kernel: every probe variant at that kernel's own byte
    counts (one or two streams read, one written) and launch pattern (a graph of one launch per
    layer over distinct buffers), the fastest kept, beside the kernel's per-launch time. Then the
    step itself built of those fastest probes: the step's 170 path launches in the step's order,
    each replaced by its kernel's best probe over buffers of its own, captured in one graph and
    timed like the step (no weight-gradient stage 2: its partials are not algorithmic bytes)."""
    import torch

    T, H, HQ, HK, D, L = (cfg[k] for k in ("T", "H", "HQ", "HK", "D", "layers"))
    e = 2
    kinds = {  # kernel -> (streams read, bytes per stream, launches per step)
        "rmsnorm_fwd": (1, e * T * H, 2 * L + 1),
        "rmsnorm_bwd": (2, e * T * H, 2 * L + 1),
        "rope_fwd": (1, e * T * (HQ + HK) * D, L),
        "rope_bwd": (1, e * T * (HQ + HK) * D, L),
    }
    bufs = {name: [[torch.empty(nbytes, device=dev, dtype=torch.uint8) for _ in range(n_src + 1)]
                   for _ in range(launches)]
            for name, (n_src, nbytes, launches) in kinds.items()}
    out, best = {}, {}
    for name, (n_src, nbytes, launches) in kinds.items():
        res = _probe_sweep(bufs[name], n_src, reps)
        us, v = res[0]
        best[name] = v
        algo = (n_src + 1) * nbytes
        k_us = kernel_us.get(name)
        out[name] = {"probe_us": round(us, 3), "probe": _vname(v),
                     "probe_GB/s": round(algo / (us * 1e-6) / 1e9, 1), "launches_per_step": launches,
                     "runners_up": [{"us": round(u2, 3), "probe": _vname(v2)} for u2, v2 in res[1:4]],
                     "kernel_us": None if k_us is None else round(k_us, 3),
                     "kernel_over_probe": None if k_us is None else round(k_us / us, 4)}
        log(f"stream ceiling {name}: best probe {us:.2f} us ({_vname(v)}), kernel "
            f"{k_us if k_us is None else round(k_us, 2)} us")

    def probe_step():
        nf = lambda i: _probe_launch(best["rmsnorm_fwd"], bufs["rmsnorm_fwd"][i], 1)
        nb = lambda i: _probe_launch(best["rmsnorm_bwd"], bufs["rmsnorm_bwd"][i], 2)
        rf = lambda l: _probe_launch(best["rope_fwd"], bufs["rope_fwd"][l], 1)
        rb = lambda l: _probe_launch(best["rope_bwd"], bufs["rope_bwd"][l], 1)
        for l in range(L):
            nf(2 * l)
            rf(l)
            nf(2 * l + 1)
        nf(2 * L)
        nb(2 * L)
        for l in reversed(range(L)):
            nb(2 * l + 1)
            rb(l)
            nb(2 * l)
    gr = capture(probe_step)
    time_graph(gr, 3)
    ev_ms, wall_ms = time_graph(gr, 20)
    pstep = max(ev_ms, wall_ms)
    del gr, bufs
    torch.cuda.empty_cache()
    sum_ms = sum(v["probe_us"] * v["launches_per_step"] for v in out.values()) * 1e-3
    floor = launch_floor(dev, cfg, kinds, reps)
    step_bytes = sum((n_src + 1) * nbytes * launches for n_src, nbytes, launches in kinds.values())
    log(f"probe step {pstep:.3f} ms ({step_bytes / (pstep * 1e-3) / 1e9:.0f} GB/s); kernel step "
        f"{step_ms:.3f} ms")
    return {"what": "benchlib probes (out = a (+ b), non-temporal 16-byte buffer loads and stores) "
                    f"at each kernel's bytes and launch pattern, fastest of {len(PROBE_VARIANTS)} "
                    "variants: one-shot grids with 1/2/4/8 chunks per stream per lane (256 or 512 "
                    "threads), strided grids of 256-2048 blocks with 1-8 chunks per stream per lane "
                    "and the next step's chunks issued before this step's stores",
            "kernels": out,
            "probe_step_ms": round(pstep, 4),
            "probe_step_GB/s": round(step_bytes / (pstep * 1e-3) / 1e9, 1),
            "probe_step_frac_of_peak": round(step_bytes / (pstep * 1e-3) / 1e9 / PEAK_GBS, 4),
            "probe_sum_ms": round(sum_ms, 4),
            "step_ms": round(step_ms, 4),
            "step_over_probe_step": round(step_ms / pstep, 4),
            "floor": floor}


def launch_floor(dev, cfg, kinds, reps):
    """The fixed cost of the step's launch structure, measured in the same run:
      launch_us     the time per launch of a graph of 57 nearly empty launches (a probe over 16
                    bytes, one block): what each dependent launch costs before any data moves
                    (the command processor's end-of-kernel and dispatch work);
      launch_ms     launch_us times the step's launches (time no kernel design removes while
                    every op is its own launch);
      asymptote     the rate of one streaming launch over 1 GiB per stream (1 read + 1 write,
                    2 reads + 1 write), fastest probe variant."""
    import torch

    n = 57
    tiny = [[torch.empty(16, device=dev, dtype=torch.uint8) for _ in range(2)] for _ in range(n)]

    def empties():
        for bs in tiny:
            _probe_launch(("strided", 1, 256, 1), bs, 1)
    gr = capture(empties)
    time_graph(gr, 2)
    ms, _ = time_graph(gr, reps)
    launch_us = ms * 1e3 / n
    del gr, tiny

    big = 1 << 30
    rates, names = {}, {}
    bufs = [torch.empty(big, device=dev, dtype=torch.uint8) for _ in range(3)]
    for n_src in (1, 2):
        res = _probe_sweep([[bufs[0], bufs[1], bufs[2]] if n_src == 2 else [bufs[0], bufs[2]]],
                           n_src, 3)
        us, v = res[0]
        rates[n_src] = (n_src + 1) * big / (us * 1e-6) / 1e9
        names[n_src] = _vname(v)
    del bufs
    torch.cuda.empty_cache()
    launches = sum(v[2] for v in kinds.values()) + 1  # + the batched weight-gradient reduce
    log(f"launch floor: {launch_us:.2f} us per launch x {launches} launches; 1 GiB stream "
        f"asymptotes 1R1W {rates[1]:.0f} / 2R1W {rates[2]:.0f} GB/s")
    return {"launch_us": round(launch_us, 3), "launches_per_step": launches,
            "launch_ms": round(launches * launch_us * 1e-3, 4),
            "asymptote_GB/s": {"1R1W": round(rates[1], 1), "2R1W": round(rates[2], 1)},
            "asymptote_probe": {"1R1W": names[1], "2R1W": names[2]}}


def _flush_buffer(dev):
    import torch

    return torch.empty(512 << 20, device=dev, dtype=torch.uint8)  # 2x the 256 MB Infinity Cache


def time_flushed(g, flush, reps):
    """Median event time of one replay of graph g with the Infinity Cache flushed before each
    replay (a 512 MB write outside the timed region)."""
    import torch

    times = []
    for _ in range(reps):
        flush.fill_(1)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    return statistics.median(times)


def run_small_configs(dev, reps):
    """Configs 1-3 as whole forward + backward steps, fp16: each timed
    cache-resident (graph replays back to back; the inputs fit the 256 MB Infinity Cache) and
    with the cache flushed before each replay (HBM-resident inputs)."""
    import torch

    from solution.body import _hip

    g = torch.Generator(device=dev).manual_seed(0)
    hf = torch.float16
    eps, theta, D = 1e-6, 1e6, 128

    def rn(*shape):
        return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(hf)

    inv = (1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float) / D))).to(dev)

    def norm_set(T, H):
        t = dict(x=rn(T, H), dy=rn(T, H), w=1 + 0.02 * torch.randn(H, generator=g, device=dev))
        t.update(y=torch.empty(T, H, device=dev, dtype=hf), dx=torch.empty(T, H, device=dev, dtype=hf),
                 rstd=torch.empty(T, device=dev), dw=torch.empty(H, device=dev),
                 ws=torch.empty(_hip.rmsnorm_partials(T, H), H, device=dev))
        return t

    def norm_step(t):
        _hip.rmsnorm_fwd(t["x"], t["w"], t["y"], eps, rstd=t["rstd"])
        _hip.rmsnorm_bwd([t["dy"]], t["x"], t["w"], eps, rstd=t["rstd"], dx=t["dx"], dw=t["dw"],
                         workspace=t["ws"])

    def rope_set(shape_q, shape_k):
        t = dict(q=rn(*shape_q), k=rn(*shape_k), dqo=rn(*shape_q), dko=rn(*shape_k))
        for a, b in (("qo", "q"), ("ko", "k"), ("dq", "q"), ("dk", "k")):
            t[a] = torch.empty_like(t[b])
        return t

    lens3 = torch.randint(64, 1025, (8,), generator=torch.Generator().manual_seed(0)).tolist()
    T3 = sum(lens3)
    cu3 = torch.tensor([0] + list(itertools.accumulate(lens3)), dtype=torch.int32, device=dev)
    c1 = norm_set(2048, 1536)
    c2 = rope_set((4, 12, 512, D), (4, 2, 512, D))   # contiguous [B, H, S, D]
    c3n, c3r = norm_set(T3, 1536), rope_set((1, T3, 12, D), (1, T3, 2, D))

    def rope2(t, sign, src_q, src_k, dst_q, dst_k):
        # [B, H, S, D] tensors seen as (B, S, H, D) views; positions 0..S-1 per row
        _hip.rope(t[src_q].transpose(1, 2), t[src_k].transpose(1, 2), t[dst_q].transpose(1, 2),
                  t[dst_k].transpose(1, 2), inv, sign)

    def c2_step():
        rope2(c2, 1.0, "q", "k", "qo", "ko")
        rope2(c2, -1.0, "dqo", "dko", "dq", "dk")

    def c3_step():
        norm_step(c3n)
        _hip.rope(c3r["q"], c3r["k"], c3r["qo"], c3r["ko"], inv, 1.0, cu_seqlens=cu3)
        _hip.rope(c3r["dqo"], c3r["dko"], c3r["dq"], c3r["dk"], inv, -1.0, cu_seqlens=cu3)

    e = 2
    nb = lambda T, H: norm_fwd_bytes(T, H, e, True) + norm_bwd_bytes(T, H, e, True)  # noqa: E731
    cases = {
        "config1": ("RMSNorm fwd + bwd (y, rstd; dx, dw), x [4, 512, 1536] fp16", lambda: norm_step(c1),
                    nb(2048, 1536), 2048),
        "config2": ("RoPE fwd + bwd on the padded [B, H, S, D] layout, q [4, 12, 512, 128], k "
                    "[4, 2, 512, 128] fp16, positions 0..511 per row", c2_step,
                    2 * rope_bytes(2048, 12, 2, D, e), 2048),
        "config3": (f"varlen: 8 sequences {lens3} (T={T3}, cu_seqlens int32) RMSNorm [T, 1536] + "
                    "RoPE q [T, 12, 128] k [T, 2, 128], fp16, fwd + bwd", c3_step,
                    nb(T3, 1536) + 2 * rope_bytes(T3, 12, 2, D, e), T3),
    }
    flush = _flush_buffer(dev)
    out = {}
    per_graph = 10
    for name, (what, fn, nbytes, T) in cases.items():
        gr = capture(fn)
        time_graph(gr, 3)
        res_ms, _ = time_graph(gr, reps)
        fl_ms = time_flushed(gr, flush, reps)
        # the same step captured 10 times in one graph: a graph replay's own start-up (several
        # microseconds, a large share of these short steps) spread over 10 steps, as in a
        # training step that captures many layers in one graph
        gr10 = capture(lambda: [fn() for _ in range(per_graph)])
        time_graph(gr10, 2)
        g10_ms = time_graph(gr10, reps)[0] / per_graph
        row = {"workload": what, "bytes_per_step": nbytes, "tokens": T}
        for tag, ms in (("cache_resident", res_ms), ("flushed", fl_ms),
                        ("cache_resident_10_steps_per_graph", g10_ms)):
            gbs = nbytes / (ms * 1e-3) / 1e9
            row[tag] = {"us_per_step": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                        "frac_of_peak": round(gbs / PEAK_GBS, 4), "tokens_per_s": round(T / (ms * 1e-3), 1)}
        log(f"{name}: cache-resident {res_ms * 1e3:.1f} us, flushed {fl_ms * 1e3:.1f} us, "
            f"10 steps per graph {g10_ms * 1e3:.1f} us per step ({nbytes / 1e6:.1f} MB)")
        out[name] = row
        del gr, gr10
    del flush, c1, c2, c3n, c3r
    torch.cuda.empty_cache()
    return out


def run_config4_other_rstd(dev, steps, save_rstd):
    """Config 4's step graph with the other rstd mode (saved by the forward and read by the
    backward, or recomputed from x in the backward); returns the JSON object."""
    import torch

    body = Body(CFG4, save_rstd, dev)
    torch.cuda.synchronize()
    g = capture(body.step)
    time_graph(g, 2)
    ev_ms, wall_ms = time_graph(g, steps)
    ms = max(ev_ms, wall_ms)
    nbytes = body.step_bytes()
    gbs = nbytes / (ms * 1e-3) / 1e9
    mode = "saved" if save_rstd else "recomputed"
    log(f"config 4, rstd {mode}: {ms:.3f} ms per step, {gbs:.0f} GB/s = {gbs / PEAK_GBS:.1%} of peak")
    del g, body
    torch.cuda.empty_cache()
    return {"rstd": mode, "ms_per_step": round(ms, 4), "GB/s": round(gbs, 1),
            "frac_of_peak": round(gbs / PEAK_GBS, 4), "bytes_per_step": nbytes}


def capture(fn, warm=True):
    import torch

    if warm:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(g, reps):
    """(event ms per replay, wall ms per replay) over `reps` back-to-back replays."""
    import torch

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    return e0.elapsed_time(e1) / reps, (t1 - t0) * 1e3 / reps


def api_bytes(T, H, k_dy, fwd, x_bytes=4):
    """The reference API's pattern (AddRMSNorm in the packed decoder): fp32 residual r, bf16
    delta / y / dys, fp32 r_out / dr_out / dr, bf16 ddelta, rstd saved, frozen weight (no dw).
    x_bytes: the backward's xhat source, the fp32 r_out (4) or, in save-output mode, y (2)."""
    if fwd:  # r_in, delta -> r_out, y, rstd
        return T * H * (4 + 2 + 4 + 2) + 4 * T
    # k dys, x (r_out or y), dr_out -> dr, ddelta; rstd read
    return T * H * (2 * k_dy + x_bytes + 4 + 4 + 2) + 4 * T


def run_api_variant(dev, reps, n_sets=6):
    """Times the reference API's own calls at the config-4 shape (T = 8192, H = 1536): the
    add_rmsnorm forward, and the backward of the input norm (3 consumers) and of the
    post-attention norm (2 consumers), each in a graph over n_sets distinct tensor sets."""
    import torch

    from solution.body import _hip

    T, H, eps = CFG4["B"] * CFG4["S"], CFG4["H"], CFG4["eps"]
    g = torch.Generator(device=dev).manual_seed(7)
    bf = torch.bfloat16

    def rn(dt, *shape):
        return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(dt)

    sets = []
    for _ in range(n_sets):
        sets.append(dict(r=rn(torch.float32, T, H), d=rn(bf, T, H), ro=torch.empty(T, H, device=dev),
                         y=torch.empty(T, H, device=dev, dtype=bf), rstd=torch.rand(T, device=dev) + 0.5,
                         w=1 + 0.02 * torch.randn(H, generator=g, device=dev),
                         dys=[rn(bf, T, H) for _ in range(3)], dro=rn(torch.float32, T, H),
                         dr=torch.empty(T, H, device=dev), dd=torch.empty(T, H, device=dev, dtype=bf)))
    calls = {
        "add_rmsnorm_fwd": (lambda: [_hip.rmsnorm_fwd(s["r"], s["w"], s["y"], eps, delta=s["d"], r_out=s["ro"],
                                                      rstd=s["rstd"]) for s in sets], api_bytes(T, H, 0, True)),
        "add_rmsnorm_bwd_3dy": (lambda: [_hip.rmsnorm_bwd(s["dys"], s["r"], s["w"], eps, rstd=s["rstd"],
                                                          dr_out=s["dro"], dr=s["dr"], dx=s["dd"]) for s in sets],
                                api_bytes(T, H, 3, False)),
        "add_rmsnorm_bwd_2dy": (lambda: [_hip.rmsnorm_bwd(s["dys"][:2], s["r"], s["w"], eps, rstd=s["rstd"],
                                                          dr_out=s["dro"], dr=s["dr"], dx=s["dd"]) for s in sets],
                                api_bytes(T, H, 2, False)),
        # the reference decoder's default (NORM_SAVE_OUTPUT): xhat recovered from the saved y
        # (y / w; a weight of 1 + 0.02 N(0, 1) has no exact channels)
        "add_rmsnorm_bwd_3dy_from_y": (lambda: [_hip.rmsnorm_bwd(s["dys"], s["y"], s["w"], eps, from_y=True,
                                                                 rstd=s["rstd"], dr_out=s["dro"], dr=s["dr"],
                                                                 dx=s["dd"]) for s in sets],
                                       api_bytes(T, H, 3, False, x_bytes=2)),
    }
    out = {}
    for name, (fn, nbytes) in calls.items():
        kg = capture(fn)
        time_graph(kg, 2)
        ms, _ = time_graph(kg, reps)
        us = ms * 1e3 / n_sets
        out[name] = {"us": round(us, 2), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1), "bytes": nbytes}
        log(f"api {name}: {us:.2f} us/launch, {nbytes / (us * 1e-6) / 1e9:.0f} GB/s")
    del sets
    torch.cuda.empty_cache()
    return {"workload": "the reference API's calls at T=8192, H=1536: add_rmsnorm forward (fp32 r_in + "
                        "bf16 delta -> fp32 r_out, bf16 y, rstd) and AddRMSNorm backward with 3 or 2 "
                        "bf16 dys and fp32 dr_out -> fp32 dr + bf16 ddelta (frozen weight, rstd saved)"
                        "; the 3-dy backward also in save-output mode (xhat from the bf16 y)",
            "kernels": out}


def attn_flops(lengths, HQ, D):
    """Algorithmic causal attention FLOPs: (forward, backward). Each (query, key <= query) pair
    of a head costs 2 D multiply-adds per product: QK^T and PV forward (4 D), S, dP, dV, dK, dQ
    backward (10 D)."""
    pairs = sum(n * (n + 1) // 2 for n in lengths)
    return 4 * D * HQ * pairs, 10 * D * HQ * pairs


PEAK_BF16_TFLOPS = 2500.0


def run_attention(dev, reps):
    """The varlen causal attention kernels (esep_attn_fwd / esep_attn_bwd, bf16) at the config-4
    shape (8 rows of 1024, 12/2 heads) and the config-5 shape (29 packed sequences, 28/4 heads),
    graphed and timed with HIP events (best of three runs), beside the reference's per-row SDPA loop
    (packed.py:404-436, torch's scaled_dot_product_attention on the same GPU, eager)."""
    import torch

    from solution.body import _hip

    out = {}
    for name, lengths, HQ, HK in (("config4", [CFG4["S"]] * CFG4["B"], CFG4["HQ"], CFG4["HK"]),
                                  ("config5", config5_lengths(CFG5), CFG5["HQ"], CFG5["HK"])):
        D = 128
        T = sum(lengths)
        g = torch.Generator(device=dev).manual_seed(11)
        bf = torch.bfloat16

        def rn(*shape):
            return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(bf)

        q, k, v, do = rn(T, HQ, D), rn(T, HK, D), rn(T, HK, D), rn(T, HQ, D)
        o, dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        lse = torch.empty(HQ, T, device=dev)
        ws = torch.empty(_hip.attn_bwd_workspace(T, HQ, HK, D), device=dev)
        cu = torch.tensor([0] + list(itertools.accumulate(lengths)), dtype=torch.int32, device=dev)
        L, scale = max(lengths), D ** -0.5
        fwd = lambda: _hip.attn_fwd(q, k, v, o, cu, L, scale, lse=lse)
        bwd = lambda: _hip.attn_bwd(q, k, v, o, do, lse, dq, dk, dv, cu, L, scale, workspace=ws)
        ff, fb = attn_flops(lengths, HQ, D)
        res = {"tokens": T, "sequences": len(lengths), "heads": f"{HQ}/{HK}", "head_dim": D}
        for kind, fn, fl in (("fwd", fwd, ff), ("bwd", bwd, fb)):
            gr = capture(fn)
            time_graph(gr, 2)
            # best of three runs: one run swings by up to 10% with the box's clocks after the
            # preceding legs
            ms = min(time_graph(gr, reps)[0] for _ in range(3))
            tf = fl / (ms * 1e-3) / 1e12
            res[kind] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1), "frac": round(tf / PEAK_BF16_TFLOPS, 4)}
            log(f"attention {name} {kind}: {ms:.3f} ms, {tf:.0f} TFLOP/s = {tf / PEAK_BF16_TFLOPS:.1%} of bf16 MFMA peak")
            del gr
        # the reference's per-row loop, forward + backward, eager
        qr, kr, vr = (t.detach().clone().requires_grad_() for t in (q, k, v))

        def ref_step():
            outs = []
            for qs, ks, vs in zip(qr.split(lengths), kr.split(lengths), vr.split(lengths)):
                n = qs.shape[0]
                qh = qs.reshape(n, HK, HQ // HK, D).permute(1, 2, 0, 3)
                kh = ks.permute(1, 0, 2).unsqueeze(1).expand(HK, HQ // HK, n, D)
                vh = vs.permute(1, 0, 2).unsqueeze(1).expand(HK, HQ // HK, n, D)
                oo = torch.nn.functional.scaled_dot_product_attention(qh, kh, vh, is_causal=True, scale=scale)
                outs.append(oo.permute(2, 0, 1, 3))
            torch.autograd.backward(torch.cat(outs, 0), do.view(T, HK, HQ // HK, D))

        ref_step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n_ref = max(3, reps // 4)
        e0.record()
        for _ in range(n_ref):
            ref_step()
        e1.record()
        torch.cuda.synchronize()
        ref_ms = e0.elapsed_time(e1) / n_ref
        ours = res["fwd"]["ms"] + res["bwd"]["ms"]
        res["reference_loop_fwd_bwd_ms"] = round(ref_ms, 4)
        res["speedup_vs_reference_loop"] = round(ref_ms / ours, 2)
        log(f"attention {name}: fwd+bwd {ours:.3f} ms vs the reference's per-row SDPA loop {ref_ms:.3f} ms")
        out[name] = res
        del q, k, v, do, o, dq, dk, dv, lse, ws, qr, kr, vr
        torch.cuda.empty_cache()
    return {"workload": "varlen causal GQA attention, bf16, head_dim 128, fwd (o, lse) and bwd "
                        "(dq, dk, dv): config4 = 8 rows of 1024 tokens, 12/2 heads; config5 = the "
                        "29 packed sequences of config 5, 28/4 heads",
            "peak_TFLOP/s": PEAK_BF16_TFLOPS, **out}


def run_swiglu(dev, reps, n_sets=4):
    """The SwiGLU kernels at the Qwen2.5-1.5B MLP shape (T = 8192 tokens, intermediate 8960,
    bf16): forward reads gate and up and writes h (3 x 2 bytes per element), backward reads
    dh, gate, up and writes dgate, dup (5 x 2 bytes). Graphs over n_sets distinct buffers."""
    import torch

    from solution.body import _hip

    T, I = CFG4["B"] * CFG4["S"], 8960
    g = torch.Generator(device=dev).manual_seed(13)
    rn = lambda: torch.randn(T, I, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    sets = [dict(g=rn(), u=rn(), d=rn()) for _ in range(n_sets)]
    for s_ in sets:
        s_["h"], s_["dg"], s_["du"] = (torch.empty(T, I, device=dev, dtype=torch.bfloat16) for _ in range(3))
    out = {}
    for kind, fn, nbytes in (
            ("fwd", lambda: [_hip.swiglu_fwd(s_["g"], s_["u"], s_["h"]) for s_ in sets], 3 * 2 * T * I),
            ("bwd", lambda: [_hip.swiglu_bwd(s_["d"], s_["g"], s_["u"], s_["dg"], s_["du"]) for s_ in sets],
             5 * 2 * T * I)):
        gr = capture(fn)
        time_graph(gr, 2)
        ms, _ = time_graph(gr, reps)
        us = ms * 1e3 / n_sets
        gbs = nbytes / (us * 1e-6) / 1e9
        out[kind] = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4),
                     "bytes": nbytes}
        log(f"swiglu {kind}: {us:.1f} us, {gbs:.0f} GB/s = {gbs / PEAK_GBS:.1%} of peak")
        del gr
    del sets
    torch.cuda.empty_cache()
    return {"workload": "SwiGLU silu(gate) * up of the Qwen2.5-1.5B MLP, T=8192, intermediate 8960, "
                        "bf16, forward and backward", **out}


def run_lora_dropout(dev, reps, n_sets=4):
    """The LoRA-dropout kernels at the q_proj LoRA input of config 4 (T = 8192 tokens x 1536,
    bf16, p = 0.05): forward reads x and writes x_d (2 x 2 bytes per element); backward reads x
    and g and writes x_d and dx (4 x 2 bytes)."""
    import torch

    from solution.body import _hip

    T, H, p = CFG4["B"] * CFG4["S"], CFG4["H"], 0.05
    g = torch.Generator(device=dev).manual_seed(17)
    rn = lambda: torch.randn(T, H, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    key = torch.randint(0, 2 ** 63 - 1, (1,), device=dev, dtype=torch.int64)
    sets = [dict(x=rn(), g=rn(), xd=torch.empty(T, H, device=dev, dtype=torch.bfloat16),
                 dx=torch.empty(T, H, device=dev, dtype=torch.bfloat16)) for _ in range(n_sets)]
    out = {}
    for kind, fn, nbytes in (
            ("fwd", lambda: [_hip.lora_dropout_fwd(s_["x"], key, s_["xd"], p) for s_ in sets], 2 * 2 * T * H),
            ("bwd", lambda: [_hip.lora_dropout_bwd(s_["x"], s_["g"], key, s_["xd"], s_["dx"], p)
                             for s_ in sets], 4 * 2 * T * H)):
        gr = capture(fn)
        time_graph(gr, 2)
        ms, _ = time_graph(gr, reps)
        us = ms * 1e3 / n_sets
        gbs = nbytes / (us * 1e-6) / 1e9
        out[kind] = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4),
                     "bytes": nbytes}
        log(f"lora dropout {kind}: {us:.2f} us, {gbs:.0f} GB/s = {gbs / PEAK_GBS:.1%} of peak")
        del gr
    del sets
    torch.cuda.empty_cache()
    return {"workload": "LoRA dropout (Philox mask regenerated from a device key) on the q_proj LoRA "
                        "input of config 4: T=8192 x 1536, bf16, p=0.05", **out}


def run_nf4(dev, reps):
    """NF4 dequantization of the four Qwen2.5-1.5B projection shapes of one layer (q, k, v, o,
    gate, up, down: 1536x1536 x2, 256x1536 x2, 8960x1536 x2, 1536x8960) to fp16: per element
    0.5 byte of codes in, 2 bytes out, plus one scale byte per 64 (algorithmic bytes)."""
    import torch

    from solution.body import _hip

    shapes = [(1536, 1536), (256, 1536), (256, 1536), (1536, 1536), (8960, 1536), (8960, 1536),
              (1536, 8960)]
    g = torch.Generator(device=dev).manual_seed(19)
    tabs = dict(code2=torch.sort(torch.randn(256, generator=g, device=dev))[0],
                offset=torch.tensor([0.01], device=dev),
                nf4=torch.linspace(-1, 1, 16, device=dev))
    ws = []
    for n, k in shapes:
        nb = n * k // 64
        ws.append(dict(packed=torch.randint(0, 256, (nb * 32,), generator=g, device=dev, dtype=torch.uint8),
                       absmax=torch.randint(0, 256, (nb,), generator=g, device=dev, dtype=torch.uint8),
                       absmax2=torch.rand((nb + 255) // 256, generator=g, device=dev),
                       out=torch.empty(n, k, device=dev, dtype=torch.float16)))
    elems = sum(n * k for n, k in shapes)
    nbytes = elems // 2 + elems // 64 + 2 * elems
    items = [(w["packed"], w["absmax"], w["absmax2"], tabs["code2"], tabs["offset"], tabs["nf4"], w["out"])
             for w in ws]
    res = {}
    for key, fn in (("multi", lambda: _hip.nf4_dequant_multi(items)),
                    ("per_weight", lambda: [_hip.nf4_dequant(*it) for it in items])):
        gr = capture(fn)
        time_graph(gr, 2)
        ms, _ = time_graph(gr, reps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[key] = (ms, gbs)
        log(f"nf4 dequant (one layer, 7 weights, {key}): {ms * 1e3:.1f} us, {gbs:.0f} GB/s = "
            f"{gbs / PEAK_GBS:.1%} of peak")
        del gr
    del ws, items
    torch.cuda.empty_cache()
    ms, gbs = res["multi"]
    return {"workload": "NF4 double-quant dequantization to fp16 of one Qwen2.5-1.5B layer's seven "
                        "projection weights in one launch (esep_nf4_dequant_multi)",
            "us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4),
            "bytes": nbytes, "per_weight_launches_us": round(res["per_weight"][0] * 1e3, 2)}


def run_lm_head(dev, reps):
    """The fused LM head (solution.head.fused_linear_ce) on the Qwen2.5-1.5B head: N = 8192 rows
    (config 4's tokens), H = 1536, V = 151936, fp16 weight and hidden states, every 7th row
    ignored. Reported: the row kernel esep_head_row_softmax alone on one 4096-row chunk
    (statistics only: one read of the chunk; with g on every row: two reads and one write, the
    algorithmic bytes), and the whole op (forward with the dX precompute, then backward) at the
    default chunk and at the reference's 256-row chunk, with its two GEMMs' FLOP rate."""
    import torch

    from solution.body import _hip
    from solution.head import op as head

    N, H, V, rows = CFG4["B"] * CFG4["S"], CFG4["H"], head.VOCAB, 4096
    g = torch.Generator(device=dev).manual_seed(23)
    out = {}
    z = (torch.randn(rows, V, generator=g, device=dev) * 3).to(torch.float16)
    tgt = torch.randint(0, V, (rows,), generator=g, device=dev)
    cew = torch.ones(rows, device=dev)
    st = [torch.empty(rows, device=dev) for _ in range(3)] + [torch.empty(rows, device=dev, dtype=torch.int32)]
    for kind, wg, nbytes in (("row_stats", False, rows * V * 2), ("row_stats_g", True, 3 * rows * V * 2)):
        gr = capture(lambda: _hip.head_row_softmax(z, tgt, cew, *st, wg, head.G_SCALE))
        time_graph(gr, 2)
        ms, _ = time_graph(gr, reps)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[kind] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4),
                     "bytes": nbytes, "rows": rows}
        log(f"lm head {kind} ({rows} x {V}): {ms * 1e3:.1f} us, {gbs:.0f} GB/s = {gbs / PEAK_GBS:.1%} of peak")
        del gr
    del z, st
    torch.cuda.empty_cache()
    w = (torch.randn(V, H, generator=g, device=dev) * 0.02).to(torch.float16)
    x = torch.randn(N, H, generator=g, device=dev).to(torch.float16)
    target = torch.randint(0, V, (N,), generator=g, device=dev)
    target[::7] = -100
    ce_w = torch.full((N,), 1.0 / N, device=dev)
    flops = 2 * (2 * N * H * V) * 6 / 7 + 2 * N * H * V / 7  # dX GEMM on the weighted rows only

    def step(chunk):
        xg = x.detach().requires_grad_(True)
        loss, _ = head.fused_linear_ce(xg, w, target, ce_w, chunk_rows=chunk)
        loss.backward()

    for key, chunk in (("op", head.CHUNK_ROWS), ("op_chunk256_reference_setting", 256)):
        for _ in range(2):
            step(chunk)
        torch.cuda.synchronize()
        n = max(reps // 4, 3)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            step(chunk)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / n
        tfs = flops / (ms * 1e-3) / 1e12
        out[key] = {"ms": round(ms, 3), "chunk_rows": chunk, "TFLOP/s": round(tfs, 1),
                    "frac_mfma_fp16": round(tfs / PEAK_BF16_TFLOPS, 4)}
        log(f"lm head {key} (chunk {chunk}): {ms:.3f} ms, {tfs:.0f} TFLOP/s of GEMM work")
    del w, x
    torch.cuda.empty_cache()
    return {"workload": f"fused linear + cross-entropy over the Qwen2.5-1.5B head: N={N}, H={H}, "
                        f"V={V}, fp16, forward (stats + dX) and backward; row kernel on one "
                        f"{rows}-row chunk", "gemm_flops": int(flops), **out}


def run_packed_decoder(dev, reps, layers=28):
    """The reference's patch point end to end (solution/body/packed.py): a Qwen2.5-1.5B-shaped
    Qwen2Model (random weights on the device, `layers` decoder layers, hidden 1536, 12 / 2
    heads, MLP 8960) in the reference's training setup (fp32 master weights, bf16 autocast; base
    frozen except q_proj / v_proj, as a LoRA run freezes it), forward + backward on 8 rows padded
    to 1024 tokens with lengths U[512, 1024] (seed 0): the patched forward (pad removal, HIP
    norms, RoPE, varlen attention, SwiGLU recompute MLP) against HF's original forward (sdpa)
    on the same GPU and inputs."""
    import torch
    from transformers import Qwen2Config, Qwen2Model
    from transformers.models.qwen2 import modeling_qwen2

    from solution import body
    from solution.body import _hip

    body.patch()
    cfg = Qwen2Config(vocab_size=151936, hidden_size=1536, intermediate_size=8960,
                      num_hidden_layers=layers, num_attention_heads=12, num_key_value_heads=2,
                      head_dim=128, max_position_embeddings=32768, rms_norm_eps=1e-6,
                      rope_theta=1e6, use_cache=False, tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    with torch.device(dev):
        model = Qwen2Model(cfg)
    for name, p in model.named_parameters():
        p.requires_grad_(name.endswith(("q_proj.weight", "v_proj.weight")))
    model.train()
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(512, 1025, (8,), generator=g)
    ids = torch.randint(0, cfg.vocab_size, (8, 1024), generator=g).to(dev)
    mask = (torch.arange(1024)[None, :] < lens[:, None]).long().to(dev)

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = model(input_ids=ids, attention_mask=mask).last_hidden_state
        out.float().square().mean().backward()

    def timed():
        """ms per step, and the step's peak device memory above what was allocated before it
        (weights, their gradients and the inputs), in GB."""
        for _ in range(2):
            step()
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated(dev)
        torch.cuda.reset_peak_memory_stats(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            step()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps, (torch.cuda.max_memory_allocated(dev) - base) / 1e9

    with _hip.count_launches() as names:
        step()
        torch.cuda.synchronize()
    ours, ours_gb = timed()
    # the reference's memory-for-time switch the other way: the MLP keeps its [T, intermediate]
    # activations instead of recomputing them in backward
    from solution.body import packed

    packed.RECOMPUTE_MLP = False
    try:
        keep, keep_gb = timed()
    finally:
        packed.RECOMPUTE_MLP = True
    cls = modeling_qwen2.Qwen2Model
    patched = cls.forward
    cls.forward = patched.__wrapped__
    try:
        hf, hf_gb = timed()
    finally:
        cls.forward = patched
    log(f"packed decoder ({layers} layers): {ours:.2f} ms vs HF's original forward {hf:.2f} ms; "
        f"step peak memory {ours_gb:.2f} vs {hf_gb:.2f} GB; without the MLP recompute "
        f"{keep:.2f} ms, {keep_gb:.2f} GB")
    del model
    torch.cuda.empty_cache()
    return {"workload": f"Qwen2.5-1.5B-shaped Qwen2Model, {layers} layers, random weights, fp32 master "
                        "weights under bf16 autocast, q/v projections trainable, forward + backward on "
                        "8 rows padded to 1024 tokens (lengths U[512, 1024], seed 0): the patched "
                        "packed forward against HF's original forward (sdpa) on the same GPU",
            "layers": layers, "tokens": int(lens.sum()), "padded_tokens": 8 * 1024,
            "ours_ms": round(ours, 3), "hf_original_ms": round(hf, 3), "speedup": round(hf / ours, 2),
            "step_peak_GB": {"ours": round(ours_gb, 3), "hf_original": round(hf_gb, 3),
                             "what": "peak device memory of the timed steps above what was "
                                     "allocated before them (weights, gradients, inputs)"},
            "without_mlp_recompute": {"ms": round(keep, 3), "step_peak_GB": round(keep_gb, 3),
                                      "what": "packed.RECOMPUTE_MLP off: the MLP keeps its "
                                              "[T, intermediate] activations for backward"},
            "hip_launches_per_step": len(names), "kernels": sorted(set(names))}


def kernel_rooflines(body, reps):
    """Per-launch time of each entry point: a graph of one launch per layer of that kernel
    alone (distinct tensors, as in the sweep), replayed `reps` times, timed with HIP events
    on the replay stream. Returns {name: (us_per_launch, algorithmic_bytes_per_launch, launches_per_step)}."""
    c, T = body.cfg, body.T
    L = c["layers"]
    # With the deferred schedule the norm backward launch is stage 1 (dx and the partials; its
    # algorithmic bytes exclude the 4H of dw, which stage 2 writes); stage 2 is one batched
    # launch per step whose algorithmic bytes are the 2L + 1 weight gradients.
    bwd_bytes = norm_bwd_bytes(T, c["H"], 2, body.save_rstd) - (4 * c["H"] if body.deferred else 0)
    kinds = {
        "rmsnorm_fwd": (lambda: [body.norm_fwd(i) for i in range(2 * L + 1)], 2 * L + 1,
                        norm_fwd_bytes(T, c["H"], 2, body.save_rstd)),
        "rmsnorm_bwd": (lambda: [body.norm_bwd(i) for i in range(2 * L + 1)], 2 * L + 1, bwd_bytes),
        "rope_fwd": (lambda: [body.rope_fwd(l) for l in range(L)], L,
                     rope_bytes(T, c["HQ"], c["HK"], c["D"], 2)),
        "rope_bwd": (lambda: [body.rope_bwd(l) for l in range(L)], L,
                     rope_bytes(T, c["HQ"], c["HK"], c["D"], 2)),
    }
    launches = {}
    if body.deferred:
        # one launch per step; timed as 8 launches in one graph, since a graph of a single
        # 15 us kernel adds the replay's own start-up (~6 us) to every launch
        kinds["dgamma_stage2"] = (lambda: [body.dgamma_stage2() for _ in range(8)], 1,
                                  (2 * L + 1) * 4 * c["H"])
        launches["dgamma_stage2"] = 8
    out = {}
    for name, (fn, n, nbytes) in kinds.items():
        g = capture(fn)
        time_graph(g, 2)
        ms, _ = time_graph(g, reps)
        out[name] = (ms * 1e3 / launches.get(name, n), nbytes, n)
        us = out[name][0]
        log(f"{name}: {us:.2f} us/launch, {nbytes / (us * 1e-6) / 1e9:.0f} GB/s")
    return out


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# The GPU box gives the job of its one GPU a share of 16 host cores (OMP_NUM_THREADS=16 there),
# whatever os.sched_getaffinity reports; the CPU legs use at most that many threads.
CPU_SHARE = 16


def _cpu_threads():
    return max(1, min(len(os.sched_getaffinity(0)), CPU_SHARE))


def _cpu_threads_note():
    return (f"{_cpu_threads()} threads: os.sched_getaffinity reports "
            f"{len(os.sched_getaffinity(0))} cores, capped at the box's {CPU_SHARE}-core share "
            f"for one GPU's job")


def _cpu_time(fn, budget_s, min_reps=5):
    """Median wall time of fn() over at least min_reps runs (after one warm-up), stopping at
    budget_s or 20 runs."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_reps or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_configs(cfg5, budget_s=2.0):
    """The same PyTorch-eager fp32 HF path on the host cores for configs 1-3 (whole) and config
    5 (its longest-sequence share: one 4096-token sequence at H = 3584, 28/4 heads), forward +
    autograd backward; GB/s from the same byte formulas with 4-byte (fp32) elements."""
    import torch

    from oracle import hf_eager

    threads = _cpu_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    eps, theta, D = 1e-6, 1e6, 128

    def inv(d):
        return 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float) / d))

    def norm_pass(x, w, dy):
        xr, wr = x.detach().requires_grad_(), w.detach().requires_grad_()
        torch.autograd.grad(hf_eager.rms_norm(xr, wr, eps), [xr, wr], dy)

    def rope_pass(q, k, dq, dk, pos):
        qr, kr = q.detach().requires_grad_(), k.detach().requires_grad_()
        cos, sin = hf_eager.rotary_cos_sin(inv(q.shape[-1]), pos, qr.dtype)
        qe, ke = hf_eager.apply_rotary_pos_emb(qr, kr, cos, sin, unsqueeze_dim=1)
        torch.autograd.grad([qe, ke], [qr, kr], [dq, dk])

    def norm_case(T, H):
        x, dy = torch.randn(T, H, generator=g), torch.randn(T, H, generator=g)
        w = 1 + 0.02 * torch.randn(H, generator=g)
        return lambda: norm_pass(x, w, dy)

    def rope_case(B, S, HQ, HK, pos):
        q, dq = torch.randn(B, HQ, S, D, generator=g), torch.randn(B, HQ, S, D, generator=g)
        k, dk = torch.randn(B, HK, S, D, generator=g), torch.randn(B, HK, S, D, generator=g)
        return lambda: rope_pass(q, k, dq, dk, pos)

    e = 4
    lens3 = torch.randint(64, 1025, (8,), generator=torch.Generator().manual_seed(0)).tolist()
    T3 = sum(lens3)
    pos3 = torch.cat([torch.arange(n) for n in lens3])[None, :]
    c1 = norm_case(2048, 1536)
    c2 = rope_case(4, 512, 12, 2, torch.arange(512).expand(4, 512))
    c3n, c3r = norm_case(T3, 1536), rope_case(1, T3, 12, 2, pos3)
    H5, HQ5, HK5 = cfg5["H"], cfg5["HQ"], cfg5["HK"]
    c5n, c5r = norm_case(4096, H5), rope_case(1, 4096, HQ5, HK5, torch.arange(4096)[None, :])
    nb = lambda T, H: norm_fwd_bytes(T, H, e, True) + norm_bwd_bytes(T, H, e, True)  # noqa: E731
    cases = {
        "config1": (c1, nb(2048, 1536), 2048, "the whole config"),
        "config2": (c2, 2 * rope_bytes(2048, 12, 2, D, e), 2048, "the whole config"),
        "config3": (lambda: (c3n(), c3r()), nb(T3, 1536) + 2 * rope_bytes(T3, 12, 2, D, e), T3,
                    "the whole config"),
        "config5": (lambda: (c5n(), c5n(), c5r()),
                    2 * nb(4096, H5) + 2 * rope_bytes(4096, HQ5, HK5, D, e), 4096,
                    "one 4096-token sequence of the 65536 (2 norms + q/k RoPE per token, as the "
                    "GPU step)"),
    }
    out = {}
    for name, (fn, nbytes, T, sample) in cases.items():
        t, reps = _cpu_time(fn, budget_s)
        out[name] = {"GB/s": round(nbytes / t / 1e9, 2), "tokens_per_s": round(T / t, 1),
                     "ms": round(t * 1e3, 3), "reps": reps, "cores": threads,
                     "cpu_model": _cpu_model(), "kind": "port", "sample": sample}
        log(f"CPU {name}: {t * 1e3:.2f} ms ({out[name]['GB/s']} GB/s, {threads} threads)")
    return out


def cpu_baseline(cfg, budget_s=12.0, batch=2):
    """PyTorch-eager fp32 HF path (oracle/hf_eager.py) on the host cores: one layer of the
    workload (2 RMSNorms + q/k RoPE, forward + autograd backward) on `batch` of its 8 rows
    (the per-token cost does not depend on the batch)."""
    import torch

    from oracle import hf_eager

    threads = _cpu_threads()
    torch.set_num_threads(threads)
    model = _cpu_model()
    S, H, HQ, HK, D, eps = (cfg[k] for k in ("S", "H", "HQ", "HK", "D", "eps"))
    B = batch
    T = B * S
    g = torch.Generator().manual_seed(0)
    xs = [torch.randn(T, H, generator=g) for _ in range(2)]
    ws = [1 + 0.02 * torch.randn(H, generator=g) for _ in range(2)]
    dys = [torch.randn(T, H, generator=g) for _ in range(2)]
    q = torch.randn(B, HQ, S, D, generator=g)
    k = torch.randn(B, HK, S, D, generator=g)
    dq, dk = torch.randn(B, HQ, S, D, generator=g), torch.randn(B, HK, S, D, generator=g)
    inv = 1.0 / (cfg["theta"] ** (torch.arange(0, D, 2, dtype=torch.float) / D))
    pos = torch.arange(S).expand(B, S)
    times = []
    t_start = time.perf_counter()
    hf_eager.body_step(xs, ws, q, k, dys, dq, dk, inv, pos, eps)  # warm-up (allocator, threads)
    while len(times) < 2 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        hf_eager.body_step(xs, ws, q, k, dys, dq, dk, inv, pos, eps)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    e = 4
    layer_bytes = 2 * (norm_fwd_bytes(T, H, e, True) + norm_bwd_bytes(T, H, e, True)) + \
        2 * rope_bytes(T, HQ, HK, D, e)
    return {"value": round(layer_bytes / t / 1e9, 2), "unit": "GB/s", "cores": threads,
            "cores_note": _cpu_threads_note(), "cpu_model": model, "kind": "port",
            "sample": f"one layer of config 4 (2 RMSNorm + q/k RoPE, fwd + autograd bwd) on "
                      f"{B} of its 8 rows (T={T}), fp32 PyTorch eager (HF Qwen2RMSNorm / apply_rotary_pos_emb "
                      f"restated), median of {len(times)} reps, {t * 1e3:.1f} ms per layer; "
                      f"bytes counted with e=4",
            # a full sweep is L layers plus the final norm (~ half a layer)
            "tokens_per_s": round(T / (t * (cfg["layers"] + 0.5)), 1)}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--rstd", choices=["saved", "recomputed"], default="saved")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--no-config5", action="store_true", help="skip the config 5 stress line")
    ap.add_argument("--no-attention", action="store_true", help="skip the attention measurement")
    ap.add_argument("--no-lm-head", action="store_true", help="skip the fused LM head measurement")
    ap.add_argument("--no-packed", action="store_true",
                    help="skip the end-to-end packed decoder against HF's original forward")
    ap.add_argument("--packed-only", action="store_true",
                    help="profiling run: only the end-to-end packed decoder leg (its log line, "
                         "no JSON)")
    ap.add_argument("--pmc-kernel", choices=["rmsnorm_fwd", "rmsnorm_bwd", "rope_fwd", "rope_bwd"],
                    help="counter-collection run: a calibration copy of 256 MiB (read 256 MiB, "
                         "write 256 MiB) three times, then one launch per layer of this kernel "
                         "at config 4; no timing, no JSON (for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (--gpus {args.gpus} "
              "requested). The path shards by tokens with no communication except one H-float "
              "all-reduce of the norm weight gradients; run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    from solution.body import _hip

    _hip.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.packed_only:
        run_packed_decoder(dev, 5)
        return 0
    cfg = CFG4
    save_rstd = args.rstd == "saved"
    log(f"allocating config 4 ({cfg['layers']} layers, T={cfg['B'] * cfg['S']}) on {torch.cuda.get_device_name(dev)}")
    body = Body(cfg, save_rstd, dev)
    torch.cuda.synchronize()
    if args.pmc_kernel:
        src = torch.ones(128 << 20, device=dev, dtype=torch.bfloat16)  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        L = cfg["layers"]
        if args.pmc_kernel.startswith("rmsnorm"):
            fn = body.norm_fwd if args.pmc_kernel == "rmsnorm_fwd" else body.norm_bwd
            for i in range(2 * L + 1):
                fn(i)
        else:
            fn = body.rope_fwd if args.pmc_kernel == "rope_fwd" else body.rope_bwd
            for l in range(L):
                fn(l)
        torch.cuda.synchronize()
        log(f"pmc run done: {args.pmc_kernel}")
        return 0
    log("capturing the step graph")
    g = capture(body.step)
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    ev_ms, wall_ms = time_graph(g, args.steps)
    step_bytes = body.step_bytes()
    ms = max(ev_ms, wall_ms)
    gbs = step_bytes / (ms * 1e-3) / 1e9
    log(f"step {ms:.3f} ms (events {ev_ms:.3f}), {gbs:.0f} GB/s = {gbs / PEAK_GBS:.1%} of peak")

    kr = kernel_rooflines(body, args.kernel_reps)
    name, (us, nbytes, n) = max(kr.items(), key=lambda kv: kv[1][0] * kv[1][2])
    achieved = nbytes / (us * 1e-6) / 1e9
    # HBM bytes per launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE runs (bench.py
    # --pmc-kernel), each scaled by the counter's reading on a 256 MiB copy
    traffic = None
    tpath = ROOT / "profiles" / "hbm_traffic_config4.json"
    if tpath.exists() and save_rstd:
        traffic = json.loads(tpath.read_text()).get(name, {}).get("traffic_bytes")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic, "kernel": name,
                "us_per_launch": round(us, 3), "bytes_per_launch": nbytes,
                "all_kernels": {k: {"us": round(v[0], 3), "GB/s": round(v[1] / (v[0] * 1e-6) / 1e9, 1),
                                    "launches_per_step": v[2]} for k, v in kr.items()}}
    # the same kernel's average duration in the committed rocprofv3 kernel-trace summary of
    # this workload, when there is one: the fraction from the trace beside the event one
    ppath = ROOT / "profiles" / "kernel_trace_config4.json"
    if ppath.exists() and save_rstd:
        prof = json.loads(ppath.read_text()).get(name)
        if prof and prof.get("avg_us"):
            roofline["frac_trace"] = round(nbytes / (prof["avg_us"] * 1e-6) / 1e9 / PEAK_GBS, 4)
            roofline["trace_avg_us"] = prof["avg_us"]

    c4dims = dict(T=body.T, H=cfg["H"], HQ=cfg["HQ"], HK=cfg["HK"], D=cfg["D"], layers=cfg["layers"])
    del g
    del body
    torch.cuda.empty_cache()
    ceiling = stream_ceiling(dev, c4dims, {k: v[0] for k, v in kr.items()}, args.kernel_reps, ms)
    small = run_small_configs(dev, args.kernel_reps)
    c4_other = run_config4_other_rstd(dev, max(args.steps // 3, 5), not save_rstd)
    c4_per_call = run_config4_per_call_dgamma(dev, max(args.steps // 3, 5), save_rstd)
    c5 = None if args.no_config5 else run_config5(dev, max(args.steps // 3, 5))
    api = run_api_variant(dev, max(args.steps // 3, 5))
    attn = None if args.no_attention else run_attention(dev, max(args.steps // 3, 5))
    swi = run_swiglu(dev, max(args.steps // 3, 5))
    lora = run_lora_dropout(dev, max(args.steps // 3, 5))
    nf4 = run_nf4(dev, max(args.steps // 3, 5))
    lmh = None if args.no_lm_head else run_lm_head(dev, max(args.steps // 3, 5))
    pdec = None if args.no_packed else run_packed_decoder(dev, 5)

    cpu = None
    if not args.no_cpu:
        log("CPU baseline (PyTorch eager fp32, one layer)")
        cpu = cpu_baseline(cfg)
        log(f"CPU: {cpu['value']} GB/s on {cpu['cores']} threads")
        # the same eager path on the other configs, each beside its GPU figures
        for name, row in cpu_configs(CFG5).items():
            target = c5 if name == "config5" else small[name]
            if target is not None:
                target["cpu"] = row

    T = cfg["B"] * cfg["S"]
    out = {
        "metric": "RMSNorm+RoPE fwd+bwd achieved HBM GB/s (% of peak), Qwen2.5-1.5B shape",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "config4: 28-layer Qwen2.5-1.5B body sweep, 2 RMSNorm + q/k RoPE "
                               "per layer + final norm, forward then backward (dx, dw, dq, dk)",
                   "tokens": T, "batch": cfg["B"], "seq_len": cfg["S"], "hidden": cfg["H"],
                   "q_heads": cfg["HQ"], "kv_heads": cfg["HK"], "head_dim": cfg["D"],
                   "io_dtype": "bf16", "rstd": args.rstd, "graph": True,
                   "dgamma": "stage 2 deferred to one batched launch per step (the Python API's "
                             "schedule in a loss.backward() pass, norm_rope.DEFER_WEIGHT_GRAD)",
                   "bytes_per_step": step_bytes},
        "frac_of_peak": round(gbs / PEAK_GBS, 4),
        "tokens_per_s": round(T / (ms * 1e-3), 1),
        "ms_per_step_events": round(ev_ms, 4),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "stream_ceiling": ceiling,
        "config4_other_rstd": c4_other,
        "config4_per_call_dgamma": c4_per_call,
        "config1": small["config1"],
        "config2": small["config2"],
        "config3": small["config3"],
        "config5": c5,
        "api_variant": api,
        "attention": attn,
        "swiglu": swi,
        "lora_dropout": lora,
        "nf4_dequant": nf4,
        "lm_head": lmh,
        "packed_decoder": pdec,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
