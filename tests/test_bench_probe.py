"""The streaming probes bench.py holds the path kernels against (libesep_probe.so, built from
esep-soup-kernels_amd/benchlib/probe.hip; measurement code, outside the product library).

CPU: the library loads and rejects bad arguments before launching anything. GPU: every variant
computes out = a (+ b) exactly, also where the last block of a one-shot grid or the last step of
a strided walk is partial."""

import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "esep-soup-kernels_amd"))

import benchlib  # noqa: E402


def test_probe_validation():
    h = benchlib.lib()
    O, S = benchlib.ONESHOT, benchlib.STRIDED
    assert h.esep_probe_stream(O, 1, 256, 1, None, None, 64, 64, None) == -1
    assert h.esep_probe_stream(O, 1, 256, 1, 64, None, 64, 40, None) == -2      # not 16-byte sized
    assert h.esep_probe_stream(O, 1, 256, 1, 64, None, 64, 1 << 32, None) == -2  # over 4 GiB - 16
    assert h.esep_probe_stream(O, 1, 256, 1, 64, 8, 64, 64, None) == -3        # misaligned b
    assert h.esep_probe_stream(2, 1, 256, 1, 64, None, 64, 64, None) == -4     # mode
    assert h.esep_probe_stream(O, 3, 256, 1, 64, None, 64, 64, None) == -4     # u
    assert h.esep_probe_stream(S, 1, 128, 1, 64, None, 64, 64, None) == -4     # threads
    assert h.esep_probe_stream(S, 1, 256, 0, 64, None, 64, 64, None) == -2     # no blocks
    assert h.esep_probe_stream(O, 1, 256, 1, 64, None, 64, 0, None) == 0       # nothing to do
    assert benchlib.grid(O, 4, 256, 16 * 1024 * 4 + 16, 7) == 5
    assert benchlib.grid(S, 4, 256, 1 << 20, 7) == 7


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["oneshot", "strided"])
@pytest.mark.parametrize("two", [False, True])
def test_probe_values(mode, two):
    import torch

    m = benchlib.ONESHOT if mode == "oneshot" else benchlib.STRIDED
    g = torch.Generator(device="cuda").manual_seed(7)
    n = (1 << 20) + 4 * 37  # int32 elements: ragged against every grid
    a = torch.randint(0, 1 << 30, (n,), generator=g, device="cuda", dtype=torch.int32)
    b = torch.randint(0, 1 << 30, (n,), generator=g, device="cuda", dtype=torch.int32) if two else None
    want = a + b if two else a
    for u in (1, 2, 4, 8):
        for threads in (256, 512):
            out = torch.full_like(a, -1)
            benchlib.stream(a, out, b, mode=m, u=u, threads=threads, blocks=37)
            torch.cuda.synchronize()
            assert torch.equal(out, want), (mode, two, u, threads)
