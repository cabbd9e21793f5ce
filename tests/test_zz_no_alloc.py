"""esep_rmsnorm_bwd_noalloc (the norm backward with a weight gradient whose partials live in the
library's own device scratch array) against esep_rmsnorm_bwd with a caller workspace: dx and
dw bit for bit, on two calls in a row with the second one smaller (the array keeps the first
call's contents, which the second must not read), then a wider row; and the size limit."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
EPS = 1e-6


def _lib():
    from solution.body import _hip

    return _hip, _hip.lib()


def _inputs(T, n, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(T, n, generator=g, device=DEV).to(torch.bfloat16)
    dy = torch.randn(T, n, generator=g, device=DEV).to(torch.bfloat16)
    w = 1 + 0.02 * torch.randn(n, generator=g, device=DEV)
    rstd = torch.empty(T, device=DEV)
    return x, dy, w, rstd


def _noalloc(lib, x, dy, w, rstd, dx, dw):
    T, n = x.shape
    arr = (ctypes.c_void_p * 5)(dy.data_ptr())
    return lib.esep_rmsnorm_bwd_noalloc(arr, 1, 2, n, None, x.data_ptr(), 2, n, 0, rstd.data_ptr(),
                                        w.data_ptr(), None, None, 0, None, dx.data_ptr(), 2, n,
                                        dw.data_ptr(), 0, T, n, EPS,
                                        torch.cuda.current_stream().cuda_stream)


def test_noalloc_matches_workspace_entry_point():
    hip, lib = _lib()
    for T, n, seed in ((8192, 1536, 1), (300, 1536, 2), (4097, 3584, 3)):
        x, dy, w, rstd = _inputs(T, n, seed)
        hip.rmsnorm_fwd(x, w, torch.empty_like(x), EPS, rstd=rstd)
        dx_ref, dw_ref = torch.empty_like(x), torch.empty(n, device=DEV)
        hip.rmsnorm_bwd([dy], x, w, EPS, rstd=rstd, dx=dx_ref, dw=dw_ref)
        dx, dw = torch.full_like(x, float("nan")), torch.full((n,), float("nan"), device=DEV)
        rc = _noalloc(lib, x, dy, w, rstd, dx, dw)
        assert rc == 0, lib.esep_last_error()
        torch.cuda.synchronize()
        assert torch.equal(dx, dx_ref), (T, n)
        assert torch.equal(dw, dw_ref), (T, n)


def test_noalloc_rejects_partials_beyond_the_scratch():
    hip, lib = _lib()
    arr = (ctypes.c_void_p * 5)(64)
    # 65536 x 16384: 512 partial rows of 16384 floats, 4x the 2^21-float scratch
    rc = lib.esep_rmsnorm_bwd_noalloc(arr, 1, 2, 16384, None, 64, 2, 16384, 0, None, 64, None, None,
                                      0, None, 64, 2, 16384, 64, 0, 65536, 16384, EPS, None)
    assert rc == -2 and b"scratch" in lib.esep_last_error()
    rc = lib.esep_rmsnorm_bwd_noalloc(arr, 1, 2, 8, None, 64, 2, 8, 0, None, 64, None, None,
                                      0, None, 64, 2, 8, None, 0, 4, 8, EPS, None)
    assert rc == -1 and b"dw is required" in lib.esep_last_error()


def test_noalloc_stream_on_the_current_device():
    """A stream of the current device (not torch's current stream) is accepted and gives the same
    bits as the workspace entry point on it."""
    hip, lib = _lib()
    x, dy, w, rstd = _inputs(1000, 1536, 9)
    hip.rmsnorm_fwd(x, w, torch.empty_like(x), EPS, rstd=rstd)
    dx_ref, dw_ref = torch.empty_like(x), torch.empty(1536, device=DEV)
    hip.rmsnorm_bwd([dy], x, w, EPS, rstd=rstd, dx=dx_ref, dw=dw_ref)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        dx, dw = torch.full_like(x, float("nan")), torch.full((1536,), float("nan"), device=DEV)
        assert _noalloc(lib, x, dy, w, rstd, dx, dw) == 0, lib.esep_last_error()
    s.synchronize()
    assert torch.equal(dx, dx_ref) and torch.equal(dw, dw_ref)


@pytest.mark.skipif(torch.cuda.device_count() < 2, reason="needs a second GPU for a stream on "
                    "another device; this pool's boxes have one")
def test_noalloc_rejects_a_stream_of_another_device():
    hip, lib = _lib()
    x, dy, w, rstd = _inputs(64, 1536, 10)
    dx, dw = torch.empty_like(x), torch.empty(1536, device=DEV)
    other = torch.cuda.Stream(device=1)
    arr = (ctypes.c_void_p * 5)(dy.data_ptr())
    with torch.cuda.device(0):
        rc = lib.esep_rmsnorm_bwd_noalloc(arr, 1, 2, 1536, None, x.data_ptr(), 2, 1536, 0,
                                          rstd.data_ptr(), w.data_ptr(), None, None, 0, None,
                                          dx.data_ptr(), 2, 1536, dw.data_ptr(), 0, 64, 1536, EPS,
                                          other.cuda_stream)
    assert rc == -1  # ESEP_EINVAL
    assert b"device" in lib.esep_last_error()
