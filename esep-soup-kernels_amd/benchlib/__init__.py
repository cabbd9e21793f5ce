"""ctypes binding of libesep_probe.so, the streaming probes bench.py holds the path kernels
against (probe.hip). Measurement code only: nothing in solution/ imports it."""

import ctypes
from pathlib import Path

LIB = Path(__file__).resolve().parent / "libesep_probe.so"
ONESHOT, STRIDED = 0, 1
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise RuntimeError(f"{LIB} is not built (python esep-soup-kernels_amd/build.py)")
        h = ctypes.CDLL(str(LIB))
        h.esep_probe_stream.restype = ctypes.c_int
        h.esep_probe_stream.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_int64, ctypes.c_void_p]
        h.esep_probe_grid.restype = ctypes.c_int
        h.esep_probe_grid.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                      ctypes.c_int]
        _lib = h
    return _lib


def stream(a, out, b=None, mode=STRIDED, u=2, threads=512, blocks=256):
    """out = a (+ b) over out's bytes on torch's current stream (contiguous device tensors, a and
    b at least as large as out)."""
    import torch

    nbytes = out.numel() * out.element_size()
    for t in (a, b):
        if t is not None and (not t.is_contiguous() or t.numel() * t.element_size() < nbytes):
            raise ValueError("probe inputs must be contiguous and as large as out")
    rc = lib().esep_probe_stream(mode, u, threads, blocks, a.data_ptr(),
                                 None if b is None else b.data_ptr(), out.data_ptr(), nbytes,
                                 torch.cuda.current_stream(out.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(f"esep_probe_stream failed: {rc}")


def grid(mode, u, threads, nbytes, blocks):
    return lib().esep_probe_grid(mode, u, threads, nbytes, blocks)
