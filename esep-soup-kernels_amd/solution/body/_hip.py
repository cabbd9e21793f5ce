"""ctypes binding of libesep_body.so, the HIP kernels of the decoder-body path (gfx950).

This module is the only place that talks to the C ABI (include/esep_body.h). It loads the
library that build.py compiled next to this file, declares every entry point's signature,
turns a non-zero status into EsepError (with the library's message), and passes torch's
current HIP stream so that every launch is ordered with the surrounding torch work.

There is no fallback: a missing library, a CPU tensor or an unsupported dtype is an error.

Launch accounting: every entry point records the name of the reference Triton kernel it
replaces (`_add_rmsnorm_fwd`, `_add_rmsnorm_bwd`, `_rope_kernel`; reference
solution/body/norm_rope.py:83, :116, :356), so tests can count launches the way the
reference's tests wrap JITFunction.run (reference solution/test_body_norm_rope.py:200-211).
"""

import contextlib
import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libesep_body.so")
ABI_VERSION = 1

F32, F16, BF16, I32, I64 = 0, 1, 2, 3, 4
_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16,
       torch.int32: I32, torch.int64: I64}

# Entry points and their C signatures (include/esep_body.h).
_vp, _i32, _i64, _f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
_I64x3 = ctypes.c_int64 * 3
_I64x2 = ctypes.c_int64 * 2
_VP5 = ctypes.c_void_p * 5
SIGNATURES = {
    "esep_abi_version": (_i32, []),
    "esep_last_error": (ctypes.c_char_p, []),
    "esep_rmsnorm_fwd": (_i32, [_vp, _i32, _i64, _vp, _i32, _i64, _vp, _vp, _i64, _vp, _i32, _i64,
                                _vp, _vp, _vp, _i32, _i64, _i64, _f32, _vp]),
    "esep_rmsnorm_partials": (_i64, [_i64, _i64]),
    "esep_rmsnorm_bwd": (_i32, [_vp, _i32, _i32, _i64, _vp, _vp, _i32, _i64, _i32, _vp, _vp, _vp,
                                _vp, _i32, _vp, _vp, _i32, _i64, _vp, _i64, _vp, _i32, _i64, _i64,
                                _f32, _vp]),
    "esep_rmsnorm_bwd_noalloc": (_i32, [_vp, _i32, _i32, _i64, _vp, _vp, _i32, _i64, _i32, _vp,
                                        _vp, _vp, _vp, _i32, _vp, _vp, _i32, _i64, _vp, _i32,
                                        _i64, _i64, _f32, _vp]),
    "esep_dgamma_reduce": (_i32, [_vp, _i64, _i64, _vp, _i32, _vp]),
    "esep_dgamma_reduce_batch": (_i32, [_vp, _i32, _i64, _i32, _vp]),
    "esep_attn_fwd": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i32, _i64, _i32,
                             _i32, _i32, _vp, _i32, _i32, _f32, _vp]),
    "esep_attn_bwd_workspace": (_i64, [_i64, _i32, _i32, _i32]),
    "esep_swiglu_fwd": (_i32, [_vp, _vp, _vp, _i64, _i32, _vp]),
    "esep_lora_dropout_fwd": (_i32, [_vp, _vp, _vp, _i64, _f32, _i32, _vp]),
    "esep_nf4_dequant": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _vp]),
    "esep_head_row_softmax": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32,
                                     _f32, _i32, _vp]),
    "esep_nf4_dequant_multi": (_i32, [_vp, _i32, _i32, _vp]),
    "esep_lora_dropout_bwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _f32, _i32, _i32, _vp]),
    "esep_swiglu_bwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i32, _vp]),
    "esep_attn_bwd": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp,
                             _vp, _i64, _vp, _i64, _vp, _i64, _i32, _i64, _i32, _i32, _i32, _vp,
                             _i32, _i32, _f32, _vp]),
    "esep_rope": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i64,
                         _i32, _i32, _i32, _vp, _i32, _vp, _vp, _i32, _vp, _f32, _vp]),
}


class EsepError(RuntimeError):
    """A call into libesep_body.so failed (bad argument or launch error)."""


_lib = None
_lock = threading.Lock()


def lib():
    """The loaded library (loaded once, signatures declared). Raises if it is not built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise EsepError(f"{LIB_PATH} is not built: run "
                                    "`python esep-soup-kernels_amd/build.py` (or __graft_entry__.build())")
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype, fn.argtypes = res, args
                got = handle.esep_abi_version()
                if got != ABI_VERSION:
                    raise EsepError(f"libesep_body.so ABI {got}, this binding expects {ABI_VERSION}")
                _lib = handle
    return _lib


# ---------------------------------------------------------------------------------------
# launch accounting
# ---------------------------------------------------------------------------------------
_counters = []


def _record(name):
    for c in _counters:
        c.append(name)


@contextlib.contextmanager
def count_launches():
    """Collects the reference kernel names of every library launch made inside the block."""
    names = []
    _counters.append(names)
    try:
        yield names
    finally:
        _counters.remove(names)


# ---------------------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------------------
def _check(rc, what):
    if rc != 0:
        msg = lib().esep_last_error().decode(errors="replace")
        raise EsepError(f"{what} failed (status {rc}): {msg}")


def dtype_code(dt):
    try:
        return _DT[dt]
    except KeyError:
        raise EsepError(f"unsupported dtype {dt}") from None


def _dev(*tensors):
    """Device of the first tensor; every given tensor must be a HIP tensor on it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise EsepError(f"libesep_body kernels need device (HIP) tensors, got {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise EsepError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _p(t):
    return None if t is None else t.data_ptr()


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _rows_ld(t, n):
    """Leading dimension of a [rows, n] tensor whose last dim is contiguous. The column stride
    is checked whenever a row has more than one element (a one-row view such as t[:, ::2] or an
    expanded row has a non-unit column stride too); a multi-row tensor must not overlap its
    rows (row stride >= n, so an expanded stride 0 is rejected)."""
    if t.dim() != 2 or t.shape[1] != n or (n > 1 and t.stride(1) != 1):
        raise EsepError(f"expected a [rows, {n}] tensor with unit column stride, got "
                        f"{tuple(t.shape)} / {t.stride()}")
    if t.shape[0] > 1 and t.stride(0) < n:
        raise EsepError(f"rows of a [rows, {n}] tensor overlap (row stride {t.stride(0)})")
    return t.stride(0) if t.shape[0] > 1 else n


# ---------------------------------------------------------------------------------------
# entry points
# ---------------------------------------------------------------------------------------
def rmsnorm_fwd(x, w, y, eps, delta=None, r_out=None, rstd=None, slot=None, xs=None,
                n_special=0, name="_add_rmsnorm_fwd"):
    """y = w * rmsnorm(x (+ delta)) row-wise; optional r_out, rstd, exact-channel xs.
    x, delta, r_out, y: [rows, n] (unit column stride); w fp32 [n]; rstd fp32 [rows]."""
    rows, n = x.shape
    dev = _dev(x, delta, w, r_out, y, rstd, slot, xs)
    if w.dtype != torch.float32 or not w.is_contiguous() or w.numel() != n:
        raise EsepError("w must be a contiguous fp32 [n] tensor")
    rc = lib().esep_rmsnorm_fwd(
        _p(x), dtype_code(x.dtype), _rows_ld(x, n),
        _p(delta), dtype_code(delta.dtype) if delta is not None else 0,
        _rows_ld(delta, n) if delta is not None else 0,
        _p(w), _p(r_out), _rows_ld(r_out, n) if r_out is not None else 0,
        _p(y), dtype_code(y.dtype), _rows_ld(y, n),
        _p(rstd), _p(slot), _p(xs), int(n_special), rows, n, float(eps), _stream(dev))
    _check(rc, "esep_rmsnorm_fwd")
    _record(name)


def rmsnorm_partials(rows, n):
    """Rows of the fp32 weight-gradient workspace esep_rmsnorm_bwd needs for this shape."""
    return int(lib().esep_rmsnorm_partials(int(rows), int(n)))


def rmsnorm_bwd(dys, x, w, eps, from_y=False, rstd=None, dr_out=None, slot=None, xs=None,
                n_special=0, dr=None, dx=None, dw=None, workspace=None, partials=None,
                name="_add_rmsnorm_bwd"):
    """Backward of rmsnorm_fwd; see esep_rmsnorm_bwd. dys: list of [rows, n] tensors of one
    dtype (their sum is dy). dr: fp32 [rows, n] out; dx: low-precision [rows, n] out;
    dw: [n] out, reduced through a [P, n] fp32 workspace (P = rmsnorm_partials(rows, n));
    pass `workspace` to reuse one, else it is allocated here. Without dw, `partials` (an fp32
    [P, n] tensor) receives the weight-gradient partials for a later dgamma_reduce."""
    rows, n = x.shape
    dev = _dev(x, w, rstd, dr_out, slot, xs, dr, dx, dw, *dys)
    if len(dys) > 5:
        raise EsepError("at most 5 gradients of y")
    if w.dtype != torch.float32 or not w.is_contiguous() or w.numel() != n:
        raise EsepError("w must be a contiguous fp32 [n] tensor")
    if len({d.dtype for d in dys}) > 1:
        raise EsepError("all gradients of y must share one dtype")
    lds = {_rows_ld(d, n) for d in dys}
    if len(lds) > 1:
        raise EsepError("all gradients of y must share one row stride")
    ld_dy = lds.pop() if lds else n
    outs = [t for t in (dr_out, dr, dx) if t is not None]
    louts = {_rows_ld(t, n) for t in outs}
    if len(louts) > 1:
        raise EsepError("dr_out, dr and dx must share one row stride")
    ld_out = louts.pop() if louts else n
    part = None
    n_part = 0
    if dw is not None and partials is not None:
        raise EsepError("pass either dw (reduced here) or partials (reduced later), not both")
    if partials is not None:
        n_part = rmsnorm_partials(rows, n)
        if (partials.dtype != torch.float32 or not partials.is_contiguous()
                or tuple(partials.shape) != (n_part, n) or partials.device != dev):
            raise EsepError(f"partials must be a contiguous fp32 [{n_part}, {n}] tensor")
        part = partials
    elif dw is not None:
        n_part = rmsnorm_partials(rows, n)
        if workspace is not None:
            if (workspace.dtype != torch.float32 or not workspace.is_contiguous()
                    or workspace.numel() < n_part * n or workspace.device != dev):
                raise EsepError(f"workspace must be a contiguous fp32 tensor of >= {n_part}x{n}")
            part = workspace
        else:
            part = torch.empty((max(n_part, 1), n), device=dev, dtype=torch.float32)
    arr = _VP5(*([d.data_ptr() for d in dys] + [None] * (5 - len(dys))))
    rc = lib().esep_rmsnorm_bwd(
        arr, len(dys), dtype_code(dys[0].dtype) if dys else 0, ld_dy,
        _p(dr_out), _p(x), dtype_code(x.dtype), _rows_ld(x, n), int(bool(from_y)),
        _p(rstd), _p(w), _p(slot), _p(xs), int(n_special),
        _p(dr), _p(dx), dtype_code(dx.dtype) if dx is not None else 0, ld_out,
        _p(part), n_part, _p(dw), dtype_code(dw.dtype) if dw is not None else 0,
        rows, n, float(eps), _stream(dev))
    _check(rc, "esep_rmsnorm_bwd")
    _record(name)


def dgamma_reduce(partials, dw, name="_dgamma_reduce"):
    """dw[j] = sum_p partials[p, j] (fp32 [P, n] contiguous) in the fixed order of
    esep_dgamma_reduce; dw: [n] fp32 / fp16 / bf16 out."""
    dev = _dev(partials, dw)
    if partials.dtype != torch.float32 or not partials.is_contiguous() or partials.dim() != 2:
        raise EsepError("partials must be a contiguous fp32 [P, n] tensor")
    P, n = partials.shape
    if not dw.is_contiguous() or dw.numel() != n:
        raise EsepError(f"dw must be a contiguous [{n}] tensor")
    rc = lib().esep_dgamma_reduce(_p(partials) if P else None, P, n, _p(dw), dtype_code(dw.dtype),
                                  _stream(dev))
    _check(rc, "esep_dgamma_reduce")
    _record(name)


class DgammaItem(ctypes.Structure):
    """esep_dgamma_item (include/esep_body.h)."""
    _fields_ = [("partials", _vp), ("n_partials", _i64), ("dw", _vp)]


DGAMMA_BATCH_MAX = 64


def dgamma_reduce_batch(partials, dws, name="_dgamma_reduce_batch"):
    """Stage 2 of several norms in one launch (esep_dgamma_reduce_batch): dws[i] gets exactly
    what dgamma_reduce(partials[i], dws[i]) would write. partials: fp32 [P_i, n] contiguous
    tensors (P_i may differ), dws: contiguous [n] tensors of one float dtype."""
    if len(partials) != len(dws) or not 1 <= len(dws) <= DGAMMA_BATCH_MAX:
        raise EsepError(f"1..{DGAMMA_BATCH_MAX} (partials, dw) pairs per launch")
    dev = _dev(*partials, *dws)
    n = dws[0].numel()
    arr = (DgammaItem * len(dws))()
    for i, (part, dw) in enumerate(zip(partials, dws)):
        if part.dtype != torch.float32 or not part.is_contiguous() or part.dim() != 2:
            raise EsepError("partials must be contiguous fp32 [P, n] tensors")
        if part.shape[1] != n or dw.numel() != n or not dw.is_contiguous() or dw.dtype != dws[0].dtype:
            raise EsepError(f"every dw must be a contiguous [{n}] tensor of one dtype")
        arr[i] = DgammaItem(_p(part) if part.shape[0] else None, part.shape[0], _p(dw))
    rc = lib().esep_dgamma_reduce_batch(ctypes.cast(arr, _vp), len(dws), n, dtype_code(dws[0].dtype),
                                        _stream(dev))
    _check(rc, "esep_dgamma_reduce_batch")
    _record(name)


def rope(q, k, qo, ko, inv_freq, sign, q_delta=None, positions=None, cu_seqlens=None,
         name="_rope_kernel"):
    """Rotate q and k (4-D (B, S, H, D) views with unit last stride) into qo / ko.
    positions: None (pos = s), or an int32/int64 tensor broadcastable as (B, S) given as a
    (B, S) view; cu_seqlens: int32 [n_seq + 1] (B must be 1)."""
    dev = _dev(q, k, qo, ko, inv_freq, q_delta, positions, cu_seqlens)
    B, S, HQ, D = q.shape
    HK = k.shape[2]
    for t in (q, k, qo, ko) + ((q_delta,) if q_delta is not None else ()):
        if t.stride(3) != 1 and t.shape[3] > 1:
            raise EsepError("rope tensors need a unit stride on the head dim")
    if inv_freq.dtype != torch.float32 or not inv_freq.is_contiguous() or inv_freq.numel() != D // 2:
        raise EsepError("inv_freq must be a contiguous fp32 [D/2] tensor")
    dt = dtype_code(q.dtype)
    if any(t.dtype != q.dtype for t in (k, qo, ko) + ((q_delta,) if q_delta is not None else ())):
        raise EsepError("q, k, q_delta and the outputs must share one dtype")

    def st(t):
        return _I64x3(t.stride(0), t.stride(1), t.stride(2))

    pos_ptr, pos_dt, pos_st = None, 0, None
    if positions is not None:
        if positions.dtype not in (torch.int32, torch.int64) or positions.dim() != 2:
            raise EsepError("positions must be an int32/int64 (B, S) view")
        pos_ptr, pos_dt = positions.data_ptr(), dtype_code(positions.dtype)
        pos_st = _I64x2(positions.stride(0) if positions.shape[0] > 1 else 0,
                        positions.stride(1) if positions.shape[1] > 1 else 0)
    cu_ptr, n_seq = None, 0
    if cu_seqlens is not None:
        if cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1 or not cu_seqlens.is_contiguous():
            raise EsepError("cu_seqlens must be a contiguous int32 [n_seq + 1] tensor")
        cu_ptr, n_seq = cu_seqlens.data_ptr(), cu_seqlens.numel() - 1
    rc = lib().esep_rope(
        q.data_ptr(), st(q), _p(q_delta), st(q_delta) if q_delta is not None else None,
        k.data_ptr(), st(k), qo.data_ptr(), st(qo), ko.data_ptr(), st(ko),
        dt, B, S, HQ, HK, D, pos_ptr, pos_dt, pos_st, cu_ptr, n_seq,
        inv_freq.data_ptr(), float(sign), _stream(dev))
    _check(rc, "esep_rope")
    _record(name)


def _tokens_ld(t, name):
    """Token stride of a [T, H, D] tensor whose heads and head dim are packed (stride D, 1)."""
    if t.dim() != 3 or (t.shape[2] > 1 and t.stride(2) != 1) or (t.shape[1] > 1 and t.stride(1) != t.shape[2]):
        raise EsepError(f"{name} must be a [T, H, D] tensor with contiguous heads")
    return t.stride(0)


def attn_fwd(q, k, v, o, cu_seqlens, max_seqlen, scale, lse=None, name="_attn_fwd"):
    """Varlen causal attention forward (esep_attn_fwd). q, o: [T, HQ, D]; k, v: [T, HK, D];
    cu_seqlens int32 [n_seq + 1] on the device; lse: fp32 [HQ, T] out or None."""
    dev = _dev(q, k, v, o, cu_seqlens, lse)
    T, HQ, D = q.shape
    HK = k.shape[1]
    if k.shape != (T, HK, D) or v.shape != (T, HK, D) or o.shape != (T, HQ, D):
        raise EsepError("attention shapes: q, o [T, HQ, D] and k, v [T, HK, D]")
    if any(t.dtype != q.dtype for t in (k, v, o)):
        raise EsepError("q, k, v and o must share one dtype")
    if cu_seqlens.dtype != torch.int32 or not cu_seqlens.is_contiguous():
        raise EsepError("cu_seqlens must be a contiguous int32 tensor")
    if lse is not None and (lse.dtype != torch.float32 or not lse.is_contiguous() or lse.shape != (HQ, T)):
        raise EsepError("lse must be a contiguous fp32 [HQ, T] tensor")
    rc = lib().esep_attn_fwd(
        _p(q), _tokens_ld(q, "q"), _p(k), _tokens_ld(k, "k"), _p(v), _tokens_ld(v, "v"),
        _p(o), _tokens_ld(o, "o"), _p(lse), dtype_code(q.dtype), T, HQ, HK, D, _p(cu_seqlens),
        cu_seqlens.numel() - 1, int(max_seqlen), float(scale), _stream(dev))
    _check(rc, "esep_attn_fwd")
    _record(name)


def attn_bwd_workspace(T, HQ, HK, D):
    """Floats of fp32 workspace esep_attn_bwd needs for this shape."""
    return int(lib().esep_attn_bwd_workspace(int(T), int(HQ), int(HK), int(D)))


def attn_bwd(q, k, v, o, dout, lse, dq, dk, dv, cu_seqlens, max_seqlen, scale, workspace=None,
             name="_attn_bwd"):
    """Backward of attn_fwd (esep_attn_bwd): dq [T, HQ, D], dk, dv [T, HK, D] out. `workspace`
    is a contiguous fp32 tensor of >= attn_bwd_workspace(T, HQ, HK, D) elements (allocated here
    when not given)."""
    dev = _dev(q, k, v, o, dout, lse, dq, dk, dv, cu_seqlens, workspace)
    T, HQ, D = q.shape
    HK = k.shape[1]
    for t, shp in ((o, (T, HQ, D)), (dout, (T, HQ, D)), (dq, (T, HQ, D)), (k, (T, HK, D)),
                   (v, (T, HK, D)), (dk, (T, HK, D)), (dv, (T, HK, D))):
        if tuple(t.shape) != shp or t.dtype != q.dtype:
            raise EsepError("attention backward shapes / dtypes do not match q [T, HQ, D], k [T, HK, D]")
    if lse.dtype != torch.float32 or not lse.is_contiguous() or tuple(lse.shape) != (HQ, T):
        raise EsepError("lse must be a contiguous fp32 [HQ, T] tensor")
    if cu_seqlens.dtype != torch.int32 or not cu_seqlens.is_contiguous():
        raise EsepError("cu_seqlens must be a contiguous int32 tensor")
    need = attn_bwd_workspace(T, HQ, HK, D)
    if workspace is None:
        workspace = torch.empty(max(need, 1), device=dev, dtype=torch.float32)
    elif (workspace.dtype != torch.float32 or not workspace.is_contiguous()
          or workspace.numel() < need or workspace.device != dev):
        raise EsepError(f"workspace must be a contiguous fp32 tensor of >= {need} elements")
    rc = lib().esep_attn_bwd(
        _p(q), _tokens_ld(q, "q"), _p(k), _tokens_ld(k, "k"), _p(v), _tokens_ld(v, "v"),
        _p(o), _tokens_ld(o, "o"), _p(dout), _tokens_ld(dout, "dout"), _p(lse), _p(workspace),
        _p(dq), _tokens_ld(dq, "dq"), _p(dk), _tokens_ld(dk, "dk"), _p(dv), _tokens_ld(dv, "dv"),
        dtype_code(q.dtype), T, HQ, HK, D, _p(cu_seqlens), cu_seqlens.numel() - 1,
        int(max_seqlen), float(scale), _stream(dev))
    _check(rc, "esep_attn_bwd")
    _record(name)


def _flat(t, name):
    if not t.is_contiguous():
        raise EsepError(f"{name} must be contiguous")
    return t


def swiglu_fwd(gate, up, out, name="_swiglu_fwd"):
    """out = silu(gate) * up (esep_swiglu_fwd); contiguous tensors of one dtype and size; out
    may be gate itself."""
    dev = _dev(gate, up, out)
    if gate.numel() != up.numel() or gate.numel() != out.numel():
        raise EsepError("gate, up and out must have the same number of elements")
    if up.dtype != gate.dtype or out.dtype != gate.dtype:
        raise EsepError("gate, up and out must share one dtype")
    rc = lib().esep_swiglu_fwd(_p(_flat(gate, "gate")), _p(_flat(up, "up")), _p(_flat(out, "out")),
                               gate.numel(), dtype_code(gate.dtype), _stream(dev))
    _check(rc, "esep_swiglu_fwd")
    _record(name)


def swiglu_bwd(dout, gate, up, dgate, dup, name="_swiglu_bwd"):
    """(dgate, dup) of out = silu(gate) * up (esep_swiglu_bwd); dgate may be gate and dup may
    be up."""
    dev = _dev(dout, gate, up, dgate, dup)
    n = gate.numel()
    if any(t.numel() != n for t in (dout, up, dgate, dup)):
        raise EsepError("dout, gate, up, dgate and dup must have the same number of elements")
    if any(t.dtype != gate.dtype for t in (dout, up, dgate, dup)):
        raise EsepError("dout, gate, up, dgate and dup must share one dtype")
    rc = lib().esep_swiglu_bwd(_p(_flat(dout, "dout")), _p(_flat(gate, "gate")), _p(_flat(up, "up")),
                               _p(_flat(dgate, "dgate")), _p(_flat(dup, "dup")), n,
                               dtype_code(gate.dtype), _stream(dev))
    _check(rc, "esep_swiglu_bwd")
    _record(name)


def _key(key, dev):
    if key.dtype != torch.int64 or key.numel() < 1 or key.device != dev:
        raise EsepError("key must be an int64 tensor on the same device")
    return key


def lora_dropout_fwd(x, key, xd, p, name="_lora_dropout_fwd"):
    """xd = x * keep / (1 - p) with keep regenerated from the int64 device key
    (esep_lora_dropout_fwd)."""
    dev = _dev(x, key, xd)
    if x.dtype != xd.dtype or x.numel() != xd.numel():
        raise EsepError("x and xd must share dtype and size")
    rc = lib().esep_lora_dropout_fwd(_p(_flat(x, "x")), _p(_key(key, dev)), _p(_flat(xd, "xd")),
                                     x.numel(), float(p), dtype_code(x.dtype), _stream(dev))
    _check(rc, "esep_lora_dropout_fwd")
    _record(name)


def lora_dropout_bwd(x, g, key, xd, dx, p, accumulate=False, name="_lora_dropout_bwd"):
    """xd = x * keep / (1 - p) (regenerated) and dx = [dx +] g * keep / (1 - p)
    (esep_lora_dropout_bwd); dx may be g itself."""
    dev = _dev(x, g, key, xd, dx)
    n = x.numel()
    if any(t.numel() != n or t.dtype != x.dtype for t in (g, xd, dx)):
        raise EsepError("x, g, xd and dx must share dtype and size")
    rc = lib().esep_lora_dropout_bwd(_p(_flat(x, "x")), _p(_flat(g, "g")), _p(_key(key, dev)),
                                     _p(_flat(xd, "xd")), _p(_flat(dx, "dx")), n, float(p),
                                     int(bool(accumulate)), dtype_code(x.dtype), _stream(dev))
    _check(rc, "esep_lora_dropout_bwd")
    _record(name)


def nf4_dequant(packed, absmax, absmax2, code2, offset, nf4, out, name="_nf4_dequant"):
    """out = NF4 double-quant dequantization (esep_nf4_dequant). packed uint8 (n_blocks * 32
    bytes, any contiguous view), absmax uint8 [n_blocks], absmax2 / code2 / offset / nf4 fp32
    device tensors, out: n_blocks * 64 contiguous elements (fp16 / bf16 / fp32)."""
    dev = _dev(packed, absmax, absmax2, code2, offset, nf4, out)
    nb = absmax.numel()
    if packed.dtype != torch.uint8 or packed.numel() != nb * 32 or absmax.dtype != torch.uint8:
        raise EsepError("packed must hold n_blocks * 32 uint8 and absmax n_blocks uint8")
    for t, nm in ((absmax2, "absmax2"), (code2, "code2"), (offset, "offset"), (nf4, "nf4")):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise EsepError(f"{nm} must be a contiguous fp32 tensor")
    if absmax2.numel() < (nb + 255) // 256 or code2.numel() < 256 or nf4.numel() < 16 or offset.numel() < 1:
        raise EsepError("nf4 tables too small")
    if out.numel() != nb * 64 or not out.is_contiguous():
        raise EsepError("out must be n_blocks * 64 contiguous elements")
    rc = lib().esep_nf4_dequant(_p(packed), _p(absmax.contiguous()), _p(absmax2), _p(code2),
                                _p(offset), _p(nf4), _p(out), dtype_code(out.dtype), nb, _stream(dev))
    _check(rc, "esep_nf4_dequant")
    _record(name)


class Nf4Weight(ctypes.Structure):
    """esep_nf4_weight (include/esep_body.h)."""
    _fields_ = [("packed", _vp), ("absmax", _vp), ("absmax2", _vp), ("code2", _vp),
                ("offset", _vp), ("nf4", _vp), ("out", _vp), ("n_blocks", _i64)]


NF4_MULTI_MAX = 8


def nf4_dequant_multi(items, name="_nf4_dequant_multi"):
    """Several NF4 weights in one launch (esep_nf4_dequant_multi). items: sequence of
    (packed, absmax, absmax2, code2, offset, nf4, out) tuples, each as for nf4_dequant; every out
    shares one dtype."""
    if not 1 <= len(items) <= NF4_MULTI_MAX:
        raise EsepError(f"1..{NF4_MULTI_MAX} weights per launch")
    dev = _dev(*[t for it in items for t in it])
    arr = (Nf4Weight * len(items))()
    dts = set()
    for k, (packed, absmax, absmax2, code2, offset, nf4, out) in enumerate(items):
        nb = absmax.numel()
        if packed.dtype != torch.uint8 or packed.numel() != nb * 32 or absmax.dtype != torch.uint8:
            raise EsepError("packed must hold n_blocks * 32 uint8 and absmax n_blocks uint8")
        for t, nm in ((absmax2, "absmax2"), (code2, "code2"), (offset, "offset"), (nf4, "nf4")):
            if t.dtype != torch.float32 or not t.is_contiguous():
                raise EsepError(f"{nm} must be a contiguous fp32 tensor")
        if (absmax2.numel() < (nb + 255) // 256 or code2.numel() < 256 or nf4.numel() < 16
                or offset.numel() < 1):
            raise EsepError("nf4 tables too small")
        if out.numel() != nb * 64 or not out.is_contiguous():
            raise EsepError("out must be n_blocks * 64 contiguous elements")
        if not (packed.is_contiguous() and absmax.is_contiguous()):
            raise EsepError("packed and absmax must be contiguous")
        dts.add(out.dtype)
        arr[k] = Nf4Weight(_p(packed), _p(absmax), _p(absmax2), _p(code2), _p(offset), _p(nf4),
                           _p(out), nb)
    if len(dts) != 1:
        raise EsepError("every output must share one dtype")
    rc = lib().esep_nf4_dequant_multi(ctypes.cast(arr, _vp), len(items), dtype_code(dts.pop()),
                                      _stream(dev))
    _check(rc, "esep_nf4_dequant_multi")
    _record(name)


def head_row_softmax(z, target, cew, lse, tlogit, ent, amax, write_g, g_scale,
                     name="head_row_softmax_kernel"):
    """Softmax statistics of the logits chunk z [rows, V] (fp16 / bf16, unit column stride) and,
    with write_g, g = (softmax - onehot) * g_scale written over the rows whose cew is != 0
    (esep_head_row_softmax). target int64 [rows]; cew fp32 [rows]; lse / tlogit / ent fp32 and
    amax int32 outputs of [rows]."""
    dev = _dev(z, target, cew, lse, tlogit, ent, amax)
    rows, V = z.shape
    ld = _rows_ld(z, V)
    for t, dt, nm in ((target, torch.int64, "target"), (cew, torch.float32, "cew"),
                      (lse, torch.float32, "lse"), (tlogit, torch.float32, "tlogit"),
                      (ent, torch.float32, "ent"), (amax, torch.int32, "amax")):
        if t.dtype != dt or t.numel() != rows or (rows > 1 and t.stride(0) != 1):
            raise EsepError(f"{nm} must be a contiguous {dt} tensor of {rows} elements")
    rc = lib().esep_head_row_softmax(_p(z), ld, _p(target), _p(cew), _p(lse), _p(tlogit), _p(ent),
                                     _p(amax), rows, V, 1 if write_g else 0, float(g_scale),
                                     dtype_code(z.dtype), _stream(dev))
    _check(rc, "esep_head_row_softmax")
    _record(name)
