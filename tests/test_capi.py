"""The C ABI boundary without a GPU: libesep_body.so loads, exports every entry point that
include/esep_body.h declares with the binding's signature, reports its ABI version, and
rejects bad arguments before touching the device (negative status + message)."""

import ctypes
import re
from pathlib import Path

import pytest

from solution.body import _hip

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "esep_body.h"


def declared():
    text = HEADER.read_text()
    return re.findall(r"^(?:const char\*|int64_t|int)\s+(esep_\w+)\(", text, flags=re.M)


def test_header_declares_the_binding_surface():
    names = declared()
    assert sorted(names) == sorted(_hip.SIGNATURES), names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_hip.LIB_PATH))
    for name in declared():
        assert hasattr(lib, name), name


def test_abi_version():
    assert _hip.lib().esep_abi_version() == _hip.ABI_VERSION
    m = re.search(r"#define ESEP_ABI_VERSION (\d+)", HEADER.read_text())
    assert int(m.group(1)) == _hip.ABI_VERSION


def _fwd(lib, **kw):
    a = dict(x=1, x_dt=0, ld_x=8, delta=None, delta_dt=0, ld_d=0, w=1, r_out=None, ld_r=0,
             y=1, y_dt=0, ld_y=8, rstd=None, slot=None, xs=None, k=0, rows=4, n=8, eps=1e-6,
             stream=None)
    a.update(kw)
    return lib.esep_rmsnorm_fwd(*a.values())


def test_rmsnorm_fwd_validation():
    lib = _hip.lib()
    assert _fwd(lib, n=0) == -2 and b"n=0" in lib.esep_last_error()
    assert _fwd(lib, n=16385) == -2
    assert _fwd(lib, rows=-1) == -2
    assert _fwd(lib, x_dt=7) == -1
    assert _fwd(lib, x=None) == -1
    assert _fwd(lib, k=2) == -1 and b"n_special" in lib.esep_last_error()
    assert _fwd(lib, ld_x=4) == -2
    assert _fwd(lib, rows=0) == 0  # nothing to do, nothing launched
    assert _fwd(lib, x=None, rows=0) == -1  # arguments are checked even for empty inputs


def test_rmsnorm_bwd_validation():
    lib = _hip.lib()
    Arr = ctypes.c_void_p * 5

    def bwd(**kw):
        a = dict(dys=Arr(1), n_dy=1, dy_dt=2, ld_dy=8, dr_out=None, x=1, x_dt=2, ld_x=8, from_y=0,
                 rstd=None, w=1, slot=None, xs=None, k=0, dr=None, dx=1, dx_dt=2, ld_out=8,
                 part=None, n_part=0, dw=None, dw_dt=0, rows=4, n=8, eps=1e-6, stream=None)
        a.update(kw)
        return lib.esep_rmsnorm_bwd(*a.values())

    assert bwd(n_dy=6) == -1
    assert bwd(dys=Arr(None)) == -1
    assert bwd(from_y=1) == -1 and b"rstd" in lib.esep_last_error()
    assert bwd(dw=1) == -1  # no partials workspace
    assert bwd(dw=1, part=64, n_part=3) == -2 and b"needs 1" in lib.esep_last_error()
    assert bwd(part=64, n_part=3) == -2  # partials only: the count is checked too
    assert bwd(dw=1, dw_dt=3, part=64, n_part=1) == -1  # int32 dw
    # the partials are read and written as 16-byte vectors: a misaligned buffer is refused
    assert bwd(dw=1, part=8, n_part=1) == -3 and b"aligned" in lib.esep_last_error()
    assert bwd(part=4, n_part=1) == -3
    assert bwd(rows=0) == 0


def test_dgamma_reduce_validation():
    lib = _hip.lib()
    assert lib.esep_dgamma_reduce(1, 4, 0, 1, 0, None) == -2
    assert lib.esep_dgamma_reduce(1, 4, 16385, 1, 0, None) == -2
    assert lib.esep_dgamma_reduce(1, -1, 8, 1, 0, None) == -2
    assert lib.esep_dgamma_reduce(1, 4, 8, None, 0, None) == -1
    assert lib.esep_dgamma_reduce(None, 4, 8, 1, 0, None) == -1
    assert lib.esep_dgamma_reduce(1, 4, 8, 1, 3, None) == -1 and b"dgamma" in lib.esep_last_error()
    assert lib.esep_dgamma_reduce(8, 4, 8, 1, 0, None) == -3 and b"aligned" in lib.esep_last_error()


def test_dgamma_reduce_batch_validation():
    """esep_dgamma_reduce_batch checks the item count, n, the dtype and every item's pointers and
    partial count before launching anything."""
    lib = _hip.lib()

    def call(n_items=2, n=8, dt=0, **kw):
        arr = (_hip.DgammaItem * 65)()
        for i in range(65):
            f = dict(partials=64, n_partials=4, dw=64)
            if i == 1:
                f.update(kw)
            arr[i] = _hip.DgammaItem(*f.values())
        return lib.esep_dgamma_reduce_batch(ctypes.cast(arr, ctypes.c_void_p), n_items, n, dt, None)

    assert call(n_items=0) == -1 and call(n_items=65) == -1
    assert lib.esep_dgamma_reduce_batch(None, 1, 8, 0, None) == -1
    assert call(n=0) == -2 and call(n=16385) == -2
    assert call(dt=3) == -1
    assert call(dw=None) == -1 and b"item 1" in lib.esep_last_error()
    assert call(partials=None) == -1
    assert call(n_partials=-1) == -2
    assert call(partials=72) == -3 and b"item 1" in lib.esep_last_error()
    assert _hip.DGAMMA_BATCH_MAX == int(re.search(r"#define ESEP_DGAMMA_BATCH_MAX (\d+)",
                                                  HEADER.read_text()).group(1))


def test_rope_validation():
    lib = _hip.lib()
    S3 = ctypes.c_int64 * 3
    st = S3(0, 128, 128)

    def rope(**kw):
        a = dict(q=1, qs=st, qd=None, qds=None, k=1, ks=st, qo=1, qos=st, ko=1, kos=st, dt=1,
                 B=1, S=4, HQ=1, HK=1, D=128, pos=None, pos_dt=0, pos_s=None, cu=None, n_seq=0,
                 inv=1, sign=1.0, stream=None)
        a.update(kw)
        return lib.esep_rope(*a.values())

    assert rope(D=96) == -2
    assert rope(dt=5) == -1
    assert rope(inv=None) == -1
    assert rope(pos=1, pos_dt=3, pos_s=(ctypes.c_int64 * 2)(0, 1), cu=1, n_seq=1) == -1
    assert rope(cu=1, n_seq=1, B=2) == -1
    assert rope(HQ=0, HK=0) == -2
    assert rope(S=0) == 0


@pytest.mark.parametrize("rows,n", [(1, 1536), (37, 1536), (8192, 1536), (65536, 3584),
                                    (4557, 1536), (100000, 24), (8192, 16384)])
def test_partition_depends_on_shape_only(rows, n):
    """The weight-gradient partition: at most 256 partial rows (512 from 2^26 elements on),
    every row covered, and a pure function of (rows, n) (the C ABI takes no device argument)."""
    p = _hip.rmsnorm_partials(rows, n)
    assert 1 <= p <= (512 if rows * n >= 1 << 26 else 256) and p == _hip.rmsnorm_partials(rows, n)
    assert _hip.rmsnorm_partials(0, n) == 0


def test_attention_validation():
    """esep_attn_fwd / esep_attn_bwd reject bad arguments before launching anything."""
    lib = _hip.lib()

    def fwd(**kw):
        a = dict(q=16, q_rs=256, k=16, k_rs=256, v=16, v_rs=256, o=16, o_rs=256, lse=None, dt=2,
                 T=4, HQ=2, HK=2, D=128, cu=16, n_seq=1, max_seqlen=4, scale=0.1, stream=None)
        a.update(kw)
        return lib.esep_attn_fwd(*a.values())

    assert fwd(dt=0) == -1 and b"dtype" in lib.esep_last_error()  # fp32 not taken
    assert fwd(D=96) == -2
    assert fwd(HQ=3, HK=2) == -2  # query heads must be a multiple of kv heads
    assert fwd(q_rs=128) == -2  # token stride below HQ * D
    assert fwd(k_rs=(1 << 22) + 8) == -2 and b"above" in lib.esep_last_error()
    assert fwd(k_rs=1 << 22, v_rs=1 << 22, T=0) == 0  # the cap itself is accepted
    assert fwd(q=None) == -1
    assert fwd(cu=None) == -1
    assert fwd(q=8) == -3 and b"alignment" in lib.esep_last_error()
    assert fwd(q_rs=260) == -3
    assert fwd(scale=0.0) == -1
    assert fwd(T=0) == 0 and fwd(n_seq=0) == 0  # nothing to do, nothing launched

    def bwd(**kw):
        a = dict(q=16, q_rs=256, k=16, k_rs=256, v=16, v_rs=256, o=16, o_rs=256, do=16,
                 do_rs=256, lse=16, ws=16, dq=16, dq_rs=256, dk=16, dk_rs=256, dv=16, dv_rs=256,
                 dt=1, T=4, HQ=2, HK=2, D=128, cu=16, n_seq=1, max_seqlen=4, scale=0.1,
                 stream=None)
        a.update(kw)
        return lib.esep_attn_bwd(*a.values())

    assert bwd(dt=4) == -1
    assert bwd(lse=None) == -1 and bwd(ws=None) == -1
    assert bwd(dk=None) == -1
    assert bwd(ws=8) == -3
    assert bwd(dv_rs=100) == -2
    assert bwd(do_rs=(1 << 22) + 8) == -2
    assert bwd(T=0) == 0


def test_attention_workspace_size():
    """Per-query delta (rounded up to 4 floats) plus the dK/dV partials when the query heads of a
    kv head are split over blocks: a pure function of the shape."""
    ws = _hip.attn_bwd_workspace
    assert ws(0, 12, 2, 128) == 0 and ws(8, 3, 2, 128) == 0
    # 1 sequence of 65536 tokens, 28/4 heads: 256-key blocks already fill the GPU, no split
    assert ws(65536, 28, 4, 128) == 28 * 65536
    # 8192 tokens, 12/2 heads: 32 x 2 blocks; the smallest divisor s of the 6 query heads of a
    # kv head with 64 s >= 384 blocks is 6
    assert ws(8192, 12, 2, 128) == 12 * 8192 + 2 * 6 * 8192 * 2 * 128
    # 4096 tokens: 16 x 2 blocks, s = 6 (all 6 query heads apart: 32 x 6 = 192 blocks)
    assert ws(4096, 12, 2, 128) == 12 * 4096 + 2 * 6 * 4096 * 2 * 128
    # 32768 tokens, 28/4 heads: 128 x 4 = 512 blocks already, no split
    assert ws(32768, 28, 4, 128) == 28 * 32768
    # 16384 tokens, 28/4 heads: 64 x 4 = 256 blocks; s = 7 (the only divisor of 7 above 1)
    assert ws(16384, 28, 4, 128) == 28 * 16384 + 2 * 7 * 16384 * 4 * 128
    assert ws(3, 1, 1, 64) == 4  # delta rounded up to a multiple of 4 floats


def test_head_row_softmax_validation():
    """esep_head_row_softmax rejects bad arguments before launching anything."""
    lib = _hip.lib()

    def call(**kw):
        a = dict(z=16, ld=1024, target=16, cew=16, lse=16, tlogit=16, ent=16, amax=16, rows=4,
                 V=1000, write_g=1, g_scale=1024.0, dt=1, stream=None)
        a.update(kw)
        return lib.esep_head_row_softmax(*a.values())

    assert call(dt=0) == -1 and b"fp16 or bf16" in lib.esep_last_error()
    assert call(dt=4) == -1
    assert call(V=0) == -2 and call(V=(1 << 30) + 1) == -2
    assert call(ld=999) == -2 and b"ld" in lib.esep_last_error()
    assert call(rows=-1) == -2
    assert call(z=None) == -1 and call(amax=None) == -1
    assert call(cew=None) == -1  # the CE weights decide which rows get g
    assert call(z=17) == -3
    assert call(rows=0) == 0  # nothing to do, nothing launched


def test_nf4_dequant_multi_validation():
    """esep_nf4_dequant_multi checks the weight count, every weight's pointers, sizes and
    alignment, and the output dtype before launching anything."""
    lib = _hip.lib()

    def call(n=2, dt=1, **kw):
        arr = (_hip.Nf4Weight * 9)()
        for i in range(9):
            f = dict(packed=64, absmax=64, absmax2=64, code2=64, offset=64, nf4=64, out=64, n_blocks=4)
            if i == 1:
                f.update(kw)
            arr[i] = _hip.Nf4Weight(*f.values())
        return lib.esep_nf4_dequant_multi(ctypes.cast(arr, ctypes.c_void_p), n, dt, None)

    assert call(n=0) == -1 and call(n=9) == -1
    assert lib.esep_nf4_dequant_multi(None, 1, 1, None) == -1
    assert call(dt=3) == -1
    assert call(out=None) == -1 and b"weight 1" in lib.esep_last_error()
    assert call(n_blocks=-1) == -2
    assert call(packed=68) == -3 and call(out=72) == -3


def test_apply_installs_the_patches_idempotently():
    """solution.apply() (the reference's entry, solution/__init__.py:19-25) patches Qwen2MLP and
    Qwen2Model once; a second call changes nothing. CPU only: no kernel runs."""
    import solution
    from transformers.models.qwen2 import modeling_qwen2 as mq

    mlp0, model0 = mq.Qwen2MLP.forward, mq.Qwen2Model.forward
    try:
        solution.apply()
        mlp1, model1 = mq.Qwen2MLP.forward, mq.Qwen2Model.forward
        assert getattr(mlp1, "_esep_swiglu", False) and mlp1.__wrapped__ is mlp0
        assert model1 is not model0
        solution.apply()
        assert mq.Qwen2MLP.forward is mlp1 and mq.Qwen2Model.forward is model1
    finally:
        mq.Qwen2MLP.forward, mq.Qwen2Model.forward = mlp0, model0

