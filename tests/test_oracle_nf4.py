"""Pins of the NF4 dequantization oracle (oracle/nf4_ref.py) on the CPU.

* Known answers built by hand: a byte 0x7F (high nibble 7 -> NF4 0.0, low nibble 15 -> 1.0) with
  scale 2 gives (0, 2); nibble order (element 2i in the high nibble) and the per-64 / per-256
  scale indexing checked on a hand-made state.
* The nested scale is rounded twice in float32 (multiply, then add): a case where a fused
  multiply-add gives a different float32 must follow the two-rounding result.
* Round trip: quantize_nf4 then dequantize_nf4 reconstructs a weight within the NF4 step of each
  block's scale, and every NF4 code value times its block scale is reproduced exactly.
* A planted mistake (nibbles swapped) fails the known answers.
"""

import numpy as np
import pytest

from oracle import nf4_ref as ref


def _state(nb, scale=2.0):
    code2 = np.zeros(256, dtype=np.float32)
    code2[1] = 1.0
    return np.ones(nb, dtype=np.uint8), np.full((nb + 255) // 256, scale, dtype=np.float32), code2


def test_known_answers():
    absmax, absmax2, code2 = _state(1)
    packed = np.full(32, 0x7F, dtype=np.uint8)
    w = ref.dequantize_nf4(packed, absmax, absmax2, code2, 0.0, out_dtype=np.float32)
    assert w.size == 64 and np.all(w[0::2] == 0.0) and np.all(w[1::2] == 2.0)
    packed[0] = 0x0F  # element 0 -> code 0 (-1), element 1 -> code 15 (+1)
    w = ref.dequantize_nf4(packed, absmax, absmax2, code2, 0.5, out_dtype=np.float32)
    assert w[0] == -2.5 and w[1] == 2.5  # scale = 1 * 2 + 0.5


def test_block_and_second_level_indexing():
    nb = 600  # 3 second-level groups
    absmax = np.ones(nb, dtype=np.uint8)
    absmax2 = np.array([1.0, 2.0, 4.0], dtype=np.float32)
    code2 = np.zeros(256, dtype=np.float32)
    code2[1] = 1.0
    packed = np.full(nb * 32, 0xFF, dtype=np.uint8)  # every element NF4 +1 -> W = scale
    w = ref.dequantize_nf4(packed, absmax, absmax2, code2, 0.0, out_dtype=np.float32)
    blocks = w.reshape(nb, 64)
    assert np.all(blocks[:256] == 1.0) and np.all(blocks[256:512] == 2.0) and np.all(blocks[512:] == 4.0)


def test_two_roundings_not_fused():
    a, b, c = np.float32(1.0000001), np.float32(3.0000002), np.float32(-3.0000005)
    two = np.float32(np.float32(a * b) + c)
    fused = np.float32(np.float64(a) * np.float64(b) + np.float64(c))
    assert two != fused  # the case distinguishes the two
    code2 = np.zeros(256, dtype=np.float32)
    code2[1] = a
    w = ref.dequantize_nf4(np.full(32, 0xFF, dtype=np.uint8), np.ones(1, dtype=np.uint8),
                           np.array([b], dtype=np.float32), code2, c, out_dtype=np.float32)
    assert np.all(w == two)


def test_quantize_round_trip():
    rng = np.random.default_rng(0)
    w = (rng.standard_normal(64 * 1000) * 0.02).astype(np.float32)
    w[:64] *= 50
    packed, absmax, absmax2, code2, offset = ref.quantize_nf4(w)
    got = ref.dequantize_nf4(packed, absmax, absmax2, code2, offset, out_dtype=np.float32)
    scale = np.abs(w.reshape(-1, 64)).max(axis=1)
    err = np.abs(got - w).reshape(-1, 64).max(axis=1)
    # half the widest NF4 gap of the block's scale, plus the nested-scale error
    assert np.all(err <= 0.17 * scale + 0.05 * scale.max()), (err / scale).max()


def test_planted_nibble_swap_is_caught():
    def bad(packed, *args, **kw):
        p = np.asarray(packed, dtype=np.uint8)
        return ref.dequantize_nf4(((p & 15) << 4) | (p >> 4), *args, **kw)

    absmax, absmax2, code2 = _state(1)
    w = bad(np.full(32, 0x7F, dtype=np.uint8), absmax, absmax2, code2, 0.0, out_dtype=np.float32)
    with pytest.raises(AssertionError):
        assert np.all(w[0::2] == 0.0) and np.all(w[1::2] == 2.0)
