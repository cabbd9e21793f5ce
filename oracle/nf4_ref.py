"""CPU oracle for the NF4 (double-quant) dequantization (test infrastructure only: imported by
tests/, never by the product path).

Restates the storage format the reference's kernel decodes (solution/nf4/dequant.py:1-22; the
format of QLoRA, Dettmers et al. 2023, as bitsandbytes stores a Linear4bit weight W[N, K]):
  * packed: uint8, N*K/2 bytes over the row-major flattened weight; byte i holds element 2i in
    its high nibble and element 2i + 1 in its low nibble; a nibble indexes the 16-entry NF4 table.
  * one scale per 64 consecutive elements, stored double-quantized: absmax[b] (uint8) indexes a
    256-entry table code2, times one fp32 absmax2[b // 256], plus a scalar fp32 offset:
        scale[b] = fp32(fp32(code2[absmax[b]] * absmax2[b // 256]) + offset)
        W[e]     = fp16(fp32(nf4[nibble(e)] * scale[e // 64]))
    every step rounded separately (no fused multiply-add), in float32 numpy arithmetic.

quantize_nf4 builds such a state from a float weight (block absmax, nearest NF4 code, the
scales' mean as offset, nested 8-bit quantization of (scale - offset) per 256 with a symmetric
256-entry table): enough to generate realistic test inputs; the dequantization above is what is
pinned (tests/test_oracle_nf4.py).
"""

import numpy as np

# The NF4 data type of the QLoRA paper (normal-float 4-bit quantiles, exact 0, endpoints +-1).
NF4 = np.array([-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
                -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
                0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
                0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
                0.7229568362236023, 1.0], dtype=np.float32)

BLOCK, BLOCK2 = 64, 256


def code2_table():
    """A symmetric 256-entry map on [-1, 1] for the nested scale quantization (signed, finer near
    0, monotone): sign * (i / 127)^2 for i = 0..127 on both sides, padded to 256."""
    pos = (np.arange(128, dtype=np.float64) / 127.0) ** 2
    table = np.concatenate([-pos[::-1], pos])
    return table.astype(np.float32)


def dequantize_nf4(packed, absmax, absmax2, code2, offset, nf4=NF4, out_dtype=np.float16):
    """W (flattened, N*K elements) from the packed bytes and the nested scale state."""
    packed = np.asarray(packed, dtype=np.uint8).reshape(-1)
    absmax = np.asarray(absmax, dtype=np.uint8).reshape(-1)
    nb = absmax.size
    b = np.arange(nb)
    scale = (np.asarray(code2, dtype=np.float32)[absmax] *
             np.asarray(absmax2, dtype=np.float32)[b // BLOCK2]).astype(np.float32)
    scale = (scale + np.float32(offset)).astype(np.float32)
    hi = (packed >> 4).astype(np.int64)
    lo = (packed & 15).astype(np.int64)
    nib = np.stack([hi, lo], axis=1).reshape(-1)            # element 2i, 2i + 1
    vals = (np.asarray(nf4, dtype=np.float32)[nib] *
            np.repeat(scale, BLOCK)[: nib.size]).astype(np.float32)
    return vals.astype(out_dtype)


def quantize_nf4(w, nf4=NF4):
    """(packed uint8 [N*K/2], absmax uint8 [N*K/64], absmax2 fp32 [ceil(nb/256)], code2 fp32
    [256], offset fp32) for a float weight with N*K a multiple of 64."""
    w = np.asarray(w, dtype=np.float32).reshape(-1)
    blocks = w.reshape(-1, BLOCK)
    scale = np.abs(blocks).max(axis=1).astype(np.float32)
    scale[scale == 0] = 1.0
    normed = blocks / scale[:, None]
    nib = np.abs(normed[..., None] - nf4[None, None, :]).argmin(axis=-1).reshape(-1).astype(np.uint8)
    packed = ((nib[0::2] << 4) | nib[1::2]).astype(np.uint8)
    offset = np.float32(scale.mean())
    c = scale - offset
    nb = c.size
    n2 = (nb + BLOCK2 - 1) // BLOCK2
    cpad = np.zeros(n2 * BLOCK2, dtype=np.float32)
    cpad[:nb] = c
    absmax2 = np.abs(cpad.reshape(n2, BLOCK2)).max(axis=1).astype(np.float32)
    absmax2[absmax2 == 0] = 1.0
    code2 = code2_table()
    normed2 = cpad.reshape(n2, BLOCK2) / absmax2[:, None]
    q = np.abs(normed2.reshape(-1)[:nb, None] - code2[None, :]).argmin(axis=1).astype(np.uint8)
    return packed, q, absmax2, code2, offset
