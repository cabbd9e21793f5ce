"""CPU oracle for the LoRA dropout path (test infrastructure only: imported by tests/, never by
the product path).

* philox4x32_10: the counter-based generator of Salmon, Moraes, Dror and Shaw, "Parallel Random
  Numbers: As Easy as 1, 2, 3" (SC 2011), 10 rounds, restated from the paper in numpy uint32 /
  uint64 arithmetic. Pinned to the paper's published known-answer vectors in
  tests/test_oracle_lora.py.
* dropout_mask: this build's mask layout (the reference's layout, solution/body/lora.py:61-65, is
  tied to its Triton block size and its bits are not part of the contract; what is kept is the
  law and the regeneration): element e is kept iff uniform(e) >= p, with
  uniform(e) = (word e % 4 of philox(counter = e // 4, key)) >> 8, times 2^-24 (24-bit uniforms
  on [0, 1)).
* The LoRA math of solution/body/lora.py:2-52 in float64: out = base + scaling * (x_d A^T) B^T
  with x_d = x * keep / (1 - p), and its gradients.
"""

import numpy as np

M0, M1 = 0xD2511F53, 0xCD9E8D57  # round multipliers
W0, W1 = 0x9E3779B9, 0xBB67AE85  # key schedule (Weyl) increments
MASK32 = 0xFFFFFFFF


def philox4x32_10(ctr, key):
    """ctr: uint32 array [..., 4]; key: uint32 array [..., 2] (broadcast). Returns uint32 [..., 4]."""
    c = np.asarray(ctr, dtype=np.uint64) & MASK32
    k = np.asarray(key, dtype=np.uint64) & MASK32
    c0, c1, c2, c3 = (c[..., i].copy() for i in range(4))
    k0 = np.broadcast_to(k[..., 0], c0.shape).copy()
    k1 = np.broadcast_to(k[..., 1], c0.shape).copy()
    for r in range(10):
        if r:
            k0 = (k0 + W0) & MASK32
            k1 = (k1 + W1) & MASK32
        p0 = c0 * np.uint64(M0)
        p1 = c2 * np.uint64(M1)
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK32
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK32
        c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
    return np.stack([c0, c1, c2, c3], axis=-1).astype(np.uint32)


def key_words(key):
    """The 63-bit key (int64) as the generator's two 32-bit key words (low, high)."""
    key = int(key)
    return np.array([key & MASK32, (key >> 32) & MASK32], dtype=np.uint32)


def uniforms(key, n):
    """24-bit uniforms on [0, 1) of elements 0 .. n - 1."""
    nc = (n + 3) // 4
    cnt = np.arange(nc, dtype=np.uint64)
    ctr = np.zeros((nc, 4), dtype=np.uint64)
    ctr[:, 0] = cnt & MASK32
    ctr[:, 1] = cnt >> np.uint64(32)
    words = philox4x32_10(ctr, key_words(key)).reshape(-1)[:n]
    return (words >> np.uint32(8)).astype(np.float64) * 2.0 ** -24


def dropout_mask(key, n, p):
    """Keep mask (bool [n]) of elements 0 .. n - 1 for dropout probability p."""
    return uniforms(key, n) >= p


def lora_fwd(x, base, a, b, keep, p, scaling):
    """base + scaling * (x_d A^T) B^T, x_d = x * keep / (1 - p) (keep None: no dropout)."""
    x, base, a, b = (np.asarray(t, dtype=np.float64) for t in (x, base, a, b))
    xd = x if keep is None else x * keep.reshape(x.shape) / (1.0 - p)
    return base + scaling * (xd @ a.T) @ b.T


def lora_bwd(x, a, b, dout, keep, p, scaling):
    """(dx, dbase, dA, dB) of lora_fwd for upstream dout."""
    x, a, b, dout = (np.asarray(t, dtype=np.float64) for t in (x, a, b, dout))
    k = np.ones_like(x) if keep is None else keep.reshape(x.shape).astype(np.float64)
    inv = 1.0 if keep is None else 1.0 / (1.0 - p)
    xd = x * k * inv
    xa = xd @ a.T
    dxa = scaling * dout @ b
    db = scaling * dout.T @ xa
    da = dxa.T @ xd
    dx = (dxa @ a) * k * inv
    return dx, dout, da, db
