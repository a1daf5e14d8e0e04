"""The division step of the KIVI quantisation ladder (csrc/zkv_common.hpp,
div_recip): q = x * r, r = 1 / b, then q + (x - q b) r with two fused
multiply-adds.  For bf16 operands with normal quotients it must equal the
IEEE fp32 division bit for bit, which the bit-exact pack and stage-2 kernels
rely on (quant_pack.py's bf16 ladder, S:2003-2009).

In the normal range the rounding of every step depends only on the operands'
significands (scaling x or b by a power of two scales every intermediate by
the same power), so every pair of bf16 significands covers every pair of
normal bf16 operands; x / 15 is checked for every bf16 x.  The fused
multiply-adds are modelled exactly: x - q b is exact in float64 (8 + 24 + 8
significant bits), e * r too (24 + 24 bits), and q + e r is rounded once to
float32 through an exact two-sum.
"""
import numpy as np


def _fma_step(q0: np.ndarray, e: np.ndarray, r: np.ndarray) -> np.ndarray:
    """float32 round-to-nearest-even of q0 + e * r computed exactly."""
    a = q0.astype(np.float64)
    p = e.astype(np.float64) * r.astype(np.float64)        # exact: 48 significant bits
    s = a + p
    bb = s - a                                               # two-sum: s + err == a + p exactly
    err = (a - (s - bb)) + (p - bb)
    c = s.astype(np.float32)
    c64 = c.astype(np.float64)
    toward = np.where(s > c64, np.float32(np.inf), np.float32(-np.inf)).astype(np.float32)
    other = np.nextafter(c, toward)
    mid = (c64 + other.astype(np.float64)) / 2.0            # exact in float64
    at_mid = (c64 != s) & (s == mid)
    up = np.maximum(c, other)
    down = np.minimum(c, other)
    out = c.copy()
    out = np.where(at_mid & (err > 0), up, out)
    out = np.where(at_mid & (err < 0), down, out)
    return out.astype(np.float32)


def div_recip(x: np.ndarray, b: np.ndarray) -> np.ndarray:
    x = x.astype(np.float32)
    b = b.astype(np.float32)
    r = (np.float32(1.0) / b).astype(np.float32)             # IEEE, correctly rounded
    q0 = (x * r).astype(np.float32)
    # x - q0 b: exact in float64, then one rounding (the first multiply-add)
    e = (x.astype(np.float64) - q0.astype(np.float64) * b.astype(np.float64)).astype(np.float32)
    return _fma_step(q0, e, r)


def _bf16_from_bits(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def test_every_bf16_significand_pair():
    sig = 1.0 + np.arange(128, dtype=np.float64) / 128.0
    xs, bs = np.meshgrid(sig, sig, indexing="ij")
    for shift in (-3, -1, 0, 1, 3):
        x = (xs * 2.0 ** shift).astype(np.float32).ravel()
        b = bs.astype(np.float32).ravel()
        ref = x / b
        got = div_recip(x, b)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
            f"{int((got != ref).sum())} mismatches at shift {shift}"


def test_every_bf16_over_15():
    bits = np.arange(0x0080, 0x7F80, dtype=np.uint32)       # positive normal bf16
    x = _bf16_from_bits(bits)
    keep = (x >= np.float32(2.0 ** -120)) & (x <= np.float32(2.0 ** 127))   # the fast range
    x = x[keep]
    b = np.full_like(x, 15.0)
    assert np.array_equal(div_recip(x, b).view(np.uint32), (x / b).view(np.uint32))
    assert np.array_equal(div_recip(-x, b).view(np.uint32), (-x / b).view(np.uint32))


def test_step_catches_a_dropped_correction():
    """Without the correction (q0 alone) the quotient is wrong on some pairs,
    so the exhaustive tests above can tell the two apart."""
    sig = 1.0 + np.arange(128, dtype=np.float64) / 128.0
    xs, bs = np.meshgrid(sig, sig, indexing="ij")
    x, b = xs.astype(np.float32).ravel(), bs.astype(np.float32).ravel()
    q0 = (x * (np.float32(1.0) / b).astype(np.float32)).astype(np.float32)
    assert (q0 != x / b).any()


def test_zeros_keep_their_sign_only_with_the_select():
    """The step maps -0 to +0 (the kernel's div15_bf16 returns x for zeros)."""
    z = np.array([0.0, -0.0], dtype=np.float32)
    got = div_recip(z, np.full(2, 15.0, dtype=np.float32))
    assert np.array_equal(got.view(np.uint32), np.zeros(2, dtype=np.uint32))
