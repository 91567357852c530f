"""The exact three-term bf16 split behind the f32 attention kernels
(candle-3d_amd/csrc/common.hpp, split3_bf16; used by attn_f32x3_kernel and
the exact-probability P v of attn_mfma_kernel): x = x1 + x2 + x3 with each
term a bf16 value, x1 = RNE_bf16(x), x2 = RNE_bf16(x - x1), x3 = x - x1 - x2.

Checked over every f32 significand of one binade (the split scales with the
exponent while x3 stays normal):
- the three terms sum to x exactly and x3 is exactly representable in bf16;
- |x2| <= 2^-8 |x| and |x3| <= 2^-17 |x|, so the products the kernels drop,
  x2 y3 + x3 y2 + x3 y3, stay below 2^-24 |x y| for every pair of operands.
A split with truncation instead of RNE (a plausible slip) leaves
|x2| up to 2^-7 |x| and fails the bound."""
import numpy as np


def bf16_rne(a):
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


def bf16_trunc(a):
    return (np.asarray(a, np.float32).view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


def split3(x, rnd=bf16_rne):
    x1 = rnd(x)
    r1 = (x - x1).astype(np.float32)
    x2 = rnd(r1)
    x3 = (r1 - x2).astype(np.float32)
    return x1, x2, x3


def binade():
    m = np.arange(1 << 23, dtype=np.uint32)
    return ((np.uint32(127) << 23) | m).view(np.float32)


def test_split_is_exact_and_terms_are_bf16():
    x = binade()
    x1, x2, x3 = split3(x)
    for t in (x1, x2, x3):
        assert np.array_equal(bf16_rne(t), t)
    s = x1.astype(np.float64) + x2.astype(np.float64) + x3.astype(np.float64)
    assert np.array_equal(s, x.astype(np.float64))


def test_dropped_products_stay_below_2_pow_minus_24():
    x = binade()
    _, x2, x3 = split3(x)
    r2 = float(np.max(np.abs(x2) / x))
    r3 = float(np.max(np.abs(x3) / x))
    assert r2 <= 2.0 ** -8 and r3 <= 2.0 ** -17, (np.log2(r2), np.log2(r3))
    # worst case over independent operands: x2 y3 + x3 y2 + x3 y3
    assert 2 * r2 * r3 + r3 * r3 < 2.0 ** -24


def test_truncating_split_would_break_the_bound():
    x = binade()
    _, x2, x3 = split3(x, bf16_trunc)
    r2 = float(np.max(np.abs(x2) / x))
    r3 = float(np.max(np.abs(x3) / x))
    assert 2 * r2 * r3 >= 2.0 ** -24
