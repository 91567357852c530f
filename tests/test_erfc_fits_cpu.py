"""The erfc forms behind GELU-erf (candle-3d_amd/csrc/pointwise.hip,
erfc_nonneg<DEG>): t * exp(-z^2 + P(t)), t = 1 / (1 + z/2). Each degree's
coefficients are read from the kernel source and evaluated with the kernel's
f32 steps emulated: t from the rounded 1 + z/2, FMA Horner steps rounded to
f32, and the exponent argument as the kernel forms it -- rounded to f32 twice
(fma(-z, z, P), then times log2(e)) for degrees 7 / 5, carried in two parts
for degree 9 (z^2 = hi + lo, TwoSum, n = rint(a log2 e) split off, FMA
remainder). The relative error of erfc against scipy's is held to the bound
the source states for that degree over z in [0, 9]. v_exp_f32 and v_rcp_f32
add at most about one f32 ulp each on top (not emulated)."""
import os
import re

import numpy as np
import pytest

scipy_special = pytest.importorskip("scipy.special")

SRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "candle-3d_amd", "csrc",
                   "pointwise.hip")
BOUND = {9: 3.6e-7, 7: 8.2e-6, 5: 5.5e-5}
L2E = float(np.float32(1.4426950408889634))
L2E_LO = float(np.float32(1.925963033500011e-8))


def coefficients():
    text = open(SRC).read()
    body = text[text.index("__device__ __forceinline__ float erfc_nonneg(float z) {"):]
    body = body[:body.index("constexpr float log2e")]
    out = {}
    for deg, block in ((9, r"DEG == 9\) \{(.*?)\}"), (7, r"DEG == 7\) \{(.*?)\}"), (5, r"DEG == 5, [^;]*;(.*)")):
        m = re.search(block, body, flags=re.S)
        nums = re.findall(r"(-?\d+\.\d+(?:e-?\d+)?)f", m.group(1))
        out[deg] = [np.float32(float(v)) for v in nums]
        assert len(out[deg]) == deg + 1, (deg, nums)
    return out


def _f32(x):
    """Round to f32 (the result of one f32 operation computed exactly in f64)."""
    return np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float64)


def kernel_erfc(deg, z):
    c = [float(v) for v in coefficients()[deg]]  # highest degree first, as in the Horner steps
    t = _f32(1.0 / _f32(0.5 * z + 1.0))
    p = np.full_like(t, c[0])
    for k in c[1:]:
        p = _f32(p * t + k)                       # fmaf: one rounding
    if deg == 9:
        hi = _f32(z * z)
        lo = z * z - hi                           # exact remainder of the f32 square
        a = _f32(p - hi)
        ae = (p - hi) - a                         # TwoSum error, exact
        a_lo = _f32(ae - lo)
        n = np.rint(_f32(a * L2E))
        r = _f32(a * L2E - n)
        r = _f32(a * L2E_LO + r)
        r = _f32(a_lo * L2E + r)
        return t * np.exp2(r) * np.exp2(n)
    return t * np.exp2(_f32(_f32(-z * z + p) * L2E))


@pytest.mark.parametrize("deg", [9, 7, 5])
def test_erfc_fit_relative_error(deg):
    z = np.linspace(0.0, 9.0, 200001).astype(np.float32).astype(np.float64)
    exact = scipy_special.erfc(z)
    rel = np.abs(kernel_erfc(deg, z) - exact) / exact
    assert rel.max() <= BOUND[deg], f"degree {deg}: max relative error {rel.max():.3g}"


def test_one_rounding_of_the_argument_would_exceed_the_f32_bound():
    """Rounding the degree-9 argument to f32 before the exp2 (the simple
    form degrees 7 / 5 use) exceeds the 3.6e-7 bound by an order of
    magnitude near z = 8.4: the two-part argument is what keeps it."""
    c = [float(v) for v in coefficients()[9]]
    z = np.linspace(8.0, 9.0, 20001).astype(np.float32).astype(np.float64)
    t = _f32(1.0 / _f32(0.5 * z + 1.0))
    p = np.full_like(t, c[0])
    for k in c[1:]:
        p = _f32(p * t + k)
    simple = t * np.exp2(_f32(_f32(-z * z + p) * L2E))
    rel = np.abs(simple - scipy_special.erfc(z)) / scipy_special.erfc(z)
    assert rel.max() > 10 * BOUND[9]
