"""The erfc forms behind GELU-erf (candle-3d_amd/csrc/pointwise.hip,
erfc_nonneg<DEG>): t * exp(-z^2 + P(t)), t = 1 / (1 + z/2). Each degree's
coefficients are read from the kernel source and evaluated with f32 Horner
steps, as the kernel does, and the relative error of erfc against scipy's is
held to the bound the source states for that degree over z in [0, 9]."""
import os
import re

import numpy as np
import pytest

scipy_special = pytest.importorskip("scipy.special")

SRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "candle-3d_amd", "csrc",
                   "pointwise.hip")
BOUND = {9: 3.6e-7, 7: 2.7e-6, 5: 5.1e-5}


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


@pytest.mark.parametrize("deg", [9, 7, 5])
def test_erfc_fit_relative_error(deg):
    c = coefficients()[deg]  # highest degree first, as in the Horner steps
    z = np.linspace(0.0, 9.0, 200001).astype(np.float32)
    t = (np.float32(1.0) / (np.float32(0.5) * z + np.float32(1.0))).astype(np.float32)
    p = np.full_like(t, c[0])
    for k in c[1:]:
        p = (p * t + k).astype(np.float32)
    approx = t.astype(np.float64) * np.exp(-(z.astype(np.float64) ** 2) + p.astype(np.float64))
    exact = scipy_special.erfc(z.astype(np.float64))
    rel = np.abs(approx - exact) / exact
    assert rel.max() <= BOUND[deg], f"degree {deg}: max relative error {rel.max():.3g}"
