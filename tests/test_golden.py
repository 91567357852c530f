"""The oracle against the committed golden fixtures.

tests/golden/*.npz hold seeded inputs and float64 expectations evaluated by
tests/golden/make_golden.py straight from the reference ops' definitions
(torch / numpy in f64, no code shared with the oracle). Each case names the
reference code whose definition it evaluates.
"""
import os

import numpy as np
import pytest

import lux3d_oracle as orc
from conftest import assert_vs_f64

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


def test_layer_norm():
    """ops::layer_norm (LayerNorm::forward, runtime/vggt.rs:104) f32 and bf16."""
    g = load("layer_norm")
    assert_vs_f64(orc.layer_norm(g["x"], g["w"], g["b"], float(g["eps"])), g["y"], "f32", "L1 f32")
    xb = orc.bf16_bits(g["x_bf16"])
    e = float(g["eps_bf16"])
    assert_vs_f64(orc.layer_norm(xb, None, None, e, dt=orc.BF16), g["y_bf16_noaffine"], "bf16", "L1 bf16")
    assert_vs_f64(orc.layer_norm_no_affine(xb, e, dt=orc.BF16), g["y_bf16_noaffine"], "bf16", "L3 bf16")


def test_residual_layer_norm():
    """LayerScale + residual + LN (runtime/vggt.rs:113-124): h bit-exact."""
    g = load("residual_layer_norm")
    h, y = orc.residual_layer_norm(orc.bf16_bits(g["x"]), orc.bf16_bits(g["a"]), g["gamma"], g["w"], g["b"],
                                   float(g["eps"]), dt=orc.BF16)
    assert np.array_equal(h, orc.bf16_bits(g["h"]))
    assert_vs_f64(y, g["y"], "bf16", "F1 y")


def _pieces(g):
    c = g["x"].shape[-1]
    te, mod = g["t_emb"], g["modulation"]
    return ({k: np.ascontiguousarray(te[:, i * c:(i + 1) * c]) for i, k in enumerate(("shift", "scale", "gate"))},
            {k: np.ascontiguousarray(mod[i * c:(i + 1) * c]) for i, k in enumerate(("shift", "scale", "gate"))})


def test_adaln_ragged():
    """`(modulation + t_emb).chunk(6)`, modulate and gate on a ragged batch
    (runtime/trellis2_blocks.rs:617-645, 693-717)."""
    g = load("adaln_ragged")
    p, b = _pieces(g)
    xb, hb = orc.bf16_bits(g["x"]), orc.bf16_bits(g["h"])
    y = orc.adaln_modulate(xb, g["offsets"], p["shift"], p["scale"], shift_base=b["shift"],
                           scale_base=b["scale"], eps=1e-6, dt=orc.BF16)
    assert_vs_f64(y, g["y"], "bf16", "M1")
    y = orc.adaln_modulate(xb, g["offsets"], p["shift"], p["scale"], p["gate"], b["shift"], b["scale"], b["gate"],
                           eps=1e-6, dt=orc.BF16)
    assert_vs_f64(y, g["y_gate"], "bf16", "M1'")
    o = orc.gated_residual(xb, hb, g["offsets"], p["gate"], b["gate"], dt=orc.BF16)
    assert_vs_f64(o, g["gated_residual"], "bf16", "G1")


def test_rms_norm_heads():
    """RmsNormHeads::rms_norm_heads (runtime/triposg_dit.rs:509-522) on the q
    slice of a [B, L, H, 3D] qkv, transposed to [B, H, L, D]."""
    g = load("rms_norm_heads")
    d = g["w"].shape[0]
    q = np.ascontiguousarray(g["qkv"][..., :d].transpose(0, 2, 1, 3))
    assert_vs_f64(orc.rms_norm_heads(orc.bf16_bits(q), g["w"], 1e-6, dt=orc.BF16), g["y"], "bf16", "N1")


def test_rope2d_vggt():
    """apply_layernorm_rope with Rope2d::embeddings (runtime/attention_math.rs:14-150)."""
    g = load("rope2d_vggt")
    c, s = orc.rope2d_tables(g["positions"], g["q"].shape[-1], float(g["base"]))
    y = orc.layernorm_rope2d(orc.bf16_bits(g["q"]), g["w"], g["b"], float(g["eps"]), c, s, dt=orc.BF16)
    assert_vs_f64(y, g["y"], "bf16", "R1")


def test_rope3d_trellis():
    """Trellis2QkRmsNorm + Trellis2Rope3d (runtime/trellis2_blocks.rs:84-161, 288-320)."""
    g = load("rope3d_trellis")
    d = g["x"].shape[-1]
    c, s = orc.rope3d_tables(g["coords"], d, float(g["base"]))
    # angles reach 63 rad: f32 angle rounding alone moves cos/sin by ~1e-5
    np.testing.assert_allclose(c, g["cos"], rtol=0, atol=2e-5)
    np.testing.assert_allclose(s, g["sin"], rtol=0, atol=2e-5)
    x = orc.bf16_bits(g["x"][0])
    y = orc.qk_l2norm_rope3d(x, g["gamma"], c, s, dt=orc.BF16)
    assert_vs_f64(y, g["y"][0], "bf16", "N2+R2")


def test_rope2d_dinov3():
    """DINOv3 RoPE tables and apply_rotary_to_patches (runtime/trellis2_dino.rs:140-187, 406-445)."""
    g = load("rope2d_dinov3")
    gh, gw = (int(v) for v in g["grid"])
    c, s = orc.dinov3_rope_tables(gh, gw, g["x"].shape[-1], 100.0)
    np.testing.assert_allclose(c, g["cos64"], rtol=0, atol=4e-6)
    np.testing.assert_allclose(s, g["sin64"], rtol=0, atol=4e-6)
    y = orc.dinov3_rope_apply(g["x"], 5, g["cos"], g["sin"])
    assert_vs_f64(y, g["y"], "f32", "R3")


@pytest.mark.parametrize("name", ["gelu_erf", "gelu_tanh", "silu"])
def test_activations(name):
    """Tensor::gelu_erf / gelu / silu (runtime/nn_blocks.rs:233, trellis2_blocks.rs:560, :236)."""
    g = load("activations")
    # the fixture is the exact f64 GELU; candle's f32 tanh form cancels for x < -3
    assert_vs_f64(getattr(orc, name)(g["x"]), g[name], "f32", name, floor_frac=0.3 if name == "gelu_tanh" else None)


def _spacing_cols(freqs, t):
    """Per-element slack for a frequency that libm's expf rounds 1 ulp away
    from the correctly rounded one: |t| * ulp(freq), for both halves."""
    sp = np.spacing(freqs.astype(np.float32)).astype(np.float64)
    col = np.concatenate([sp, sp])
    return np.abs(t.astype(np.float64))[:, None] * col[None, :]


@pytest.mark.parametrize("dim", [4, 256, 2048])
def test_timestep_embedding(dim):
    """timestep_embedding (runtime/trellis2_blocks.rs:184-204, cos first) and
    TripoSgDiT::timestep_embedding (runtime/triposg_dit.rs:280-297, sin first)."""
    g = load("timestep")
    t = g["t"]
    slack = _spacing_cols(g[f"freqs_{dim}"], t)
    for cos_first, key in ((True, "cos_first"), (False, "sin_first")):
        got = orc.timestep_embedding(t, dim, cos_first=cos_first).astype(np.float64)
        want = g[f"{key}_{dim}"]
        scale = float(np.sqrt(np.mean(want ** 2)))
        err = np.abs(got - want)
        assert np.all(err <= 1e-5 * np.maximum(np.abs(want), scale) + slack), (key, dim, float(err.max()))


def test_dequant_q8_0():
    """QTensor::dequantize for Q8_0 (runtime/nn_blocks.rs:140): the exact product q * d."""
    g = load("q8_0")
    y = orc.dequant_q8_0(g["blocks"], orc.F32)
    assert np.array_equal(y.astype(np.float64), g["y"])
    assert np.array_equal(orc.dequant_q8_0(g["blocks"], orc.BF16), orc.bf16_bits(g["y"].astype(np.float32)))
