"""The HIP path (liblux3d_fused through the C ABI) against the committed
golden fixtures (tests/golden/*.npz: float64 expectations evaluated from the
reference ops' definitions by tests/golden/make_golden.py)."""
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from conftest import assert_vs_f64  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def ops(dev):
    from lux3d_fused import ops as _ops
    return _ops


def to_dev(a, dev, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dtype)


def host(t):
    """f32 tensor -> numpy f32; bf16 -> uint16 bits."""
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def test_layer_norm(dev, ops):
    g = load("layer_norm")
    y = ops.layer_norm(to_dev(g["x"], dev), to_dev(g["w"], dev), to_dev(g["b"], dev), float(g["eps"]))
    assert_vs_f64(host(y), g["y"], "f32", "L1 f32")
    y = ops.layer_norm_no_affine(to_dev(g["x_bf16"], dev, torch.bfloat16), float(g["eps_bf16"]))
    assert_vs_f64(host(y), g["y_bf16_noaffine"], "bf16", "L3 bf16")


def test_residual_layer_norm(dev, ops):
    g = load("residual_layer_norm")
    bf = torch.bfloat16
    h, y = ops.residual_layer_norm(to_dev(g["x"], dev, bf), to_dev(g["a"], dev, bf), to_dev(g["gamma"], dev),
                                   to_dev(g["w"], dev), to_dev(g["b"], dev), float(g["eps"]))
    assert np.array_equal(host(h), host(to_dev(g["h"], dev, bf)))
    assert_vs_f64(host(y), g["y"], "bf16", "F1 y")


def test_adaln_ragged(dev, ops):
    g = load("adaln_ragged")
    c = g["x"].shape[-1]
    x = to_dev(g["x"], dev, torch.bfloat16)
    h = to_dev(g["h"], dev, torch.bfloat16)
    te, mod = to_dev(g["t_emb"], dev), to_dev(g["modulation"], dev)
    off = to_dev(g["offsets"], dev, torch.int64)
    # strided [S, C] views of t_emb and slices of modulation: no copies
    sh, sc, gt = (te[:, i * c:(i + 1) * c] for i in range(3))
    bsh, bsc, bgt = (mod[i * c:(i + 1) * c] for i in range(3))
    y = ops.adaln_modulate(x, sh, sc, shift_base=bsh, scale_base=bsc, seg_offsets=off, eps=1e-6)
    assert_vs_f64(host(y), g["y"], "bf16", "M1")
    y = ops.adaln_modulate(x, sh, sc, gt, shift_base=bsh, scale_base=bsc, gate_base=bgt, seg_offsets=off, eps=1e-6)
    assert_vs_f64(host(y), g["y_gate"], "bf16", "M1'")
    o = ops.gated_residual(x, h, gt, gate_base=bgt, seg_offsets=off)
    assert_vs_f64(host(o), g["gated_residual"], "bf16", "G1")


def test_rms_norm_heads(dev, ops):
    g = load("rms_norm_heads")
    d = g["w"].shape[0]
    qkv = to_dev(g["qkv"], dev, torch.bfloat16)
    q = qkv[..., :d].transpose(1, 2)            # strided [B, H, L, D] view
    y = ops.rms_norm_heads(q, to_dev(g["w"], dev), 1e-6)
    assert_vs_f64(host(y), g["y"], "bf16", "N1")


def test_rope2d_vggt(dev, ops):
    g = load("rope2d_vggt")
    q = to_dev(g["q"], dev, torch.bfloat16)
    w, b = to_dev(g["w"], dev), to_dev(g["b"], dev)
    eps, base = float(g["eps"]), float(g["base"])
    pos = to_dev(g["positions"], dev, torch.int32)
    emb = ops.Rope2d(base).embeddings(pos, q.shape[-1])
    assert_vs_f64(host(ops.apply_layernorm_rope(q, (w, b, eps), emb)), g["y"], "bf16", "R1 tables")
    qo, ko = ops.qk_layernorm_rope2d(q, q, (w, b, eps), (w, b, eps), positions=pos, base=base)
    assert_vs_f64(host(qo), g["y"], "bf16", "R1 positions q")
    assert_vs_f64(host(ko), g["y"], "bf16", "R1 positions k")


def test_rope3d_trellis(dev, ops):
    g = load("rope3d_trellis")
    x = to_dev(g["x"], dev, torch.bfloat16)
    gamma = to_dev(g["gamma"], dev)
    coords = to_dev(g["coords"], dev, torch.int32)
    rope = ops.Trellis2Rope3d(x.shape[-1], float(g["base"]))
    c, s = rope.cos_sin(coords)
    np.testing.assert_allclose(host(c), g["cos"], rtol=0, atol=2e-5)
    np.testing.assert_allclose(host(s), g["sin"], rtol=0, atol=2e-5)
    qo, ko = ops.qk_l2norm_rope3d(x, x, gamma, gamma, coords=coords, rope_base=float(g["base"]))
    assert_vs_f64(host(qo), g["y"], "bf16", "N2+R2 coords")
    qo, _ = ops.qk_l2norm_rope3d(x, x, gamma, gamma, cos=c, sin=s)
    assert_vs_f64(host(qo), g["y"], "bf16", "N2+R2 tables")


def test_rope2d_dinov3(dev, ops):
    g = load("rope2d_dinov3")
    x = to_dev(g["x"], dev)
    qo, ko = ops.apply_rotary_to_patches(x, x, to_dev(g["cos"], dev), to_dev(g["sin"], dev), 5)
    assert_vs_f64(host(qo), g["y"], "f32", "R3 q")
    assert_vs_f64(host(ko), g["y"], "f32", "R3 k")


@pytest.mark.parametrize("name,fn", [("gelu_erf", "gelu_erf"), ("gelu_tanh", "gelu"), ("silu", "silu")])
def test_activations(dev, ops, name, fn):
    g = load("activations")
    y = getattr(ops, fn)(to_dev(g["x"], dev))
    # the fixture is the exact f64 GELU; the kernel follows candle's f32 tanh
    # form, which cancels for x < -3 (those tail elements hold only the floor)
    assert_vs_f64(host(y), g[name], "f32", name, floor_frac=0.3 if name == "gelu_tanh" else None)


@pytest.mark.parametrize("dim", [4, 256, 2048])
def test_timestep_embedding(dev, ops, dim):
    """With the golden (correctly rounded) frequencies passed in, the only
    difference left is the device sin / cos."""
    g = load("timestep")
    t = to_dev(g["t"], dev)
    f = to_dev(g[f"freqs_{dim}"], dev)
    for cos_first, key in ((True, "cos_first"), (False, "sin_first")):
        y = ops.timestep_embedding(t, dim, cos_first=cos_first, freqs=f)
        assert_vs_f64(host(y), g[f"{key}_{dim}"], "f32", f"{key} {dim}")


def test_dequant_q8_0(dev, ops):
    g = load("q8_0")
    blocks = to_dev(g["blocks"], dev, torch.uint8)
    y = ops.dequantize_q8_0(blocks, (g["y"].size,), torch.float32)
    assert np.array_equal(host(y).astype(np.float64), g["y"])
    y = ops.dequantize_q8_0(blocks, (g["y"].size,), torch.bfloat16)
    want = torch.from_numpy(g["y"].astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(host(y), want)
