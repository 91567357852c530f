"""Pins the CPU oracle (oracle/lux3d_oracle.c) before it is trusted as the
parity reference. Every function is checked against something other than a
retyping of its own formula:
  - the reference's own known-answer tests (file:line cited per test),
  - an independent implementation (torch in float64),
  - closed forms, special cases and invariants of the mathematics
    (identity rotations, norm preservation, RoPE's relative-position
    property, exact products for Q8_0).
Each check is chosen so that a plausible slip (wrong sign, swapped halves,
wrong axis, dropped term, eps in the wrong place) fails it.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import lux3d_oracle as orc
from lux3d_fused import synth

from conftest import assert_bf16_close, assert_f32_close

orc.set_threads(4)


def f64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


def to_bf16_bits(a64: np.ndarray) -> np.ndarray:
    """float64 -> f32 -> bf16 bits (torch RNE), for expected values."""
    t = torch.from_numpy(np.asarray(a64, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


# ---------------------------------------------------------------------------
# conversions
# ---------------------------------------------------------------------------

def test_bf16_rounding_matches_torch_and_half_nan_rule():
    x = np.concatenate([synth.normal(1, 100000) * np.float32(1e3),
                        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 3.3895314e38, 1e-40], dtype=np.float32)])
    # ties: exact halfway patterns (low 16 bits 0x8000) with even and odd lsb
    ties = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x7F7F8000], dtype=np.uint32).view(np.float32)
    x = np.concatenate([x, ties])
    got = orc.bf16_bits(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    # half 2.x: NaN keeps sign + top payload and is made quiet (| 0x40)
    nans = np.array([0x7F800001, 0xFF812345, 0x7FC00000], dtype=np.uint32)
    got = orc.bf16_bits(nans.view(np.float32))
    assert list(got) == [0x7F80 | 0x40, 0xFF81 | 0x40, 0x7FC0 | 0x40]


def test_f16_conversions_match_numpy():
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = bits.view(np.float16)
    finite = np.isfinite(vals)
    out = np.array([orc.LIB.or_f16_to_f32(int(b)) for b in bits[::7]], dtype=np.float32)
    assert np.array_equal(out[finite[::7]], vals[::7][finite[::7]].astype(np.float32))
    x = np.concatenate([synth.normal(3, 50000) * np.float32(3e3), synth.normal(4, 50000) * np.float32(1e-5)])
    got = np.array([orc.LIB.or_f32_to_f16(float(v)) for v in x[::5]], dtype=np.uint16)
    assert np.array_equal(got, x[::5].astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------------------
# LayerNorm family
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("slow", [False, True])
def test_layer_norm_matches_torch_f64(slow):
    x = synth.normal(10, 64 * 1024).reshape(64, 1024) * np.float32(2.0) + np.float32(0.5)
    w = synth.normal(11, 1024, 1.0, 0.02)
    b = synth.normal(12, 1024, 0.0, 0.02)
    y = orc.layer_norm(x, w, b, 1e-5, slow=slow)
    ref = F.layer_norm(f64(x), (1024,), f64(w), f64(b), eps=1e-5).numpy()
    assert_f32_close(y, ref, what="L1/L2 vs torch")


def test_layer_norm_bf16_single_rounding():
    x32 = synth.normal(13, 16 * 2048).reshape(16, 2048)
    xb = orc.bf16_bits(x32)
    y = orc.layer_norm(xb, None, None, 1e-6, dt=orc.BF16)
    ref = F.layer_norm(f64(orc.bf16_to_f32(xb)), (2048,), eps=1e-6).numpy()
    assert_bf16_close(y, to_bf16_bits(ref), tol=1, what="bf16 LN")


def test_layer_norm_invariants():
    x = synth.normal(14, 8 * 512).reshape(8, 512)
    y = orc.layer_norm(x, None, None, 1e-12)
    assert np.allclose(y.mean(axis=1), 0.0, atol=1e-6)
    assert np.allclose((y.astype(np.float64) ** 2).mean(axis=1), 1.0, atol=1e-5)
    # shift invariance. candle's fast path uses var = E[x^2] - mean^2 (one
    # pass), which cancels for offset rows; the composed (two-pass) path does not.
    y2 = orc.layer_norm(x + np.float32(0.5), None, None, 1e-12)
    assert np.max(np.abs(y2 - y)) < 5e-5
    ys = orc.layer_norm(x, None, None, 1e-12, slow=True)
    ys2 = orc.layer_norm(x + np.float32(7.0), None, None, 1e-12, slow=True)
    assert np.max(np.abs(ys2 - ys)) < 5e-6
    # constant rows: (x - mean) == 0 exactly, so the output is the bias exactly
    c = np.full((3, 256), 1.25, dtype=np.float32)
    b = synth.normal(15, 256)
    for fn in (lambda: orc.layer_norm(c, np.ones(256, np.float32), b, 1e-5),
               lambda: orc.layer_norm(c, np.ones(256, np.float32), b, 1e-5, slow=True)):
        assert np.array_equal(fn(), np.broadcast_to(b, c.shape))
    # eps inside the sqrt: var = 0 rows of L3 give 0 / sqrt(eps) = 0
    assert np.array_equal(orc.layer_norm_no_affine(c, 1e-6), np.zeros_like(c))


def test_layer_norm_no_affine_matches_torch():
    x = synth.normal(16, 32 * 1536).reshape(32, 1536)
    y = orc.layer_norm_no_affine(x, 1e-6)
    assert_f32_close(y, F.layer_norm(f64(x), (1536,), eps=1e-6).numpy(), what="L3")


def test_residual_layer_norm_reductions():
    x = synth.normal(17, 16 * 1024).reshape(16, 1024)
    a = synth.normal(18, 16 * 1024).reshape(16, 1024)
    w = synth.normal(19, 1024, 1.0, 0.02)
    b = synth.normal(20, 1024, 0.0, 0.02)
    # gamma = 0: h == x exactly, y == L1(x)
    h, y = orc.residual_layer_norm(x, a, np.zeros(1024, np.float32), w, b, 1e-5)
    assert np.array_equal(h, x)
    assert np.array_equal(y, orc.layer_norm(x, w, b, 1e-5))
    # gamma absent (F3): h == x + a
    h, y = orc.residual_layer_norm(x, a, None, w, b, 1e-5)
    assert np.array_equal(h, (x + a).astype(np.float32))
    # LayerScale gamma ~ N(1e-5, 1e-6): y vs torch on the f64 sum
    g = synth.normal(21, 1024, 1e-5, 1e-6)
    h, y = orc.residual_layer_norm(x, a, g, w, b, 1e-5)
    ref_h = f64(x) + f64(a) * f64(g)
    assert np.max(np.abs(h - ref_h.numpy())) < 1e-6
    assert_f32_close(y, F.layer_norm(ref_h, (1024,), f64(w), f64(b), eps=1e-5).numpy(), what="F1")
    # bf16: the norm reads the stored (rounded) residual stream
    xb, ab = orc.bf16_bits(x), orc.bf16_bits(a)
    hb, yb = orc.residual_layer_norm(xb, ab, g, w, b, 1e-5, dt=orc.BF16)
    assert np.array_equal(yb, orc.layer_norm(hb, w, b, 1e-5, dt=orc.BF16))


# ---------------------------------------------------------------------------
# AdaLN modulate / gate / MV
# ---------------------------------------------------------------------------

def test_chunk_modulation_order_kat():
    """tests/trellis2_blocks.rs:205-225: chunk(6) of [1..12] with C = 2."""
    from lux3d_fused.ops import chunk_modulation
    mod = torch.arange(1, 13, dtype=torch.float32).reshape(1, 12)
    chunks = chunk_modulation(mod)
    want = [[1, 2], [3, 4], [5, 6], [7, 8], [9, 10], [11, 12]]
    for c, w in zip(chunks, want):
        assert tuple(c.shape) == (1, 1, 2)
        assert c.flatten().tolist() == w


def test_adaln_modulate_against_torch_and_reductions():
    rows, C = 40, 256
    x = synth.normal(30, rows * C).reshape(rows, C)
    offs = np.array([0, 15, 40], dtype=np.int64)
    t_emb = synth.normal(31, 2 * 6 * C, 0.0, 0.1).reshape(2, 6 * C)
    modulation = synth.normal(32, 6 * C, 0.0, 0.1)
    piece = lambda k: np.ascontiguousarray(t_emb[:, k * C:(k + 1) * C])  # noqa: E731
    base = lambda k: modulation[k * C:(k + 1) * C]  # noqa: E731
    y = orc.adaln_modulate(x, offs, piece(0), piece(1), None, base(0), base(1), None, eps=1e-6)
    n = F.layer_norm(f64(x), (C,), eps=1e-6)
    ref = torch.empty_like(n)
    for s in range(2):
        r0, r1 = offs[s], offs[s + 1]
        mv = f64(modulation) + f64(t_emb[s])       # mod_vec = modulation + t_emb
        sh, sc = mv[0:C], mv[C:2 * C]              # chunk order: shift_msa, scale_msa, ...
        ref[r0:r1] = n[r0:r1] * (1.0 + sc) + sh
    assert_f32_close(y, ref.numpy(), what="M1 ragged")
    # scale = shift = 0 reduces to L3 exactly
    z = np.zeros((2, C), np.float32)
    assert np.array_equal(orc.adaln_modulate(x, offs, z, z, eps=1e-6), orc.layer_norm_no_affine(x, 1e-6))
    # gate variant (vggt.rs:399-405): gate = 0 gives x back exactly
    yg = orc.adaln_modulate(x, offs, piece(0), piece(1), z, eps=1e-6)
    assert np.array_equal(yg, x)
    # gate = 1 gives modulated + x
    yg1 = orc.adaln_modulate(x, offs, piece(0), piece(1), np.ones((2, C), np.float32), eps=1e-6)
    y0 = orc.adaln_modulate(x, offs, piece(0), piece(1), eps=1e-6)
    assert np.array_equal(yg1, (y0 + x).astype(np.float32))


def test_gated_residual():
    rows, C = 30, 128
    x = synth.normal(33, rows * C).reshape(rows, C)
    h = synth.normal(34, rows * C).reshape(rows, C)
    offs = np.array([0, 10, 30], dtype=np.int64)
    g = synth.normal(35, 2 * C, 0.0, 0.1).reshape(2, C)
    out = orc.gated_residual(x, h, offs, g)
    ref = f64(x).clone()
    ref[:10] += f64(h[:10]) * f64(g[0])
    ref[10:] += f64(h[10:]) * f64(g[1])
    assert np.max(np.abs(out - ref.numpy())) < 1e-6
    assert np.array_equal(orc.gated_residual(x, h, offs, np.zeros((2, C), np.float32)), x)


def test_gated_residual_modulate_against_torch_and_reductions():
    """G1 then L3 + M1 on the stored residual stream (trellis2_blocks.rs:
    708-713; :637-642 ungated): torch f64 on the same ragged segments, and
    the reductions that a dropped or misplaced term would break."""
    rows, C = 40, 256
    x = synth.normal(36, rows * C).reshape(rows, C)
    h = synth.normal(37, rows * C).reshape(rows, C)
    offs = np.array([0, 17, 40], dtype=np.int64)
    t_emb = synth.normal(38, 2 * 6 * C, 0.0, 0.1).reshape(2, 6 * C)
    modulation = synth.normal(39, 6 * C, 0.0, 0.1)
    piece = lambda k: np.ascontiguousarray(t_emb[:, k * C:(k + 1) * C])  # noqa: E731
    base = lambda k: modulation[k * C:(k + 1) * C]  # noqa: E731
    # the sparse block's MLP half: gate_msa (chunk 2), then scale_mlp / shift_mlp (chunks 4 / 3)
    xo, y = orc.gated_residual_modulate(x, h, offs, piece(2), piece(3), piece(4), base(2), base(3), base(4))
    ref_x = torch.empty((rows, C), dtype=torch.float64)
    ref_y = torch.empty((rows, C), dtype=torch.float64)
    for s in range(2):
        r0, r1 = offs[s], offs[s + 1]
        mv = f64(modulation) + f64(t_emb[s])
        g, sh, sc = mv[2 * C:3 * C], mv[3 * C:4 * C], mv[4 * C:5 * C]
        ref_x[r0:r1] = f64(x[r0:r1]) + f64(h[r0:r1]) * g
        n = F.layer_norm(f64(xo[r0:r1]), (C,), eps=1e-6)   # the norm reads the stored x_out
        ref_y[r0:r1] = n * (1.0 + sc) + sh
    assert np.max(np.abs(xo - ref_x.numpy())) < 1e-6
    assert_f32_close(y, ref_y.numpy(), what="G1 + M1 ragged")
    # gate = 0: x_out == x exactly, y == the plain modulate of x
    z = np.zeros((2, C), np.float32)
    xo0, y0 = orc.gated_residual_modulate(x, h, offs, z, piece(3), piece(4))
    assert np.array_equal(xo0, x)
    assert np.array_equal(y0, orc.adaln_modulate(x, offs, piece(3), piece(4), eps=1e-6))
    # no gate (the dense block's cross-attention add): x_out == x + h exactly
    xo1, y1 = orc.gated_residual_modulate(x, h, offs, None, z, z)
    assert np.array_equal(xo1, (x + h).astype(np.float32))
    # scale = shift = 0: y is L3 of the stored x_out
    assert np.array_equal(y1, orc.layer_norm_no_affine(xo1, 1e-6))
    # bf16: x_out equals the gated residual, y the modulate of the stored x_out
    xb, hb = orc.bf16_bits(x), orc.bf16_bits(h)
    xob, yb = orc.gated_residual_modulate(xb, hb, offs, piece(2), piece(3), piece(4), dt=orc.BF16)
    assert np.array_equal(xob, orc.gated_residual(xb, hb, offs, piece(2), dt=orc.BF16))
    assert np.array_equal(yb, orc.adaln_modulate(xob, offs, piece(3), piece(4), eps=1e-6, dt=orc.BF16))


# ---------------------------------------------------------------------------
# Head norms
# ---------------------------------------------------------------------------

def test_rms_norm_heads_matches_torch():
    x = synth.normal(40, 2 * 4 * 16 * 128).reshape(2, 4, 16, 128)
    w = synth.normal(41, 128, 1.0, 0.02)
    y = orc.rms_norm_heads(x, w, 1e-6)
    xd = f64(x)
    ref = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6) * f64(w)
    assert_f32_close(y, ref.numpy(), what="N1")
    # scale invariance for norms far above eps
    y2 = orc.rms_norm_heads(x * np.float32(64.0), w, 1e-6)
    assert np.max(np.abs(y2 - y)) < 1e-5


def test_qk_l2norm_kat():
    """tests/trellis2_blocks.rs:126-153: [3, 4, 0, 0], gamma 1 -> [1.2, 1.6, 0, 0];
    gamma 2 -> [2.4, 3.2, 0, 0] (F.normalize * gamma * sqrt(4))."""
    x = np.array([[[3.0, 4.0, 0.0, 0.0]]], dtype=np.float32)
    y = orc.qk_l2norm(x, np.ones((1, 4), np.float32))
    assert np.allclose(y.reshape(-1), [1.2, 1.6, 0.0, 0.0], atol=1e-6)
    y = orc.qk_l2norm(x, np.full((1, 4), 2.0, np.float32))
    assert np.allclose(y.reshape(-1), [2.4, 3.2, 0.0, 0.0], atol=1e-6)
    # zero vector: clamp(0, 1e-12) keeps it zero (no NaN)
    assert np.array_equal(orc.qk_l2norm(np.zeros((1, 2, 4), np.float32), np.ones((2, 4), np.float32)),
                          np.zeros((1, 2, 4), np.float32))
    # per-head gamma is indexed by head
    xs = synth.normal(42, 5 * 3 * 64).reshape(5, 3, 64)
    g = synth.normal(43, 3 * 64, 1.0, 0.1).reshape(3, 64)
    y = orc.qk_l2norm(xs, g)
    ref = F.normalize(f64(xs), dim=-1) * f64(g) * 8.0
    assert_f32_close(y, ref.numpy(), what="N2")


# ---------------------------------------------------------------------------
# R1: VGGT 2D RoPE
# ---------------------------------------------------------------------------

def _rope2d_rotate(t, pos, d=64, base=100.0):
    c, s = orc.rope2d_tables(pos, d, base)
    return orc.rope2d_apply(t, c, s), c, s


def test_rope2d_specials_are_identity_and_tables_closed_form():
    pos = synth.vggt_positions(1, 3, 4)           # 5 specials at (0, 0)
    c, s = orc.rope2d_tables(pos, 64, 100.0)
    assert np.all(c[0, :5] == 1.0) and np.all(s[0, :5] == 0.0)
    # frequency index 0 has inv_freq exactly 1: angle == position. y-half (dims
    # 0..31) follows pos_y, x-half (32..63) pos_x; sin_alt negates the first
    # quarter of each half.
    tok = 5 + 2 * 4 + 3                            # patch (y=2, x=3) -> pos (3, 4)
    assert tuple(pos[0, tok]) == (3, 4)
    assert c[0, tok, 0] == np.float32(math.cos(3.0)) and c[0, tok, 16] == np.float32(math.cos(3.0))
    assert c[0, tok, 32] == np.float32(math.cos(4.0))
    assert s[0, tok, 0] == -np.float32(math.sin(3.0)) and s[0, tok, 16] == np.float32(math.sin(3.0))
    assert s[0, tok, 48] == np.float32(math.sin(4.0))
    # the k-th frequency is 100^(-2k/32), checked in f64
    for k in (1, 7, 15):
        ang = 3.0 * 100.0 ** (-2.0 * k / 32.0)
        assert abs(c[0, tok, k] - math.cos(ang)) < 2e-7


def test_rope2d_rotation_properties():
    n = 40
    pos = np.stack([synth.uniform(50, n, 0, 37).astype(np.int32),
                    synth.uniform(51, n, 0, 37).astype(np.int32)], axis=1)[None]
    q = synth.normal(52, 1 * 2 * n * 64).reshape(1, 2, n, 64)
    k = synth.normal(53, 1 * 2 * n * 64).reshape(1, 2, n, 64)
    rq, _, _ = _rope2d_rotate(q, pos)
    # norm preservation on each rotated pair (j, j^16)
    e_in = q[..., :16] ** 2 + q[..., 16:32] ** 2
    e_out = rq[..., :16] ** 2 + rq[..., 16:32] ** 2
    assert np.max(np.abs(e_in - e_out)) < 1e-4
    # relative-position property: <R(p)q, R(p')k> depends only on p - p'
    shift = np.array([[[7, 11]]], dtype=np.int32)
    rk, _, _ = _rope2d_rotate(k, pos)
    rq2, _, _ = _rope2d_rotate(q, pos + shift)
    rk2, _, _ = _rope2d_rotate(k, pos + shift)
    d1 = np.einsum("bhnd,bhnd->bhn", rq.astype(np.float64), rk.astype(np.float64))
    d2 = np.einsum("bhnd,bhnd->bhn", rq2.astype(np.float64), rk2.astype(np.float64))
    assert np.max(np.abs(d1 - d2)) < 2e-4
    # as a complex rotation: (t[j] + i t[j+16]) * e^{i*angle} per y/x half
    c, s = orc.rope2d_tables(pos, 64, 100.0)
    zq = q[..., 0:16].astype(np.float64) + 1j * q[..., 16:32]
    ang = np.arctan2(-s[:, None, :, 0:16].astype(np.float64), c[:, None, :, 0:16])
    want = zq * np.exp(1j * ang)
    assert np.max(np.abs(rq[..., 0:16] - want.real)) < 2e-5
    assert np.max(np.abs(rq[..., 16:32] - want.imag)) < 2e-5


def test_layernorm_rope2d_is_ln_then_rope():
    pos = synth.vggt_positions(1, 5, 6)
    n = pos.shape[1]
    q = synth.normal(54, 2 * n * 64).reshape(1, 2, n, 64)
    w, b = synth.normal(55, 64, 1.0, 0.05), synth.normal(56, 64, 0.0, 0.05)
    c, s = orc.rope2d_tables(pos, 64, 100.0)
    fused = orc.layernorm_rope2d(q, w, b, 1e-5, c, s)
    ln = F.layer_norm(f64(q), (64,), f64(w), f64(b), eps=1e-5).numpy().astype(np.float32)
    assert_f32_close(fused, orc.rope2d_apply(ln, c, s), what="L2+R1")
    # a LayerNorm without bias (candle_nn::LayerNorm, bias None) stops at n * w
    nob = orc.layernorm_rope2d(q, w, None, 1e-5, c, s)
    ln0 = F.layer_norm(f64(q), (64,), f64(w), None, eps=1e-5).numpy().astype(np.float32)
    assert_f32_close(nob, orc.rope2d_apply(ln0, c, s), what="L2 (no bias)+R1")
    assert np.array_equal(nob, orc.layernorm_rope2d(q, w, np.zeros(64, np.float32), 1e-5, c, s))


# ---------------------------------------------------------------------------
# R2: TRELLIS.2 3D RoPE
# ---------------------------------------------------------------------------

def test_rope3d_tables_kat():
    """tests/trellis2_blocks.rs:43-73 (head_dim 12: freq_dim 2, freqs [1, 1e4^-0.5])."""
    coords = np.array([[1, 0, 0], [0, 1, 0]], dtype=np.int32)
    c, s = orc.rope3d_tables(coords, 12)
    assert c.shape == (2, 6)
    freq2 = 1.0 / 10000.0 ** 0.5
    for tok, co in enumerate(coords):
        angles = [co[0] * 1.0, co[0] * freq2, co[1] * 1.0, co[1] * freq2, co[2] * 1.0, co[2] * freq2]
        for j, a in enumerate(angles):
            assert abs(c[tok, j] - math.cos(a)) < 1e-6
            assert abs(s[tok, j] - math.sin(a)) < 1e-6


def test_rope3d_apply_kat():
    """tests/trellis2_blocks.rs:78-111: complex product per interleaved pair,
    the zero-angle pairs are the identity, energy is preserved."""
    coords = np.array([[1, 0, 0]], dtype=np.int32)
    c, s = orc.rope3d_tables(coords, 12)
    x = np.array([1.0, 0.0, 2.0, 3.0, 5.0, 0.0, 7.0, 1.0, 0.0, 2.0, 4.0, 4.0], dtype=np.float32)
    out = orc.rope3d_apply(x.reshape(1, 1, 1, 12), c, s).reshape(-1)
    freq2 = 1.0 / 10000.0 ** 0.5
    phases = [(1.0, 1.0), (freq2, freq2), (0.0, 0.0)]
    for pair in range(6):
        ac, as_ = (math.cos(phases[pair][0]), math.sin(phases[pair][1])) if pair < 2 else (1.0, 0.0)
        re, im = x[2 * pair], x[2 * pair + 1]
        assert abs(out[2 * pair] - (re * ac - im * as_)) < 1e-5
        assert abs(out[2 * pair + 1] - (re * as_ + im * ac)) < 1e-5
    e_in = float((x.reshape(-1, 2) ** 2).sum())
    e_out = float((out.reshape(-1, 2) ** 2).sum())
    assert abs(e_in - e_out) < 1e-4


def test_rope3d_head128_layout_and_pad_pair():
    """head_dim 128: 21 freqs per axis, axis-major (x, y, z), pair 63 is pad."""
    coords = np.array([[5, 9, 13]], dtype=np.int32)
    c, s = orc.rope3d_tables(coords, 128)
    assert c.shape == (1, 64)
    assert c[0, 63] == 1.0 and s[0, 63] == 0.0
    for axis, val in enumerate((5, 9, 13)):
        for i in (0, 1, 20):
            ang = val * 10000.0 ** (-i / 21.0)
            assert abs(c[0, axis * 21 + i] - math.cos(ang)) < 2e-6
    x = synth.normal(60, 3 * 2 * 128).reshape(1, 3, 2, 128)
    coords3 = np.array([[5, 9, 13], [0, 0, 0], [63, 1, 2]], dtype=np.int32)
    c3, s3 = orc.rope3d_tables(coords3, 128)
    y = orc.rope3d_apply(x, c3, s3)
    assert np.array_equal(y[0, 1], x[0, 1])                    # coord (0,0,0): identity
    assert np.array_equal(y[..., 126:], x[..., 126:])          # pad pair untouched
    g = np.ones((2, 128), np.float32)
    fused = orc.qk_l2norm_rope3d(x.reshape(3, 2, 128), g, c3, s3)
    two = orc.rope3d_apply(orc.qk_l2norm(x.reshape(3, 2, 128), g).reshape(1, 3, 2, 128), c3, s3)
    assert_f32_close(fused.reshape(-1), two.reshape(-1), what="N2+R2 fused vs composed")


# ---------------------------------------------------------------------------
# R3: DINOv3 RoPE
# ---------------------------------------------------------------------------

def test_dinov3_tables_kat():
    """runtime/trellis2_dino.rs:516-569 (head_dim 8, 2x2 grid, inv_freq [1, 0.1])."""
    c, s = orc.dinov3_rope_tables(2, 2, 8, 100.0)
    inv = [1.0, 1.0 / 100.0 ** 0.5]
    two_pi = 2.0 * math.pi
    for y in range(2):
        cy = 2.0 * ((y + 0.5) / 2) - 1.0
        for x in range(2):
            cx = 2.0 * ((x + 0.5) / 2) - 1.0
            half = [two_pi * cy * f for f in inv] + [two_pi * cx * f for f in inv]
            row = half + half
            for j, a in enumerate(row):
                assert abs(c[y * 2 + x, j] - math.cos(a)) < 1e-6
                assert abs(s[y * 2 + x, j] - math.sin(a)) < 1e-6


def test_dinov3_rotate_half_and_prefix_kat():
    """runtime/trellis2_dino.rs:571-644: rotate_half([1..8]) = [-5..-8, 1..4];
    prefix tokens pass through; patches get q*c + rotate_half(q)*s."""
    x = np.arange(1, 9, dtype=np.float32).reshape(1, 1, 1, 8)
    rh = orc.dinov3_rope_apply(x, 0, np.zeros((1, 8), np.float32), np.ones((1, 8), np.float32))
    assert rh.reshape(-1).tolist() == [-5.0, -6.0, -7.0, -8.0, 1.0, 2.0, 3.0, 4.0]
    npfx, patches, hd = 3, 2, 8
    q = (0.1 * (np.arange((npfx + patches) * hd, dtype=np.float32) + 1.0)).reshape(1, 1, npfx + patches, hd)
    cval, sval = 0.5, math.sqrt(0.5)
    out = orc.dinov3_rope_apply(q, npfx, np.full((patches, hd), cval, np.float32),
                                np.full((patches, hd), sval, np.float32))
    assert np.array_equal(out[0, 0, :npfx], q[0, 0, :npfx])
    qp = q[0, 0, npfx]
    for d in range(hd):
        partner = -qp[d + hd // 2] if d < hd // 2 else qp[d - hd // 2]
        assert abs(out[0, 0, npfx, d] - (qp[d] * cval + partner * sval)) < 1e-5


# ---------------------------------------------------------------------------
# Activations
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("act", ["gelu_erf", "gelu_tanh", "silu"])
def test_activations_match_torch_f64(act):
    x = np.concatenate([synth.normal(70, 200000) * np.float32(4.0),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 30.0, -30.0, 10.0, -10.0], np.float32)])
    fn = {"gelu_erf": orc.gelu_erf, "gelu_tanh": orc.gelu_tanh, "silu": orc.silu}[act]
    tf = {"gelu_erf": lambda t: F.gelu(t), "gelu_tanh": lambda t: F.gelu(t, approximate="tanh"),
          "silu": F.silu}[act]
    ref = tf(f64(x)).numpy()
    # candle's f32 Gelu 0.5*x*(1 + tanh(u)) cancels for x < -3 (1 + tanh(u)
    # loses relative accuracy, and is exactly 0 below x = -5.3): against the
    # exact f64 GELU those tail elements hold only the absolute floor
    tail = 0.3 if act == "gelu_tanh" else None
    assert_f32_close(fn(x), ref, what=act, floor_frac=tail)
    xb = orc.bf16_bits(x)
    refb = tf(f64(orc.bf16_to_f32(xb))).numpy()
    assert_bf16_close(fn(xb, dt=orc.BF16), to_bf16_bits(refb), tol=1, what=act + " bf16", floor_frac=tail)


# ---------------------------------------------------------------------------
# Timestep embeddings
# ---------------------------------------------------------------------------

def test_timestep_embedding_kat_and_conventions():
    """tests/trellis2_blocks.rs:157-171 (t = 500, dim 4, cos first)."""
    emb = orc.timestep_embedding(np.array([500.0], np.float32), 4, cos_first=True).reshape(-1)
    f1 = math.exp(-math.log(10000.0) / 2.0)
    want = [math.cos(500.0), math.cos(500.0 * f1), math.sin(500.0), math.sin(500.0 * f1)]
    assert np.allclose(emb, want, atol=1e-5)
    # TripoSG is the same table with the halves swapped (sin first, dim = width)
    t = synth.uniform(71, 5, 0.0, 1000.0)
    a = orc.timestep_embedding(t, 2048, cos_first=True)
    b = orc.timestep_embedding(t, 2048, cos_first=False)
    assert np.array_equal(a[:, :1024], b[:, 1024:]) and np.array_equal(a[:, 1024:], b[:, :1024])
    # odd dim: zero pad at the end
    odd = orc.timestep_embedding(t, 7, cos_first=True)
    assert np.all(odd[:, 6] == 0.0)
    # frequencies follow 10000^(-i/half) (f64 check, small t keeps the arguments exact-ish)
    small = orc.timestep_embedding(np.array([1.0], np.float32), 256, cos_first=True).reshape(-1)
    i = np.arange(128)
    assert np.max(np.abs(small[:128] - np.cos(10000.0 ** (-i / 128.0)))) < 2e-7


def _libm_timestep_freqs(dim):
    """The reference's host frequency loop: f32 argument, libm expf."""
    import ctypes
    import ctypes.util
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.argtypes, libm.expf.restype = [ctypes.c_float], ctypes.c_float
    half = dim // 2
    nlp = np.float32(-math.log(10000.0))
    return np.array([libm.expf(float((nlp * np.float32(i)) / np.float32(half))) for i in range(half)], np.float32)


def test_timestep_frequencies_rounded_once():
    """The device path's frequencies, exp(x) in f64 rounded once to f32, are
    the f32 nearest the exact exp(x) of the reference's f32 argument at the
    configs' dims (mpmath at 200 bits); and the given-frequency form of the
    oracle, fed the reference's libm table, reproduces its own T1 / T2 bit
    for bit. glibc's expf is not correctly rounded everywhere (dim 2048,
    i = 457: 0.5004 ulp), so that table and the rounded-once one can differ
    in the last bit of a frequency; the GPU tests hold the device path to
    the rounded-once table."""
    mpmath = pytest.importorskip("mpmath")
    mpmath.mp.prec = 200
    for dim in (256, 2048, 255):
        f = orc.timestep_freqs_rounded_once(dim)
        half = dim // 2
        nlp = np.float32(-math.log(10000.0))
        x = (nlp * np.arange(half, dtype=np.float32)) / np.float32(half)
        for i in range(half):
            exact = mpmath.exp(mpmath.mpf(float(x[i])))
            err = abs(mpmath.mpf(float(f[i])) - exact)
            ulp = mpmath.mpf(float(np.spacing(f[i])))
            assert err <= ulp / 2, (dim, i)
        t = synth.uniform(72, 3, 0.0, 1000.0)
        libm = _libm_timestep_freqs(dim)
        for cos_first in (True, False):
            if dim % 2 and not cos_first:
                continue
            assert np.array_equal(orc.timestep_embedding(t, dim, cos_first, freqs=libm),
                                  orc.timestep_embedding(t, dim, cos_first))


# ---------------------------------------------------------------------------
# Q8_0
# ---------------------------------------------------------------------------

def _quantize_q8_0_py(x):
    """BlockQ8_0::from_float restated independently (numpy f32 arithmetic,
    numpy's own binary16 rounding)."""
    x = np.asarray(x, np.float32).reshape(-1, 32)
    out = np.empty((x.shape[0], 34), np.uint8)
    for b, xs in enumerate(x):
        a = np.abs(xs)
        a = a[~np.isnan(a)]
        amax = np.float32(a.max()) if a.size else np.float32(0.0)
        amax = max(amax, np.float32(0.0))
        d = np.float32(amax / np.float32(127.0))
        idv = np.float32(1.0) / d if d != 0 else np.float32(0.0)
        v = (xs * idv).astype(np.float32)
        with np.errstate(invalid="ignore"):
            r = np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))  # half away from zero
            q = np.where(np.isnan(r), 0, np.clip(r, -128, 127)).astype(np.int8)
        out[b, 0:2] = np.array([d], np.float16).view(np.uint8)
        out[b, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def test_quantize_q8_0_matches_restatement_and_bounds():
    """or_quantize_q8_0 (candle's BlockQ8_0::from_float, k_quants.rs) against
    an independent numpy restatement on random and special blocks, plus what
    the format fixes: |q| <= 127, the largest |x| of a block maps to +-127,
    and q * d reconstructs x within d / 2 (+ the f16 rounding of d)."""
    rng = np.random.default_rng(5)
    blocks = [rng.normal(0, 1, 32), rng.normal(0, 1e-3, 32), rng.uniform(-1e4, 1e4, 32), np.zeros(32),
              np.full(32, -2.5), np.arange(32) - 15.5, np.r_[np.full(31, 0.25), 127.0],
              np.r_[np.nan, rng.normal(0, 1, 31)], np.r_[np.inf, rng.normal(0, 1, 31)],
              np.r_[1e-40, np.zeros(31)], np.r_[70000.0, rng.normal(0, 1, 31)]]
    x = np.concatenate([np.asarray(b, np.float32) for b in blocks])
    got = orc.quantize_q8_0(x)
    assert np.array_equal(got, _quantize_q8_0_py(x))
    xr = rng.normal(0, 3, 32 * 64).astype(np.float32)
    g = orc.quantize_q8_0(xr).reshape(-1, 34)
    q = g[:, 2:].view(np.int8).astype(np.int32)
    d = g[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    xb = xr.reshape(-1, 32)
    assert np.abs(q).max() <= 127
    assert np.all(np.abs(q[np.arange(len(xb)), np.abs(xb).argmax(1)]) == 127)
    amax = np.abs(xb).max(1)
    err = np.abs(q * d[:, None] - xb)
    assert np.all(err <= (amax / 127.0)[:, None] * (0.5 + 127 * 2.0 ** -11) * 1.0001)


def test_q8_0_linear_int8_brute_force():
    """or_q8_0_linear_int8 (candle's CPU QMatMul for Q8_0: x quantized per row,
    integer block dots, sumf += (f32)isum * wd * xd in block order, + bias)
    against a Python loop in the same f32 order on tiny shapes; the integer
    block dots against numpy int64; and one block in closed form."""
    rng = np.random.default_rng(6)
    M, N, K = 3, 5, 96
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    wblk = synth.q8_0_blocks(7, N * K // 32)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    y = orc.q8_0_linear_int8(x, wblk, N, bias)
    xq = orc.quantize_q8_0(x).reshape(M, K // 32, 34)
    wq = wblk.reshape(N, K // 32, 34)
    want = np.empty((M, N), np.float32)
    for m in range(M):
        for n in range(N):
            s = np.float32(0.0)
            for b in range(K // 32):
                xi = xq[m, b, 2:].view(np.int8).astype(np.int64)
                wi = wq[n, b, 2:].view(np.int8).astype(np.int64)
                isum = int((xi * wi).sum())
                assert abs(isum) < 2 ** 24  # exact in f32 as well
                xd = np.float32(xq[m, b, 0:2].copy().view(np.float16)[0])
                wd = np.float32(wq[n, b, 0:2].copy().view(np.float16)[0])
                s = np.float32(s + np.float32(np.float32(np.float32(isum) * wd) * xd))
            want[m, n] = np.float32(s + bias[n])
    assert np.array_equal(y, want)
    # one block, closed form: x = 127 * e_3 quantizes to d = 1, q = 127 e_3,
    # so with weight values -16..15 at d = 1: y = 127 * (3 - 16)
    x1 = np.zeros((1, 32), np.float32)
    x1[0, 3] = 127.0
    wb = np.zeros(34, np.uint8)
    wb[0:2] = np.array([1.0], np.float16).view(np.uint8)
    wb[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    assert orc.q8_0_linear_int8(x1, wb, 1)[0, 0] == np.float32(127 * -13)


def test_q8_0_dequant_brute_force():
    scales = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF,
                       0x1234, 0x2E66, 0x7C00, 0xFC00, 0x7E00], dtype=np.uint16)
    qs = np.arange(-128, 128, dtype=np.int16).astype(np.int8).reshape(8, 32)
    blocks = np.empty((len(scales) * 8, 34), dtype=np.uint8)
    for si, sc in enumerate(scales):
        for r in range(8):
            blocks[si * 8 + r, 0] = sc & 0xFF          # little-endian f16 scale
            blocks[si * 8 + r, 1] = sc >> 8
            blocks[si * 8 + r, 2:] = qs[r].view(np.uint8)
    d = np.repeat(scales.view(np.float16).astype(np.float32), 8 * 32)
    q = np.tile(qs.reshape(-1).astype(np.float32), len(scales))
    with np.errstate(invalid="ignore"):
        exact = (q * d).astype(np.float32)                 # exact: <= 7 x 11 significant bits
    got32 = orc.dequant_q8_0(blocks, orc.F32)
    assert np.array_equal(np.isnan(got32), np.isnan(exact))
    fin = ~np.isnan(exact)
    assert np.array_equal(got32[fin].view(np.uint32), exact[fin].view(np.uint32))
    got_b = orc.dequant_q8_0(blocks, orc.BF16)
    want_b = torch.from_numpy(exact).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got_b[fin], want_b[fin])
    assert np.all((got_b[~fin] & 0x7FFF) > 0x7F80)
    got_h = orc.dequant_q8_0(blocks, orc.F16)
    with np.errstate(over="ignore", invalid="ignore"):
        want_h = exact.astype(np.float16).view(np.uint16)
    assert np.array_equal(got_h[fin], want_h[fin])


def test_threads_do_not_change_results():
    x = synth.normal(80, 300 * 1024).reshape(300, 1024)
    w = synth.normal(81, 1024, 1.0, 0.02)
    orc.set_threads(1)
    a = orc.layer_norm(x, w, None, 1e-5)
    orc.set_threads(7)
    b = orc.layer_norm(x, w, None, 1e-5)
    orc.set_threads(4)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------------------
# Q8_0 quantized linear (dequantize-then-matmul)
# ---------------------------------------------------------------------------

def _dequant_bf16_numpy(blocks, n, k):
    """The bf16 weight the linear uses, decoded with numpy alone: f16 scale,
    int8 values, exact product, RNE to bf16 (torch)."""
    b = np.asarray(blocks, dtype=np.uint8).reshape(n * (k // 32), 34)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)          # [blocks, 1]
    q = b[:, 2:].view(np.int8).astype(np.float32)
    w = (q * d).reshape(n, k)
    return torch.from_numpy(w).to(torch.bfloat16).to(torch.float64).numpy()


def test_q8_0_linear_matches_numpy_f64_matmul():
    m, k, n = 37, 256, 45
    x = orc.bf16_bits(synth.normal(90, m * k).reshape(m, k))
    blocks = synth.q8_0_blocks(91, n * k // 32)
    bias = synth.normal(92, n, 0.0, 0.5)
    y = orc.q8_0_linear(x, blocks, n, bias, orc.F32)
    want = orc.bf16_to_f32(x).astype(np.float64) @ _dequant_bf16_numpy(blocks, n, k).T + bias.astype(np.float64)
    # f64 sums in a different order, then one rounding to f32
    assert np.all(np.abs(y - want) <= 2.0 ** -23 * np.abs(want) + 1e-30)
    yb = orc.q8_0_linear(x, blocks, n, bias, orc.BF16)
    assert np.array_equal(yb, to_bf16_bits(want))


def test_q8_0_linear_identity_weight_and_brute_force():
    # identity weight (d = 1.0, q = 1 on the diagonal) returns x exactly
    k = 64
    blocks = np.zeros((k, k // 32, 34), dtype=np.uint8)
    blocks[:, :, 0], blocks[:, :, 1] = 0x00, 0x3C                    # f16 1.0, little-endian
    for i in range(k):
        blocks[i, i // 32, 2 + i % 32] = 1
    x = orc.bf16_bits(synth.normal(93, 5 * k).reshape(5, k))
    assert np.array_equal(orc.q8_0_linear(x, blocks.reshape(-1), k, None, orc.BF16), x)
    # pure-Python brute force on a tiny case, decoding the bytes by hand
    m, k, n = 2, 32, 3
    x = orc.bf16_bits(synth.normal(94, m * k).reshape(m, k))
    raw = synth.q8_0_blocks(95, n).reshape(n, 34)
    xf = orc.bf16_to_f32(x)
    got = orc.q8_0_linear(x, raw.reshape(-1), n, None, orc.F32)
    for i in range(m):
        for j in range(n):
            d = float(np.frombuffer(bytes(raw[j, 0:2]), dtype="<f2")[0])
            acc = 0.0
            for t in range(k):
                qv = int(raw[j, 2 + t]) - 256 * (raw[j, 2 + t] > 127)
                w = float(torch.tensor(qv * d, dtype=torch.float32).to(torch.bfloat16).item())
                acc += float(xf[i, t]) * w
            assert abs(got[i, j] - acc) <= 2.0 ** -23 * abs(acc) + 1e-30, (i, j)


def test_q8_0_linear_f32_activations():
    """f32 x with the exact f32 weights q * d: against a numpy f64 matmul of
    the dequantized weight decoded independently, an identity weight, and a
    pure-Python brute force on the block bytes."""
    m, k, n = 7, 96, 10
    x = synth.normal(97, m * k).reshape(m, k).astype(np.float32)
    blocks = synth.q8_0_blocks(98, n * k // 32)
    bias = synth.normal(99, n, 0.0, 0.5)
    raw = blocks.reshape(n, k // 32, 34)
    d = raw[:, :, 0:2].copy().view(np.float16).astype(np.float64)          # [n, k/32, 1]
    q = raw[:, :, 2:].view(np.int8).astype(np.float64)                      # [n, k/32, 32]
    w = (q * d).reshape(n, k)
    want = x.astype(np.float64) @ w.T + bias.astype(np.float64)
    got = orc.q8_0_linear(x, blocks, n, bias, orc.F32)
    assert np.all(np.abs(got - want) <= 2.0 ** -24 * np.abs(want) + 1e-30)
    gb = orc.q8_0_linear(x, blocks, n, bias, orc.BF16)
    assert np.array_equal(gb, to_bf16_bits(want))
    # identity weight (d = 1, q = 1 on the diagonal) returns x exactly
    kk = 64
    ident = np.zeros((kk, kk // 32, 34), dtype=np.uint8)
    ident[:, :, 0], ident[:, :, 1] = 0x00, 0x3C
    for i in range(kk):
        ident[i, i // 32, 2 + i % 32] = 1
    xi = synth.normal(100, 3 * kk).reshape(3, kk).astype(np.float32)
    assert np.array_equal(orc.q8_0_linear(xi, ident.reshape(-1), kk, None, orc.F32), xi)
    # brute force
    for i in range(m):
        for j in range(n):
            acc = float(bias[j])
            for t in range(k):
                blk = raw[j, t // 32]
                dd = float(np.frombuffer(bytes(blk[0:2]), dtype="<f2")[0])
                qv = int(blk[2 + t % 32]) - 256 * (blk[2 + t % 32] > 127)
                acc += float(x[i, t]) * (qv * dd)
            assert abs(got[i, j] - acc) <= 2.0 ** -23 * abs(acc) + 1e-30, (i, j)


def _pattern_f32(index):
    """The reference's sparse-attention test inputs (tests/trellis2_sparse.rs:23-25)."""
    return ((np.asarray(index) % 23).astype(np.float32) - np.float32(11.0)) * np.float32(0.1)


def test_sdpa_matches_scipy_softmax_on_reference_test_inputs():
    """The shapes of the reference's naive-attention tests
    (tests/trellis2_sparse.rs:521-623: H=2, T=17 self and T=9 over Tkv=7
    cross, head_dim 8, scale 1/sqrt(8)) with its pattern_f32 inputs, against
    scipy.special.softmax and numpy matmuls in f64."""
    from scipy.special import softmax
    for t, tkv, seeds in [(17, 17, (1, 2, 3)), (9, 7, (4, 5, 6))]:
        h, hd = 2, 8
        q, k, v = (_pattern_f32(np.arange(h * n * hd) * 7 + s * 3).reshape(h, n, hd)
                   for n, s in ((t, seeds[0]), (tkv, seeds[1]), (tkv, seeds[2])))
        scale = 1.0 / np.sqrt(np.float32(hd))
        got = orc.sdpa(q, k, v, float(np.float32(scale)))
        q64, k64, v64 = (a.astype(np.float64) for a in (q, k, v))
        want = softmax(q64 @ k64.transpose(0, 2, 1) * float(np.float32(scale)), axis=-1) @ v64
        assert np.all(np.abs(got - want) <= 2.0 ** -23 * np.abs(want) + 1e-30)


def test_sdpa_closed_forms_and_key_permutation():
    rng = np.random.default_rng(11)
    # identical keys: uniform weights, the output is the mean of the values
    q = rng.standard_normal((3, 5, 16)).astype(np.float32)
    k = np.repeat(rng.standard_normal((3, 1, 16)).astype(np.float32), 9, axis=1)
    v = rng.standard_normal((3, 9, 16)).astype(np.float32)
    got = orc.sdpa(q, k, v, 0.25)
    want = np.broadcast_to(v.astype(np.float64).mean(axis=1, keepdims=True), got.shape)
    assert np.all(np.abs(got - want) <= 2.0 ** -22 * np.abs(want) + 1e-7)
    # one key: the output is that value row for every query
    got = orc.sdpa(q, k[:, :1], v[:, :1], 0.25)
    assert np.array_equal(got, np.broadcast_to(v[:, :1], got.shape))
    # a dominant key (score gap > 200 after scaling) takes all the weight
    k2 = rng.standard_normal((1, 6, 4)).astype(np.float32)
    k2[0, 4] = 100.0
    q2 = np.ones((1, 2, 4), dtype=np.float32)
    v2 = rng.standard_normal((1, 6, 4)).astype(np.float32)
    assert np.array_equal(orc.sdpa(q2, k2, v2, 1.0), np.broadcast_to(v2[:, 4:5], (1, 2, 4)))
    # permuting the (key, value) pairs leaves the output unchanged (up to the
    # order of the f64 sums); a mixed-up transpose or index would not
    perm = rng.permutation(9)
    q3 = rng.standard_normal((2, 7, 16)).astype(np.float32)
    k3 = rng.standard_normal((2, 9, 16)).astype(np.float32)
    v3 = rng.standard_normal((2, 9, 16)).astype(np.float32)
    a = orc.sdpa(q3, k3, v3, 0.3)
    b = orc.sdpa(q3, k3[:, perm], v3[:, perm], 0.3)
    assert np.all(np.abs(a - b) <= 2.0 ** -22 * np.abs(a) + 1e-7)


def test_sdpa_bf16_inputs_round_once():
    rng = np.random.default_rng(12)
    q, k, v = (orc.bf16_bits(rng.standard_normal((2, n, 64))) for n in (33, 70, 70))
    got, wabs = orc.sdpa(q, k, v, 0.125, dt=orc.BF16, with_abs=True)
    from scipy.special import softmax
    q64, k64, v64 = (orc.bf16_to_f32(a).astype(np.float64) for a in (q, k, v))
    p = softmax(q64 @ k64.transpose(0, 2, 1) * 0.125, axis=-1)
    want = p @ v64
    assert np.array_equal(got, to_bf16_bits(want))
    assert np.allclose(wabs, p @ np.abs(v64), rtol=1e-6)


def test_sdpa_f32_bar_rejects_bf16_probabilities():
    """The bar the GPU exact_sdpa_heads path is held to (attention_math.rs:
    244-259: f32 scores, softmax and P v), |err| <= 1e-5 * wabs +
    2^-23 |want| against the oracle's f32 output, at the DINOv3 length (1029
    tokens, D 64, 4 heads): the exact f64 attention passes it everywhere,
    and the same attention with the probabilities rounded to bf16 before
    P v (the exact_query_chunked_sdpa path's rounding) fails it on most
    outputs, so the bar can tell the two arithmetics apart."""
    rng = np.random.default_rng(13)
    q, k, v = (orc.bf16_bits(rng.standard_normal((4, 1029, 64))) for _ in range(3))
    want, wabs = orc.sdpa(q, k, v, 0.125, dt=orc.BF16, out_dt=orc.F32, with_abs=True)
    q64, k64, v64 = (torch.from_numpy(orc.bf16_to_f32(a).astype(np.float64)) for a in (q, k, v))
    s = (q64 @ k64.transpose(1, 2)) * 0.125
    p = torch.exp(s - s.amax(-1, keepdim=True))
    bound = 1e-5 * wabs.astype(np.float64) + 2.0 ** -23 * np.abs(want.astype(np.float64))
    exact = ((p @ v64) / p.sum(-1, keepdim=True)).numpy()
    assert np.all(np.abs(exact - want) <= bound)
    pb = p.to(torch.float32).to(torch.bfloat16).to(torch.float64)
    rounded = ((pb @ v64) / pb.sum(-1, keepdim=True)).numpy()
    assert np.mean(np.abs(rounded - want) > bound) > 0.5


# ---- TRELLIS.2 sparse ops ---------------------------------------------------

def _delta(k):
    return np.array([k // 9 - 1, (k % 9) // 3 - 1, k % 3 - 1])


def _grid_with_holes(res=4):
    """The reference's 4^3 grid skipping every 5th row-major cell
    (tests/trellis2_sparse.rs:72-85)."""
    return np.array([[x, y, z] for x in range(res) for y in range(res) for z in range(res)
                     if (x * res * res + y * res + z) % 5 != 0], dtype=np.int32)


def test_sparse_neighbors_kats_and_brute_force():
    # kernel_offset_delta KATs (tests/trellis2_sparse.rs:50-66) through a pair of voxels
    for k, want in ((0, (-1, -1, -1)), (13, (0, 0, 0)), (26, (1, 1, 1)), (5, (-1, 0, 1))):
        assert tuple(_delta(k)) == want
        if k == 13:
            continue
        c = np.array([[5, 5, 5], [5 + want[0], 5 + want[1], 5 + want[2]]], dtype=np.int32)
        nbr = orc.sparse_neighbors(c)
        assert nbr[0, k] == 1 and nbr[0, 13] == 0 and nbr[1, 26 - k] == 0
        assert (nbr[0] >= 0).sum() == 2
    # CoordMap KAT (tests/trellis2_sparse.rs:67-77)
    nbr = orc.sparse_neighbors(np.array([[0, 0, 0], [1, 0, 3], [7, 2, 5]]))
    assert list(nbr[:, 13]) == [0, 1, 2] and (nbr >= 0).sum() == 3
    # brute force over all pairs on the reference's grid with holes
    coords = _grid_with_holes()
    nbr = orc.sparse_neighbors(coords)
    for i in range(len(coords)):
        for k in range(27):
            hit = np.nonzero((coords == coords[i] + _delta(k)).all(axis=1))[0]
            assert nbr[i, k] == (hit[0] if hit.size else -1), (i, k)
    # a later duplicate overwrites (HashMap::insert)
    nbr = orc.sparse_neighbors(np.array([[2, 2, 2], [2, 2, 2]]))
    assert list(nbr[:, 13]) == [1, 1]


def _pattern(idx):
    return ((np.asarray(idx) % 23).astype(np.float32) - np.float32(11.0)) * np.float32(0.1)


def _dense_conv_torch(coords, x, w27, bias, res):
    """F.conv3d (padding 1) in f64 on the densified grid, read at the active sites."""
    import torch.nn.functional as F
    cin, cout = x.shape[1], w27.shape[1]
    dense = torch.zeros((1, cin, res, res, res), dtype=torch.float64)
    for i, (a, b, c) in enumerate(coords):
        dense[0, :, a, b, c] = torch.from_numpy(x[i].astype(np.float64))
    wt = torch.from_numpy(w27.astype(np.float64)).reshape(3, 3, 3, cout, cin).permute(3, 4, 0, 1, 2)
    bt = None if bias is None else torch.from_numpy(bias.astype(np.float64))
    y = F.conv3d(dense, wt, bt, padding=1)[0]
    return np.stack([y[:, a, b, c].numpy() for a, b, c in coords])


def test_sparse_conv3d_matches_dense_conv3d():
    # the reference's parity case (tests/trellis2_sparse.rs:67-162): 3 -> 5 channels
    coords = _grid_with_holes()
    cin, cout = 3, 5
    x = np.array([[_pattern(i * 13 + c * 7) for c in range(cin)] for i in range(len(coords))], dtype=np.float32)
    w27 = np.zeros((27, cout, cin), dtype=np.float32)
    for o in range(cout):
        for k in range(27):
            for c in range(cin):
                w27[k, o, c] = _pattern(o * 31 + k * 5 + c * 3) * np.float32(0.5)
    bias = np.array([((o * 3) % 7) * 0.02 - 0.06 for o in range(cout)], dtype=np.float32)
    got = orc.sparse_conv3d(x, orc.sparse_neighbors(coords), w27, bias)
    want = _dense_conv_torch(coords, x, w27, bias, 4)
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()
    # a larger random case
    rng = np.random.default_rng(4)
    res = 8
    cells = rng.choice(res ** 3, 200, replace=False)
    coords = np.stack([cells // 64, (cells // 8) % 8, cells % 8], axis=1).astype(np.int32)
    x = rng.standard_normal((200, 16)).astype(np.float32)
    w27 = rng.standard_normal((27, 8, 16)).astype(np.float32)
    got = orc.sparse_conv3d(x, orc.sparse_neighbors(coords), w27, None)
    want = _dense_conv_torch(coords, x, w27, None, res)
    assert np.all(np.abs(got - want) <= 2.0 ** -23 * np.abs(want) + 1e-12)


def test_sparse_conv3d_identity_and_shift_kernels():
    """tests/trellis2_sparse.rs:164-237: the centre tap as identity returns x;
    the +x tap (k = 22) returns the +x neighbour's features or zero."""
    coords = np.array([[0, 0, 0], [1, 0, 0], [1, 1, 0], [3, 0, 0]], dtype=np.int32)
    x = _pattern(np.arange(8)).reshape(4, 2)
    nbr = orc.sparse_neighbors(coords)
    w = np.zeros((27, 2, 2), dtype=np.float32)
    w[13] = np.eye(2)
    assert np.array_equal(orc.sparse_conv3d(x, nbr, w), x)
    w = np.zeros((27, 2, 2), dtype=np.float32)
    w[22] = np.eye(2)
    want = np.stack([x[1], np.zeros(2), np.zeros(2), np.zeros(2)]).astype(np.float32)
    assert np.array_equal(orc.sparse_conv3d(x, nbr, w), want)


def test_channel_to_spatial_kat_and_round_trip():
    # tests/trellis2_sparse.rs:274-318
    coords = np.array([[0, 0, 0], [1, 0, 0], [0, 1, 1]], dtype=np.int32)
    feats = (np.arange(48, dtype=np.float32) / 10.0).reshape(3, 16)
    logits = -np.ones((3, 8), dtype=np.float32)
    logits[0, [0, 3, 5]] = 1.0
    logits[1, 1] = 1.0
    oc, of, src, sub = orc.channel_to_spatial(coords, feats, logits)
    assert oc.tolist() == [[0, 0, 0], [1, 1, 0], [1, 0, 1], [3, 0, 0]]
    flat = feats.reshape(24, 2)
    assert np.array_equal(of, flat[[0, 3, 5, 9]]) and src.tolist() == [0, 3, 5, 9]
    assert sub[0, 0] == 1 and sub[0, 1] == 0 and sub.reshape(-1)[9] == 1 and sub.size == 24
    # S2C (numpy, trellis2_sparse.rs:365-412) then C2S with the occupancy as logits returns the input
    rng = np.random.default_rng(9)
    cells = rng.choice(8 ** 3, 60, replace=False)
    child = np.stack([cells // 64, (cells // 8) % 8, cells % 8], axis=1).astype(np.int32)
    cf = rng.standard_normal((60, 4)).astype(np.float32)
    parents = sorted({tuple(c // 2) for c in child})
    pidx = {p: i for i, p in enumerate(parents)}
    s2c = np.zeros((len(parents), 8 * 4), dtype=np.float32)
    occ = -np.ones((len(parents), 8), dtype=np.float32)
    for i, c in enumerate(child):
        p, s = pidx[tuple(c // 2)], int(c[0] % 2 + 2 * (c[1] % 2) + 4 * (c[2] % 2))
        s2c[p, s * 4:(s + 1) * 4] = cf[i]
        occ[p, s] = 1.0
    oc, of, _, _ = orc.channel_to_spatial(np.array(parents, dtype=np.int32), s2c, occ)
    order = np.lexsort((child[:, 2], child[:, 1], child[:, 0]))
    got = {tuple(c): tuple(f) for c, f in zip(oc, of)}
    assert len(got) == 60 and all(got[tuple(child[i])] == tuple(cf[i]) for i in order)
