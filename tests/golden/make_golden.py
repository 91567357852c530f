"""Writes the golden fixtures of tests/golden/*.npz.

Each fixture holds seeded inputs (the reference's LCG, lux3d_fused.synth)
and expected outputs computed in float64 with torch / numpy straight from the
mathematical definitions of the reference ops, independently of the C oracle
and of the HIP kernels. Both are checked against these files:
  tests/test_golden.py      (oracle, CPU)
  tests/test_gpu_golden.py  (liblux3d_fused, GPU)
Expected values are stored in float64; bf16 inputs are stored as the f32
values they decode to (each exactly representable in bf16).

Run:  python tests/golden/make_golden.py
"""
import math
import os
import sys

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "candle-3d_amd"))
from lux3d_fused import synth  # noqa: E402


def bf16_round(a):
    """f32 values -> nearest bf16 values (RNE), returned as f32."""
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)
    return t.to(torch.float32).numpy()


def t64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


def save(name, **arrays):
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
    print(name, {k: v.shape for k, v in arrays.items()})


def layer_norm():
    # configs[0]-like row LN (f32) and a bf16 variant, eps 1e-6 / 1e-5
    x = synth.normal(synth.config_seed(0) + 900, 16 * 1024).reshape(16, 1024)
    w = synth.normal(901, 1024, 1.0, 0.02)
    b = synth.normal(902, 1024, 0.0, 0.02)
    y = F.layer_norm(t64(x), (1024,), t64(w), t64(b), eps=1e-6).numpy()
    xb = bf16_round(synth.normal(903, 12 * 2048).reshape(12, 2048))
    yb = F.layer_norm(t64(xb), (2048,), eps=1e-5).numpy()
    save("layer_norm", x=x, w=w, b=b, y=y, eps=np.float64(1e-6), x_bf16=xb, y_bf16_noaffine=yb,
         eps_bf16=np.float64(1e-5))


def residual_layer_norm():
    # F1: h = x + a*gamma (two f32 roundings); y = LN(h)
    shape = (2, 5, 1024)
    x = bf16_round(synth.normal(910, 10 * 1024).reshape(shape))
    a = bf16_round(synth.normal(911, 10 * 1024).reshape(shape))
    g = synth.normal(912, 1024, 1.0, 0.02)
    w = synth.normal(913, 1024, 1.0, 0.02)
    b = synth.normal(914, 1024, 0.0, 0.02)
    h32 = (x + (a * g).astype(np.float32)).astype(np.float32)   # the reference rounds the product, then the sum
    h = bf16_round(h32)                                          # stored residual stream (bf16)
    y = F.layer_norm(t64(h), (1024,), t64(w), t64(b), eps=1e-5).numpy()
    save("residual_layer_norm", x=x, a=a, gamma=g, w=w, b=b, h=h, y=y, eps=np.float64(1e-5))


def adaln_ragged():
    # ragged 2-segment AdaLN modulate with the `modulation + t_emb` add, and the gate
    C = 256
    sizes = (7, 13)
    n = sum(sizes)
    x = bf16_round(synth.normal(920, n * C).reshape(n, C))
    t_emb = synth.normal(921, 2 * 6 * C, 0.0, 0.1).reshape(2, 6 * C)
    mod = synth.normal(922, 6 * C, 0.0, 0.1)
    offs = np.array([0, sizes[0], n], dtype=np.int64)
    h = bf16_round(synth.normal(923, n * C).reshape(n, C))
    nrm = F.layer_norm(t64(x), (C,), eps=1e-6)
    y = torch.empty_like(nrm)
    yg = torch.empty_like(nrm)
    gres = torch.empty_like(nrm)
    for s in range(2):
        r0, r1 = offs[s], offs[s + 1]
        mv = t64(mod) + t64(t_emb[s])
        sh, sc, gt = mv[0:C], mv[C:2 * C], mv[2 * C:3 * C]
        y[r0:r1] = nrm[r0:r1] * (1.0 + sc) + sh
        yg[r0:r1] = gt * y[r0:r1] + t64(x[r0:r1])
        gres[r0:r1] = t64(x[r0:r1]) + t64(h[r0:r1]) * gt
    save("adaln_ragged", x=x, h=h, t_emb=t_emb, modulation=mod, offsets=offs, y=y.numpy(), y_gate=yg.numpy(),
         gated_residual=gres.numpy())


def rms_norm_heads():
    B, L, H, D = 2, 9, 4, 128
    qkv = bf16_round(synth.normal(930, B * L * H * 3 * D).reshape(B, L, H, 3 * D))
    w = synth.normal(931, D, 1.0, 0.02)
    q = t64(qkv[..., 0:D]).transpose(1, 2)                       # [B, H, L, D]
    y = q / torch.sqrt((q * q).mean(-1, keepdim=True) + 1e-6) * t64(w)
    save("rms_norm_heads", qkv=qkv, w=w, y=y.numpy())


def rope2d_vggt():
    # QK LayerNorm + VGGT 2D RoPE on a [1, 3, 5 + 3*4, 64] head view; angles
    # from the frequency law 100^(-2k/32) in float64, positions (y+1, x+1)
    B, H, D, ph, pw = 1, 3, 64, 3, 4
    pos = synth.vggt_positions(B, ph, pw)
    N = pos.shape[1]
    q = bf16_round(synth.normal(940, B * H * N * D).reshape(B, H, N, D))
    w = synth.normal(941, D, 1.0, 0.05)
    b = synth.normal(942, D, 0.0, 0.05)
    n = F.layer_norm(t64(q), (D,), t64(w), t64(b), eps=1e-5).numpy()
    out = np.empty_like(n)
    inv = 100.0 ** (-2.0 * np.arange(16) / 32.0)
    for t in range(N):
        for axis in range(2):
            ang = pos[0, t, axis] * inv                         # 16 angles for this half
            c, s = np.cos(ang), np.sin(ang)
            lo = n[0, :, t, axis * 32: axis * 32 + 16]
            hi = n[0, :, t, axis * 32 + 16: axis * 32 + 32]
            out[0, :, t, axis * 32: axis * 32 + 16] = lo * c - hi * s   # rotate-half per half
            out[0, :, t, axis * 32 + 16: axis * 32 + 32] = hi * c + lo * s
    save("rope2d_vggt", q=q, w=w, b=b, positions=pos, y=out, eps=np.float64(1e-5), base=np.float64(100.0))


def rope3d_trellis():
    # L2 q/k norm + 3D RoPE from voxel coords: 21 freqs/axis 1e4^(-i/21),
    # interleaved (re, im) pairs, pad pair 63 unrotated
    L, H, D = 11, 2, 128
    coords = synth.unique_voxels(950, L, 64)
    x = bf16_round(synth.normal(951, L * H * D).reshape(1, L, H, D))
    g = synth.normal(952, H * D, 1.0, 0.05).reshape(H, D)
    xn = F.normalize(t64(x), dim=-1) * t64(g) * math.sqrt(D)
    xn = xn.numpy()
    f = 10000.0 ** (-np.arange(21) / 21.0)
    ang = np.zeros((L, 64))
    for a in range(3):
        ang[:, a * 21:(a + 1) * 21] = coords[:, a:a + 1] * f[None, :]
    z = xn[..., 0::2] + 1j * xn[..., 1::2]
    z = z * np.exp(1j * ang)[None, :, None, :]
    out = np.empty_like(xn)
    out[..., 0::2] = z.real
    out[..., 1::2] = z.imag
    save("rope3d_trellis", x=x, gamma=g, coords=coords, y=out, cos=np.cos(ang), sin=np.sin(ang),
         base=np.float64(10000.0))


def rope2d_dinov3():
    # DINOv3: 5 prefix tokens untouched, patch centres on a 2x3 grid
    B, H, D, gh, gw = 1, 2, 64, 2, 3
    S = 5 + gh * gw
    x = synth.normal(960, B * H * S * D).reshape(B, H, S, D)
    inv = 1.0 / 100.0 ** (np.arange(16) * 4.0 / 64.0)
    cos = np.empty((gh * gw, D))
    sin = np.empty((gh * gw, D))
    for yy in range(gh):
        for xx in range(gw):
            cy = 2.0 * ((yy + 0.5) / gh) - 1.0
            cx = 2.0 * ((xx + 0.5) / gw) - 1.0
            half = np.concatenate([2 * math.pi * cy * inv, 2 * math.pi * cx * inv])
            ang = np.concatenate([half, half])
            cos[yy * gw + xx] = np.cos(ang)
            sin[yy * gw + xx] = np.sin(ang)
    out = x.astype(np.float64).copy()
    p = x[:, :, 5:].astype(np.float64)
    rh = np.concatenate([-p[..., 32:], p[..., :32]], axis=-1)
    out[:, :, 5:] = p * cos + rh * sin
    save("rope2d_dinov3", x=x, cos=cos.astype(np.float32), sin=sin.astype(np.float32), y=out,
         cos64=cos, sin64=sin, grid=np.array([gh, gw]))


def activations():
    x = np.concatenate([synth.normal(970, 4096) * np.float32(3.0),
                        np.array([0.0, -0.0, 1e-3, -1e-3, 4.0, -4.0, 8.0, -8.0], np.float32)])
    xd = t64(x)
    save("activations", x=x, gelu_erf=F.gelu(xd).numpy(), gelu_tanh=F.gelu(xd, approximate="tanh").numpy(),
         silu=F.silu(xd).numpy())


def timestep():
    # The reference's f32 steps (trellis2_blocks.rs:189-203, triposg_dit.rs:286-297):
    # arg = f32(f32(-ln(1e4) * i) / half); freq = exp(arg) rounded once to f32
    # (f64 exp: the correctly rounded expf); angle = f32(t * freq). sin / cos of
    # that angle in f64. t = 500 with dim 4 is the reference's KAT input
    # (tests/trellis2_blocks.rs:157-171).
    t = np.concatenate([np.array([0.0, 0.5, 1.0, 500.0], np.float32), synth.uniform(980, 4, 0.0, 1000.0)])
    out = {}
    for dim in (4, 256, 2048):
        half = dim // 2
        nlp = np.float32(-math.log(10000.0))
        arg = (nlp * np.arange(half, dtype=np.float32)) / np.float32(half)
        freq = np.exp(arg.astype(np.float64)).astype(np.float32)
        ang = (t[:, None] * freq[None, :]).astype(np.float64)
        out[f"freqs_{dim}"] = freq
        out[f"cos_first_{dim}"] = np.concatenate([np.cos(ang), np.sin(ang)], axis=1)
        out[f"sin_first_{dim}"] = np.concatenate([np.sin(ang), np.cos(ang)], axis=1)
    save("timestep", t=t, **out)


def q8_0():
    blocks = synth.q8_0_blocks(990, 24)
    b = blocks.reshape(24, 34)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(24, 1)
    q = b[:, 2:].view(np.int8).astype(np.float64)
    save("q8_0", blocks=blocks, y=(q * d).reshape(-1))


if __name__ == "__main__":
    layer_norm()
    residual_layer_norm()
    adaln_ragged()
    rms_norm_heads()
    rope2d_vggt()
    rope3d_trellis()
    rope2d_dinov3()
    activations()
    timestep()
    q8_0()
