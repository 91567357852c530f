"""GPU parity of the head family at head dims other than 64 / 128 and on
unaligned views (the generic head kernel), plus the reference's own
known-answer tests, which use head dims 4, 6 and 12
(tests/trellis2_blocks.rs:43-171), run through the HIP path.

Tolerances as in test_gpu_parity.py (conftest.py).
"""
import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from conftest import assert_bf16_close, assert_f16_close, assert_f32_close  # noqa: E402


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def ops(dev):
    from lux3d_fused import ops as _ops
    return _ops


@pytest.fixture(scope="module")
def orc():
    import lux3d_oracle as o
    o.set_threads(16)
    return o


@pytest.fixture(scope="module")
def synth():
    from lux3d_fused import synth as s
    return s


TDT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def to_dev(a, dev, dt="f32"):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev).to(TDT[dt])


def host(t, dt):
    """f32 -> numpy f32; bf16 -> uint16 bits; f16 -> numpy float16 (the oracle's encodings)."""
    t = t.detach().contiguous().cpu()
    if dt == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def check(got, want, dt, what):
    g = host(got, dt)
    if dt == "f32":
        assert_f32_close(g, want, what=what)
    elif dt == "bf16":
        assert_bf16_close(g, want, what=what)
    else:
        assert_f16_close(g.view(np.uint16), np.asarray(want).view(np.uint16), what=what)


def odt(orc, dt):
    return {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}[dt]


def misaligned(t):
    """The same values in a view that starts 1 element into a fresh buffer
    (2 or 4 bytes off 16-byte alignment)."""
    flat = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    v = flat[1:].view(t.shape)
    v.copy_(t)
    return v


@pytest.mark.parametrize("dt,D,source", [("bf16", 12, "tables"), ("bf16", 12, "positions"), ("f32", 32, "tables"),
                                         ("bf16", 96, "positions"), ("f32", 96, "positions"),
                                         ("f16", 64, "positions"), ("f16", 64, "tables"), ("f16", 12, "positions")])
def test_qk_layernorm_rope2d_any_dim(dev, ops, orc, synth, dt, D, source):
    print(f"\n[case] qk_layernorm_rope2d D={D} dt={dt} source={source}", flush=True)
    B, H, ph, pw = 2, 3, 4, 5
    pos = synth.vggt_positions(B, ph, pw)
    N = pos.shape[1]
    qkv = synth.normal(201, B * N * 3 * H * D).reshape(B, N, 3, H, D)
    perm = to_dev(qkv, dev, dt).permute(2, 0, 3, 1, 4)
    q, k = perm[0], perm[1]
    w, b = synth.normal(202, D, 1.0, 0.05), synth.normal(203, D, 0.0, 0.05)
    T = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    cos, sin = orc.rope2d_tables(pos, D, 100.0)
    if source == "tables":
        emb = ops.Rope2d(100.0).embeddings(T(pos), D)
        qo, ko = ops.qk_layernorm_rope2d(q, k, (T(w), T(b), 1e-5), (T(w), T(b), 1e-5), emb)
    else:
        qo, ko = ops.qk_layernorm_rope2d(q, k, (T(w), T(b), 1e-5), (T(w), T(b), 1e-5), positions=T(pos), base=100.0)
    torch.cuda.synchronize()
    for got, src, what in ((qo, q, "q"), (ko, k, "k")):
        want = orc.layernorm_rope2d(np.ascontiguousarray(host(src, dt)), w, b, 1e-5, cos, sin, dt=odt(orc, dt))
        check(got, want, dt, what)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_head_kernels_on_unaligned_views(dev, ops, orc, synth, dt):
    """D = 64 / 128 views that are not 16-byte aligned take the generic kernel."""
    print(f"\n[case] unaligned head views dt={dt}", flush=True)
    T = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    # VGGT QK LN + RoPE, D = 64
    B, H, ph, pw, D = 1, 4, 6, 6, 64
    pos = synth.vggt_positions(B, ph, pw)
    N = pos.shape[1]
    q = misaligned(to_dev(synth.normal(211, B * H * N * D).reshape(B, H, N, D), dev, dt))
    w, b = synth.normal(212, D, 1.0, 0.05), synth.normal(213, D, 0.0, 0.05)
    cos, sin = orc.rope2d_tables(pos, D, 100.0)
    qo, _ = ops.qk_layernorm_rope2d(q, q, (T(w), T(b), 1e-5), (T(w), T(b), 1e-5), positions=T(pos), base=100.0)
    # TRELLIS.2 L2 + 3D RoPE, D = 128
    L, H3, D3 = 50, 2, 128
    coords = synth.unique_voxels(214, L, 64)
    x = misaligned(to_dev(synth.normal(215, L * H3 * D3).reshape(1, L, H3, D3), dev, dt))
    g = synth.normal(216, H3 * D3, 1.0, 0.05).reshape(H3, D3)
    xo, _ = ops.qk_l2norm_rope3d(x, x, T(g), T(g), coords=T(coords))
    # TripoSG RMS, D = 128
    r = misaligned(to_dev(synth.normal(217, 2 * 3 * 20 * 128).reshape(2, 3, 20, 128), dev, dt))
    rw = synth.normal(218, 128, 1.0, 0.05)
    ro = ops.rms_norm_heads(r, T(rw), 1e-6)
    torch.cuda.synchronize()
    check(qo, orc.layernorm_rope2d(np.ascontiguousarray(host(q, dt)), w, b, 1e-5, cos, sin, dt=odt(orc, dt)), dt,
          "unaligned QK LN + RoPE")
    c3, s3 = orc.rope3d_tables(coords, D3)
    check(xo, orc.qk_l2norm_rope3d(np.ascontiguousarray(host(x, dt)).reshape(L, H3, D3), g, c3, s3,
                                   dt=odt(orc, dt)).reshape(1, L, H3, D3), dt, "unaligned L2 + RoPE3d")
    check(ro, orc.rms_norm_heads(np.ascontiguousarray(host(r, dt)), rw, 1e-6, dt=odt(orc, dt)), dt, "unaligned RMS")


@pytest.mark.parametrize("dt,D", [("bf16", 4), ("bf16", 96), ("bf16", 130), ("f16", 128), ("f16", 96)])
def test_rms_norm_heads_any_dim(dev, ops, orc, synth, dt, D):
    print(f"\n[case] rms_norm_heads D={D} dt={dt}", flush=True)
    B, L, H = 2, 33, 5
    qkv = to_dev(synth.normal(221, B * L * H * 3 * D).reshape(B, L, H, 3 * D), dev, dt)
    q, k = qkv[..., :D].transpose(1, 2), qkv[..., D:2 * D].transpose(1, 2)
    wq, wk = synth.normal(222, D, 1.0, 0.05), synth.normal(223, D, 1.0, 0.05)
    T = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    qo, ko = ops.rms_norm_heads(q, T(wq), 1e-6, k=k, k_weight=T(wk))
    torch.cuda.synchronize()
    check(qo, orc.rms_norm_heads(np.ascontiguousarray(host(q, dt)), wq, 1e-6, dt=odt(orc, dt)), dt, "q")
    check(ko, orc.rms_norm_heads(np.ascontiguousarray(host(k, dt)), wk, 1e-6, dt=odt(orc, dt)), dt, "k")


@pytest.mark.parametrize("dt,D,source", [("f32", 6, "coords"), ("f32", 12, "coords"), ("f32", 12, "tables"),
                                         ("f32", 36, "coords"), ("f16", 128, "coords"), ("f16", 12, "tables")])
def test_qk_l2norm_rope3d_any_dim(dev, ops, orc, synth, dt, D, source):
    print(f"\n[case] qk_l2norm_rope3d D={D} dt={dt} source={source}", flush=True)
    L, H = 40, 2
    coords = synth.unique_voxels(231, L, 64)
    qkv = to_dev(synth.normal(232, L * 3 * H * D).reshape(1, L, 3, H, D), dev, dt)
    q, k = qkv[:, :, 0], qkv[:, :, 1]
    gq = synth.normal(233, H * D, 1.0, 0.05).reshape(H, D)
    T = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    cos, sin = orc.rope3d_tables(coords, D)
    if source == "coords":
        qo, ko = ops.qk_l2norm_rope3d(q, k, T(gq), T(gq), coords=T(coords))
    else:
        qo, ko = ops.qk_l2norm_rope3d(q, k, T(gq), T(gq), cos=T(cos), sin=T(sin))
    torch.cuda.synchronize()
    for got, src, what in ((qo, q, "q"), (ko, k, "k")):
        want = orc.qk_l2norm_rope3d(np.ascontiguousarray(host(src, dt)).reshape(L, H, D), gq, cos, sin, dt=odt(orc, dt))
        check(got, want.reshape(1, L, H, D), dt, what)


@pytest.mark.parametrize("dt,D", [("f32", 32), ("f32", 48), ("f16", 64), ("f16", 32)])
def test_dinov3_rope_any_dim(dev, ops, orc, synth, dt, D):
    print(f"\n[case] dinov3 rope D={D} dt={dt}", flush=True)
    B, H, grid = 1, 3, 4
    S = 5 + grid * grid
    cos, sin = orc.dinov3_rope_tables(grid, grid, D)
    x = to_dev(synth.normal(241, B * H * S * D).reshape(B, H, S, D), dev, dt)
    T = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    qo, _ = ops.apply_rotary_to_patches(x, x, T(cos), T(sin), 5)
    torch.cuda.synchronize()
    check(qo, orc.dinov3_rope_apply(np.ascontiguousarray(host(x, dt)), 5, cos, sin, dt=odt(orc, dt)), dt, "q")


# ---------------------------------------------------------------------------
# The reference's known-answer tests (tests/trellis2_blocks.rs), on the GPU
# ---------------------------------------------------------------------------

def test_kat_rope_tables_head_dim_12(dev, ops):
    """rope_tables_match_reference_formula (tests/trellis2_blocks.rs:43-74):
    head_dim 12 -> 2 freqs per axis [1, 10000^-0.5], axis-major angles."""
    coords = torch.tensor([[1, 0, 0], [0, 1, 0]], dtype=torch.int32, device=dev)
    cos, sin = ops.Trellis2Rope3d(12).cos_sin(coords)
    cos, sin = cos.cpu().numpy(), sin.cpu().numpy()
    assert cos.shape == (2, 6)
    freq2 = np.float32(1.0) / np.float32(10000.0) ** np.float32(0.5)
    for t, c in enumerate(([1, 0, 0], [0, 1, 0])):
        angles = [c[0] * 1.0, c[0] * freq2, c[1] * 1.0, c[1] * freq2, c[2] * 1.0, c[2] * freq2]
        for j, a in enumerate(angles):
            assert abs(cos[t][j] - math.cos(a)) < 1e-6, (t, j)
            assert abs(sin[t][j] - math.sin(a)) < 1e-6, (t, j)


def test_kat_rope_apply_complex_product(dev, ops):
    """rope_apply_matches_complex_product_and_preserves_norm (:79-111)."""
    rope = ops.Trellis2Rope3d(12)
    cos, sin = rope.cos_sin(torch.tensor([[1, 0, 0]], dtype=torch.int32, device=dev))
    x = [1.0, 0.0, 2.0, 3.0, 5.0, 0.0, 7.0, 1.0, 0.0, 2.0, 4.0, 4.0]
    xs = torch.tensor(x, dtype=torch.float32, device=dev).reshape(1, 1, 1, 12)
    out = rope.apply(xs, cos, sin).reshape(-1).cpu().numpy()
    freq2 = 1.0 / 10000.0 ** 0.5
    phases = [(1.0, 1.0), (freq2, freq2), (0.0, 0.0)]
    for pair in range(6):
        ac, as_ = (math.cos(phases[pair][0]), math.sin(phases[pair][1])) if pair < 2 else (1.0, 0.0)
        re, im = x[2 * pair], x[2 * pair + 1]
        assert abs(out[2 * pair] - (re * ac - im * as_)) < 1e-5, pair
        assert abs(out[2 * pair + 1] - (re * as_ + im * ac)) < 1e-5, pair
    e_in = sum(x[2 * i] ** 2 + x[2 * i + 1] ** 2 for i in range(6))
    e_out = float(np.sum(out.astype(np.float64) ** 2))
    assert abs(e_in - e_out) < 1e-4


def test_kat_qk_rms_norm(dev, ops):
    """qk_rms_norm_matches_reference (:126-153): [3, 4, 0, 0] -> [1.2, 1.6, 0, 0],
    gamma 2 -> [2.4, 3.2, 0, 0]."""
    xs = torch.tensor([3.0, 4.0, 0.0, 0.0], device=dev).reshape(1, 1, 1, 4)
    for g, want in ((1.0, [1.2, 1.6, 0.0, 0.0]), (2.0, [2.4, 3.2, 0.0, 0.0])):
        gamma = torch.full((1, 4), g, device=dev)
        out = ops.Trellis2QkRmsNorm(gamma).forward(xs).reshape(-1).cpu().numpy()
        assert np.all(np.abs(out - np.array(want, dtype=np.float32)) < 1e-6), out


def test_kat_timestep_embedding(dev, ops):
    """timestep_embedding_matches_reference (:157-171): t = 500, dim 4."""
    t = torch.tensor([500.0], device=dev)
    out = ops.timestep_embedding(t, 4, cos_first=True).reshape(-1).cpu().numpy()
    f1 = np.float32(math.exp(-math.log(10000.0) / 2.0))
    want = [math.cos(500.0), math.cos(np.float32(500.0) * f1), math.sin(500.0), math.sin(np.float32(500.0) * f1)]
    assert np.all(np.abs(out - np.array(want, dtype=np.float32)) < 1e-5), out


@pytest.mark.parametrize("D", [64, 128])
def test_head_kernel_64bit_offsets_match_32bit(dev, ops, D):
    """The vector head kernel forms its offsets in 32 bits (24-bit products)
    when every byte offset of the views is below 2^31 and every stride of an
    axis longer than 1 below 2^24, else in 64 bits. A batch stride of
    2^24 + 64 elements takes the 64-bit instance; its q and k equal, bit for
    bit, the same rows normalised from compact tensors (32-bit instance)."""
    B, H, L = 2, 4, 40
    sb = (1 << 24) + 64
    print(f"\n[case] head kernel 64-bit offsets D={D} batch stride {sb}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(11 + D)
    q = torch.randn(B, H, L, D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(B, H, L, D, generator=g).to(torch.bfloat16).to(dev)
    wq = (torch.rand(D, generator=g) + 0.5).to(dev)
    wk = (torch.rand(D, generator=g) + 0.5).to(dev)
    bq = torch.zeros(sb * B, dtype=torch.bfloat16, device=dev)
    bk = torch.zeros(sb * B, dtype=torch.bfloat16, device=dev)
    qv = bq.as_strided((B, H, L, D), (sb, L * D, D, 1))
    kv = bk.as_strided((B, H, L, D), (sb, L * D, D, 1))
    qv.copy_(q)
    kv.copy_(k)
    got_q, got_k = ops.rms_norm_heads(qv, wq, 1e-6, k=kv, k_weight=wk)
    want_q, want_k = ops.rms_norm_heads(q, wq, 1e-6, k=k, k_weight=wk)
    torch.cuda.synchronize()
    assert torch.equal(got_q, want_q) and torch.equal(got_k, want_k)
