"""GPU parity of the attention entries that apply q's head norm / rotation in
the attention kernel's Q load:

- lux3d_sdpa_rms_norm_heads (TripoSG, triposg_dit.rs:446-455),
- lux3d_sdpa_l2norm_rope3d (TRELLIS.2, trellis2_blocks.rs:417-436),
- lux3d_sdpa_dinov3_rope (DINOv3, trellis2_dino.rs:385-393).

Each fused result must equal, bit for bit, the two launches it replaces (the
head op, whose own parity is pinned in test_gpu_parity.py, followed by
lux3d_sdpa or lux3d_sdpa_heads_f32), at the configuration shapes and on the
fallback layouts (where the entry runs those two launches itself). A small
case of each is also checked end to end against the oracle's head op
followed by its double-precision attention, with the attention bound of
test_gpu_attention.py plus the head op's own tolerance on q.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TDT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
ULP = {"bf16": 2.0 ** -7, "f16": 2.0 ** -10, "f32": 2.0 ** -23}


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


def _print_case(**kw):
    print("\n[case] " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def host(t, dt):
    t = t.detach().contiguous().cpu()
    if dt == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def to_f64(a, dt):
    if dt == "bf16":
        return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return np.asarray(a).astype(np.float64)


def odt(orc, dt):
    return {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}[dt]


def assert_end_to_end(orc, got, q_oracle, k, v, scale, dt, exact_heads=False):
    """got against the oracle's attention over the oracle's normalised q: the
    matrix-core bound of test_gpu_attention.py, widened by 2 output ulp for
    the head op's own tolerance on q (and f32 probabilities for
    exact_sdpa_heads)."""
    want, wabs = orc.sdpa(q_oracle, host(k, dt), host(v, dt), scale, dt=odt(orc, dt), with_abs=True)
    g, w = to_f64(host(got, dt), dt), to_f64(want, dt)
    u = ULP[dt] if not (exact_heads and dt == "f32") else 2.0 ** -20
    bound = 2 * u * np.abs(w) + (4 * u + 1e-6) * wabs.astype(np.float64) + 1e-6
    err = np.abs(g - w)
    assert np.all(err <= bound), f"worst err {err.max():.3e}"


def _thirds(dev, b, n, h, d, dt, seed):
    """q, k, v as TripoSGAttnProcessor's per-head thirds of cat([q, k, v])
    reshaped to [B, L, H, 3D] (triposg_dit.rs:438-452), each transposed to a
    [B, H, L, D] view (no contiguous copy)."""
    w = d
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = (torch.randn((b, n, h, 3 * w), generator=g) * 1.5 + 0.25).to(dev).to(TDT[dt])
    return (x[..., w - d:w].transpose(1, 2), x[..., w:w + d].transpose(1, 2), x[..., 2 * w:2 * w + d].transpose(1, 2))


# ---------------------------------------------------------------------------
# TripoSG: per-head RMSNorm
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("b,n,h,d,dt,case", [
    (2, 2048, 16, 128, "bf16", "fused"),        # configs[2]: TripoSG DiT self-attention, CFG pair
    (1, 300, 4, 64, "f16", "fused"),
    (1, 129, 2, 128, "bf16", "bf16_weight"),
    (1, 200, 2, 128, "bf16", "unaligned_weight"),  # runs the two launches
    (1, 100, 2, 128, "f32", "fused"),             # f32: the two launches
])
def test_sdpa_rms_norm_heads_equals_the_two_launches(dev, ops, b, n, h, d, dt, case):
    _print_case(op="sdpa_rms_norm_heads", b=b, n=n, h=h, d=d, dt=dt, case=case)
    q, k, v = _thirds(dev, b, n, h, d, dt, seed=n + d)
    g = torch.Generator(device="cpu").manual_seed(5)
    w = (1 + 0.1 * torch.randn(d + 1, generator=g)).to(dev)
    qw = w[1:] if case == "unaligned_weight" else w[:d]
    if case == "bf16_weight":
        qw = qw.to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(d, generator=g)).to(dev)
    k_n = ops.rms_norm_heads(k, kw, 1e-6)
    scale = 1.0 / np.sqrt(d)
    fused = ops.sdpa_rms_norm_heads(q, qw, 1e-6, k_n, v, scale)
    two = ops.sdpa(ops.rms_norm_heads(q, qw, 1e-6), k_n, v, scale)
    torch.cuda.synchronize()
    assert torch.isfinite(fused.float()).all()
    assert torch.equal(fused, two)


def test_sdpa_rms_norm_heads_against_oracle(dev, ops, orc):
    b, n, h, d, dt = 1, 333, 2, 128, "bf16"
    _print_case(op="sdpa_rms_norm_heads oracle", b=b, n=n, h=h, d=d)
    q, k, v = _thirds(dev, b, n, h, d, dt, seed=11)
    qw = (1 + 0.1 * torch.randn(d, generator=torch.Generator().manual_seed(3))).to(dev)
    scale = 1.0 / np.sqrt(d)
    fused = ops.sdpa_rms_norm_heads(q, qw, 1e-6, k, v, scale)
    torch.cuda.synchronize()
    qo = orc.rms_norm_heads(host(q, dt), qw.cpu().numpy(), 1e-6, dt=orc.BF16)
    assert_end_to_end(orc, fused, qo, k, v, scale, dt)


# ---------------------------------------------------------------------------
# TRELLIS.2: L2 norm + 3D RoPE
# ---------------------------------------------------------------------------

def _trellis_case(dev, ops, b, n, h, d, dt, seed, tables_dt=torch.float32):
    """q, k, v [B, L, H, D] (Trellis2SelfAttention's layout), coords of n
    voxels, the cos / sin tables, gammas [H, D]."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    qkv = (torch.randn((b, n, 3, h, d), generator=g) * 1.5).to(dev).to(TDT[dt])
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]          # [B, L, H, D] views
    coords = torch.randint(0, 64, (n, 3), generator=g, dtype=torch.int32).to(dev)
    cos, sin = ops.Trellis2Rope3d(d).cos_sin(coords)
    cos, sin = cos.to(tables_dt), sin.to(tables_dt)
    qg = (1 + 0.1 * torch.randn((h, d + 1), generator=g)).to(dev)
    kg = (1 + 0.1 * torch.randn((h, d), generator=g)).to(dev)
    return q, k, v, cos, sin, qg, kg


@pytest.mark.parametrize("b,n,h,d,dt,case", [
    (1, 40000, 12, 128, "bf16", "fused"),       # configs[3]: the 40k-voxel batch element
    (2, 517, 4, 64, "bf16", "bf16_tables"),
    (1, 300, 3, 128, "f16", "fused"),
    (1, 250, 2, 128, "bf16", "unaligned_gamma"),  # runs the two launches
    (1, 90, 2, 64, "f32", "fused"),               # f32: the two launches
])
def test_sdpa_l2norm_rope3d_equals_the_two_launches(dev, ops, b, n, h, d, dt, case):
    _print_case(op="sdpa_l2norm_rope3d", b=b, n=n, h=h, d=d, dt=dt, case=case)
    q, k, v, cos, sin, qg, kg = _trellis_case(dev, ops, b, n, h, d, dt, seed=n + h,
                                              tables_dt=torch.bfloat16 if case == "bf16_tables" else torch.float32)
    gamma = qg.reshape(-1)[1:h * d + 1] if case == "unaligned_gamma" else qg[:, :d].contiguous()
    q_n, k_n = ops.qk_l2norm_rope3d(q, k, gamma.reshape(h, d), kg, cos=cos, sin=sin)
    scale = 1.0 / np.sqrt(d)
    # the attention takes [B, H, L, D] views of the [B, L, H, D] buffers
    fused = ops.sdpa_l2norm_rope3d(q.transpose(1, 2), gamma, cos, sin, k_n.transpose(1, 2), v.transpose(1, 2), scale)
    two = ops.sdpa(q_n.transpose(1, 2), k_n.transpose(1, 2), v.transpose(1, 2), scale)
    torch.cuda.synchronize()
    assert torch.isfinite(fused.float()).all()
    assert torch.equal(fused, two)


def test_sdpa_l2norm_rope3d_against_oracle(dev, ops, orc):
    b, n, h, d, dt = 1, 301, 2, 128, "bf16"
    _print_case(op="sdpa_l2norm_rope3d oracle", b=b, n=n, h=h, d=d)
    q, k, v, cos, sin, qg, _ = _trellis_case(dev, ops, b, n, h, d, dt, seed=23)
    gamma = qg[:, :d].contiguous()
    scale = 1.0 / np.sqrt(d)
    fused = ops.sdpa_l2norm_rope3d(q.transpose(1, 2), gamma, cos, sin, k.transpose(1, 2), v.transpose(1, 2), scale)
    torch.cuda.synchronize()
    qo = orc.qk_l2norm_rope3d(host(q, dt)[0], gamma.cpu().numpy(), cos.cpu().numpy(), sin.cpu().numpy(),
                              dt=orc.BF16)                        # [L, H, D]
    qo = np.ascontiguousarray(qo.transpose(1, 0, 2))[None]        # [1, H, L, D]
    assert_end_to_end(orc, fused, qo, k.transpose(1, 2), v.transpose(1, 2), scale, dt)


# ---------------------------------------------------------------------------
# DINOv3: rotate_half RoPE past the prefix tokens
# ---------------------------------------------------------------------------

def _dino_case(dev, orc, b, s, h, d, dt, prefix, seed, grid=None):
    """q, k, v as to_heads views ([B, S, H, D] transposed to [B, H, S, D]) and
    the rope tables [S - prefix, D]."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn((3, b, s, h, d), generator=g).to(dev).to(TDT[dt])
    q, k, v = (x[i].transpose(1, 2) for i in range(3))
    if grid is not None:
        cos, sin = orc.dinov3_rope_tables(grid, grid, d)
    else:
        ang = torch.rand((s - prefix, d), generator=g) * 6.3
        cos, sin = np.cos(ang.numpy()), np.sin(ang.numpy())
    return q, k, v, torch.from_numpy(np.ascontiguousarray(cos)).to(dev), \
        torch.from_numpy(np.ascontiguousarray(sin)).to(dev)


@pytest.mark.parametrize("b,s,h,d,dt,prefix,case", [
    (1, 1029, 16, 64, "f32", 5, "fused"),       # configs[4]: DINOv3 over 1029 tokens (f32, the reference's)
    (1, 1029, 16, 64, "bf16", 5, "fused"),
    (2, 300, 4, 128, "f32", 0, "fused"),
    (1, 260, 2, 128, "bf16", 7, "bf16_tables"),
    (1, 5000, 2, 64, "bf16", 5, "fused"),       # > 4096 queries: the two-tile exact kernel
    (1, 200, 2, 64, "f16", 5, "fused"),         # f16: the two launches
    (1, 201, 2, 64, "f32", 5, "unaligned_tables"),
])
def test_sdpa_dinov3_rope_equals_the_two_launches(dev, ops, orc, b, s, h, d, dt, prefix, case):
    _print_case(op="sdpa_dinov3_rope", b=b, s=s, h=h, d=d, dt=dt, prefix=prefix, case=case)
    q, k, v, cos, sin = _dino_case(dev, orc, b, s, h, d, dt, prefix, seed=s + d,
                                   grid=32 if s == 1029 else None)
    if case == "bf16_tables":
        cos, sin = cos.to(torch.bfloat16), sin.to(torch.bfloat16)
    if case == "unaligned_tables":
        cw = torch.zeros((s - prefix, d + 1), device=dev)
        sw = torch.zeros((s - prefix, d + 1), device=dev)
        cw[:, 1:], sw[:, 1:] = cos, sin
        cos, sin = cw[:, 1:], sw[:, 1:]
    q_r, k_r = ops.apply_rotary_to_patches(q, k, cos, sin, prefix)
    scale = 1.0 / np.sqrt(d)
    fused = ops.sdpa_dinov3_rope(q, cos, sin, prefix, k_r, v, scale)
    two = ops.exact_sdpa_heads(q_r, k_r, v, scale)
    torch.cuda.synchronize()
    assert torch.isfinite(fused.float()).all()
    assert torch.equal(fused, two)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_sdpa_dinov3_rope_against_oracle(dev, ops, orc, dt):
    b, s, h, d, prefix = 1, 5 + 16 * 16, 2, 64, 5
    _print_case(op="sdpa_dinov3_rope oracle", dt=dt)
    q, k, v, cos, sin = _dino_case(dev, orc, b, s, h, d, dt, prefix, seed=31, grid=16)
    scale = 1.0 / np.sqrt(d)
    fused = ops.sdpa_dinov3_rope(q, cos, sin, prefix, k, v, scale)
    torch.cuda.synchronize()
    qo = orc.dinov3_rope_apply(np.ascontiguousarray(host(q, dt)), prefix, cos.cpu().numpy(), sin.cpu().numpy(),
                               dt=odt(orc, dt))
    assert_end_to_end(orc, fused, qo, k, v, scale, dt, exact_heads=True)
    # the prefix tokens' q passes through: their outputs equal plain attention's
    plain = ops.exact_sdpa_heads(q, k, v, scale)
    torch.cuda.synchronize()
    assert torch.equal(fused[:, :, :prefix], plain[:, :, :prefix])


# ---------------------------------------------------------------------------
# Key groups: the wavefronts of a workgroup split each key block (D 64)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("ks", [1, 2, 4])
@pytest.mark.parametrize("b,lq,lk,h", [(1, 1029, 1029, 16), (2, 200, 700, 3), (1, 33, 128, 2)])
def test_sdpa_key_groups_exact_heads(dev, ops, orc, monkeypatch, ks, b, lq, lk, h):
    """exact_sdpa_heads (bf16 in, f32 out) with the keys of every block split
    over 1, 2 or 4 wavefronts and merged in LDS: every output within the f32
    bar of the oracle (|err| <= 1e-5 wabs + 2^-23 |want|), at the DINOv3
    shape (partial last key block, a partial query tile) and cross shapes."""
    monkeypatch.setenv("LUX3D_ATTN_KS", str(ks))
    d = 64
    _print_case(op="sdpa key groups exact", ks=ks, b=b, lq=lq, lk=lk, h=h)
    g = torch.Generator(device="cpu").manual_seed(lq + lk + ks)
    q = torch.randn((b, h, lq, d), generator=g).to(dev).to(torch.bfloat16)
    k = (torch.randn((b, h, lk, d), generator=g) * 1.5).to(dev).to(torch.bfloat16)
    v = torch.randn((b, h, lk, d), generator=g).to(dev).to(torch.bfloat16)
    out = torch.empty((b, h, lq, d), dtype=torch.float32, device=dev)
    ops.exact_sdpa_heads(q, k, v, 0.125, out=out)
    torch.cuda.synchronize()
    want, wabs = orc.sdpa(host(q, "bf16"), host(k, "bf16"), host(v, "bf16"), 0.125, dt=orc.BF16, out_dt=orc.F32,
                          with_abs=True)
    err = np.abs(out.cpu().numpy().astype(np.float64) - want.astype(np.float64))
    bound = 1e-5 * wabs.astype(np.float64) + 2.0 ** -23 * np.abs(want.astype(np.float64))
    assert np.all(err <= bound + 1e-30), f"worst err {err.max():.3e}"


@pytest.mark.parametrize("ks", [2, 4])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_sdpa_key_groups_rounded_probabilities(dev, ops, orc, monkeypatch, ks, dt):
    """lux3d_sdpa (probabilities rounded to the input type) with key groups:
    the matrix-core bound of test_gpu_attention.py against the oracle."""
    monkeypatch.setenv("LUX3D_ATTN_KS", str(ks))
    b, lq, lk, h, d = 1, 1029, 1029, 8, 64
    _print_case(op="sdpa key groups", ks=ks, dt=dt)
    g = torch.Generator(device="cpu").manual_seed(7 + ks)
    qkv = torch.randn((b, lq, 3, h, d), generator=g).to(dev).to(TDT[dt]).permute(2, 0, 3, 1, 4)
    q, k, v = qkv[0], qkv[1], qkv[2]
    got = ops.sdpa(q, k, v, 0.125)
    torch.cuda.synchronize()
    want, wabs = orc.sdpa(host(q, dt), host(k, dt), host(v, dt), 0.125, dt=odt(orc, dt), with_abs=True)
    gg, w = to_f64(host(got, dt), dt), to_f64(want, dt)
    bound = ULP[dt] * np.abs(w) + (ULP[dt] + 1e-6) * wabs.astype(np.float64)
    err = np.abs(gg - w)
    assert np.all(err <= bound + 1e-30), f"worst err {err.max():.3e}"


@pytest.mark.parametrize("ks", [2, 4])
def test_sdpa_dinov3_rope_key_groups_equals_the_two_launches(dev, ops, orc, monkeypatch, ks):
    """The fused DINOv3 rotation with key groups equals the rotation launch
    followed by exact_sdpa_heads on the same key groups, bit for bit, and
    repeated calls agree (the merge order is fixed)."""
    monkeypatch.setenv("LUX3D_ATTN_KS", str(ks))
    b, s, h, d, prefix = 1, 1029, 16, 64, 5
    _print_case(op="sdpa_dinov3_rope key groups", ks=ks)
    q, k, v, cos, sin = _dino_case(dev, orc, b, s, h, d, "bf16", prefix, seed=91, grid=32)
    q_r, k_r = ops.apply_rotary_to_patches(q, k, cos, sin, prefix)
    fused = ops.sdpa_dinov3_rope(q, cos, sin, prefix, k_r, v, 0.125)
    again = ops.sdpa_dinov3_rope(q, cos, sin, prefix, k_r, v, 0.125)
    two = ops.exact_sdpa_heads(q_r, k_r, v, 0.125)
    torch.cuda.synchronize()
    assert torch.equal(fused, two) and torch.equal(fused, again)
