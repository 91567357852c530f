"""GPU parity: every fused HIP op (through the C ABI) against the CPU oracle
on the same seeded inputs, at the BASELINE.json config shapes and at edge
cases (odd widths, unaligned/strided views, empty inputs, ragged segments).

Tolerances: bf16 <= 2 ulp, f32 <= 1e-5 relative to the output scale,
Q8_0 dequant and table/index math bit-exact (see conftest.py).
"""
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


def dev_tensor(a: np.ndarray, dt: str, dev):
    """numpy f32 -> device tensor of dtype `dt` (RNE for bf16/f16)."""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev).to(TDT[dt])


def host_view(t, dt: str) -> np.ndarray:
    """Device tensor -> numpy in the oracle's encoding (f32, or uint16 bits)."""
    t = t.detach().contiguous().cpu()
    if dt == "f32":
        return t.numpy()
    if dt == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()  # float16


def oracle_dt(orc, dt):
    return {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}[dt]


def check(got_dev, want, dt, what):
    got = host_view(got_dev, dt)
    if dt == "f32":
        return assert_f32_close(got, want, what=what)
    if dt == "bf16":
        return assert_bf16_close(got, want, what=what)
    return assert_f16_close(got.view(np.uint16), np.asarray(want).view(np.uint16), what=what)


def sync():
    torch.cuda.synchronize()


# ---------------------------------------------------------------------------
# LayerNorm family
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dt,rows,d,eps", [
    ("f32", 1374, 1024, 1e-6),     # configs[0]: DINOv2 norm inside VGGT
    ("bf16", 8 * 1374, 1024, 1e-5),
    ("f16", 300, 2048, 1e-5),
    ("bf16", 1029, 1024, 1e-5),    # multi-wave rows (short job)
    ("f32", 37, 1000, 1e-5),       # d % 8 != 0: generic kernel
    ("bf16", 5, 1536, 1e-6),
    ("f32", 3, 4096, 1e-5),
])
def test_layer_norm(dev, ops, orc, synth, dt, rows, d, eps):
    print(f"\n[case] layer_norm dt={dt} rows={rows} d={d}", flush=True)
    x = synth.normal(synth.config_seed(0), rows * d).reshape(rows, d)
    w = synth.normal(11, d, 1.0, 0.02)
    b = synth.normal(12, d, 0.0, 0.02)
    xd = dev_tensor(x, dt, dev)
    y = ops.layer_norm(xd, torch.from_numpy(w).to(dev), torch.from_numpy(b).to(dev), eps)
    sync()
    want = orc.layer_norm(host_view(xd, dt), w, b, eps, dt=oracle_dt(orc, dt))
    check(y, want, dt, "layer_norm")


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_layer_norm_no_affine_and_views(dev, ops, orc, synth, dt):
    print(f"\n[case] layer_norm_no_affine dt={dt}", flush=True)
    rows, d = 2 * 2048, 2048
    x = synth.normal(synth.config_seed(2), rows * d).reshape(rows, d)
    xd = dev_tensor(x, dt, dev)
    y = ops.layer_norm_no_affine(xd, 1e-6)
    sync()
    want = orc.layer_norm_no_affine(host_view(xd, dt), 1e-6, dt=oracle_dt(orc, dt))
    check(y, want, dt, "layer_norm_no_affine")
    # a row-strided view (every other row) and an unaligned view (offset 1 col)
    big = dev_tensor(synth.normal(5, 64 * 520).reshape(64, 520), dt, dev)
    v = big[::2, :512]
    y2 = ops.layer_norm_no_affine(v, 1e-6)
    u = big[:, 1:513]
    y3 = ops.layer_norm_no_affine(u, 1e-6)
    sync()
    check(y2, orc.layer_norm_no_affine(host_view(v, dt), 1e-6, dt=oracle_dt(orc, dt)), dt, "strided rows")
    check(y3, orc.layer_norm_no_affine(host_view(u, dt), 1e-6, dt=oracle_dt(orc, dt)), dt, "unaligned rows")


def test_layer_norm_empty_and_errors(dev, ops):
    from lux3d_fused import Lux3dError
    x = torch.empty((0, 1024), dtype=torch.bfloat16, device=dev)
    y = ops.layer_norm_no_affine(x, 1e-6)
    sync()
    assert y.shape == (0, 1024)
    with pytest.raises(Lux3dError):
        ops.layer_norm(torch.zeros((4, 64), device=dev), torch.zeros(32, device=dev), None, 1e-5)


@pytest.mark.parametrize("dt,shape,gamma", [
    ("bf16", (8, 1374, 1024), (1.0, 0.02)),     # configs[1]: VGGT residual(+LayerScale)+LN
    ("f32", (1, 1029, 1024), (1e-5, 1e-6)),     # configs[4]: DINOv3 LayerScale+residual+LN
    ("bf16", (1, 1029, 1024), (1e-5, 1e-6)),
    ("bf16", (2, 2049, 2048), None),            # TripoSG plain residual + LN (F3)
    ("f32", (3, 7, 200), (1.0, 0.1)),           # generic kernel
    ("bf16", (1, 4099, 1024), (1.0, 0.02)),     # persistent rows: odd row count (a row past the end)
    ("f16", (3, 1373, 1024), None),             # persistent rows: f16, no LayerScale, odd row count
    ("bf16", (1, 2048, 1024), (1.0, 0.02)),     # the first job size on the persistent kernel
    ("bf16", (1, 65537, 1024), (1.0, 0.02)),    # 64 rows per wavefront, one more for some
])
def test_residual_layer_norm(dev, ops, orc, synth, dt, shape, gamma):
    print(f"\n[case] residual_layer_norm dt={dt} shape={shape} gamma={gamma}", flush=True)
    n = int(np.prod(shape))
    d = shape[-1]
    seed = synth.config_seed(1)
    x = synth.normal(seed, n).reshape(shape)
    a = synth.normal(seed + 100, n).reshape(shape)
    g = synth.normal(seed + 200, d, *gamma) if gamma else None
    w = synth.normal(seed + 300, d, 1.0, 0.02)
    b = synth.normal(seed + 400, d, 0.0, 0.02)
    xd, ad = dev_tensor(x, dt, dev), dev_tensor(a, dt, dev)
    gd = torch.from_numpy(g).to(dev) if gamma else None
    h, y = ops.residual_layer_norm(xd, ad, gd, torch.from_numpy(w).to(dev), torch.from_numpy(b).to(dev), 1e-5)
    sync()
    hw, yw = orc.residual_layer_norm(host_view(xd, dt), host_view(ad, dt), g, w, b, 1e-5, dt=oracle_dt(orc, dt))
    # h = x + a*gamma is one product and one add in both implementations: exact
    if dt == "f32":
        assert np.array_equal(host_view(h, dt), hw), "residual stream h must be bit-exact"
    else:
        assert np.array_equal(host_view(h, dt), hw), "residual stream h must be bit-exact"
    check(y, yw, dt, "residual_layer_norm y")


def test_residual_layer_norm_strided_rows(dev, ops, orc, synth):
    """Row-strided x and branch views on the long-job path (rows of 1024 in
    2048-wide buffers)."""
    print("\n[case] residual_layer_norm strided rows bf16 [5000, 1024] of [5000, 2048]", flush=True)
    rows, d = 5000, 1024
    seed = synth.config_seed(1) + 31
    xw = synth.normal(seed, rows * 2 * d).reshape(rows, 2 * d)
    aw = synth.normal(seed + 1, rows * 2 * d).reshape(rows, 2 * d)
    g = synth.normal(seed + 2, d, 1.0, 0.02)
    w = synth.normal(seed + 3, d, 1.0, 0.02)
    b = synth.normal(seed + 4, d, 0.0, 0.02)
    xwd, awd = dev_tensor(xw, "bf16", dev), dev_tensor(aw, "bf16", dev)
    xd, ad = xwd[:, d:], awd[:, :d]
    h, y = ops.residual_layer_norm(xd, ad, torch.from_numpy(g).to(dev), torch.from_numpy(w).to(dev),
                                   torch.from_numpy(b).to(dev), 1e-5)
    sync()
    hw, yw = orc.residual_layer_norm(host_view(xd, "bf16"), host_view(ad, "bf16"), g, w, b, 1e-5, dt=orc.BF16)
    assert np.array_equal(host_view(h, "bf16"), hw), "residual stream h must be bit-exact"
    check(y, yw, "bf16", "residual_layer_norm y (strided rows)")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_residual_layer_norm_persistent_equals_row_kernel(dev, ops, synth, dt):
    """The long jobs (>= 2048 rows of 1024, 2-byte) run the persistent kernel,
    the short ones row_kernel; both compute each row with the same element
    mapping, arithmetic and reduction order, so a row's h and y do not depend
    on which of them ran: the first 2000 rows of a 6001-row job, run again as
    a job of their own, come out bit for bit the same."""
    print(f"\n[case] residual_layer_norm persistent vs row kernel dt={dt}", flush=True)
    rows, d, part = 6001, 1024, 2000
    seed = synth.config_seed(1) + 57
    x = dev_tensor(synth.normal(seed, rows * d).reshape(rows, d), dt, dev)
    a = dev_tensor(synth.normal(seed + 1, rows * d).reshape(rows, d), dt, dev)
    g = torch.from_numpy(synth.normal(seed + 2, d, 1.0, 0.02)).to(dev)
    w = torch.from_numpy(synth.normal(seed + 3, d, 1.0, 0.02)).to(dev)
    b = torch.from_numpy(synth.normal(seed + 4, d, 0.0, 0.02)).to(dev)
    h, y = ops.residual_layer_norm(x, a, g, w, b, 1e-5)
    h2, y2 = ops.residual_layer_norm(x[:part].contiguous(), a[:part].contiguous(), g, w, b, 1e-5)
    sync()
    assert torch.equal(h[:part].view(torch.int16), h2.view(torch.int16))
    assert torch.equal(y[:part].view(torch.int16), y2.view(torch.int16))


@pytest.mark.parametrize("dt,shape,gamma,pdt", [
    ("bf16", (1, 700, 1024), None, None),           # no LayerScale, no affine
    ("bf16", (1, 700, 1024), (1.0, 0.1), "bf16"),   # 2-byte parameters
    ("f32", (1, 700, 1024), (1e-5, 1e-6), "f16"),
    ("f32", (2, 300, 2048), None, "f32"),           # 2048-wide rows: 256 threads per row
    ("bf16", (2, 300, 2048), (1.0, 0.1), "f32"),
])
def test_residual_layer_norm_short_jobs(dev, ops, orc, synth, dt, shape, gamma, pdt):
    """Jobs under 2048 rows run one row per workgroup and issue the LayerNorm
    parameters ahead of the residual store; every parameter dtype and the
    absent ones take that path."""
    print(f"\n[case] residual_layer_norm short job dt={dt} shape={shape} gamma={gamma} params={pdt}", flush=True)
    n = int(np.prod(shape))
    d = shape[-1]
    seed = synth.config_seed(4) + 17
    x = synth.normal(seed, n).reshape(shape)
    a = synth.normal(seed + 1, n).reshape(shape)

    def param(s, mean, std):
        t = torch.from_numpy(synth.normal(s, d, mean, std)).to(dev).to(TDT[pdt if pdt else "f32"])
        return t, t.float().cpu().numpy()

    gd, g = param(seed + 2, *gamma) if gamma else (None, None)
    wd, w = param(seed + 3, 1.0, 0.02) if pdt else (None, None)
    bd, b = param(seed + 4, 0.0, 0.02) if pdt else (None, None)
    xd, ad = dev_tensor(x, dt, dev), dev_tensor(a, dt, dev)
    h, y = ops.residual_layer_norm(xd, ad, gd, wd, bd, 1e-5)
    sync()
    hw, yw = orc.residual_layer_norm(host_view(xd, dt), host_view(ad, dt), g, w, b, 1e-5, dt=oracle_dt(orc, dt))
    assert np.array_equal(host_view(h, dt), hw), "residual stream h must be bit-exact"
    check(y, yw, dt, "residual_layer_norm y (short job)")


# ---------------------------------------------------------------------------
# AdaLN modulate / gated residual (dense and ragged)
# ---------------------------------------------------------------------------

def test_adaln_modulate_dense_cfg2(dev, ops, orc, synth):
    print("\n[case] adaln_modulate dense configs[2]", flush=True)
    B, L, C = 2, 2048, 2048
    seed = synth.config_seed(2)
    x = synth.normal(seed, B * L * C).reshape(B, L, C)
    shift = synth.normal(seed + 1, B * C, 0.0, 0.1).reshape(B, C)
    scale = synth.normal(seed + 2, B * C, 0.0, 0.1).reshape(B, C)
    xd = dev_tensor(x, "bf16", dev)
    y = ops.adaln_modulate(xd, torch.from_numpy(shift).to(dev), torch.from_numpy(scale).to(dev), eps=1e-6)
    sync()
    want = orc.adaln_modulate(host_view(xd, "bf16"), np.array([0, L, 2 * L]), shift, scale, eps=1e-6, dt=orc.BF16)
    check(y, want, "bf16", "adaln dense")


def _ragged_cfg3(synth, C=1536, sizes=(24000, 40000)):
    seed = synth.config_seed(3)
    n = sum(sizes)
    x = synth.normal(seed, n * C).reshape(n, C)
    t_emb = synth.normal(seed + 1, len(sizes) * 6 * C, 0.0, 0.1).reshape(len(sizes), 6 * C)
    modulation = synth.normal(seed + 2, 6 * C, 0.0, 0.1)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    return x, t_emb, modulation, offs


@pytest.mark.parametrize("with_gate", [False, True])
def test_adaln_modulate_ragged_cfg3(dev, ops, orc, synth, with_gate):
    print(f"\n[case] adaln_modulate ragged configs[3] gate={with_gate}", flush=True)
    C = 1536
    x, t_emb, modulation, offs = _ragged_cfg3(synth, C)
    xd = dev_tensor(x, "bf16", dev)
    te = torch.from_numpy(t_emb).to(dev)
    md = torch.from_numpy(modulation).to(dev)
    pieces = ops.chunk_modulation(te)       # [S, 1, C] views of t_emb (no copies)
    base = md.chunk(6)                       # the block's `modulation` parameter
    y = ops.adaln_modulate(xd, pieces[0], pieces[1], pieces[2] if with_gate else None,
                           shift_base=base[0], scale_base=base[1], gate_base=base[2] if with_gate else None,
                           seg_offsets=torch.from_numpy(offs).to(dev), eps=1e-6)
    sync()
    sl = lambda k: np.ascontiguousarray(t_emb[:, k * C:(k + 1) * C])  # noqa: E731
    bl = lambda k: modulation[k * C:(k + 1) * C]  # noqa: E731
    want = orc.adaln_modulate(host_view(xd, "bf16"), offs, sl(0), sl(1), sl(2) if with_gate else None,
                              bl(0), bl(1), bl(2) if with_gate else None, eps=1e-6, dt=orc.BF16)
    check(y, want, "bf16", "adaln ragged")


@pytest.mark.parametrize("ragged", [False, True])
def test_gated_residual(dev, ops, orc, synth, ragged):
    print(f"\n[case] gated_residual ragged={ragged}", flush=True)
    if ragged:
        C = 1536
        x, t_emb, modulation, offs = _ragged_cfg3(synth, C)
        h = synth.normal(77, x.size).reshape(x.shape)
        gate_seg = np.ascontiguousarray(t_emb[:, 2 * C:3 * C])
        gate_base = modulation[2 * C:3 * C]
    else:
        B, L, C = 2, 2048, 2048
        x = synth.normal(synth.config_seed(2), B * L * C).reshape(B * L, C)
        h = synth.normal(78, x.size).reshape(x.shape)
        gate_seg = synth.normal(79, B * C, 0.0, 0.1).reshape(B, C)
        gate_base = None
        offs = np.array([0, L, 2 * L], dtype=np.int64)
    xd, hd = dev_tensor(x, "bf16", dev), dev_tensor(h, "bf16", dev)
    gd = torch.from_numpy(gate_seg).to(dev)
    gb = torch.from_numpy(gate_base).to(dev) if gate_base is not None else None
    so = torch.from_numpy(offs).to(dev) if ragged else None
    out = ops.gated_residual(xd, hd, gd, gate_base=gb, seg_offsets=so)
    sync()
    want = orc.gated_residual(host_view(xd, "bf16"), host_view(hd, "bf16"), offs, gate_seg, gate_base, dt=orc.BF16)
    check(out, want, "bf16", "gated_residual")


# Segment boundaries that fall inside a workgroup of several rows: those
# workgroups read the segment pieces per row, the others share them in LDS.
STRADDLE = [((2049, 1, 1027, 2000), 1536), ((1031, 1031, 1031), 2048)]


@pytest.mark.parametrize("sizes,C", STRADDLE)
@pytest.mark.parametrize("with_gate", [False, True])
def test_adaln_modulate_straddling_segments(dev, ops, orc, synth, sizes, C, with_gate):
    print(f"\n[case] adaln_modulate segments {sizes} C={C} gate={with_gate}", flush=True)
    S, n = len(sizes), sum(sizes)
    x = synth.normal(91, n * C).reshape(n, C)
    t_emb = synth.normal(92, S * 6 * C, 0.0, 0.1).reshape(S, 6 * C)
    modulation = synth.normal(93, 6 * C, 0.0, 0.1)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    xd = dev_tensor(x, "bf16", dev)
    pieces = ops.chunk_modulation(torch.from_numpy(t_emb).to(dev))
    base = torch.from_numpy(modulation).to(dev).chunk(6)
    y = ops.adaln_modulate(xd, pieces[0], pieces[1], pieces[2] if with_gate else None,
                           shift_base=base[0], scale_base=base[1], gate_base=base[2] if with_gate else None,
                           seg_offsets=torch.from_numpy(offs).to(dev), eps=1e-6)
    sync()
    sl = lambda k: np.ascontiguousarray(t_emb[:, k * C:(k + 1) * C])  # noqa: E731
    bl = lambda k: modulation[k * C:(k + 1) * C]  # noqa: E731
    want = orc.adaln_modulate(host_view(xd, "bf16"), offs, sl(0), sl(1), sl(2) if with_gate else None,
                              bl(0), bl(1), bl(2) if with_gate else None, eps=1e-6, dt=orc.BF16)
    check(y, want, "bf16", "adaln straddling segments")


@pytest.mark.parametrize("sizes,C", STRADDLE)
def test_gated_residual_straddling_segments(dev, ops, orc, synth, sizes, C):
    print(f"\n[case] gated_residual segments {sizes} C={C}", flush=True)
    S, n = len(sizes), sum(sizes)
    x = synth.normal(94, n * C).reshape(n, C)
    h = synth.normal(95, n * C).reshape(n, C)
    gate_seg = synth.normal(96, S * C, 0.0, 0.1).reshape(S, C)
    gate_base = synth.normal(97, C, 0.0, 0.1)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    xd, hd = dev_tensor(x, "bf16", dev), dev_tensor(h, "bf16", dev)
    out = ops.gated_residual(xd, hd, torch.from_numpy(gate_seg).to(dev), gate_base=torch.from_numpy(gate_base).to(dev),
                             seg_offsets=torch.from_numpy(offs).to(dev))
    sync()
    want = orc.gated_residual(host_view(xd, "bf16"), host_view(hd, "bf16"), offs, gate_seg, gate_base, dt=orc.BF16)
    check(out, want, "bf16", "gated_residual straddling segments")


def test_adaln_modulate_dense_uneven_segments(dev, ops, orc, synth):
    """Equal segments without offsets ([B, L, C] with L not a multiple of the
    rows per workgroup)."""
    print("\n[case] adaln_modulate dense B=3 L=1031", flush=True)
    B, L, C = 3, 1031, 2048
    x = synth.normal(98, B * L * C).reshape(B, L, C)
    shift = synth.normal(99, B * C, 0.0, 0.1).reshape(B, C)
    scale = synth.normal(100, B * C, 0.0, 0.1).reshape(B, C)
    xd = dev_tensor(x, "bf16", dev)
    y = ops.adaln_modulate(xd, torch.from_numpy(shift).to(dev), torch.from_numpy(scale).to(dev), eps=1e-6)
    sync()
    want = orc.adaln_modulate(host_view(xd, "bf16"), np.array([0, L, 2 * L, 3 * L]), shift, scale, eps=1e-6,
                              dt=orc.BF16)
    check(y, want, "bf16", "adaln dense uneven")


# ---------------------------------------------------------------------------
# VGGT: QK LayerNorm + 2D RoPE
# ---------------------------------------------------------------------------

def _vggt_qkv(synth, dev, dt, B=8, H=16, D=64, ph=37, pw=37):
    N = 5 + ph * pw
    seed = synth.config_seed(1)
    qkv = synth.normal(seed + 7, B * N * 3 * H * D).reshape(B, N, 3, H, D)
    qkv_d = dev_tensor(qkv, dt, dev)
    perm = qkv_d.permute(2, 0, 3, 1, 4)  # [3, B, H, N, D] (vggt.rs:163-165)
    pos = synth.vggt_positions(B, ph, pw)
    return perm[0], perm[1], pos, N


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_rope2d_tables(dev, ops, orc, synth, dt):
    print(f"\n[case] rope2d_tables dt={dt}", flush=True)
    pos = synth.vggt_positions(2, 37, 37)
    emb = ops.Rope2d(100.0).embeddings(torch.from_numpy(pos).to(dev), 64)
    sync()
    c, s = orc.rope2d_tables(pos, 64, 100.0)
    got_c = emb.cos_full.cpu().numpy().reshape(c.shape)
    got_s = emb.sin_alt_full.cpu().numpy().reshape(s.shape)
    # device sincosf vs libm: within 2 f32 ulp of |value| <= 1
    assert np.max(np.abs(got_c - c)) <= 2.5e-7
    assert np.max(np.abs(got_s - s)) <= 2.5e-7
    # specials (position (0, 0)) are the identity rotation exactly
    assert np.all(got_c[:, :5] == 1.0) and np.all(got_s[:, :5] == 0.0)


@pytest.mark.parametrize("dt,source", [("bf16", "tables"), ("bf16", "positions"), ("f32", "tables"),
                                       ("f32", "positions")])
def test_qk_layernorm_rope2d_cfg1(dev, ops, orc, synth, dt, source):
    print(f"\n[case] qk_layernorm_rope2d configs[1] dt={dt} source={source}", flush=True)
    B = 8
    q, k, pos, N = _vggt_qkv(synth, dev, dt, B=B)
    D = 64
    qw, qb = synth.normal(21, D, 1.0, 0.02), synth.normal(22, D, 0.0, 0.02)
    kw, kb = synth.normal(23, D, 1.0, 0.02), synth.normal(24, D, 0.0, 0.02)
    T = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    cos, sin = orc.rope2d_tables(pos, D, 100.0)
    if source == "tables":
        emb = ops.RopeEmbeddings(T(cos).unsqueeze(1), T(sin).unsqueeze(1))
        qo, ko = ops.qk_layernorm_rope2d(q, k, (T(qw), T(qb), 1e-5), (T(kw), T(kb), 1e-5), emb)
    else:
        qo, ko = ops.qk_layernorm_rope2d(q, k, (T(qw), T(qb), 1e-5), (T(kw), T(kb), 1e-5),
                                         positions=T(pos), base=100.0)
    sync()
    assert qo.is_contiguous() and qo.shape == (B, 16, N, D)
    odt = oracle_dt(orc, dt)
    qh = np.ascontiguousarray(host_view(q, dt))
    kh = np.ascontiguousarray(host_view(k, dt))
    check(qo, orc.layernorm_rope2d(qh, qw, qb, 1e-5, cos, sin, dt=odt), dt, "q")
    check(ko, orc.layernorm_rope2d(kh, kw, kb, 1e-5, cos, sin, dt=odt), dt, "k")


@pytest.mark.parametrize("dt,source", [("bf16", "positions"), ("f32", "tables")])
def test_qk_layernorm_rope2d_without_bias(dev, ops, orc, synth, dt, source):
    """A LayerNorm without bias (candle_nn::LayerNorm, bias None: n * w) on the
    q / k heads: the bias is NULL at the C ABI."""
    print(f"\n[case] qk_layernorm_rope2d without bias dt={dt} source={source}", flush=True)
    q, k, pos, N = _vggt_qkv(synth, dev, dt, B=2, ph=13, pw=11)
    D = 64
    qw, kw = synth.normal(25, D, 1.0, 0.1), synth.normal(26, D, 1.0, 0.1)
    T = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    cos, sin = orc.rope2d_tables(pos, D, 100.0)
    if source == "tables":
        emb = ops.RopeEmbeddings(T(cos).unsqueeze(1), T(sin).unsqueeze(1))
        qo, ko = ops.qk_layernorm_rope2d(q, k, (T(qw), None, 1e-5), (T(kw), None, 1e-5), emb)
    else:
        qo, ko = ops.qk_layernorm_rope2d(q, k, (T(qw), None, 1e-5), (T(kw), None, 1e-5), positions=T(pos), base=100.0)
    sync()
    odt = oracle_dt(orc, dt)
    check(qo, orc.layernorm_rope2d(np.ascontiguousarray(host_view(q, dt)), qw, None, 1e-5, cos, sin, dt=odt), dt, "q")
    check(ko, orc.layernorm_rope2d(np.ascontiguousarray(host_view(k, dt)), kw, None, 1e-5, cos, sin, dt=odt), dt, "k")


def test_rope_fused_and_single_tensor(dev, ops, orc, synth):
    print("\n[case] rope_fused / layernorm_rope_fused single tensor", flush=True)
    q, k, pos, N = _vggt_qkv(synth, dev, "bf16", B=2, ph=9, pw=11)
    cos, sin = orc.rope2d_tables(pos, 64, 100.0)
    T = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    r = ops.rope_fused(q, T(cos), T(sin))
    w, b = synth.normal(31, 64, 1.0, 0.02), synth.normal(32, 64, 0.0, 0.02)
    ln = ops.layernorm_rope_fused(k, T(w), T(b), 1e-5, T(cos), T(sin))
    sync()
    check(r, orc.rope2d_apply(np.ascontiguousarray(host_view(q, "bf16")), cos, sin, dt=orc.BF16), "bf16", "rope")
    check(ln, orc.layernorm_rope2d(np.ascontiguousarray(host_view(k, "bf16")), w, b, 1e-5, cos, sin, dt=orc.BF16),
          "bf16", "layernorm_rope")


# ---------------------------------------------------------------------------
# TripoSG: per-head RMSNorm on the re-split q/k views
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dt,L", [("bf16", 2048), ("bf16", 2049), ("f32", 257)])
def test_rms_norm_heads_cfg2(dev, ops, orc, synth, dt, L):
    print(f"\n[case] rms_norm_heads dt={dt} L={L}", flush=True)
    B, H, D = 2, 16, 128
    seed = synth.config_seed(2)
    qkv = synth.normal(seed + 9, B * L * H * 3 * D).reshape(B, L, H, 3 * D)
    qd = dev_tensor(qkv, dt, dev)
    q = qd[..., 0:D].transpose(1, 2)       # [B, H, L, D] strided (triposg_dit.rs:439-449)
    k = qd[..., D:2 * D].transpose(1, 2)
    wq, wk = synth.normal(41, D, 1.0, 0.02), synth.normal(42, D, 1.0, 0.02)
    T = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    qo, ko = ops.rms_norm_heads(q, T(wq), 1e-6, k=k, k_weight=T(wk))
    sync()
    odt = oracle_dt(orc, dt)
    check(qo, orc.rms_norm_heads(np.ascontiguousarray(host_view(q, dt)), wq, 1e-6, dt=odt), dt, "q")
    check(ko, orc.rms_norm_heads(np.ascontiguousarray(host_view(k, dt)), wk, 1e-6, dt=odt), dt, "k")


# ---------------------------------------------------------------------------
# TRELLIS.2: L2 q/k norm + 3D RoPE on ragged voxel tokens
# ---------------------------------------------------------------------------

def _slat_coords(synth, sizes=(24000, 40000), res=64):
    return np.concatenate([synth.unique_voxels(synth.config_seed(3) + 10 * i, n, res)
                           for i, n in enumerate(sizes)], axis=0)


@pytest.mark.parametrize("source", ["coords", "tables"])
def test_qk_l2norm_rope3d_cfg3(dev, ops, orc, synth, source):
    print(f"\n[case] qk_l2norm_rope3d configs[3] source={source}", flush=True)
    H, D = 12, 128
    coords = _slat_coords(synth)
    N = coords.shape[0]
    qkv = synth.normal(synth.config_seed(3) + 5, N * 3 * H * D).reshape(1, N, 3, H, D)
    qkvd = dev_tensor(qkv, "bf16", dev)
    q, k = qkvd[:, :, 0], qkvd[:, :, 1]       # [1, N, H, D] views (split_heads :404-407)
    gq, gk = synth.normal(51, H * D, 1.0, 0.02).reshape(H, D), synth.normal(52, H * D, 1.0, 0.02).reshape(H, D)
    T = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    cos, sin = orc.rope3d_tables(coords, D)
    if source == "coords":
        qo, ko = ops.qk_l2norm_rope3d(q, k, T(gq), T(gk), coords=T(coords))
    else:
        qo, ko = ops.qk_l2norm_rope3d(q, k, T(gq), T(gk), cos=T(cos), sin=T(sin))
    sync()
    qh = np.ascontiguousarray(host_view(q, "bf16")).reshape(N, H, D)
    kh = np.ascontiguousarray(host_view(k, "bf16")).reshape(N, H, D)
    check(qo, orc.qk_l2norm_rope3d(qh, gq, cos, sin, dt=orc.BF16).reshape(1, N, H, D), "bf16", "q")
    check(ko, orc.qk_l2norm_rope3d(kh, gk, cos, sin, dt=orc.BF16).reshape(1, N, H, D), "bf16", "k")


def test_rope3d_tables_and_norm_only(dev, ops, orc, synth):
    print("\n[case] rope3d tables / norm only / rope only", flush=True)
    coords = _slat_coords(synth, sizes=(3000,))
    T = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    rope = ops.Trellis2Rope3d(128)
    c, s = rope.cos_sin(T(coords))
    sync()
    cw, sw = orc.rope3d_tables(coords, 128)
    assert np.max(np.abs(c.cpu().numpy() - cw)) <= 2.5e-7
    assert np.max(np.abs(s.cpu().numpy() - sw)) <= 2.5e-7
    x = synth.normal(61, 3000 * 12 * 128).reshape(1, 3000, 12, 128)
    xd = dev_tensor(x, "f32", dev)
    g = synth.normal(62, 12 * 128, 1.0, 0.02).reshape(12, 128)
    n_only = ops.Trellis2QkRmsNorm(T(g)).forward(xd)
    r_only = rope.apply(xd, T(cw), T(sw))
    sync()
    check(n_only, orc.qk_l2norm(x.reshape(3000, 12, 128), g).reshape(x.shape), "f32", "l2 norm only")
    check(r_only, orc.rope3d_apply(x, cw, sw), "f32", "rope3d only")


# ---------------------------------------------------------------------------
# DINOv3 2D RoPE
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_dinov3_rope(dev, ops, orc, synth, dt):
    print(f"\n[case] dinov3 rope dt={dt}", flush=True)
    B, H, D, grid = 1, 16, 64, 32
    S = 5 + grid * grid
    cos, sin = orc.dinov3_rope_tables(grid, grid, D)
    q = synth.normal(71, B * S * H * D).reshape(B, S, H, D)
    qd = dev_tensor(q, dt, dev).transpose(1, 2)     # to_heads: [B, H, S, D] view
    kd = dev_tensor(q[:, :, ::-1], dt, dev).transpose(1, 2)
    T = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    qo, ko = ops.apply_rotary_to_patches(qd, kd, T(cos), T(sin), 5)
    sync()
    odt = oracle_dt(orc, dt)
    check(qo, orc.dinov3_rope_apply(np.ascontiguousarray(host_view(qd, dt)), 5, cos, sin, dt=odt), dt, "q")
    check(ko, orc.dinov3_rope_apply(np.ascontiguousarray(host_view(kd, dt)), 5, cos, sin, dt=odt), dt, "k")
    # prefix tokens pass through bit-exactly
    assert np.array_equal(host_view(qo, dt)[:, :, :5], np.ascontiguousarray(host_view(qd, dt))[:, :, :5])


# ---------------------------------------------------------------------------
# Activations
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("act", ["gelu_tanh", "gelu_erf", "silu"])
@pytest.mark.parametrize("dt,n", [("bf16", 2 * 2048 * 8192), ("f32", 1 << 20), ("f16", 100003),
                                  ("bf16", 13)])
def test_activations(dev, ops, orc, synth, act, dt, n):
    print(f"\n[case] {act} dt={dt} n={n}", flush=True)
    x = synth.normal(synth.config_seed(2) + 3, n) * np.float32(3.0)
    if n > 1000:
        x[:8] = [0.0, -0.0, -10.0, 10.0, -5.5, 5.5, -30.0, 30.0]
    xd = dev_tensor(x, dt, dev)
    fn = {"gelu_tanh": ops.gelu, "gelu_erf": ops.gelu_erf, "silu": ops.silu}[act]
    y = fn(xd)
    sync()
    ofn = {"gelu_tanh": orc.gelu_tanh, "gelu_erf": orc.gelu_erf, "silu": orc.silu}[act]
    want = ofn(host_view(xd, dt), dt=oracle_dt(orc, dt))
    check(y, want, dt, act)


# ---------------------------------------------------------------------------
# Timestep embeddings
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dim,cos_first", [(256, True), (2048, False), (2048, True), (256, False), (255, True)])
def test_timestep_embedding(dev, ops, orc, synth, dim, cos_first):
    print(f"\n[case] timestep_embedding dim={dim} cos_first={cos_first}", flush=True)
    t = synth.uniform(synth.config_seed(2) + 4, 2, 0.0, 1000.0)
    td = torch.from_numpy(t).to(dev)
    freqs = torch.tensor(ops.host_timestep_freqs(dim), dtype=torch.float32, device=dev)
    y = ops.timestep_embedding(td, dim, cos_first, freqs=freqs)
    y_dev = ops.timestep_embedding(td, dim, cos_first)
    sync()
    want = orc.timestep_embedding(t, dim, cos_first)
    got = y.cpu().numpy()
    # identical frequencies: only sin/cos rounding differs (<= 2 ulp of |v| <= 1)
    assert np.max(np.abs(got - want)) <= 2.5e-7
    # device-computed frequencies (exp in f64, rounded once): bit for bit the
    # rounded-once table (tests/test_oracle_pins.py pins it to the exact exp),
    # and the same 2.5e-7 bar against the oracle given that table
    cr = orc.timestep_freqs_rounded_once(dim)
    y_cr = ops.timestep_embedding(td, dim, cos_first, freqs=torch.from_numpy(cr).to(dev))
    sync()
    assert np.array_equal(y_dev.cpu().numpy(), y_cr.cpu().numpy())
    assert np.max(np.abs(y_dev.cpu().numpy() - orc.timestep_embedding(t, dim, cos_first, freqs=cr))) <= 2.5e-7


# ---------------------------------------------------------------------------
# Q8_0 dequant (bit-exact)
# ---------------------------------------------------------------------------

def _edge_blocks():
    """Every int8 value against scale bit patterns covering +-0, subnormals,
    normals, 65504, +-inf and NaNs."""
    scales = np.array([0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF, 0x7C00,
                       0xFC00, 0x7E00, 0x7C01, 0xFE01, 0x1234, 0x2E66], dtype=np.uint16)
    qs = np.arange(-128, 128, dtype=np.int16).astype(np.int8).reshape(8, 32)
    blocks = []
    for s in scales:
        for row in qs:
            b = np.empty(34, dtype=np.uint8)
            b[0:2] = np.array([s], dtype=np.uint16).view(np.uint8)
            b[2:] = row.view(np.uint8)
            blocks.append(b)
    return np.concatenate(blocks)


@pytest.mark.parametrize("out", ["bf16", "f32", "f16"])
@pytest.mark.parametrize("which", ["cfg4", "edge"])
def test_dequant_q8_0(dev, ops, orc, synth, out, which):
    print(f"\n[case] dequant_q8_0 {which} -> {out}", flush=True)
    if which == "cfg4":
        blocks = synth.q8_0_blocks(synth.config_seed(4), 4096 * 1024 // 32)
        shape = (4096, 1024)
    else:
        blocks = _edge_blocks()
        shape = (blocks.size // 34 * 32,)
    bd = torch.from_numpy(blocks).to(dev)
    y = ops.dequantize_q8_0(bd, shape, TDT[out])
    sync()
    want = orc.dequant_q8_0(blocks, oracle_dt(orc, out))
    got = host_view(y, out).reshape(-1)
    if out == "f32":
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "f32 dequant must be bit-exact"
    else:
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), f"{out} dequant must be bit-exact"
    # unaligned output (scalar stores) must agree too
    buf = torch.empty(int(np.prod(shape)) + 1, dtype=TDT[out], device=dev)
    from lux3d_fused import _lib
    ops_desc = ops.desc
    _lib.call("lux3d_dequant_q8_0", ops_desc(bd), ops_desc(buf[1:]), None)
    sync()
    got2 = host_view(buf[1:], out).reshape(-1)
    assert np.array_equal(got2.view(np.uint32 if out == "f32" else np.uint16),
                          want.view(np.uint32 if out == "f32" else np.uint16))
    # blocks that are only 2-byte aligned (direct kernel) and a block count
    # that leaves a ragged last workgroup (staged kernel's tail)
    raw = torch.empty(blocks.size + 2, dtype=torch.uint8, device=dev)
    raw[2:] = bd
    y3 = ops.dequantize_q8_0(raw[2:], shape, TDT[out])
    nb = blocks.size // 34 - 5
    y4 = ops.dequantize_q8_0(bd[:nb * 34], (nb * 32,), TDT[out])
    sync()
    u = np.uint32 if out == "f32" else np.uint16
    assert np.array_equal(host_view(y3, out).reshape(-1).view(u), want.view(u)), "2-byte aligned blocks"
    assert np.array_equal(host_view(y4, out).reshape(-1).view(u), want[:nb * 32].view(u)), "ragged block count"


def test_empty_inputs_are_no_ops(dev, ops, synth):
    """Zero rows / tokens / queries / blocks: every entry returns OK and an
    empty result without launching (candle's ops on empty tensors are
    no-ops)."""
    print("\n[case] empty inputs", flush=True)
    bf = torch.bfloat16
    C = 1024
    x0 = torch.empty((0, C), dtype=bf, device=dev)
    g = torch.ones(C, device=dev)
    h, y = ops.residual_layer_norm(x0, x0, g, g, torch.zeros(C, device=dev), 1e-5)
    assert h.shape == (0, C) and y.shape == (0, C)
    assert ops.gated_residual(x0, x0, g).shape == (0, C)
    assert ops.gelu_erf(x0).shape == (0, C) and ops.gelu(x0).shape == (0, C) and ops.silu(x0).shape == (0, C)
    q = torch.empty((2, 0, 3, 16, 64), dtype=bf, device=dev)
    qv, kv = q[:, :, 0].permute(0, 2, 1, 3), q[:, :, 1].permute(0, 2, 1, 3)
    w64, b64 = torch.ones(64, device=dev), torch.zeros(64, device=dev)
    pos = torch.empty((2, 0, 2), dtype=torch.int32, device=dev)
    qo, ko = ops.qk_layernorm_rope2d(qv, kv, (w64, b64, 1e-5), (w64, b64, 1e-5), positions=pos)
    assert qo.shape == (2, 16, 0, 64) and ko.shape == (2, 16, 0, 64)
    r = torch.empty((2, 16, 0, 128), dtype=bf, device=dev)
    assert ops.rms_norm_heads(r, torch.ones(128, device=dev), 1e-6).shape == (2, 16, 0, 128)
    t0 = torch.empty((0,), dtype=torch.float32, device=dev)
    assert ops.timestep_embedding(t0, 256).shape == (0, 256)
    assert ops.dequantize_q8_0(torch.empty((0,), dtype=torch.uint8, device=dev), (0, 32)).shape == (0, 32)
    blocks = torch.from_numpy(synth.q8_0_blocks(5, 64 * 128 // 32)).to(dev)
    mm = ops.QMatMul.from_q8_0(blocks, 64, 128)
    assert mm.forward(torch.empty((0, 128), dtype=bf, device=dev)).shape == (0, 64)
    kk = torch.randn((1, 4, 5, 64), device=dev).to(bf)
    assert ops.sdpa(torch.empty((1, 4, 0, 64), dtype=bf, device=dev), kk, kk, 0.125).shape == (1, 4, 0, 64)
    torch.cuda.synchronize()
