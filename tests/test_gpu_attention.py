"""GPU parity of lux3d_sdpa (exact_query_chunked_sdpa / exact_sdpa_heads,
attention_math.rs:199-259) against the oracle's double-precision attention
(or_sdpa, pinned in tests/test_oracle_pins.py).

Tolerances, per output element, with want = the oracle's value and
wabs = sum_j p_j |v_j| / sum_j p_j (the oracle reports it):
- matrix-core path (bf16 / f16, D 64 / 128): the probabilities are rounded
  to the input type before the P v product, an error of at most one half
  unit in their last place relative to each p_j, so
  |err| <= ulp * |want| + ulp * wabs (+ 1e-6 * wabs for the f32 sums), with
  ulp = 2^-7 (bf16) or 2^-10 (f16);
- generic path: f32 throughout, |err| <= 1e-5 * wabs + ulp(out) * |want|.
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


def host(t, dt):
    """[..., L, D] device tensor -> contiguous numpy (bf16 as uint16 bits)."""
    t = t.detach().contiguous().cpu()
    if dt == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def to_f64(a, dt):
    if dt == "bf16":
        return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return np.asarray(a).astype(np.float64)


def oracle(orc, q, k, v, scale, dt):
    code = {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}[dt]
    return orc.sdpa(host(q, dt), host(k, dt), host(v, dt), scale, dt=code, with_abs=True)


def assert_attn_close(got, want, wabs, dt, mfma, what):
    g, w = to_f64(host(got, dt), dt), to_f64(want, dt)
    a = wabs.astype(np.float64)
    if mfma:
        bound = ULP[dt] * np.abs(w) + (ULP[dt] + 1e-6) * a
    else:
        bound = 1e-5 * a + ULP[dt] * np.abs(w)
    err = np.abs(g - w)
    bad = err > bound + 1e-30
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} outputs out of tolerance; worst err "
                           f"{err.max():.3e} (bound there {bound.reshape(-1)[np.argmax(err)]:.3e})")


def qkv_views(dev, b, n, h, d, dt, seed, kscale=1.0, rising=False):
    """q, k, v as the permuted views of a fused [B, N, 3, H, D] qkv buffer,
    the way vggt.rs:161-168 takes them."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn((b, n, 3, h, d), generator=g, dtype=torch.float32)
    x[:, :, 1] *= kscale
    if rising:  # later keys score higher: the running maximum keeps moving
        x[:, :, 1] *= torch.linspace(0.5, 3.0, n).view(1, n, 1, 1)
    qkv = x.to(dev).to(TDT[dt]).permute(2, 0, 3, 1, 4)
    return qkv[0], qkv[1], qkv[2]


def _print_case(**kw):
    print("\n[case] sdpa " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


@pytest.mark.parametrize("b,n,h,d,dt,kscale,rising", [
    (2, 1374, 4, 64, "bf16", 1.0, False),     # VGGT frame-attention tokens (37 x 37 + 5)
    (1, 2100, 16, 64, "bf16", 1.0, True),     # 16 heads, 17 query blocks each
    (2, 2100, 16, 64, "bf16", 2.0, False),
    (1, 517, 3, 128, "bf16", 2.0, True),     # TRELLIS.2 head dim, peaky and moving maxima
    (2, 300, 2, 64, "f16", 3.0, True),
    (1, 129, 2, 128, "f16", 1.0, False),
    (1, 65, 1, 64, "bf16", 1.0, False),
    (1, 63, 1, 64, "bf16", 4.0, False),
])
def test_sdpa_self_attention_mfma(dev, ops, orc, b, n, h, d, dt, kscale, rising):
    _print_case(b=b, n=n, h=h, d=d, dt=dt)
    q, k, v = qkv_views(dev, b, n, h, d, dt, 10 + n + d, kscale, rising)
    scale = 1.0 / np.sqrt(d)
    out = ops.sdpa(q, k, v, scale)
    torch.cuda.synchronize()
    want, wabs = oracle(orc, q, k, v, scale, dt)
    assert_attn_close(out, want, wabs, dt, True, f"self {b}x{h}x{n}x{d} {dt}")


@pytest.mark.parametrize("lq,lk,d", [(300, 517, 128), (1, 1, 64), (5, 1, 64), (1, 200, 128), (257, 64, 64),
                                     (40, 129, 64), (100, 200, 64), (33, 4000, 64)])
def test_sdpa_cross_attention_and_edges(dev, ops, orc, lq, lk, d):
    _print_case(lq=lq, lk=lk, d=d)
    g = torch.Generator(device="cpu").manual_seed(lq * 7 + lk)
    q = torch.randn((2, 3, lq, d), generator=g).to(dev).to(torch.bfloat16)
    k = (2 * torch.randn((2, 3, lk, d), generator=g)).to(dev).to(torch.bfloat16)
    v = torch.randn((2, 3, lk, d), generator=g).to(dev).to(torch.bfloat16)
    scale = 1.0 / np.sqrt(d)
    out = ops.sdpa(q, k, v, scale)
    torch.cuda.synchronize()
    want, wabs = oracle(orc, q, k, v, scale, "bf16")
    assert_attn_close(out, want, wabs, "bf16", True, f"cross {lq}x{lk}x{d}")


def test_sdpa_output_view_in_token_major_layout(dev, ops, orc):
    """out written straight into [B, L, H, D] (the layout the reference
    transposes to next, vggt.rs:184) through a permuted view."""
    b, n, h, d = 2, 200, 4, 64
    q, k, v = qkv_views(dev, b, n, h, d, "bf16", 77)
    buf = torch.full((b, n, h, d), 7.0, dtype=torch.bfloat16, device=dev)
    ops.sdpa(q, k, v, 0.125, out=buf.permute(0, 2, 1, 3))
    torch.cuda.synchronize()
    want, wabs = oracle(orc, q, k, v, 0.125, "bf16")
    assert_attn_close(buf.permute(0, 2, 1, 3), want, wabs, "bf16", True, "token-major out")


def _pattern_f32(index):
    return ((np.asarray(index) % 23).astype(np.float32) - np.float32(11.0)) * np.float32(0.1)


@pytest.mark.parametrize("t,tkv,seeds", [(17, 17, (1, 2, 3)), (9, 7, (4, 5, 6))])
def test_sdpa_reference_kat_f32(dev, ops, orc, t, tkv, seeds):
    """The reference's sparse self / cross attention tests
    (tests/trellis2_sparse.rs:521-623): H=2, head_dim 8, pattern_f32 inputs,
    scale 1/sqrt(8), max |diff| < 1e-5 against naive attention; here against
    the oracle, on the generic f32 kernel."""
    h, hd = 2, 8
    arrs = [_pattern_f32(np.arange(h * n * hd) * 7 + s * 3).reshape(1, h, n, hd)
            for n, s in ((t, seeds[0]), (tkv, seeds[1]), (tkv, seeds[2]))]
    q, k, v = (torch.from_numpy(a).to(dev) for a in arrs)
    scale = float(np.float32(1.0 / np.sqrt(np.float32(hd))))
    out = ops.sdpa(q, k, v, scale)
    torch.cuda.synchronize()
    want, wabs = oracle(orc, q, k, v, scale, "f32")
    got = out.cpu().numpy()
    assert np.abs(got - want).max() < 1e-5
    assert_attn_close(out, want, wabs, "f32", False, f"kat {t}x{tkv}")


@pytest.mark.parametrize("case", ["f32_unaligned", "bf16_d80", "bf16_unaligned", "f16_d32", "bf16_d256"])
def test_sdpa_generic_kernel(dev, ops, orc, case):
    _print_case(case=case)
    dt = case.split("_")[0]
    d = {"f32_unaligned": 64, "bf16_d80": 80, "bf16_unaligned": 64, "f16_d32": 32, "bf16_d256": 256}[case]
    g = torch.Generator(device="cpu").manual_seed(len(case) * 31 + d)
    lq, lk = 77, 130
    if case.endswith("_unaligned"):
        # rows start one element past a 16-byte boundary: the generic kernel takes it
        qb = torch.randn((1, 2, lq, d + 1), generator=g).to(dev).to(TDT[dt])
        q = qb[..., 1:]
    else:
        q = torch.randn((1, 2, lq, d), generator=g).to(dev).to(TDT[dt])
    k = torch.randn((1, 2, lk, d), generator=g).to(dev).to(TDT[dt])
    v = torch.randn((1, 2, lk, d), generator=g).to(dev).to(TDT[dt])
    scale = 1.0 / np.sqrt(d)
    out = ops.sdpa(q, k, v, scale)
    torch.cuda.synchronize()
    want, wabs = oracle(orc, q, k, v, scale, dt)
    assert_attn_close(out, want, wabs, dt, False, case)


@pytest.mark.parametrize("b,n,h,d,lk", [(2, 300, 3, 64, None), (1, 257, 2, 128, None), (1, 77, 2, 128, 130),
                                         (1, 1, 1, 64, 1), (1, 33, 2, 64, 1000), (1, 40, 2, 64, 96),
                                         (1, 64, 1, 128, 32)])
def test_sdpa_f32_matrix_cores(dev, ops, orc, b, n, h, d, lk):
    """f32 q, k, v with D 64 / 128 take the matrix-core kernel for f32
    (attn_f32x3_kernel: three-term bf16 splits, f32 scores and
    probabilities), held to the f32 bar: self-attention on the permuted views
    of a fused qkv buffer, and cross-attention with key counts that leave a
    partial block or fill whole blocks (no key clamp at all)."""
    _print_case(op="sdpa f32 mfma", b=b, n=n, h=h, d=d, lk=lk)
    if lk is None:
        q, k, v = qkv_views(dev, b, n, h, d, "f32", 17 + n)
    else:
        g = torch.Generator(device="cpu").manual_seed(n + lk)
        q = torch.randn((b, h, n, d), generator=g).to(dev)
        k = torch.randn((b, h, lk, d), generator=g).to(dev)
        v = torch.randn((b, h, lk, d), generator=g).to(dev)
    scale = 1.0 / np.sqrt(d)
    out = ops.sdpa(q, k, v, scale)
    torch.cuda.synchronize()
    want, wabs = oracle(orc, q, k, v, scale, "f32")
    assert_attn_close(out, want, wabs, "f32", False, f"f32 mfma {b}x{h}x{n}x{d} lk={lk}")


@pytest.mark.parametrize("b,dt", [(5, "bf16"), (6, "bf16"), (8, "bf16"), (8, "f16")])
def test_sdpa_vggt_frames_sampled(dev, ops, orc, b, dt):
    """VGGT frame attention over b frames (1374 tokens, 16 heads, D 64):
    the launcher runs 256-query workgroups for 5 and 8 frames and 128-query
    ones for 6 (whichever leaves the busiest CU less work); the oracle checks
    32 sampled queries of every head."""
    n, h, d = 1374, 16, 64
    _print_case(op="sdpa frames sampled", b=b, n=n, h=h, d=d, dt=dt)
    q, k, v = qkv_views(dev, b, n, h, d, dt, 40 + b)
    out = ops.sdpa(q, k, v, 0.125)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(b).choice(n, 32, replace=False))
    qs = np.ascontiguousarray(host(q, dt)[:, :, rows])
    odt = orc.BF16 if dt == "bf16" else orc.F16
    want, wabs = orc.sdpa(qs, host(k, dt), host(v, dt), 0.125, dt=odt, with_abs=True)
    got = out[:, :, torch.from_numpy(rows).to(dev)]
    assert_attn_close(got, want, wabs, dt, True, f"{b} frames sampled {dt}")


def test_sdpa_vggt_global_attention_sampled(dev, ops, orc):
    """VGGT global attention (8 frames x 1374 tokens = 10992 per head, 16
    heads, D 64); the oracle checks 64 sampled queries of every head."""
    b, n, h, d = 1, 8 * 1374, 16, 64
    q, k, v = qkv_views(dev, b, n, h, d, "bf16", 5)
    out = ops.sdpa(q, k, v, 0.125)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(3).choice(n, 64, replace=False))
    qs = np.ascontiguousarray(host(q, "bf16")[:, :, rows])
    want, wabs = orc.sdpa(qs, host(k, "bf16"), host(v, "bf16"), 0.125, dt=orc.BF16, with_abs=True)
    got = out[:, :, torch.from_numpy(rows).to(dev)]
    assert_attn_close(got, want, wabs, "bf16", True, "global sampled")


def test_sdpa_graph_replay_matches_eager(dev, ops):
    q, k, v = qkv_views(dev, 2, 500, 4, 128, "bf16", 9)
    eager = ops.sdpa(q, k, v, 0.088)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            ops.sdpa(q, k, v, 0.088, out=out)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("d,case", [(64, "fused"), (128, "fused"), (64, "unaligned_q"), (64, "bf16_tables"),
                                    (64, "no_bias")])
def test_sdpa_layernorm_rope2d_equals_the_two_launches(dev, ops, orc, d, case):
    """VGGT attention with q's LayerNorm + 2D RoPE in the Q load
    (vggt.rs:170-183) equals lux3d_qk_layernorm_rope2d followed by lux3d_sdpa
    bit for bit (the same arithmetic); the fused result is also checked
    against the oracle's LayerNorm+RoPE then attention."""
    from lux3d_fused import synth
    _print_case(op="sdpa_layernorm_rope2d", d=d, case=case)
    b, h = 2, 4
    pos = synth.vggt_positions(b, 37, 37)           # [b, 1374, 2]: 5 specials + the 37 x 37 grid
    n = pos.shape[1]
    g = torch.Generator(device="cpu").manual_seed(d + len(case))
    width = d + 1 if case == "unaligned_q" else d
    qkv = (torch.randn((b, n, 3, h, width), generator=g) * 2 + 0.5).to(dev).to(torch.bfloat16).permute(2, 0, 3, 1, 4)
    q_raw, k_raw, v = qkv[0][..., -d:], qkv[1][..., :d], qkv[2][..., :d]
    qw = (1 + 0.1 * torch.randn(d, generator=g)).to(dev)
    qb = (0.1 * torch.randn(d, generator=g)).to(dev) if case != "no_bias" else None
    kw = (1 + 0.1 * torch.randn(d, generator=g)).to(dev)
    kb = (0.1 * torch.randn(d, generator=g)).to(dev)
    emb = ops.Rope2d(100.0).embeddings(torch.from_numpy(pos).to(dev), d)
    if case == "bf16_tables":
        emb = ops.RopeEmbeddings(emb.cos_full.to(torch.bfloat16), emb.sin_alt_full.to(torch.bfloat16))
    k_n = ops.apply_layernorm_rope(k_raw, (kw, kb, 1e-6), emb)
    scale = 1.0 / np.sqrt(d)
    fused = ops.sdpa_layernorm_rope2d(q_raw, (qw, qb, 1e-6), emb, k_n, v, scale)
    q_n = ops.apply_layernorm_rope(q_raw, (qw, qb, 1e-6), emb)
    two = ops.sdpa(q_n, k_n, v, scale)
    torch.cuda.synchronize()
    assert torch.equal(fused, two)
    if case == "fused":
        qo = orc.layernorm_rope2d(host(q_raw, "bf16"), qw.cpu().numpy(), qb.cpu().numpy(), 1e-6,
                                  emb.cos_full.reshape(b, n, d).cpu().numpy(),
                                  emb.sin_alt_full.reshape(b, n, d).cpu().numpy(), dt=orc.BF16)
        want, wabs = orc.sdpa(qo, host(k_n, "bf16"), host(v, "bf16"), scale, dt=orc.BF16, with_abs=True)
        # the oracle's q may differ from the kernel's by the LayerNorm+RoPE
        # tolerance (2 bf16 ulp): allow that on top of the attention bound
        g64, w64 = to_f64(host(fused, "bf16"), "bf16"), to_f64(want, "bf16")
        bound = 2 * ULP["bf16"] * np.abs(w64) + 4 * ULP["bf16"] * wabs.astype(np.float64) + 1e-6
        assert np.all(np.abs(g64 - w64) <= bound)


def test_sdpa_layernorm_rope2d_vggt_frames_equals_the_two_launches(dev, ops):
    """The configs[1] shape (8 frames, 16 heads, D 64), where both the fused
    q LayerNorm + RoPE attention and lux3d_sdpa run 256-query workgroups:
    the fused result equals the two launches bit for bit."""
    from lux3d_fused import synth
    b, h, d = 8, 16, 64
    _print_case(op="sdpa_layernorm_rope2d frames", b=b, h=h, d=d)
    pos = synth.vggt_positions(b, 37, 37)
    n = pos.shape[1]
    g = torch.Generator(device="cpu").manual_seed(77)
    qkv = (torch.randn((b, n, 3, h, d), generator=g) * 2 + 0.5).to(dev).to(torch.bfloat16).permute(2, 0, 3, 1, 4)
    q_raw, k_raw, v = qkv[0], qkv[1], qkv[2]
    qw, qb = (1 + 0.1 * torch.randn(d, generator=g)).to(dev), (0.1 * torch.randn(d, generator=g)).to(dev)
    kw, kb = (1 + 0.1 * torch.randn(d, generator=g)).to(dev), (0.1 * torch.randn(d, generator=g)).to(dev)
    emb = ops.Rope2d(100.0).embeddings(torch.from_numpy(pos).to(dev), d)
    k_n = ops.apply_layernorm_rope(k_raw, (kw, kb, 1e-6), emb)
    fused = ops.sdpa_layernorm_rope2d(q_raw, (qw, qb, 1e-6), emb, k_n, v, 0.125)
    two = ops.sdpa(ops.apply_layernorm_rope(q_raw, (qw, qb, 1e-6), emb), k_n, v, 0.125)
    torch.cuda.synchronize()
    assert torch.isfinite(fused.float()).all()
    assert torch.equal(fused, two)


@pytest.mark.parametrize("dt,d,lk", [("f32", 64, 200), ("f32", 128, 77), ("bf16", 128, 200), ("bf16", 64, 130),
                                     ("f16", 128, 33)])
def test_sdpa_keys_past_lk_are_not_read(dev, ops, orc, dt, d, lk):
    """K and V are views into a larger buffer whose rows Lk .. Lk + 63 of
    every head hold NaN: every read stays inside the allocation, and a kernel
    that fetched a key past Lk would turn the masked 0 * V into NaN outputs.
    Lk leaves a partial last block on every path (32-key f32 blocks, 64-key
    bf16 / f16 blocks), including the direct-load ones (bf16 / f16 D 128)."""
    _print_case(op="sdpa nan tail", dt=dt, d=d, lk=lk)
    b, h, lq = 2, 3, 96
    g = torch.Generator(device="cpu").manual_seed(lk * 3 + d)
    buf = torch.full((2, b, h, lk + 64, d), float("nan"))
    buf[:, :, :, :lk] = torch.randn((2, b, h, lk, d), generator=g)
    buf = buf.to(dev).to(TDT[dt])
    k, v = buf[0, :, :, :lk], buf[1, :, :, :lk]
    q = torch.randn((b, h, lq, d), generator=g).to(dev).to(TDT[dt])
    scale = 1.0 / np.sqrt(d)
    out = ops.sdpa(q, k, v, scale)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all(), "a key past Lk reached the output"
    want, wabs = oracle(orc, q, k, v, scale, dt)
    assert_attn_close(out, want, wabs, dt, dt != "f32", f"nan tail {dt} d={d} lk={lk}")


def _reversed_keys(t):
    """Descriptor of [B, H, L, D] `t` read with the token order reversed
    (data at the last token, a negative token stride)."""
    from lux3d_fused import _lib
    import ctypes
    st = list(t.stride())
    ptr = t.data_ptr() + (t.shape[2] - 1) * st[2] * t.element_size()
    code = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}[t.dtype]
    return ctypes.pointer(_lib.descriptor(ptr, code, list(t.shape), [st[0], st[1], -st[2], st[3]]))


@pytest.mark.parametrize("dt,d,lk", [("f32", 64, 200), ("f32", 128, 77), ("bf16", 128, 200), ("f16", 128, 65)])
def test_sdpa_register_staged_path_matches_direct_loads(dev, ops, dt, d, lk):
    """The register-staged K / V kernels run when the direct loads cannot
    address a head's keys (a negative token stride here). Keys and values
    read backwards through a negative stride, and the same keys flipped into
    a contiguous buffer, are the same logical sequence: the two paths must
    agree bit for bit. (f32 has only the register-staged kernel, which must
    take the negative stride the same way.)"""
    from lux3d_fused import _lib
    _print_case(op="sdpa register path", dt=dt, d=d, lk=lk)
    b, h, lq = 1, 2, 130
    g = torch.Generator(device="cpu").manual_seed(lk + d)
    k = torch.randn((b, h, lk, d), generator=g).to(dev).to(TDT[dt])
    v = torch.randn((b, h, lk, d), generator=g).to(dev).to(TDT[dt])
    q = torch.randn((b, h, lq, d), generator=g).to(dev).to(TDT[dt])
    scale = 1.0 / np.sqrt(d)
    direct = ops.sdpa(q, k.flip(2).contiguous(), v.flip(2).contiguous(), scale)
    staged = torch.empty_like(direct)
    _lib.call("lux3d_sdpa", ops.desc(q), _reversed_keys(k), _reversed_keys(v), float(scale), ops.desc(staged),
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(direct, staged)
