"""GPU parity sweep over the row kernels' launch layouts: row widths that
pick one, two or four wavefronts per row and one to eight 16-byte chunks per
lane (and the generic fallback), row counts either side of the 2048-row
switch between one-row workgroups and multi-row ones (and the persistent
residual + LayerNorm kernel), and every activation dtype, for each row op
against the oracle at the usual bars (residual streams bit-exact, bf16 / f16
within 2 ulp, f32 within 1e-5 of the output scale; see conftest.py).
Inputs are seeded N(0, 1) rows and N(1, 0.05) / N(0, 0.1) parameters.

Rows of 8192 (wider than any config) are allowed 4e-5 instead of 1e-5 of
their elements on the absolute floor: there the reference's single-pass
statistics (sum2 / d - mean^2, which the oracle restates) are themselves
that noisy near zero. Against a float64 LayerNorm of the same bf16 rows the
oracle has 264 of 16,777,216 elements (1.6e-5) beyond 2 ulp that pass only
through the floor at d = 8192 (46 of 4,194,304 at d = 2048); the GPU kernel
against the oracle had 263."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from conftest import assert_bf16_close, assert_f16_close, assert_f32_close  # noqa: E402

TDT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


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


def _dev(a, dt, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev).to(TDT[dt])


def _host(t, dt):
    t = t.detach().contiguous().cpu()
    if dt == "f32":
        return t.numpy()
    if dt == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _odt(orc, dt):
    return {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}[dt]


def _check(got, want, dt, what, d):
    g = _host(got, dt)
    ff = 4e-5 if d >= 8192 else None
    if dt == "f32":
        return assert_f32_close(g, want, what=what, floor_frac=ff)
    if dt == "bf16":
        return assert_bf16_close(g, want, what=what, floor_frac=ff)
    return assert_f16_close(g.view(np.uint16), np.asarray(want).view(np.uint16), what=what, floor_frac=ff)


def _rows(seed, rows, d):
    return np.random.default_rng(seed).normal(0.0, 1.0, (rows, d)).astype(np.float32)


def _vec(seed, n, mean, std, lead=()):
    return np.random.default_rng(seed).normal(mean, std, lead + (n,)).astype(np.float32)


# (width, rows, dtype): 512 / 1024 / 1536 / 2048 / 3072 / 4096 / 8192 cover
# 1-8 chunks per lane on one wavefront and 2- / 4-wavefront rows; 640 and 200
# (chunk counts no layout divides) take the generic kernel.
LN_CASES = [(512, 5, "bf16"), (1024, 1, "f32"), (1024, 2047, "bf16"), (1024, 2048, "f16"), (1536, 2049, "bf16"),
            (2048, 1023, "f32"), (3072, 2050, "bf16"), (4096, 2048, "bf16"), (4096, 100, "f32"),
            (8192, 2048, "bf16"), (8192, 7, "f16"), (640, 300, "bf16"), (200, 9, "f32")]


@pytest.mark.parametrize("d,rows,dt", LN_CASES)
def test_sweep_layer_norm(dev, ops, orc, d, rows, dt):
    print(f"\n[case] sweep layer_norm d={d} rows={rows} dt={dt}", flush=True)
    x = _dev(_rows(d * 7 + rows, rows, d), dt, dev)
    w, b = _vec(1, d, 1.0, 0.05), _vec(2, d, 0.0, 0.1)
    y = ops.layer_norm(x, torch.from_numpy(w).to(dev), torch.from_numpy(b).to(dev), 1e-5)
    torch.cuda.synchronize()
    _check(y, orc.layer_norm(_host(x, dt), w, b, 1e-5, dt=_odt(orc, dt)), dt, f"layer_norm {d}x{rows}", d)


# 2-byte rows of 1024 from 2048 rows on take the persistent kernel (at 2051
# rows some wavefronts take one row more than others); the rest row_kernel
RESID_CASES = [(1024, 2048, "bf16"), (1024, 2051, "f16"), (1024, 1, "bf16"), (1024, 2047, "f32"),
               (2048, 2049, "bf16"), (4096, 2048, "f32"), (1536, 64, "bf16"), (8192, 2049, "bf16")]


@pytest.mark.parametrize("d,rows,dt", RESID_CASES)
def test_sweep_residual_layer_norm(dev, ops, orc, d, rows, dt):
    print(f"\n[case] sweep residual_layer_norm d={d} rows={rows} dt={dt}", flush=True)
    x = _dev(_rows(d * 11 + rows, rows, d), dt, dev)
    a = _dev(_rows(d * 13 + rows, rows, d), dt, dev)
    g, w, b = _vec(3, d, 1.0, 0.05), _vec(4, d, 1.0, 0.05), _vec(5, d, 0.0, 0.1)
    T = lambda v: torch.from_numpy(v).to(dev)  # noqa: E731
    h, y = ops.residual_layer_norm(x, a, T(g), T(w), T(b), 1e-5)
    torch.cuda.synchronize()
    hw, yw = orc.residual_layer_norm(_host(x, dt), _host(a, dt), g, w, b, 1e-5, dt=_odt(orc, dt))
    assert np.array_equal(_host(h, dt), hw), "residual stream h must be bit-exact"
    _check(y, yw, dt, f"residual_layer_norm y {d}x{rows}", d)


# (width, segment sizes, dtype, with the M1' output gate)
MOD_CASES = [(2048, (2048, 2048), "bf16", False), (1536, (1000, 1, 1048), "bf16", True),
             (1024, (350, 350), "f32", False), (4096, (1025, 1025), "f16", True),
             (3072, (1024, 1024), "bf16", False), (8192, (1024, 1024), "bf16", False),
             (640, (7, 9), "bf16", True)]


def _pieces(seed, S, d, n):
    return [_vec(seed + k, d, 0.0, 0.1, (S,)) for k in range(n)]


@pytest.mark.parametrize("d,sizes,dt,gated", MOD_CASES)
def test_sweep_adaln_modulate(dev, ops, orc, d, sizes, dt, gated):
    print(f"\n[case] sweep adaln_modulate d={d} segments={sizes} dt={dt} gate={gated}", flush=True)
    n, S = sum(sizes), len(sizes)
    x = _dev(_rows(d * 17 + n, n, d), dt, dev)
    sh, sc, gt = _pieces(20, S, d, 3)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    T = lambda v: torch.from_numpy(v).to(dev)  # noqa: E731
    y = ops.adaln_modulate(x, T(sh), T(sc), T(gt) if gated else None, seg_offsets=T(offs), eps=1e-6)
    torch.cuda.synchronize()
    want = orc.adaln_modulate(_host(x, dt), offs, sh, sc, gt if gated else None, eps=1e-6, dt=_odt(orc, dt))
    _check(y, want, dt, f"adaln_modulate {d} {sizes}", d)


GATE_CASES = [(2048, (2048, 2048), "bf16"), (1536, (1000, 1049), "f32"), (1024, (50, 50), "bf16"),
              (4096, (1024, 1024), "f16"), (640, (5, 6), "bf16")]


@pytest.mark.parametrize("d,sizes,dt", GATE_CASES)
def test_sweep_gated_residual(dev, ops, orc, d, sizes, dt):
    print(f"\n[case] sweep gated_residual d={d} segments={sizes} dt={dt}", flush=True)
    n, S = sum(sizes), len(sizes)
    x = _dev(_rows(d * 19 + n, n, d), dt, dev)
    h = _dev(_rows(d * 23 + n, n, d), dt, dev)
    (gt,) = _pieces(30, S, d, 1)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    T = lambda v: torch.from_numpy(v).to(dev)  # noqa: E731
    out = ops.gated_residual(x, h, T(gt), seg_offsets=T(offs))
    torch.cuda.synchronize()
    want = orc.gated_residual(_host(x, dt), _host(h, dt), offs, gt, dt=_odt(orc, dt))
    assert np.array_equal(_host(out, dt), want), "x + h * gate must be bit-exact"


GMOD_CASES = [(2048, (1024, 1024), "bf16", True), (1536, (1000, 1049), "bf16", True),
              (1024, (350, 350), "f32", False), (4096, (1025, 1025), "f16", True), (640, (5, 6), "f32", True)]


@pytest.mark.parametrize("d,sizes,dt,gated", GMOD_CASES)
def test_sweep_gated_residual_adaln_modulate(dev, ops, orc, d, sizes, dt, gated):
    print(f"\n[case] sweep gated_residual_adaln_modulate d={d} segments={sizes} dt={dt} gate={gated}", flush=True)
    n, S = sum(sizes), len(sizes)
    x = _dev(_rows(d * 29 + n, n, d), dt, dev)
    h = _dev(_rows(d * 31 + n, n, d), dt, dev)
    gt, sh, sc = _pieces(40, S, d, 3)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    T = lambda v: torch.from_numpy(v).to(dev)  # noqa: E731
    xo, y = ops.gated_residual_adaln_modulate(x, h, T(gt) if gated else None, T(sh), T(sc), seg_offsets=T(offs),
                                              eps=1e-6)
    torch.cuda.synchronize()
    xw, yw = orc.gated_residual_modulate(_host(x, dt), _host(h, dt), offs, gt if gated else None, sh, sc, eps=1e-6,
                                         dt=_odt(orc, dt))
    assert np.array_equal(_host(xo, dt), xw), "the residual stream x' must be bit-exact"
    _check(y, yw, dt, f"gated_residual_adaln_modulate {d} {sizes}", d)


# ---- head kernels -------------------------------------------------------------
#
# The launcher fits whole heads into a workgroup pass (threads = a multiple of
# H * D / 8 rounded to wavefronts, at most 256) and takes tb tokens per
# workgroup; H = 1, 3, 12, 24, 48, 64 give tiles of 64 down to one token and
# passes with dead items, and more heads than one workgroup holds (96 or 80
# heads of 64, 80 of 128) take the generic kernel. 2-byte rows run two rows
# per thread (four for unrotated rows of 128), f32 rows one.


def _synth():
    from lux3d_fused import synth as s
    return s


@pytest.mark.parametrize("B,ph,pw,H,dt", [(2, 5, 7, 1, "bf16"), (1, 9, 9, 3, "f32"), (2, 9, 11, 12, "bf16"),
                                          (1, 13, 13, 24, "f16"), (1, 6, 6, 48, "bf16"), (1, 4, 5, 64, "bf16"),
                                          (1, 3, 3, 96, "bf16"), (1, 3, 3, 80, "f32")])
@pytest.mark.parametrize("source", ["positions", "tables"])
def test_sweep_qk_layernorm_rope2d(dev, ops, orc, B, ph, pw, H, dt, source):
    print(f"\n[case] sweep qk_layernorm_rope2d B={B} grid={ph}x{pw} H={H} dt={dt} source={source}", flush=True)
    s, D = _synth(), 64
    N = 5 + ph * pw
    qkv = _dev(_rows(H * 37 + N, B * N * 3 * H, D).reshape(B, N, 3, H, D), dt, dev)
    perm = qkv.permute(2, 0, 3, 1, 4)  # [3, B, H, N, D] views of the packed buffer
    q, k = perm[0], perm[1]
    pos = s.vggt_positions(B, ph, pw)
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)  # noqa: E731
    qw, qb, kw, kb = _vec(51, D, 1.0, 0.05), _vec(52, D, 0.0, 0.1), _vec(53, D, 1.0, 0.05), _vec(54, D, 0.0, 0.1)
    cos, sin = orc.rope2d_tables(pos, D, 100.0)
    if source == "tables":
        emb = ops.RopeEmbeddings(T(cos).unsqueeze(1), T(sin).unsqueeze(1))
        qo, ko = ops.qk_layernorm_rope2d(q, k, (T(qw), T(qb), 1e-5), (T(kw), T(kb), 1e-5), emb)
    else:
        qo, ko = ops.qk_layernorm_rope2d(q, k, (T(qw), T(qb), 1e-5), (T(kw), T(kb), 1e-5), positions=T(pos),
                                         base=100.0)
    torch.cuda.synchronize()
    odt = _odt(orc, dt)
    _check(qo, orc.layernorm_rope2d(np.ascontiguousarray(_host(q, dt)), qw, qb, 1e-5, cos, sin, dt=odt), dt,
           f"q H={H}", D)
    _check(ko, orc.layernorm_rope2d(np.ascontiguousarray(_host(k, dt)), kw, kb, 1e-5, cos, sin, dt=odt), dt,
           f"k H={H}", D)


@pytest.mark.parametrize("B,L,H,D,dt", [(2, 33, 16, 128, "bf16"), (1, 70, 4, 64, "f32"), (1, 40, 24, 128, "bf16"),
                                        (1, 10, 64, 128, "bf16"), (1, 5, 80, 128, "f16"), (3, 17, 1, 64, "bf16")])
def test_sweep_rms_norm_heads(dev, ops, orc, B, L, H, D, dt):
    print(f"\n[case] sweep rms_norm_heads B={B} L={L} H={H} D={D} dt={dt}", flush=True)
    qkv = _dev(_rows(H * 41 + L, B * L * H, 3 * D).reshape(B, L, H, 3 * D), dt, dev)
    q, k = qkv[..., 0:D].transpose(1, 2), qkv[..., D:2 * D].transpose(1, 2)  # [B, H, L, D] strided
    wq, wk = _vec(61, D, 1.0, 0.05), _vec(62, D, 1.0, 0.05)
    T = lambda v: torch.from_numpy(v).to(dev)  # noqa: E731
    qo, ko = ops.rms_norm_heads(q, T(wq), 1e-6, k=k, k_weight=T(wk))
    torch.cuda.synchronize()
    odt = _odt(orc, dt)
    _check(qo, orc.rms_norm_heads(np.ascontiguousarray(_host(q, dt)), wq, 1e-6, dt=odt), dt, f"q H={H} D={D}", D)
    _check(ko, orc.rms_norm_heads(np.ascontiguousarray(_host(k, dt)), wk, 1e-6, dt=odt), dt, f"k H={H} D={D}", D)


@pytest.mark.parametrize("N,H,D,dt", [(500, 12, 128, "bf16"), (300, 3, 128, "f32"), (200, 16, 64, "bf16"),
                                      (64, 40, 128, "bf16"), (129, 1, 128, "f16")])
def test_sweep_qk_l2norm_rope3d(dev, ops, orc, N, H, D, dt):
    print(f"\n[case] sweep qk_l2norm_rope3d N={N} H={H} D={D} dt={dt}", flush=True)
    coords = _synth().unique_voxels(71 + N, N, 64)
    qkv = _dev(_rows(H * 43 + N, N * 3 * H, D).reshape(1, N, 3, H, D), dt, dev)
    q, k = qkv[:, :, 0], qkv[:, :, 1]  # [1, N, H, D] views
    gq, gk = _vec(63, D, 1.0, 0.05, (H,)), _vec(64, D, 1.0, 0.05, (H,))
    T = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(dev)  # noqa: E731
    qo, ko = ops.qk_l2norm_rope3d(q, k, T(gq), T(gk), coords=T(coords))
    torch.cuda.synchronize()
    cos, sin = orc.rope3d_tables(coords, D)
    odt = _odt(orc, dt)
    for got, x, g, what in ((qo, q, gq, "q"), (ko, k, gk, "k")):
        want = orc.qk_l2norm_rope3d(np.ascontiguousarray(_host(x, dt)).reshape(N, H, D), g, cos, sin, dt=odt)
        _check(got, want.reshape(1, N, H, D), dt, f"{what} H={H} D={D}", D)


# ---- activations: sizes around the 8-element chunk and unaligned starts -------
#
# A 16-byte aligned start takes the vector kernel (8 elements per thread and a
# tail); any other start the element-wise one.


@pytest.mark.parametrize("act", ["gelu_tanh", "gelu_erf", "silu"])
@pytest.mark.parametrize("dt,n,offset", [("bf16", 1, 0), ("f32", 7, 0), ("f16", 9, 0), ("bf16", 17, 1),
                                         ("f32", 1000003, 3), ("bf16", 65536, 5), ("f16", 4096, 8)])
def test_sweep_activations(dev, ops, orc, act, dt, n, offset):
    print(f"\n[case] sweep {act} dt={dt} n={n} offset={offset}", flush=True)
    x = np.random.default_rng(n + offset).normal(0.0, 3.0, n + offset).astype(np.float32)
    x[offset:offset + min(n, 6)] = [0.0, -0.0, -9.0, 9.0, -30.0, 30.0][:min(n, 6)]
    xd = _dev(x, dt, dev)[offset:]  # a contiguous view starting `offset` elements in
    fn = {"gelu_tanh": ops.gelu, "gelu_erf": ops.gelu_erf, "silu": ops.silu}[act]
    y = fn(xd)
    torch.cuda.synchronize()
    ofn = {"gelu_tanh": orc.gelu_tanh, "gelu_erf": orc.gelu_erf, "silu": orc.silu}[act]
    _check(y, ofn(np.ascontiguousarray(_host(xd, dt)), dt=_odt(orc, dt)), dt, f"{act} n={n} offset={offset}", 0)


# ---- Q8_0 dequant: block counts around the staging tile, 2-byte aligned blocks --
#
# GGUF places a tensor's blocks at 2-byte alignment: a block buffer that is
# not 16-byte aligned reads its blocks with 2-byte loads, an aligned one
# stages them through LDS in tiles of blocks; every output bit-exact.


@pytest.mark.parametrize("out", ["bf16", "f32", "f16"])
@pytest.mark.parametrize("nblocks,offset", [(1, 0), (3, 2), (63, 0), (64, 2), (65, 0), (1001, 2), (100003, 0)])
def test_sweep_dequant_q8_0(dev, ops, orc, out, nblocks, offset):
    print(f"\n[case] sweep dequant_q8_0 nblocks={nblocks} offset={offset} -> {out}", flush=True)
    blocks = _synth().q8_0_blocks(900 + nblocks, nblocks)
    buf = torch.zeros(offset + blocks.size, dtype=torch.uint8, device=dev)
    buf[offset:] = torch.from_numpy(blocks).to(dev)
    y = ops.dequantize_q8_0(buf[offset:], (nblocks * 32,), TDT[out])
    torch.cuda.synchronize()
    want = orc.dequant_q8_0(blocks, _odt(orc, out))
    got = _host(y, out).reshape(-1)
    if out == "f32":
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert np.array_equal(got.view(np.uint16), np.asarray(want).view(np.uint16))


# ---- attention at key-block boundaries on the key-group path ------------------
#
# Short launches (few 128-query tiles) split each 64-key block over two key
# groups of a workgroup (D 64); these cases put Lk just below, at and above
# the block and group sizes, with 1, 31, 64, 129 and 257 queries, through
# lux3d_sdpa (bf16 / f16, the rounded-probability bound of the attention
# tests) and exact_sdpa_heads (bf16 in, f32 arithmetic, the f32 bar).

_ATTN_CASES = [(1, 63, 64, "bf16"), (31, 64, 64, "bf16"), (129, 65, 64, "bf16"), (1, 127, 64, "bf16"),
               (31, 128, 64, "bf16"), (129, 129, 64, "bf16"), (129, 192, 64, "bf16"), (257, 1029, 64, "bf16"),
               (33, 65, 64, "f16"), (64, 128, 64, "f16"), (31, 65, 128, "bf16"), (129, 127, 128, "bf16")]


def _attn_inputs(dev, lq, lk, d, dt):
    g = torch.Generator(device="cpu").manual_seed(lq * 131 + lk * 7 + d)
    q = torch.randn((1, 3, lq, d), generator=g).to(dev).to(TDT[dt])
    k = (2 * torch.randn((1, 3, lk, d), generator=g)).to(dev).to(TDT[dt])
    v = torch.randn((1, 3, lk, d), generator=g).to(dev).to(TDT[dt])
    return q, k, v


@pytest.mark.parametrize("lq,lk,d,dt", _ATTN_CASES)
def test_sweep_sdpa_key_blocks(dev, ops, orc, lq, lk, d, dt):
    from test_gpu_attention import assert_attn_close, oracle
    print(f"\n[case] sweep sdpa lq={lq} lk={lk} d={d} dt={dt}", flush=True)
    q, k, v = _attn_inputs(dev, lq, lk, d, dt)
    scale = 1.0 / np.sqrt(d)
    out = ops.sdpa(q, k, v, scale)
    torch.cuda.synchronize()
    want, wabs = oracle(orc, q, k, v, scale, dt)
    assert_attn_close(out, want, wabs, dt, True, f"sdpa {lq}x{lk}x{d} {dt}")


@pytest.mark.parametrize("lq,lk,d", [(c[0], c[1], c[2]) for c in _ATTN_CASES if c[3] == "bf16"])
def test_sweep_exact_sdpa_heads_key_blocks(dev, ops, orc, lq, lk, d):
    from test_gpu_sdpa_heads_f32 import _check as check_exact
    print(f"\n[case] sweep exact_sdpa_heads lq={lq} lk={lk} d={d}", flush=True)
    q, k, v = _attn_inputs(dev, lq, lk, d, "bf16")
    check_exact(ops, orc, q, k, v, 1.0 / np.sqrt(d), "bf16", f"exact_sdpa_heads {lq}x{lk}x{d}")
