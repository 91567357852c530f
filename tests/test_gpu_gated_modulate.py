"""GPU parity of lux3d_gated_residual_adaln_modulate: the gated residual of
Trellis2SparseBlock::forward followed by the MLP half's AdaLN modulate
(runtime/trellis2_blocks.rs:708-713), and the ungated cross-attention add
then modulate of Trellis2DenseBlock::forward (:637-642), in one launch.

Against the oracle (or_gated_residual_modulate, pinned in
tests/test_oracle_pins.py): the residual stream x_out bit-exact, the
modulated rows y within 2 bf16 ulp (f32: 1e-5 relative; see conftest.py).
"""
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


@pytest.fixture(scope="module")
def synth():
    from lux3d_fused import synth as s
    return s


def dev_tensor(a, dt, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev).to(TDT[dt])


def host_view(t, dt):
    t = t.detach().contiguous().cpu()
    if dt == "f32":
        return t.numpy()
    if dt == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy().view(np.uint16)


def ocode(orc, dt):
    return {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}[dt]


def check_y(got, want, dt, what):
    g = host_view(got, dt)
    if dt == "f32":
        return assert_f32_close(g, want, what=what)
    if dt == "bf16":
        return assert_bf16_close(g, want, what=what)
    return assert_f16_close(g, np.asarray(want).view(np.uint16), what=what)


def run_case(dev, ops, orc, x, h, offs, t_emb, modulation, C, dt, gated=True, with_base=True, ragged=True,
             in_place=False, what=""):
    """The sparse block's MLP half: gate_msa = chunk 2, shift_mlp / scale_mlp
    = chunks 3 / 4 of modulation + t_emb (chunk_modulation order)."""
    xd, hd = dev_tensor(x, dt, dev), dev_tensor(h, dt, dev)
    x_in = host_view(xd, dt)
    pieces = ops.chunk_modulation(torch.from_numpy(t_emb).to(dev))
    base = torch.from_numpy(modulation).to(dev).chunk(6)
    so = torch.from_numpy(offs).to(dev) if ragged else None
    gb = (lambda k: base[k]) if with_base else (lambda k: None)
    xo, y = ops.gated_residual_adaln_modulate(xd, hd, pieces[2] if gated else None, pieces[3], pieces[4],
                                              gate_base=gb(2) if gated else None, shift_base=gb(3),
                                              scale_base=gb(4), seg_offsets=so, eps=1e-6,
                                              x_out=xd if in_place else None)
    torch.cuda.synchronize()
    if in_place:
        assert xo.data_ptr() == xd.data_ptr()
    sl = lambda k: np.ascontiguousarray(t_emb[:, k * C:(k + 1) * C])  # noqa: E731
    bl = (lambda k: modulation[k * C:(k + 1) * C]) if with_base else (lambda k: None)  # noqa: E731
    want_x, want_y = orc.gated_residual_modulate(x_in, host_view(hd, dt), offs, sl(2) if gated else None, sl(3),
                                                 sl(4), bl(2) if gated else None, bl(3), bl(4), eps=1e-6,
                                                 dt=ocode(orc, dt))
    got_x = host_view(xo, dt)
    assert np.array_equal(got_x, want_x), f"{what}: residual stream differs from the oracle " \
                                          f"({int((got_x != want_x).sum())} elements)"
    check_y(y, want_y, dt, what)


def test_sparse_block_cfg3_ragged(dev, ops, orc, synth):
    """ragged 24k + 40k voxels x 1536, per-segment gate / shift /
    scale on top of the block's `modulation` vector."""
    print("\n[case] gated_residual_adaln_modulate configs[3] ragged", flush=True)
    C, sizes = 1536, (24000, 40000)
    seed = synth.config_seed(3)
    n = sum(sizes)
    x = synth.normal(seed, n * C).reshape(n, C)
    h = synth.normal(seed + 5, n * C).reshape(n, C)
    t_emb = synth.normal(seed + 1, 2 * 6 * C, 0.0, 0.1).reshape(2, 6 * C)
    modulation = synth.normal(seed + 2, 6 * C, 0.0, 0.1)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    run_case(dev, ops, orc, x, h, offs, t_emb, modulation, C, "bf16", what="cfg3 ragged")


@pytest.mark.parametrize("gated", [True, False])
def test_dense_block_cfg2(dev, ops, orc, synth, gated):
    """configs[2] shape [2, 2048, 2048] dense (one segment per batch element,
    no offsets); ungated = the dense block's cross-attention add."""
    print(f"\n[case] gated_residual_adaln_modulate configs[2] dense gated={gated}", flush=True)
    B, L, C = 2, 2048, 2048
    seed = synth.config_seed(2)
    x = synth.normal(seed, B * L * C).reshape(B, L, C)
    h = synth.normal(seed + 6, B * L * C).reshape(B, L, C)
    t_emb = synth.normal(seed + 7, B * 6 * C, 0.0, 0.1).reshape(B, 6 * C)
    modulation = synth.normal(seed + 8, 6 * C, 0.0, 0.1)
    offs = np.array([0, L, 2 * L], dtype=np.int64)
    run_case(dev, ops, orc, x, h, offs, t_emb, modulation, C, "bf16", gated=gated, with_base=gated, ragged=False,
             what=f"cfg2 dense gated={gated}")


# segment boundaries inside workgroups of several rows (per-row pieces there)
@pytest.mark.parametrize("sizes,C", [((2049, 1, 1027, 2000), 1536), ((1031, 1031, 1031), 2048),
                                     ((5, 3000, 1), 1024)])
def test_straddling_segments(dev, ops, orc, synth, sizes, C):
    print(f"\n[case] gated_residual_adaln_modulate segments {sizes} C={C}", flush=True)
    S, n = len(sizes), sum(sizes)
    x = synth.normal(191, n * C).reshape(n, C)
    h = synth.normal(192, n * C).reshape(n, C)
    t_emb = synth.normal(193, S * 6 * C, 0.0, 0.1).reshape(S, 6 * C)
    modulation = synth.normal(194, 6 * C, 0.0, 0.1)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    run_case(dev, ops, orc, x, h, offs, t_emb, modulation, C, "bf16", what=f"straddling {sizes}")


@pytest.mark.parametrize("dt,C,rows", [("f32", 1024, 3000), ("f16", 2048, 700), ("f32", 1536, 900),
                                       ("bf16", 1000, 300), ("f16", 72, 50), ("bf16", 2048, 1029)])
def test_dtypes_and_widths(dev, ops, orc, synth, dt, C, rows):
    """f32 / f16, short jobs (< 2048 rows: rows split over wavefronts) and
    widths the vector kernel does not take (1000, 72: the generic kernel)."""
    print(f"\n[case] gated_residual_adaln_modulate {dt} C={C} rows={rows}", flush=True)
    x = synth.normal(201 + C, rows * C).reshape(rows, C)
    h = synth.normal(202 + C, rows * C).reshape(rows, C)
    t_emb = synth.normal(203, 2 * 6 * C, 0.0, 0.1).reshape(2, 6 * C)
    modulation = synth.normal(204, 6 * C, 0.0, 0.1)
    offs = np.array([0, rows // 3, rows], dtype=np.int64)
    run_case(dev, ops, orc, x, h, offs, t_emb, modulation, C, dt, what=f"{dt} C={C}")


def test_in_place_residual_stream(dev, ops, orc, synth):
    """x_out = x: the residual stream updated in place."""
    print("\n[case] gated_residual_adaln_modulate in place", flush=True)
    C, n = 1536, 5000
    x = synth.normal(211, n * C).reshape(n, C)
    h = synth.normal(212, n * C).reshape(n, C)
    t_emb = synth.normal(213, 2 * 6 * C, 0.0, 0.1).reshape(2, 6 * C)
    modulation = synth.normal(214, 6 * C, 0.0, 0.1)
    offs = np.array([0, 1234, n], dtype=np.int64)
    run_case(dev, ops, orc, x, h, offs, t_emb, modulation, C, "bf16", in_place=True, what="in place")


def test_equals_the_two_launches(dev, ops, synth):
    """x_out equals lux3d_gated_residual's bit for bit; y agrees with
    lux3d_adaln_modulate on that x_out within 2 ulp."""
    print("\n[case] gated_residual_adaln_modulate vs two launches", flush=True)
    C, sizes = 1536, (3000, 5000)
    n = sum(sizes)
    xd = dev_tensor(synth.normal(221, n * C).reshape(n, C), "bf16", dev)
    hd = dev_tensor(synth.normal(222, n * C).reshape(n, C), "bf16", dev)
    te = torch.from_numpy(synth.normal(223, 2 * 6 * C, 0.0, 0.1).reshape(2, 6 * C)).to(dev)
    pieces = ops.chunk_modulation(te)
    so = torch.from_numpy(np.array([0, sizes[0], n], dtype=np.int64)).to(dev)
    xo, y = ops.gated_residual_adaln_modulate(xd, hd, pieces[2], pieces[3], pieces[4], seg_offsets=so)
    x2 = ops.gated_residual(xd, hd, pieces[2], seg_offsets=so)
    y2 = ops.adaln_modulate(x2, pieces[3], pieces[4], seg_offsets=so, eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(xo, x2)
    assert_bf16_close(host_view(y, "bf16"), host_view(y2, "bf16"), what="fused vs two launches")


def test_empty_rows(dev, ops):
    x = torch.empty((0, 256), dtype=torch.bfloat16, device=dev)
    p = torch.zeros((1, 256), dtype=torch.float32, device=dev)
    xo, y = ops.gated_residual_adaln_modulate(x, x, p, p, p)
    torch.cuda.synchronize()
    assert xo.shape == (0, 256) and y.shape == (0, 256)
