"""GPU parity of the Q8_0 quantized linear (lux3d_q8_0_repack +
lux3d_q8_0_linear) against the oracle's dequantize-then-matmul
(or_q8_0_linear, pinned in tests/test_oracle_pins.py).

Tolerance: the GPU accumulates the K products in f32 on the matrix cores and
the oracle in f64, so an output may differ by the f32 accumulation error
(held to 2^-16 of sum_k |x*w|, the scale of that error) plus one unit of
the output dtype's last place.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

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


def to_f64(a, dt):
    if dt == "bf16":
        return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    if dt == "f16":
        return np.asarray(a, dtype=np.uint16).view(np.float16).astype(np.float64)
    return np.asarray(a, dtype=np.float32).astype(np.float64)


def host(t, dt):
    t = t.detach().contiguous().cpu()
    return t.numpy() if dt == "f32" else t.view(torch.int16).numpy().view(np.uint16)


def assert_gemm_close(got, want, abs_sum, dt, what):
    g, w = to_f64(got, dt), to_f64(want, dt)
    ulp = {"bf16": 2.0 ** -7, "f16": 2.0 ** -10, "f32": 2.0 ** -23}[dt]
    bound = ulp * np.abs(w) + 2.0 ** -16 * abs_sum.astype(np.float64) + 1e-30
    err = np.abs(g - w)
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} outputs out of tolerance; worst err "
                           f"{err.max():.3e} (bound there {bound.reshape(-1)[np.argmax(err)]:.3e})")


def make_problem(synth, orc, dev, m, k, n, seed, bias=True):
    x = synth.normal(seed, m * k).reshape(m, k)
    xd = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    blocks = synth.q8_0_blocks(seed + 1, n * k // 32)
    b = synth.normal(seed + 2, n, 0.0, 0.5) if bias else None
    return xd, blocks, b


# K % 64 == 0 takes the LDS-ring kernel: at these sizes (fewer than 256
# tiles of 256 rows) 160 x 128 tiles when 128 x 128 ones would exceed the CUs
# (1029 x 1024 -> 4096: 7 x 32 tiles), 128 x 128 tiles of four wavefronts
# otherwise; (77, 96, 100) takes the 128 x 128 kernel with 32-deep k-steps.
# The 256-row ring tiles: the ring-kernel test and the large sampled test
# below.
@pytest.mark.parametrize("m,k,n", [(1029, 1024, 4096), (300, 256, 200), (1, 64, 32), (129, 2048, 136), (77, 96, 100),
                                   (64, 128, 100)])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_q8_0_linear_matches_oracle(dev, ops, orc, synth, m, k, n, out):
    print(f"\n[case] q8_0_linear m={m} k={k} n={n} out={out}", flush=True)
    xd, blocks, b = make_problem(synth, orc, dev, m, k, n, 300 + m)
    bd = torch.from_numpy(blocks).to(dev)
    mm = ops.QMatMul.from_q8_0(bd, n, k)
    y = mm.forward(xd, torch.from_numpy(b).to(dev), TDT[out])
    torch.cuda.synchronize()
    want, abs_sum = orc.q8_0_linear(host(xd, "bf16"), blocks, n, b, orc.F32 if out == "f32" else orc.BF16,
                                    with_abs=True)
    assert_gemm_close(host(y, out), want, abs_sum, out, f"q8_0_linear {m}x{k}x{n}")


def test_q8_0_repack_is_exact(dev, ops, synth):
    n, k = 96, 160
    blocks = synth.q8_0_blocks(321, n * k // 32)
    qs, scales = ops.q8_0_repack(torch.from_numpy(blocks).to(dev), n, k)
    torch.cuda.synchronize()
    b = blocks.reshape(n * k // 32, 34)
    assert np.array_equal(qs.cpu().numpy().reshape(-1), b[:, 2:].view(np.int8).reshape(-1))
    assert np.array_equal(scales.cpu().numpy().reshape(-1),
                          b[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1))


def test_q8_0_linear_no_bias_f16_out_and_strided_rows(dev, ops, orc, synth):
    """No bias, f16 output, x and y as row-strided views of wider buffers."""
    m, k, n = 200, 512, 384
    xd, blocks, _ = make_problem(synth, orc, dev, m, k, n, 700, bias=False)
    xwide = torch.zeros((m, k + 64), dtype=torch.bfloat16, device=dev)
    xwide[:, :k] = xd
    ywide = torch.zeros((m, n + 32), dtype=torch.float16, device=dev)
    qs, scales = ops.q8_0_repack(torch.from_numpy(blocks).to(dev), n, k)
    from lux3d_fused import _lib
    _lib.call("lux3d_q8_0_linear", ops.desc(xwide[:, :k]), ops.desc(qs), ops.desc(scales), None,
              ops.desc(ywide[:, :n]), None)
    torch.cuda.synchronize()
    want, abs_sum = orc.q8_0_linear(host(xd, "bf16"), blocks, n, None, orc.F16, with_abs=True)
    assert_gemm_close(host(ywide[:, :n], "f16"), want, abs_sum, "f16", "f16 out, strided rows")
    assert torch.all(ywide[:, n:] == 0), "columns past n must stay untouched"


@pytest.mark.parametrize("out", ["bf16", "f32", "f16"])
@pytest.mark.parametrize("extra", [0, 3])
def test_q8_0_linear_ring_kernel(dev, ops, orc, synth, out, extra):
    """The LDS-ring kernel with 256-row tiles: x [4353, 128] -> [4353, 3700]
    is 18 x 15 = 270 tiles (not a multiple of the 8 XCDs), the last tile row
    holds one row and the last column piece 4 columns. y is a view of a buffer `extra`
    columns wider: 16-byte aligned rows (extra 0) take the LDS-staged
    epilogue, unaligned rows (extra 3) the one-element-per-store one. The
    oracle checks the first and last 40 rows and 48 sampled between."""
    m, k, n = 4353, 128, 3700
    print(f"\n[case] q8_0_linear ring kernel out={out} ldy={n + extra}", flush=True)
    xd, blocks, b = make_problem(synth, orc, dev, m, k, n, 760 + extra)
    ywide = torch.zeros((m, n + extra), dtype=TDT[out], device=dev)
    qs, scales = ops.q8_0_repack(torch.from_numpy(blocks).to(dev), n, k)
    bd = torch.from_numpy(b).to(dev)
    from lux3d_fused import _lib
    _lib.call("lux3d_q8_0_linear", ops.desc(xd), ops.desc(qs), ops.desc(scales), ops.desc(bd), ops.desc(ywide[:, :n]),
              None)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(40), np.arange(m - 40, m),
                                     np.random.default_rng(6).choice(m, 48, replace=False)]))
    code = {"bf16": orc.BF16, "f32": orc.F32, "f16": orc.F16}[out]
    want, abs_sum = orc.q8_0_linear(host(xd, "bf16")[rows], blocks, n, b, code, with_abs=True)
    assert_gemm_close(host(ywide[:, :n], out)[rows], want, abs_sum, out, "ring kernel")
    if extra:
        assert torch.all(ywide[:, n:] == 0), "columns past n must stay untouched"


def test_q8_0_linear_ring_kernel_128_row_tiles(dev, ops, orc, synth):
    """x [3800, 128] -> [3800, 4096]: 15 x 16 tiles of 256 rows would leave
    CUs idle, so the ring kernel runs with 30 x 16 tiles of 128 rows (the
    last holding 88 rows); sampled rows."""
    m, k, n = 3800, 128, 4096
    print(f"\n[case] q8_0_linear ring kernel 128-row tiles {m}x{k}x{n}", flush=True)
    xd, blocks, b = make_problem(synth, orc, dev, m, k, n, 780)
    mm = ops.QMatMul.from_q8_0(torch.from_numpy(blocks).to(dev), n, k)
    y = mm.forward(xd, torch.from_numpy(b).to(dev))
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(24), np.arange(m - 100, m),
                                     np.random.default_rng(9).choice(m, 40, replace=False)]))
    want, abs_sum = orc.q8_0_linear(host(xd, "bf16")[rows], blocks, n, b, orc.BF16, with_abs=True)
    assert_gemm_close(host(y, "bf16")[rows], want, abs_sum, "bf16", "ring kernel, 128-row tiles")


def test_q8_0_linear_large_sampled_rows(dev, ops, orc, synth):
    """A TripoSG-sized projection (x [4096, 2048] -> [4096, 8192]); the oracle
    checks a sample of 96 rows."""
    m, k, n = 4096, 2048, 8192
    xd, blocks, b = make_problem(synth, orc, dev, m, k, n, 900)
    mm = ops.QMatMul.from_q8_0(torch.from_numpy(blocks).to(dev), n, k)
    y = mm.forward(xd, torch.from_numpy(b).to(dev))
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(5).choice(m, 96, replace=False))
    xs = host(xd, "bf16")[rows]
    want, abs_sum = orc.q8_0_linear(xs, blocks, n, b, orc.BF16, with_abs=True)
    assert_gemm_close(host(y, "bf16")[rows], want, abs_sum, "bf16", "sampled rows")


# f32 activations: the reference dequantizes the weights exactly to f32
# (q * d) and sums f32 products; the kernel forms each Q8_0 block's sum of
# x q exactly-split products on the bf16 matrix cores and scales it by d, the
# same sum up to its order. The same f32 accumulation tolerance as above. (4353, 128, 3700) has 35 x 15 = 525 tiles of 128 rows,
# the last holding one row, the last column piece 116 columns.
@pytest.mark.parametrize("m,k,n", [(1029, 1024, 4096), (300, 256, 200), (1, 64, 32), (129, 2048, 136),
                                   (4353, 128, 3700)])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_q8_0_linear_f32_activations(dev, ops, orc, synth, m, k, n, out):
    print(f"\n[case] q8_0_linear f32 x m={m} k={k} n={n} out={out}", flush=True)
    x = synth.normal(1300 + m, m * k).reshape(m, k)
    xd = torch.from_numpy(x).to(dev)
    blocks = synth.q8_0_blocks(1301 + m, n * k // 32)
    b = synth.normal(1302 + m, n, 0.0, 0.5)
    mm = ops.QMatMul.from_q8_0(torch.from_numpy(blocks).to(dev), n, k)
    y = mm.forward(xd, torch.from_numpy(b).to(dev), TDT[out])
    torch.cuda.synchronize()
    rows = np.arange(m) if m <= 1100 else np.unique(np.concatenate(
        [np.arange(40), np.arange(m - 40, m), np.random.default_rng(8).choice(m, 48, replace=False)]))
    want, abs_sum = orc.q8_0_linear(np.ascontiguousarray(x[rows]), blocks, n, b,
                                    orc.F32 if out == "f32" else orc.BF16, with_abs=True)
    assert_gemm_close(host(y, out)[rows], want, abs_sum, out, f"q8_0_linear f32 x {m}x{k}x{n}")


def test_q8_0_linear_f32_strided_and_rejects_k96(dev, ops, orc, synth):
    """f32 x and bf16 y as row-strided views (x rows 16-byte aligned, y rows
    not: the one-element-per-store epilogue); f32 x with k % 64 != 0 is
    rejected before any launch."""
    from lux3d_fused import _lib
    from lux3d_fused._lib import Lux3dError
    m, k, n = 333, 320, 264
    print(f"\n[case] q8_0_linear f32 x strided m={m} k={k} n={n}", flush=True)
    x = synth.normal(1400, m * k).reshape(m, k)
    xwide = torch.zeros((m, k + 4), dtype=torch.float32, device=dev)
    xwide[:, :k] = torch.from_numpy(x).to(dev)
    ywide = torch.zeros((m, n + 3), dtype=torch.bfloat16, device=dev)
    blocks = synth.q8_0_blocks(1401, n * k // 32)
    qs, scales = ops.q8_0_repack(torch.from_numpy(blocks).to(dev), n, k)
    _lib.call("lux3d_q8_0_linear", ops.desc(xwide[:, :k]), ops.desc(qs), ops.desc(scales), None,
              ops.desc(ywide[:, :n]), None)
    torch.cuda.synchronize()
    want, abs_sum = orc.q8_0_linear(x, blocks, n, None, orc.BF16, with_abs=True)
    assert_gemm_close(host(ywide[:, :n], "bf16"), want, abs_sum, "bf16", "f32 x, strided rows")
    assert torch.all(ywide[:, n:] == 0), "columns past n must stay untouched"
    x96 = torch.zeros((4, 96), dtype=torch.float32, device=dev)
    q96, s96 = ops.q8_0_repack(torch.from_numpy(synth.q8_0_blocks(1402, 32 * 3)).to(dev), 32, 96)
    y96 = torch.zeros((4, 32), dtype=torch.float32, device=dev)
    with pytest.raises(Lux3dError, match="multiple of 64"):
        _lib.call("lux3d_q8_0_linear", ops.desc(x96), ops.desc(q96), ops.desc(s96), None, ops.desc(y96), None)


@pytest.mark.parametrize("out", ["bf16", "f32"])
@pytest.mark.parametrize("extra", [0, 3])
def test_q8_0_linear_four_wavefront_tiles(dev, ops, orc, synth, out, extra):
    """x [300, 192] -> [300, 200]: 3 x 1 tiles of 128 x 256 cannot fill the
    CUs, so the ring kernel runs 3 x 2 tiles of 128 x 128
    with four wavefronts (the last column tile holds 72 columns, the last row
    tile 44 rows). y is a view of a buffer `extra` columns wider: aligned
    rows take the staged epilogue, unaligned rows the per-element stores."""
    m, k, n = 300, 192, 200
    print(f"\n[case] q8_0_linear four-wavefront tiles out={out} ldy={n + extra}", flush=True)
    xd, blocks, b = make_problem(synth, orc, dev, m, k, n, 820 + extra)
    ywide = torch.zeros((m, n + extra), dtype=TDT[out], device=dev)
    qs, scales = ops.q8_0_repack(torch.from_numpy(blocks).to(dev), n, k)
    from lux3d_fused import _lib
    _lib.call("lux3d_q8_0_linear", ops.desc(xd), ops.desc(qs), ops.desc(scales), ops.desc(torch.from_numpy(b).to(dev)),
              ops.desc(ywide[:, :n]), None)
    torch.cuda.synchronize()
    want, abs_sum = orc.q8_0_linear(host(xd, "bf16"), blocks, n, b, orc.F32 if out == "f32" else orc.BF16,
                                    with_abs=True)
    assert_gemm_close(host(ywide[:, :n], out), want, abs_sum, out, "four-wavefront tiles")
    if extra:
        assert torch.all(ywide[:, n:] == 0), "columns past n must stay untouched"



@pytest.mark.parametrize("out", ["bf16", "f32", "f16"])
@pytest.mark.parametrize("extra", [0, 3])
@pytest.mark.parametrize("m", [1029, 1001])
def test_q8_0_linear_160_row_tiles(dev, ops, orc, synth, out, extra, m):
    """[m, 1024] -> 4096 (the configs[4] weight): 9 x 32 tiles of 128 x 128
    would exceed the 256 CUs, 7 x 32 of 160 x 128 do not, so those run (one
    per CU). The last row tile holds 69 (m 1029) or 41 (m 1001) rows; y rows
    aligned (staged epilogue) or not (per-element stores)."""
    k, n = 1024, 4096
    print(f"\n[case] q8_0_linear 160-row tiles m={m} out={out} ldy={n + extra}", flush=True)
    xd, blocks, b = make_problem(synth, orc, dev, m, k, n, 900 + m + extra)
    ywide = torch.zeros((m, n + extra), dtype=TDT[out], device=dev)
    qs, scales = ops.q8_0_repack(torch.from_numpy(blocks).to(dev), n, k)
    from lux3d_fused import _lib
    _lib.call("lux3d_q8_0_linear", ops.desc(xd), ops.desc(qs), ops.desc(scales), ops.desc(torch.from_numpy(b).to(dev)),
              ops.desc(ywide[:, :n]), None)
    torch.cuda.synchronize()
    odt = {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}[out]
    want, abs_sum = orc.q8_0_linear(host(xd, "bf16"), blocks, n, b, odt, with_abs=True)
    assert_gemm_close(host(ywide[:, :n], out), want, abs_sum, out, f"160-row tiles m={m}")
    if extra:
        assert torch.all(ywide[:, n:] == 0), "columns past n must stay untouched"
