"""GPU parity of the Q8_0 linear with candle's CPU arithmetic
(lux3d_q8_0_quantize + lux3d_q8_0_linear_int8) against the oracle's
restatement (or_quantize_q8_0, or_q8_0_linear_int8; pinned in
tests/test_oracle_pins.py). The bar is bit-exact: the activation blocks
byte for byte, and y bit for bit (the int32 block dots are exact and the
f32 fold runs in the reference's block order with every operation rounded).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


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


def special_rows(k):
    """Rows exercising the quantization's special cases: zeros, a NaN and an
    inf in a block, huge values (d overflows f16), tiny values (d subnormal
    in f16), exact half-way products, and a constant block."""
    rng = np.random.default_rng(11)
    rows = [np.zeros(k), rng.normal(0, 1, k), rng.normal(0, 1e-6, k), rng.normal(0, 1e7, k),
            np.full(k, -3.25), np.tile(np.arange(32) - 15.5, k // 32)]
    r = rng.normal(0, 1, k)
    r[5] = np.nan
    rows.append(r)
    r = rng.normal(0, 1, k)
    r[40 % k] = np.inf
    rows.append(r)
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("case", ["random", "special"])
def test_q8_0_quantize_bit_exact(dev, ops, orc, synth, case):
    print(f"\n[case] q8_0_quantize {case}", flush=True)
    if case == "random":
        x = synth.normal(91, 37 * 1024).reshape(37, 1024).astype(np.float32)
    else:
        x = special_rows(96)
    xq, xd = ops.q8_0_quantize(torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    want = orc.quantize_q8_0(x).reshape(-1, 34)
    got_q = xq.cpu().numpy().reshape(-1, 32).view(np.uint8)
    want_d = want[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    assert np.array_equal(got_q, want[:, 2:])
    got_d = xd.cpu().numpy().reshape(-1)
    assert np.array_equal(np.isnan(got_d), np.isnan(want_d))
    assert np.array_equal(got_d[~np.isnan(got_d)].view(np.uint32), want_d[~np.isnan(want_d)].view(np.uint32))


@pytest.mark.parametrize("m,n,k,bias", [(1029, 4096, 1024, True),   # configs[4]: DINOv3 ViT-L MLP fc1 shape
                                         (3, 70, 96, False),          # ragged tiles, three blocks
                                         (130, 64, 32, True),         # one block
                                         (65, 129, 2048, False),
                                         (100, 130, 64, True),        # last tile: upper wavefronts partly live
                                         (40, 64, 160, False)])       # one tile, upper wavefronts partly live
def test_q8_0_linear_int8_bit_exact(dev, ops, orc, synth, m, n, k, bias):
    print(f"\n[case] q8_0_linear_int8 m={m} n={n} k={k} bias={bias}", flush=True)
    x = synth.normal(92, m * k).reshape(m, k).astype(np.float32)
    blocks = synth.q8_0_blocks(93, n * k // 32)
    b = synth.normal(94, n, 0.0, 0.1).astype(np.float32) if bias else None
    qs, scales = ops.q8_0_repack(torch.from_numpy(blocks).to(dev), n, k)
    y = ops.q8_0_linear_int8(torch.from_numpy(x).to(dev), qs, scales,
                             torch.from_numpy(b).to(dev) if bias else None)
    torch.cuda.synchronize()
    want = orc.q8_0_linear_int8(x, blocks, n, b)
    got = y.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{int((got != want).sum())} of {got.size} differ, worst {np.abs(got - want).max()}"


def test_q8_0_linear_int8_strided_rows(dev, ops, orc, synth):
    """x rows with a stride (a column slice of a wider buffer), as the
    reference's chunked GeGLU halves arrive; y matches the contiguous x."""
    print("\n[case] q8_0_linear_int8 strided x", flush=True)
    m, n, k = 40, 96, 256
    wide = synth.normal(95, m * 2 * k).reshape(m, 2 * k).astype(np.float32)
    blocks = synth.q8_0_blocks(96, n * k // 32)
    qs, scales = ops.q8_0_repack(torch.from_numpy(blocks).to(dev), n, k)
    xd = torch.from_numpy(wide).to(dev)[:, k:]
    y = ops.q8_0_linear_int8(xd, qs, scales)
    torch.cuda.synchronize()
    want = orc.q8_0_linear_int8(np.ascontiguousarray(wide[:, k:]), blocks, n)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_q8_0_linear_int8_rejects(dev, ops):
    print("\n[case] q8_0_linear_int8 argument checks", flush=True)
    from lux3d_fused import Lux3dError
    qs = torch.zeros((64, 64), dtype=torch.int8, device=dev)
    scales = torch.zeros((64, 2), dtype=torch.float32, device=dev)
    with pytest.raises(Lux3dError):  # bf16 x: the CPU custom op takes f32 only
        ops.q8_0_linear_int8(torch.zeros((4, 64), dtype=torch.bfloat16, device=dev), qs, scales)
    with pytest.raises(Lux3dError):  # feature count differs from the weight's
        ops.q8_0_linear_int8(torch.zeros((4, 96), dtype=torch.float32, device=dev), qs, scales)
