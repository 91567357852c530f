"""Empty inputs through the C ABI: zero rows, zero tokens, zero elements,
zero Q8_0 blocks, no queries and no voxels. candle's ops return empty
tensors for them (an empty `Tensor` flows through `layer_norm`, `rope`,
`gelu`, `dequantize` with no work done); every entry point here must accept
them, launch no work over the empty input (sparse_neighbors still clears its
hash table) and return LUX3D_OK, so that the stream stays clean for the next
call. Each test ends with a synchronize (which raises on a stream error) and
one non-empty call checked against the oracle."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

from conftest import assert_bf16_close  # noqa: E402


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
    return o


def _bf16(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def _vec(dev, d, mean, std, seed):
    v = np.random.default_rng(seed).normal(mean, std, d).astype(np.float32)
    return v, torch.from_numpy(v).to(dev)


def _rows(dev, r, d, seed):
    x = torch.from_numpy(np.random.default_rng(seed).normal(0.0, 1.0, (r, d)).astype(np.float32))
    return x.to(dev).to(torch.bfloat16)


def test_empty_row_ops(dev, ops, orc):
    print("\n[case] empty rows: layer_norm, residual_layer_norm, adaln_modulate, gated_residual", flush=True)
    d = 256
    wn, w = _vec(dev, d, 1.0, 0.05, 1)
    bn, b = _vec(dev, d, 0.0, 0.1, 2)
    x0 = torch.empty((1, 0, d), dtype=torch.bfloat16, device=dev)
    p = torch.zeros((1, d), dtype=torch.float32, device=dev)
    assert ops.layer_norm(x0, w, b, 1e-5).shape == (1, 0, d)
    h, y = ops.residual_layer_norm(x0, x0, w, w, b, 1e-5)
    assert h.shape == (1, 0, d) and y.shape == (1, 0, d)
    assert ops.adaln_modulate(x0, p, p).shape == (1, 0, d)
    assert ops.adaln_modulate(x0, p, p, p).shape == (1, 0, d)
    assert ops.gated_residual(x0, x0, p).shape == (1, 0, d)
    so = torch.tensor([0, 0, 0], dtype=torch.int64, device=dev)  # two empty ragged segments
    p2 = torch.zeros((2, d), dtype=torch.float32, device=dev)
    x2 = x0.reshape(0, d)
    assert ops.adaln_modulate(x2, p2, p2, seg_offsets=so).shape == (0, d)
    assert ops.gated_residual(x2, x2, p2, seg_offsets=so).shape == (0, d)
    torch.cuda.synchronize()
    # the next non-empty call on the same stream
    x = _rows(dev, 37, d, 3)
    got = ops.layer_norm(x, w, b, 1e-5)
    torch.cuda.synchronize()
    assert_bf16_close(_bf16(got), orc.layer_norm(_bf16(x), wn, bn, 1e-5, dt=orc.BF16), what="after empty")


def test_empty_head_ops(dev, ops, orc):
    print("\n[case] empty tokens: qk_layernorm_rope2d (tables, positions), rms_norm_heads, qk_l2norm_rope3d, "
          "dinov3 rope", flush=True)
    H, D = 16, 64
    qkv = torch.empty((1, 0, 3, H, D), dtype=torch.bfloat16, device=dev)
    perm = qkv.permute(2, 0, 3, 1, 4)
    q, k = perm[0], perm[1]  # [1, H, 0, D]
    w, b = torch.ones(D, device=dev), torch.zeros(D, device=dev)
    pos = torch.empty((1, 0, 2), dtype=torch.int32, device=dev)
    qo, ko = ops.qk_layernorm_rope2d(q, k, (w, b, 1e-5), (w, b, 1e-5), positions=pos, base=100.0)
    assert qo.shape == (1, H, 0, D) and ko.shape == (1, H, 0, D)
    tab = torch.empty((1, 1, 0, D), dtype=torch.float32, device=dev)
    qo, ko = ops.qk_layernorm_rope2d(q, k, (w, b, 1e-5), (w, b, 1e-5), ops.RopeEmbeddings(tab, tab))
    assert qo.shape == (1, H, 0, D) and ko.shape == (1, H, 0, D)
    w128 = torch.ones(128, device=dev)
    qkv128 = torch.empty((1, 0, H, 3 * 128), dtype=torch.bfloat16, device=dev)
    q1, k1 = qkv128[..., 0:128].transpose(1, 2), qkv128[..., 128:256].transpose(1, 2)
    qo, ko = ops.rms_norm_heads(q1, w128, 1e-6, k=k1, k_weight=w128)
    assert qo.shape == (1, H, 0, 128) and ko.shape == (1, H, 0, 128)
    qkv3 = torch.empty((1, 0, 3, H, 128), dtype=torch.bfloat16, device=dev)
    g = torch.ones((H, 128), dtype=torch.float32, device=dev)
    coords = torch.empty((0, 3), dtype=torch.int32, device=dev)
    qo, ko = ops.qk_l2norm_rope3d(qkv3[:, :, 0], qkv3[:, :, 1], g, g, coords=coords)
    assert qo.shape == (1, 0, H, 128) and ko.shape == (1, 0, H, 128)
    cs = torch.empty((0, D), dtype=torch.float32, device=dev)
    qo, ko = ops.apply_rotary_to_patches(q, k, cs, cs, 0)
    assert qo.shape == (1, H, 0, D) and ko.shape == (1, H, 0, D)
    torch.cuda.synchronize()
    # the next non-empty call on the same stream
    n = 21
    qkv = _rows(dev, n * 3 * H, D, 4).reshape(1, n, 3, H, D)
    perm = qkv.permute(2, 0, 3, 1, 4)
    pos = np.zeros((1, n, 2), dtype=np.int32)
    pos[0, :, 0], pos[0, :, 1] = np.arange(n) // 5, np.arange(n) % 5
    wn, bn = np.ones(D, np.float32), np.zeros(D, np.float32)
    qo, _ = ops.qk_layernorm_rope2d(perm[0], perm[1], (w, b, 1e-5), (w, b, 1e-5),
                                    positions=torch.from_numpy(pos).to(dev), base=100.0)
    torch.cuda.synchronize()
    cos, sin = orc.rope2d_tables(pos, D, 100.0)
    want = orc.layernorm_rope2d(np.ascontiguousarray(_bf16(perm[0])), wn, bn, 1e-5, cos, sin, dt=orc.BF16)
    assert_bf16_close(_bf16(qo), want, what="after empty")


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_empty_pointwise(dev, ops, orc, dt):
    print(f"\n[case] empty elements: gelu_tanh, gelu_erf, silu, timestep_embedding, dequant_q8_0 ({dt})",
          flush=True)
    x0 = torch.empty((0,), dtype=dt, device=dev)
    for fn in (ops.gelu, ops.gelu_erf, ops.silu):
        assert fn(x0).shape == (0,)
        assert fn(torch.empty((4, 0, 8), dtype=dt, device=dev)).shape == (4, 0, 8)
    t0 = torch.empty((0,), dtype=torch.float32, device=dev)
    assert ops.timestep_embedding(t0, 256).shape == (0, 256)
    assert ops.timestep_embedding(t0, 256, cos_first=False).shape == (0, 256)
    blocks = torch.empty((0,), dtype=torch.uint8, device=dev)
    assert ops.dequantize_q8_0(blocks, (0, 32), dtype=dt).shape == (0, 32)
    torch.cuda.synchronize()
    # the next non-empty call on the same stream: bit-exact Q8_0 dequant
    nb = 40
    raw = np.random.default_rng(5).integers(0, 256, (nb, 34), dtype=np.uint8)
    raw[:, 0:2] = np.frombuffer(np.full(nb, 0.0123, np.float16).tobytes(), np.uint8).reshape(nb, 2)
    y = ops.dequantize_q8_0(torch.from_numpy(raw.reshape(-1)).to(dev), (nb, 32), dtype=torch.float32)
    torch.cuda.synchronize()
    want = orc.dequant_q8_0(raw.reshape(-1), out_dt=orc.F32).reshape(nb, 32)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_empty_next_rows(dev, ops, orc):
    print("\n[case] empty: sdpa (no queries), q8_0_linear / q8_0_linear_int8 (no rows), sparse_neighbors "
          "(no voxels)", flush=True)
    q0 = torch.empty((1, 4, 0, 64), dtype=torch.bfloat16, device=dev)
    kv = torch.zeros((1, 4, 10, 64), dtype=torch.bfloat16, device=dev)
    assert ops.sdpa(q0, kv, kv, 0.125).shape == (1, 4, 0, 64)
    n, k = 32, 64
    raw = np.random.default_rng(6).integers(0, 256, (n * k // 32, 34), dtype=np.uint8)
    raw[:, 0:2] = np.frombuffer(np.full(n * k // 32, 0.02, np.float16).tobytes(), np.uint8).reshape(-1, 2)
    qs, scales = ops.q8_0_repack(torch.from_numpy(raw.reshape(-1)).to(dev), n, k)
    assert ops.q8_0_linear(torch.empty((0, k), dtype=torch.bfloat16, device=dev), qs, scales).shape == (0, n)
    assert ops.q8_0_linear_int8(torch.empty((0, k), dtype=torch.float32, device=dev), qs, scales).shape == (0, n)
    assert ops.sparse_neighbors(torch.empty((0, 3), dtype=torch.int32, device=dev)).shape == (0, 27)
    torch.cuda.synchronize()
    # the next non-empty call on the same stream: neighbour indices, exact
    g = np.stack(np.meshgrid(np.arange(3), np.arange(3), np.arange(4), indexing="ij"), -1).reshape(-1, 3)
    c = np.ascontiguousarray(g[::-1], dtype=np.int32)  # 36 distinct voxels, not in scan order
    nbr = ops.sparse_neighbors(torch.from_numpy(c).to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(nbr.cpu().numpy(), orc.sparse_neighbors(c))
