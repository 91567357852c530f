"""HIP-graph capture of the fused ops (as bench.py times them): a captured
graph replayed several times, with eager work and synchronisations between
the replays, must reproduce the eager results bit-for-bit on every replay.
No memset nodes are involved: every op writes all of its outputs."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda:0")


def test_graph_replays_match_eager(dev):
    print("\n[case] graph replay of residual_layer_norm + qk_layernorm_rope2d_pos + gelu", flush=True)
    from lux3d_fused import ops, synth
    B, N, C, H, D = 2, 5 + 9 * 9, 1024, 16, 64
    T = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dt or torch.float32)  # noqa: E731
    x = T(synth.normal(1, B * N * C).reshape(B, N, C), torch.bfloat16)
    a = T(synth.normal(2, B * N * C).reshape(B, N, C), torch.bfloat16)
    g, w, b = T(synth.normal(3, C, 1.0, 0.02)), T(synth.normal(4, C, 1.0, 0.02)), T(synth.normal(5, C, 0.0, 0.02))
    qkv = T(synth.normal(6, B * N * 3 * H * D).reshape(B, N, 3, H, D), torch.bfloat16)
    perm = qkv.permute(2, 0, 3, 1, 4)
    pos = torch.from_numpy(synth.vggt_positions(B, 9, 9)).to(dev)
    qw, qb = T(synth.normal(7, D, 1.0, 0.02)), T(synth.normal(8, D, 0.0, 0.02))
    h = torch.empty_like(x)
    y = torch.empty_like(x)
    qo = torch.empty((B, H, N, D), dtype=torch.bfloat16, device=dev)
    ko = torch.empty_like(qo)
    act_in = T(synth.normal(9, 4096 * 8), torch.bfloat16)
    act_out = torch.empty_like(act_in)
    from lux3d_fused import _lib

    def run():
        s = torch.cuda.current_stream().cuda_stream
        _lib.call("lux3d_residual_layer_norm", ops.desc(x), ops.desc(a), ops.desc(g), ops.desc(w), ops.desc(b),
                  1e-5, ops.desc(h), ops.desc(y), s)
        _lib.call("lux3d_qk_layernorm_rope2d_pos", ops.desc(perm[0]), ops.desc(qw), ops.desc(qb), ops.desc(perm[1]),
                  ops.desc(qw), ops.desc(qb), 1e-5, ops.desc(pos), 100.0, ops.desc(qo), ops.desc(ko), s)
        _lib.call("lux3d_gelu_tanh", ops.desc(act_in), ops.desc(act_out), s)

    run()
    torch.cuda.synchronize()
    eager = [t.clone() for t in (h, y, qo, ko, act_out)]
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        run()
    for rep in range(4):
        for t in (h, y, qo, ko, act_out):
            t.fill_(float("nan"))           # eager work between replays (a fill kernel, not a memset node)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip((h, y, qo, ko, act_out), eager):
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"replay {rep} differs from eager"


def test_graph_replays_of_the_persistent_residual_layer_norm(dev):
    """Long 2-byte jobs of rows of 1024 run the persistent residual +
    LayerNorm kernel (its grid is sized from the device's CU count, looked up
    on the first launch): captured and replayed, bit-identical to eager."""
    print("\n[case] graph replay of the persistent residual_layer_norm [2, 2501, 1024] bf16", flush=True)
    from lux3d_fused import ops, synth, _lib
    B, N, C = 2, 2501, 1024
    T = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dt or torch.float32)  # noqa: E731
    x = T(synth.normal(21, B * N * C).reshape(B, N, C), torch.bfloat16)
    a = T(synth.normal(22, B * N * C).reshape(B, N, C), torch.bfloat16)
    g, w, b = T(synth.normal(23, C, 1.0, 0.02)), T(synth.normal(24, C, 1.0, 0.02)), T(synth.normal(25, C, 0.0, 0.02))
    h = torch.empty_like(x)
    y = torch.empty_like(x)

    def run():
        s = torch.cuda.current_stream().cuda_stream
        _lib.call("lux3d_residual_layer_norm", ops.desc(x), ops.desc(a), ops.desc(g), ops.desc(w), ops.desc(b),
                  1e-5, ops.desc(h), ops.desc(y), s)

    run()
    torch.cuda.synchronize()
    eager = [t.clone() for t in (h, y)]
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        run()
    for rep in range(4):
        for t in (h, y):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip((h, y), eager):
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"replay {rep} differs from eager"


def test_graph_replays_of_the_newer_entries(dev):
    """The same check for the fused gated residual + modulate, exact_sdpa_heads
    on bf16 (three-term probabilities), f32 attention (three-term splits) and
    the allocation-free coordinate map (its static table is cleared by its
    own first kernel on every replay, and the bad-coordinate counter by the
    same kernel)."""
    print("\n[case] graph replay of gated_residual_adaln_modulate + sdpa_heads_f32 + f32 sdpa + neighbors_noalloc",
          flush=True)
    from lux3d_fused import ops, synth, _lib
    T = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dt or torch.float32)  # noqa: E731
    rows, C = 3000, 1536
    x = T(synth.normal(11, rows * C).reshape(rows, C), torch.bfloat16)
    hh = T(synth.normal(12, rows * C).reshape(rows, C), torch.bfloat16)
    te = T(synth.normal(13, 2 * 6 * C, 0.0, 0.1).reshape(2, 6 * C))
    pieces = ops.chunk_modulation(te)
    so = torch.tensor([0, 1200, rows], dtype=torch.int64, device=dev)
    x_out, y_mod = torch.empty_like(x), torch.empty_like(x)
    qkv = T(synth.normal(14, 300 * 3 * 4 * 64).reshape(1, 300, 3, 4, 64), torch.bfloat16).permute(2, 0, 3, 1, 4)
    o_ex = torch.empty((1, 4, 300, 64), dtype=torch.bfloat16, device=dev)
    qkv32 = T(synth.normal(15, 260 * 3 * 4 * 64).reshape(1, 260, 3, 4, 64)).permute(2, 0, 3, 1, 4)
    o32 = torch.empty((1, 4, 260, 64), dtype=torch.float32, device=dev)
    rng = np.random.default_rng(16)
    flat = rng.choice(48 ** 3, size=5000, replace=False)
    c = np.stack([flat // 2304, (flat // 48) % 48, flat % 48], axis=1).astype(np.int32) - 24
    c[7, 0] = (1 << 20) + 3  # one coordinate outside the packable range
    coords = torch.from_numpy(c).to(dev)
    nbr = torch.empty((5000, 27), dtype=torch.int32, device=dev)
    bad = torch.empty((1,), dtype=torch.int32, device=dev)
    d = ops.desc

    def run():
        s = torch.cuda.current_stream().cuda_stream
        _lib.call("lux3d_gated_residual_adaln_modulate", d(x), d(hh), d(so), d(pieces[2]), None, d(pieces[3]), None,
                  d(pieces[4]), None, 1e-6, d(x_out), d(y_mod), s)
        _lib.call("lux3d_sdpa_heads_f32", d(qkv[0]), d(qkv[1]), d(qkv[2]), 0.125, d(o_ex), s)
        _lib.call("lux3d_sdpa", d(qkv32[0]), d(qkv32[1]), d(qkv32[2]), 0.125, d(o32), s)
        _lib.call("lux3d_sparse_neighbors_noalloc", d(coords), d(nbr), d(bad), s)

    outs = (x_out, y_mod, o_ex, o32, nbr, bad)
    run()
    torch.cuda.synchronize()
    eager = [t.clone() for t in outs]
    assert int(bad.item()) == 1
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        run()
    for rep in range(4):
        for t in outs:
            t.fill_(-7 if t.dtype == torch.int32 else float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(outs, eager):
            a = got.view(torch.int16) if got.dtype == torch.bfloat16 else got
            b = want.view(torch.int16) if want.dtype == torch.bfloat16 else want
            assert torch.equal(a, b), f"replay {rep} differs from eager"


def test_graph_replays_of_the_fused_attentions(dev):
    """Graph replays of the attention entries that normalise / rotate q in
    the Q load (TripoSG RMSNorm, TRELLIS.2 L2 norm + 3D RoPE, DINOv3
    rotation in f32 and bf16) and of the two-key-group attention (DINOv3's
    1029 tokens, bf16 exact and rounded probabilities): every replay equals
    the eager run bit for bit."""
    print("\n[case] graph replay of the fused attentions + key groups", flush=True)
    from lux3d_fused import ops, _lib
    g = torch.Generator(device="cpu").manual_seed(21)

    def rnd(shape, dt=torch.bfloat16, scale=1.0):
        return (torch.randn(shape, generator=g) * scale).to(dev).to(dt)

    # TripoSG: per-head thirds of [1, 300, 2, 3 * 128]
    th = rnd((1, 300, 2, 384))
    tq, tk, tv = (th[..., i * 128:(i + 1) * 128].transpose(1, 2) for i in range(3))
    tw = rnd((128,), torch.float32, 0.1) + 1
    to = torch.empty((1, 2, 300, 128), dtype=torch.bfloat16, device=dev)
    # TRELLIS.2: [1, 257, 3, 2, 128], tables [257, 64]
    tr = rnd((1, 257, 3, 2, 128))
    coords = torch.randint(0, 40, (257, 3), generator=g, dtype=torch.int32).to(dev)
    cos3, sin3 = ops.Trellis2Rope3d(128).cos_sin(coords)
    gam = rnd((2, 128), torch.float32, 0.1) + 1
    tro = torch.empty((1, 2, 257, 128), dtype=torch.bfloat16, device=dev)
    # DINOv3: [1, 16, 1029, 64] f32 and bf16 (the bf16 exact path runs two key groups)
    d32 = rnd((3, 1, 1029, 16, 64), torch.float32)
    d16 = d32.to(torch.bfloat16)
    ang = torch.rand((1024, 64), generator=g) * 6.3
    dc, ds = torch.cos(ang).to(dev), torch.sin(ang).to(dev)
    do32 = torch.empty((1, 16, 1029, 64), dtype=torch.float32, device=dev)
    do16 = torch.empty((1, 16, 1029, 64), dtype=torch.bfloat16, device=dev)
    dsd = torch.empty((1, 16, 1029, 64), dtype=torch.bfloat16, device=dev)
    d = ops.desc

    def run():
        s = torch.cuda.current_stream().cuda_stream
        _lib.call("lux3d_sdpa_rms_norm_heads", d(tq), d(tw), 1e-6, d(tk), d(tv), 0.0884, d(to), s)
        _lib.call("lux3d_sdpa_l2norm_rope3d", d(tr[:, :, 0].transpose(1, 2)), d(gam), d(cos3), d(sin3),
                  d(tr[:, :, 1].transpose(1, 2)), d(tr[:, :, 2].transpose(1, 2)), 0.0884, d(tro), s)
        _lib.call("lux3d_sdpa_dinov3_rope", d(d32[0].transpose(1, 2)), d(dc), d(ds), 5, d(d32[1].transpose(1, 2)),
                  d(d32[2].transpose(1, 2)), 0.125, d(do32), s)
        _lib.call("lux3d_sdpa_dinov3_rope", d(d16[0].transpose(1, 2)), d(dc), d(ds), 5, d(d16[1].transpose(1, 2)),
                  d(d16[2].transpose(1, 2)), 0.125, d(do16), s)
        _lib.call("lux3d_sdpa", d(d16[0].transpose(1, 2)), d(d16[1].transpose(1, 2)), d(d16[2].transpose(1, 2)),
                  0.125, d(dsd), s)

    outs = (to, tro, do32, do16, dsd)
    run()
    torch.cuda.synchronize()
    eager = [t.clone() for t in outs]
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        run()
    for rep in range(4):
        for t in outs:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(outs, eager):
            a = got.view(torch.int16) if got.dtype == torch.bfloat16 else got.view(torch.int32)
            b = want.view(torch.int16) if want.dtype == torch.bfloat16 else want.view(torch.int32)
            assert torch.equal(a, b), f"replay {rep} differs from eager"
