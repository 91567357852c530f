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
