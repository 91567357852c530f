"""Weights read from GGUF / safetensors files onto the GPU
(lux3d_fused.weights): Q8_0 tensors dequantized by the library's kernel
(bit-exact against the oracle), a Q8_0 weight used as a quantized linear
(against the oracle's dequantize-then-matmul), and float conversions (one
round to nearest even)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

import gguf_spec as gs  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def W(dev):
    from lux3d_fused import weights
    return weights


@pytest.fixture(scope="module")
def orc():
    import lux3d_oracle as o
    o.set_threads(16)
    return o


@pytest.fixture(scope="module")
def synth():
    from lux3d_fused import synth as s
    return s


def test_gguf_q8_0_weight_dequant_and_linear(tmp_path, dev, W, orc, synth):
    n, k, m = 384, 512, 77
    blocks = synth.q8_0_blocks(41, n * k // 32)
    bias = synth.normal(42, n, 0.0, 0.5)
    norm = synth.normal(43, k, 1.0, 0.02)
    p = tmp_path / "model.gguf"
    gs.write(str(p), [("blk.0.ffn.weight", gs.GGML_Q8_0, [n, k], blocks.tobytes()),
                      ("blk.0.ffn.bias", gs.GGML_F32, [n], gs.f32_bytes(bias)),
                      ("blk.0.norm.weight", gs.GGML_F16, [k], gs.f16_bytes(norm))],
             [("lux3d.family", gs.STRING, "triposg")])
    g = W.GgufFile(str(p))
    print("\n[case] gguf q8_0 dequant + linear", flush=True)
    # dequant: bit-exact against the oracle
    for dt, code in ((torch.bfloat16, orc.BF16), (torch.float32, orc.F32), (torch.float16, orc.F16)):
        got = g.get("blk.0.ffn.weight", dt, dev)
        torch.cuda.synchronize()
        want = orc.dequant_q8_0(blocks, code).reshape(n, k)
        host = got.cpu()
        host = host.numpy() if dt == torch.float32 else host.view(torch.int16).numpy().view(np.uint16)
        if dt == torch.float16:
            want = want.view(np.uint16) if want.dtype == np.float16 else want
        assert np.array_equal(host.reshape(-1).view(np.uint8), np.ascontiguousarray(want).reshape(-1).view(np.uint8))
    # quantized linear from the file
    mm = g.get_qmatmul("blk.0.ffn.weight", n, k, dev)
    x = torch.from_numpy(synth.normal(44, m * k).reshape(m, k)).to(dev).to(torch.bfloat16)
    y = mm.forward(x, g.get("blk.0.ffn.bias", torch.float32, dev), torch.float32)
    torch.cuda.synchronize()
    xb = x.cpu().view(torch.int16).numpy().view(np.uint16)
    want, abs_sum = orc.q8_0_linear(xb, blocks, n, bias.astype(np.float32), orc.F32, with_abs=True)
    err = np.abs(y.cpu().numpy().astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= 2.0 ** -23 * np.abs(want) + 2.0 ** -16 * abs_sum + 1e-30)
    # f16 -> bf16: one RNE rounding of the exact f16 value
    nb = g.get("blk.0.norm.weight", torch.bfloat16, dev).cpu()
    ref = torch.from_numpy(np.asarray(norm, dtype=np.float16).astype(np.float32)).to(torch.bfloat16)
    assert torch.equal(nb, ref)
    with pytest.raises(W.WeightsError, match="does not match expected"):
        g.get_qmatmul("blk.0.ffn.weight", k, n, dev)


def test_safetensors_to_device(tmp_path, dev, W):
    from safetensors.torch import save_file
    gen = torch.Generator().manual_seed(8)
    ts = {"qkv.weight": torch.randn(192, 64, generator=gen).to(torch.bfloat16),
          "norm.weight": torch.randn(64, generator=gen)}
    p = tmp_path / "m.safetensors"
    save_file(ts, str(p))
    s = W.SafetensorsFile(str(p))
    print("\n[case] safetensors to device", flush=True)
    a = s.get("qkv.weight", torch.bfloat16, dev)
    b = s.get("norm.weight", torch.bfloat16, dev)
    torch.cuda.synchronize()
    assert torch.equal(a.cpu(), ts["qkv.weight"])
    assert torch.equal(b.cpu(), ts["norm.weight"].to(torch.bfloat16))
