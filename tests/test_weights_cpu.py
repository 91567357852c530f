"""GGUF / safetensors readers (include/lux3d_weights.h) on the CPU: a
hand-assembled GGUF byte sequence, round trips through a writer written from
the GGUF specification (tests/gguf_spec.py) and through the independent
`safetensors` package, and malformed files (every truncation of a valid file
must be rejected, never read out of bounds)."""
import os
import struct

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import gguf_spec as gs  # noqa: E402
from lux3d_fused import synth  # noqa: E402
from lux3d_fused import weights as W  # noqa: E402


def test_gguf_hand_assembled_bytes(tmp_path):
    """One F32 tensor `w` of candle shape [2, 3], no metadata, version 3:
    24 header bytes + 41 tensor-info bytes = 65, padded to the default
    alignment 32 -> the data starts at byte 96."""
    hexs = ("47475546" "03000000"                    # "GGUF", version 3
            "0100000000000000" "0000000000000000"    # 1 tensor, 0 metadata
            "0100000000000000" "77"                  # name: len 1, "w"
            "02000000"                               # n_dims 2
            "0300000000000000" "0200000000000000"    # dims innermost first: 3, 2
            "00000000" "0000000000000000")           # F32, offset 0
    head = bytes.fromhex(hexs)
    assert len(head) == 65
    vals = np.arange(6, dtype=np.float32) * 1.5 - 2.0
    p = tmp_path / "kat.gguf"
    p.write_bytes(head + b"\0" * (96 - 65) + vals.tobytes())
    g = W.GgufFile(str(p))
    assert g.version == 3 and len(g) == 1 and g.names() == ["w"]
    w = g.info("w")
    assert w.shape == (2, 3) and w.dtype == W.GGML_F32 and w.nbytes == 24
    assert np.array_equal(g.raw("w").view(np.float32), vals)
    assert g.metadata() == {}


def _tensors():
    blocks = synth.q8_0_blocks(5, 4 * 64 // 32)
    return [
        ("blk.0.attn.qkv.weight", gs.GGML_Q8_0, [4, 64], blocks.tobytes()),
        ("blk.0.norm.weight", gs.GGML_F16, [7], gs.f16_bytes(np.linspace(-1, 1, 7))),
        ("blk.0.norm.bias", gs.GGML_F32, [3, 5], gs.f32_bytes(np.arange(15) * 0.25)),
        ("pos_embed", gs.GGML_BF16, [2, 3, 4], gs.bf16_bytes(np.arange(24) / 7.0)),
        ("conv3d.flat", gs.GGML_F16, [1, 2, 3, 4], gs.f16_bytes(np.arange(24) - 12.0)),
    ]


def _metadata():
    return [
        ("general.architecture", gs.STRING, "trellis2"),
        ("lux3d.family", gs.STRING, "trellis2"),
        ("lux3d.quantization", gs.STRING, "q8_0"),
        ("lux3d.tensor_count", gs.U32, 5),
        ("lux3d.resolved_config", gs.STRING, '{"model_channels": 1536, "name": "é漢"}'),
        ("t.u8", gs.U8, 200), ("t.i8", gs.I8, -5), ("t.u16", gs.U16, 60000), ("t.i16", gs.I16, -30000),
        ("t.i32", gs.I32, -7), ("t.f32", gs.F32, 1.5), ("t.bool", gs.BOOL, True), ("t.u64", gs.U64, 2 ** 40),
        ("t.i64", gs.I64, -2 ** 40), ("t.f64", gs.F64, -0.125),
        ("t.arr_u32", gs.ARRAY, (gs.U32, [1, 2, 3])),
        ("t.arr_str", gs.ARRAY, (gs.STRING, ["a", "bc"])),
        ("t.arr_empty", gs.ARRAY, (gs.F32, [])),
    ]


@pytest.mark.parametrize("version,alignment", [(3, None), (3, 64), (2, 32), (1, None)])
def test_gguf_round_trip(tmp_path, version, alignment):
    p = tmp_path / "m.gguf"
    tens = _tensors()
    gs.write(str(p), tens, _metadata(), version=version, alignment=alignment)
    g = W.GgufFile(str(p))
    assert g.version == version
    assert g.names() == [t[0] for t in tens]
    for name, gt, shape, raw in tens:
        w = g.info(name)
        assert (w.dtype, w.shape, w.nbytes) == (gt, tuple(shape), len(raw)), name
        assert g.raw(name).tobytes() == raw, name
        assert (w.data - g.info(tens[0][0]).data) % (alignment or 32) == 0
    md = g.metadata()
    assert md["lux3d.family"] == "trellis2" and g.metadata_string("lux3d.family") == "trellis2"
    assert g.metadata_string("lux3d.tensor_count") is None  # not a string
    assert md["lux3d.resolved_config"] == '{"model_channels": 1536, "name": "é漢"}'
    assert (md["t.u8"], md["t.i8"], md["t.u16"], md["t.i16"], md["t.i32"]) == (200, -5, 60000, -30000, -7)
    assert (md["t.f32"], md["t.bool"], md["t.u64"], md["t.i64"], md["t.f64"]) == (1.5, True, 2 ** 40, -2 ** 40, -0.125)
    assert list(md["t.arr_u32"]) == [1, 2, 3] and len(md["t.arr_empty"]) == 0
    assert md["t.arr_str"] == ("array", gs.STRING, 2)
    if alignment:
        assert md["general.alignment"] == alignment
    assert "missing" not in g and "pos_embed" in g
    with pytest.raises(W.WeightsError, match="cannot find tensor"):
        g.info("missing")


def test_gguf_unknown_type_is_listed_unsized(tmp_path):
    p = tmp_path / "q4.gguf"
    gs.write(str(p), [("a", 2, [4, 32], b"\x01" * 40), ("b", gs.GGML_F32, [2], gs.f32_bytes([1, 2]))])
    g = W.GgufFile(str(p))
    assert g.info("a").dtype == 2 and g.info("a").nbytes == 0
    assert np.array_equal(g.raw("b").view(np.float32), [1, 2])


def test_gguf_every_truncation_is_rejected(tmp_path):
    p = tmp_path / "t.gguf"
    gs.write(str(p), _tensors()[:3], _metadata()[:6])
    full = p.read_bytes()
    W.GgufFile(str(p))  # the whole file opens
    q = tmp_path / "cut.gguf"
    for n in range(len(full)):
        q.write_bytes(full[:n])
        with pytest.raises(W.WeightsError):
            W.GgufFile(str(q))


@pytest.mark.parametrize("case", ["magic", "version", "past_end", "q8_partial", "duplicate", "rank9", "align0",
                                  "huge_count", "bad_meta_type"])
def test_gguf_malformed(tmp_path, case):
    p = tmp_path / "bad.gguf"
    t = [("w", gs.GGML_F32, [2, 3], gs.f32_bytes(np.zeros(6)))]
    msg = {"magic": "bad magic", "version": "unsupported GGUF version", "past_end": "past the end",
           "q8_partial": "whole blocks", "duplicate": "duplicate tensor", "rank9": "dims",
           "align0": "alignment", "huge_count": "exceed", "bad_meta_type": "metadata"}[case]
    if case == "magic":
        p.write_bytes(b"GGUG" + b"\0" * 60)
    elif case == "version":
        gs.write(str(p), t, version=4)
    elif case == "past_end":
        data0 = gs.write(str(p), t, offsets=[4096])
        p.write_bytes(p.read_bytes()[:data0 + 24])  # the bytes for offset 0, not 4096
    elif case == "q8_partial":
        gs.write(str(p), [("q", gs.GGML_Q8_0, [2, 48], b"\0" * 102)])
    elif case == "duplicate":
        gs.write(str(p), t + t)
    elif case == "rank9":
        gs.write(str(p), [("w", gs.GGML_F32, [1] * 9, gs.f32_bytes([0]))])
    elif case == "align0":
        gs.write(str(p), t, metadata=[("general.alignment", gs.U32, 0)])
    elif case == "huge_count":
        p.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 1 << 40, 0) + b"\0" * 64)
    elif case == "bad_meta_type":
        p.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" +
                      struct.pack("<I", 99) + b"\0" * 16)
    with pytest.raises(W.WeightsError, match=msg):
        W.GgufFile(str(p))


def test_gguf_missing_file(tmp_path):
    with pytest.raises(W.WeightsError, match="cannot open"):
        W.GgufFile(str(tmp_path / "nope.gguf"))


def test_safetensors_written_by_the_safetensors_package(tmp_path):
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(3)
    ts = {
        "norm.weight": torch.randn(1024, generator=g),
        "qkv.weight": torch.randn(96, 64, generator=g).to(torch.bfloat16),
        "proj.bias": torch.randn(7, generator=g).to(torch.float16),
        "index": torch.arange(-5, 5, dtype=torch.int64),
        "mask": torch.tensor([0, 1, 255], dtype=torch.uint8),
        "q": torch.tensor([-128, 3, 127], dtype=torch.int8),
        "scalar64": torch.tensor([1.25, -2.5], dtype=torch.float64),
        "empty": torch.zeros((0, 4)),
    }
    p = tmp_path / "m.safetensors"
    save_file(ts, str(p), metadata={"format": "pt", "lux3d.family": "vggt"})
    s = W.SafetensorsFile(str(p))
    assert sorted(s.names()) == sorted(ts)
    codes = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.int64: 4, torch.uint8: 5, torch.int8: 6,
             torch.float64: -1}
    for name, t in ts.items():
        w = s.info(name)
        assert w.shape == tuple(t.shape) and w.dtype == codes[t.dtype], name
        raw = t.contiguous().view(torch.uint8).numpy().tobytes() if t.numel() else b""
        assert s.raw(name).tobytes() == raw, name
    assert s.metadata("lux3d.family") == "vggt" and s.metadata("missing") is None
    # host-side get() conversions (device "cpu"): bf16 -> f32 is exact
    assert torch.equal(s.get("qkv.weight", torch.float32, "cpu"), ts["qkv.weight"].float())


@pytest.mark.parametrize("case", ["header_size", "not_json", "bad_offsets", "size_mismatch", "trailing"])
def test_safetensors_malformed(tmp_path, case):
    p = tmp_path / "bad.safetensors"

    def put(header: str, data: bytes = b""):
        h = header.encode()
        p.write_bytes(struct.pack("<Q", len(h)) + h + data)

    if case == "header_size":
        p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    elif case == "not_json":
        put('{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}', b"\0" * 4)
    elif case == "bad_offsets":
        put('{"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}', b"\0" * 4)
    elif case == "size_mismatch":
        put('{"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}', b"\0" * 8)
    elif case == "trailing":
        put('{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}} x', b"\0" * 4)
    with pytest.raises(W.WeightsError):
        W.SafetensorsFile(str(p))


def test_safetensors_json_escapes_and_padding(tmp_path):
    name = 'odd "name" \\ é \U0001F600'
    import json
    header = json.dumps({name: {"dtype": "F16", "shape": [2], "data_offsets": [0, 4]},
                         "__metadata__": {"k": "v\nw"}}, ensure_ascii=True) + "   "
    h = header.encode()
    p = tmp_path / "esc.safetensors"
    p.write_bytes(struct.pack("<Q", len(h)) + h + np.array([1.5, -2], dtype=np.float16).tobytes())
    s = W.SafetensorsFile(str(p))
    assert s.names() == [name]
    assert s.metadata("k") == "v\nw"
    assert np.array_equal(s.raw(name).view(np.float16), [1.5, -2])
