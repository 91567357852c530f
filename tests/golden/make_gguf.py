"""Writes tests/golden/tiny_q8.gguf: a three-tensor GGUF container laid out
like the files candle-3d's quantizer writes (weights/quantize.rs:102-317:
rank-2 `*.weight` tensors in Q8_0, the rest in F16 / BF16, `lux3d.*`
metadata), written with the specification-level writer tests/gguf_spec.py.

Tensors (candle shapes):
  blocks.0.mlp.fc1.weight  Q8_0 [8, 64]: every block's scale is f16 0.5
                           (0x3800) and q[r][c] = (7 r + 3 c) % 15 - 7
  blocks.0.mlp.fc1.bias    F16 [8]: 0.25 r - 1
  blocks.0.norm.weight     BF16 [64]: 1 + c / 64
Every dequantized weight is exact in bf16, so a linear layer with
small-integer inputs has an exact expected output.

Run:  python tests/golden/make_gguf.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, ".."))
import gguf_spec as gs  # noqa: E402


def q8_weight(n, k):
    out = bytearray()
    for r in range(n):
        for b in range(k // 32):
            out += bytes([0x00, 0x38])
            out += bytes(((7 * r + 3 * (b * 32 + j)) % 15 - 7) & 0xFF for j in range(32))
    return bytes(out)


def main():
    n, k = 8, 64
    tensors = [
        ("blocks.0.mlp.fc1.weight", gs.GGML_Q8_0, [n, k], q8_weight(n, k)),
        ("blocks.0.mlp.fc1.bias", gs.GGML_F16, [n], gs.f16_bytes(0.25 * np.arange(n) - 1.0)),
        ("blocks.0.norm.weight", gs.GGML_BF16, [k], gs.bf16_bytes(1.0 + np.arange(k) / 64.0)),
    ]
    metadata = [
        ("general.architecture", gs.STRING, "trellis2"),
        ("lux3d.family", gs.STRING, "trellis2"),
        ("lux3d.quantization", gs.STRING, "q8_0"),
        ("lux3d.fallback_dtype", gs.STRING, "f16"),
        ("lux3d.tensor_count", gs.U32, len(tensors)),
    ]
    path = os.path.join(HERE, "tiny_q8.gguf")
    gs.write(path, tensors, metadata)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
