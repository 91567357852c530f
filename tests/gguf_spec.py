"""A GGUF writer written from the public ggml GGUF specification, for test
fixtures only (the container candle-3d's quantizer writes with candle's
gguf_file::write, weights/quantize.rs:280-291).

Layout: "GGUF", u32 version, tensor and metadata counts (u32 in v1, u64
from v2), metadata {string key, u32 type, value}, tensor infos {string name,
u32 n_dims, dims innermost first (u32 in v1, u64 from v2), u32 ggml type,
u64 offset}, zero padding to `general.alignment` (default 32), then each
tensor's bytes at its offset, each offset a multiple of the alignment.
Strings are {length, bytes} with a u32 length in v1 and u64 from v2.
"""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}
GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30


def _count(v, version):
    return struct.pack("<I" if version == 1 else "<Q", v)


def _string(s, version):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return _count(len(b), version) + b


def _value(t, v, version):
    if t == STRING:
        return _string(v, version)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<I", et) + _count(len(items), version)
        for it in items:
            out += _value(et, it, version)
        return out
    return struct.pack(_FMT[t], v)


def write(path, tensors, metadata=(), version=3, alignment=None, offsets=None):
    """tensors: [(name, ggml_type, candle_shape, raw_bytes)];
    metadata: [(key, type, value)] with ARRAY values as (elem_type, [items]).
    `alignment` adds a general.alignment (u32) entry; `offsets` overrides the
    tensor offsets (for malformed-file tests)."""
    meta = list(metadata)
    align = 32
    if alignment is not None:
        meta.append(("general.alignment", U32, alignment))
        align = alignment
    out = b"GGUF" + struct.pack("<I", version) + _count(len(tensors), version) + _count(len(meta), version)
    for k, t, v in meta:
        out += _string(k, version) + struct.pack("<I", t) + _value(t, v, version)
    offs, cur = [], 0
    for _, _, _, raw in tensors:
        offs.append(cur)
        cur += len(raw)
        cur = (cur + align - 1) // align * align
    if offsets is not None:
        offs = offsets
    for (name, gt, shape, _), off in zip(tensors, offs):
        dims = list(reversed(shape))
        out += _string(name, version) + struct.pack("<I", len(dims))
        for d in dims:
            out += struct.pack("<I" if version == 1 else "<Q", d)
        out += struct.pack("<I", gt) + struct.pack("<Q", off)
    pad = (-len(out)) % align
    out += b"\0" * pad
    data0 = len(out)
    body = bytearray()
    for (_, _, _, raw), off in zip(tensors, offs):
        need = off + len(raw) - len(body)
        if need > 0:
            body += b"\0" * need
        body[off:off + len(raw)] = raw
    with open(path, "wb") as f:
        f.write(out + bytes(body))
    return data0


def f16_bytes(a):
    return np.asarray(a, dtype=np.float16).tobytes()


def f32_bytes(a):
    return np.asarray(a, dtype=np.float32).tobytes()


def bf16_bytes(a):
    """RNE of f32 to bf16, as little-endian u16."""
    x = np.asarray(a, dtype=np.float32).view(np.uint32)
    r = ((x + 0x7FFF + ((x >> 16) & 1)) >> 16).astype(np.uint16)
    return r.tobytes()
