"""GGUF and safetensors readers: ctypes binding of the C ABI in
include/lux3d_weights.h (liblux3d_candle.so), mirroring VarBuilder::from_gguf
and VarBuilder::from_mmaped_safetensors (weights/mod.rs:121-140).

Files are memory-mapped by the native reader; `raw()` returns a read-only
numpy view of a tensor's bytes in the mapping (valid while the file object
lives). `get()` moves a tensor to a torch device and converts it (Q8_0 through
the library's dequant kernel); `get_qmatmul()` repacks a Q8_0 weight for the
quantized linear (QMatMul::from_qtensor, nn_blocks.rs:145-150).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Optional, Tuple

import numpy as np

from . import _lib

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "liblux3d_candle.so")

GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30
(GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL, GGUF_STRING, GGUF_ARRAY,
 GGUF_U64, GGUF_I64, GGUF_F64) = range(13)
MAX_RANK = 8

_SCALAR = {GGUF_U8: "<u1", GGUF_I8: "<i1", GGUF_U16: "<u2", GGUF_I16: "<i2", GGUF_U32: "<u4", GGUF_I32: "<i4",
           GGUF_F32: "<f4", GGUF_BOOL: "<u1", GGUF_U64: "<u8", GGUF_I64: "<i8", GGUF_F64: "<f8"}


class WeightsTensor(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("dtype", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("shape", ctypes.c_int64 * MAX_RANK),
        ("data", ctypes.c_void_p),
        ("nbytes", ctypes.c_uint64),
    ]


def _load() -> ctypes.CDLL:
    _ = _lib.LIB  # liblux3d_fused.so (and torch's HIP runtime) first
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run `make -C candle-3d_amd`")
    lib = ctypes.CDLL(LIB_PATH)
    P, WT = ctypes.c_void_p, ctypes.POINTER(WeightsTensor)
    sig = {
        "lux3d_weights_last_error": ([], ctypes.c_char_p),
        "lux3d_gguf_open": ([ctypes.c_char_p], P),
        "lux3d_gguf_close": ([P], None),
        "lux3d_gguf_version": ([P], ctypes.c_uint32),
        "lux3d_gguf_tensor_count": ([P], ctypes.c_int64),
        "lux3d_gguf_find": ([P, ctypes.c_char_p], ctypes.c_int64),
        "lux3d_gguf_tensor": ([P, ctypes.c_int64, WT], ctypes.c_int),
        "lux3d_gguf_metadata_count": ([P], ctypes.c_int64),
        "lux3d_gguf_metadata": ([P, ctypes.c_int64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int32),
                                 ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_void_p),
                                 ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
        "lux3d_gguf_metadata_find": ([P, ctypes.c_char_p], ctypes.c_int64),
        "lux3d_safetensors_open": ([ctypes.c_char_p], P),
        "lux3d_safetensors_close": ([P], None),
        "lux3d_safetensors_tensor_count": ([P], ctypes.c_int64),
        "lux3d_safetensors_find": ([P, ctypes.c_char_p], ctypes.c_int64),
        "lux3d_safetensors_tensor": ([P, ctypes.c_int64, WT], ctypes.c_int),
        "lux3d_safetensors_metadata": ([P, ctypes.c_char_p], ctypes.c_char_p),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


LIB = _load()


class WeightsError(RuntimeError):
    pass


def _err(what: str):
    raise WeightsError(f"{what}: {LIB.lux3d_weights_last_error().decode()}")


@dataclass
class Info:
    name: str
    dtype: int                 # GGUF: ggml type id; safetensors: lux3d dtype code (-1: not one)
    shape: Tuple[int, ...]     # candle order
    nbytes: int
    data: int                  # host address in the mapping


def _info(t: WeightsTensor) -> Info:
    return Info(t.name.decode(), t.dtype, tuple(t.shape[i] for i in range(t.rank)), t.nbytes, t.data or 0)


class _Mapped:
    _tensor_fn = ""
    _find_fn = ""
    _count_fn = ""

    def __len__(self):
        return getattr(LIB, self._count_fn)(self._h)

    def names(self):
        return [self.info_at(i).name for i in range(len(self))]

    def __contains__(self, name: str) -> bool:
        return getattr(LIB, self._find_fn)(self._h, name.encode()) >= 0

    def info_at(self, i: int) -> Info:
        t = WeightsTensor()
        if getattr(LIB, self._tensor_fn)(self._h, i, ctypes.byref(t)) != 0:
            _err(self._tensor_fn)
        return _info(t)

    def info(self, name: str) -> Info:
        i = getattr(LIB, self._find_fn)(self._h, name.encode())
        if i < 0:
            raise WeightsError(f"cannot find tensor {name}")
        return self.info_at(i)

    def raw(self, name: str) -> np.ndarray:
        """Read-only uint8 view of the tensor's bytes in the mapping."""
        w = self.info(name)
        if w.nbytes == 0:
            return np.zeros(0, dtype=np.uint8)
        buf = (ctypes.c_uint8 * w.nbytes).from_address(w.data)
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a


class GgufFile(_Mapped):
    """A GGUF container (weights/quantize.rs:102-317 writes it)."""
    _tensor_fn, _find_fn, _count_fn = "lux3d_gguf_tensor", "lux3d_gguf_find", "lux3d_gguf_tensor_count"

    def __init__(self, path: str):
        self._h = LIB.lux3d_gguf_open(os.fsencode(path))
        if not self._h:
            _err("lux3d_gguf_open")

    def close(self):
        if getattr(self, "_h", None):
            LIB.lux3d_gguf_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def version(self) -> int:
        return LIB.lux3d_gguf_version(self._h)

    def metadata(self) -> dict:
        """Every metadata entry decoded: scalars as Python numbers, strings as
        str, arrays of scalars as numpy arrays (arrays of strings: their
        count only, as ("array", elem_type, count))."""
        out = {}
        for i in range(LIB.lux3d_gguf_metadata_count(self._h)):
            key, t, et = ctypes.c_char_p(), ctypes.c_int32(), ctypes.c_int32()
            val, cnt = ctypes.c_void_p(), ctypes.c_uint64()
            if LIB.lux3d_gguf_metadata(self._h, i, ctypes.byref(key), ctypes.byref(t), ctypes.byref(et),
                                       ctypes.byref(val), ctypes.byref(cnt)) != 0:
                _err("lux3d_gguf_metadata")
            out[key.value.decode()] = self._decode(t.value, et.value, val.value, cnt.value)
        return out

    @staticmethod
    def _decode(t, et, addr, count):
        if t == GGUF_STRING:
            return ctypes.string_at(addr, count).decode() if count else ""
        if t == GGUF_ARRAY:
            if et in _SCALAR:
                nb = np.dtype(_SCALAR[et]).itemsize * count
                raw = ctypes.string_at(addr, nb) if count else b""
                a = np.frombuffer(raw, dtype=_SCALAR[et]).copy()
                return a.astype(bool) if et == GGUF_BOOL else a
            return ("array", et, count)
        v = np.frombuffer(ctypes.string_at(addr, np.dtype(_SCALAR[t]).itemsize), dtype=_SCALAR[t])[0]
        return bool(v) if t == GGUF_BOOL else v.item()

    def metadata_string(self, key: str) -> Optional[str]:
        """gguf_metadata_string (weights/mod.rs:656-661)."""
        v = self.metadata().get(key)
        return v if isinstance(v, str) else None

    def get(self, name: str, dtype, device):
        """VarBuilder::get: the tensor as `dtype` on `device` (Q8_0 dequantized
        exactly by the library's kernel; F16 / BF16 / F32 converted once)."""
        import torch
        from . import ops
        w = self.info(name)
        raw = torch.from_numpy(self.raw(name).copy())
        if w.dtype == GGML_Q8_0:
            return ops.dequantize_q8_0(raw.to(device), w.shape, dtype)
        src = {GGML_F32: torch.float32, GGML_F16: torch.float16, GGML_BF16: torch.bfloat16}.get(w.dtype)
        if src is None:
            raise WeightsError(f"tensor `{name}` has ggml type {w.dtype} (F32, F16, BF16 and Q8_0 are supported)")
        return raw.view(src).reshape(w.shape).to(device).to(dtype)

    def get_qmatmul(self, name: str, out_dim: int, in_dim: int, device):
        """VarBuilder::get_quantized + QMatMul::from_qtensor for a Q8_0 weight,
        with quantized_linear's shape check (nn_blocks.rs:121-127)."""
        import torch
        from . import ops
        w = self.info(name)
        if w.shape != (out_dim, in_dim):
            raise WeightsError(f"quantized linear weight shape {list(w.shape)} does not match expected "
                               f"({out_dim}, {in_dim})")
        if w.dtype != GGML_Q8_0:
            raise WeightsError(f"tensor `{name}` is not Q8_0 (ggml type {w.dtype})")
        blocks = torch.from_numpy(self.raw(name).copy()).to(device)
        return ops.QMatMul.from_q8_0(blocks, out_dim, in_dim)


class SafetensorsFile(_Mapped):
    _tensor_fn, _find_fn, _count_fn = ("lux3d_safetensors_tensor", "lux3d_safetensors_find",
                                       "lux3d_safetensors_tensor_count")

    def __init__(self, path: str):
        self._h = LIB.lux3d_safetensors_open(os.fsencode(path))
        if not self._h:
            _err("lux3d_safetensors_open")

    def close(self):
        if getattr(self, "_h", None):
            LIB.lux3d_safetensors_close(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def metadata(self, key: str) -> Optional[str]:
        v = LIB.lux3d_safetensors_metadata(self._h, key.encode())
        return None if v is None else v.decode()

    def get(self, name: str, dtype, device):
        import torch
        w = self.info(name)
        src = {_lib.F32: torch.float32, _lib.BF16: torch.bfloat16, _lib.F16: torch.float16, _lib.I32: torch.int32,
               _lib.I64: torch.int64, _lib.U8: torch.uint8, _lib.I8: torch.int8}.get(w.dtype)
        if src is None:
            raise WeightsError(f"tensor `{name}` has a dtype this reader does not convert")
        raw = torch.from_numpy(self.raw(name).copy())
        return raw.view(src).reshape(w.shape).to(device).to(dtype)
