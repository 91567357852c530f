"""ctypes binding of liblux3d_fused.so (the C ABI in include/lux3d_fused.h).

The library is built in-tree (``make -C candle-3d_amd``) and loaded from the
package's parent directory. There is no fallback: if the shared library is
missing or fails to load, importing this module raises.
"""
from __future__ import annotations

import ctypes
import os

LIB_NAME = "liblux3d_fused.so"
# LUX3D_FUSED_LIB names another build of the same library (A/B timing of
# kernel variants); it must exist, like the default
LIB_PATH = os.environ.get("LUX3D_FUSED_LIB") or os.path.join(
    os.path.dirname(os.path.dirname(os.path.abspath(__file__))), LIB_NAME)

MAX_RANK = 5

F32, BF16, F16, I32, I64, U8, I8 = 0, 1, 2, 3, 4, 5, 6

OK = 0
ERR_NULL, ERR_SHAPE, ERR_DTYPE, ERR_LAYOUT, ERR_HIP, ERR_VALUE = -1, -2, -3, -4, -5, -6
STATUS_NAMES = {
    ERR_NULL: "LUX3D_ERR_NULL",
    ERR_SHAPE: "LUX3D_ERR_SHAPE",
    ERR_DTYPE: "LUX3D_ERR_DTYPE",
    ERR_LAYOUT: "LUX3D_ERR_LAYOUT",
    ERR_HIP: "LUX3D_ERR_HIP",
    ERR_VALUE: "LUX3D_ERR_VALUE",
}


class Tensor(ctypes.Structure):
    """lux3d_tensor_t: a borrowed device tensor (pointer, dtype, shape, strides)."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("shape", ctypes.c_int64 * MAX_RANK),
        ("stride", ctypes.c_int64 * MAX_RANK),
    ]


TP = ctypes.POINTER(Tensor)
S = ctypes.c_void_p  # lux3d_stream_t

# name -> argtypes (every entry returns int)
SIGNATURES = {
    "lux3d_layer_norm": [TP, TP, TP, ctypes.c_float, TP, S],
    "lux3d_residual_layer_norm": [TP, TP, TP, TP, TP, ctypes.c_float, TP, TP, S],
    "lux3d_adaln_modulate": [TP, TP, TP, TP, TP, TP, TP, TP, ctypes.c_float, TP, S],
    "lux3d_gated_residual": [TP, TP, TP, TP, TP, TP, S],
    "lux3d_gated_residual_adaln_modulate": [TP, TP, TP, TP, TP, TP, TP, TP, TP, ctypes.c_float, TP, TP, S],
    "lux3d_qk_layernorm_rope2d": [TP, TP, TP, TP, TP, TP, ctypes.c_float, TP, TP, TP, TP, S],
    "lux3d_qk_layernorm_rope2d_pos": [TP, TP, TP, TP, TP, TP, ctypes.c_float, TP, ctypes.c_float, TP, TP, S],
    "lux3d_rope2d_tables": [TP, ctypes.c_float, TP, TP, S],
    "lux3d_rms_norm_heads": [TP, TP, TP, TP, ctypes.c_float, TP, TP, S],
    "lux3d_qk_l2norm_rope3d": [TP, TP, TP, TP, TP, TP, TP, ctypes.c_float, TP, TP, S],
    "lux3d_rope3d_tables": [TP, ctypes.c_int64, ctypes.c_float, TP, TP, S],
    "lux3d_dinov3_rope": [TP, TP, TP, TP, ctypes.c_int64, TP, TP, S],
    "lux3d_gelu_erf": [TP, TP, S],
    "lux3d_gelu_tanh": [TP, TP, S],
    "lux3d_silu": [TP, TP, S],
    "lux3d_timestep_embedding": [TP, TP, ctypes.c_int64, ctypes.c_int32, TP, S],
    "lux3d_dequant_q8_0": [TP, TP, S],
    "lux3d_q8_0_repack": [TP, ctypes.c_int64, ctypes.c_int64, TP, TP, S],
    "lux3d_q8_0_linear": [TP, TP, TP, TP, TP, S],
    "lux3d_q8_0_linear_int8": [TP, TP, TP, TP, TP, TP, TP, S],
    "lux3d_q8_0_quantize": [TP, TP, TP, S],
    "lux3d_sdpa": [TP, TP, TP, ctypes.c_float, TP, S],
    "lux3d_sdpa_heads_f32": [TP, TP, TP, ctypes.c_float, TP, S],
    "lux3d_sdpa_layernorm_rope2d": [TP, TP, TP, ctypes.c_float, TP, TP, TP, TP, ctypes.c_float, TP, S],
    "lux3d_sdpa_rms_norm_heads": [TP, TP, ctypes.c_float, TP, TP, ctypes.c_float, TP, S],
    "lux3d_sdpa_l2norm_rope3d": [TP, TP, TP, TP, TP, TP, ctypes.c_float, TP, S],
    "lux3d_sdpa_dinov3_rope": [TP, TP, TP, ctypes.c_int64, TP, TP, ctypes.c_float, TP, S],
    "lux3d_sparse_neighbors": [TP, TP, TP, TP, TP, S],
    "lux3d_sparse_neighbors_noalloc": [TP, TP, TP, S],
    "lux3d_sparse_conv3d": [TP, TP, TP, TP, TP, S],
    "lux3d_sparse_rulebook": [TP, TP, TP, S],
    "lux3d_sparse_conv3d_rulebook": [TP, TP, TP, TP, TP, TP, S],
    "lux3d_index_select_rows": [TP, TP, TP, TP, S],
    "lux3d_channel_to_spatial": [TP, TP, TP, TP, TP, TP, TP, TP, TP, S],
}


class Lux3dError(RuntimeError):
    """A non-zero lux3d_status, with the library's message."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} -> {STATUS_NAMES.get(code, code)}: {message}")
        self.fn = fn
        self.code = code


def _load() -> ctypes.CDLL:
    # PyTorch-ROCm ships its own libamdhip64.so / libhsa-runtime64.so. Import
    # it first so that liblux3d_fused.so's libamdhip64.so.7 dependency
    # resolves (by soname) to the runtime torch already loaded: two HIP
    # runtimes in one process each open the device and the second one reports
    # "no ROCm-capable device".
    import torch  # noqa: F401
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `make -C candle-3d_amd` (or __graft_entry__.build())"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    lib.lux3d_abi_version.restype = ctypes.c_int
    lib.lux3d_abi_version.argtypes = []
    lib.lux3d_last_error.restype = ctypes.c_char_p
    lib.lux3d_last_error.argtypes = []
    return lib


LIB = _load()
ABI_VERSION = LIB.lux3d_abi_version()


def call(name: str, *args) -> int:
    """Call an entry point and raise Lux3dError on a non-zero status."""
    rc = getattr(LIB, name)(*args)
    if rc != OK:
        raise Lux3dError(name, rc, LIB.lux3d_last_error().decode())
    return rc


def call_status(name: str, *args) -> tuple[int, str]:
    """Call an entry point and return (status, message) without raising."""
    rc = getattr(LIB, name)(*args)
    return rc, LIB.lux3d_last_error().decode()


def descriptor(data: int, dtype: int, shape, strides) -> Tensor:
    t = Tensor()
    t.data = data
    t.dtype = dtype
    t.rank = len(shape)
    for i, (n, s) in enumerate(zip(shape, strides)):
        t.shape[i] = int(n)
        t.stride[i] = int(s)
    return t
