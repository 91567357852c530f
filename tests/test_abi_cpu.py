"""The C ABI without a GPU: liblux3d_fused.so loads, exports every entry
point that include/lux3d_fused.h declares (and nothing is missing from the
ctypes binding), and invalid arguments are rejected on the host with the
documented status codes and a message, before any HIP call is made. The
descriptors here point at fake addresses that are never dereferenced: every
call below must fail validation."""
import ctypes
import os
import re
import subprocess

import pytest

from lux3d_fused import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lux3d_fused.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lux3d_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = header_functions()
    assert "lux3d_layer_norm" in names and "lux3d_dequant_q8_0" in names
    assert len(names) == len(_lib.SIGNATURES) + 2  # + abi_version, last_error


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (lux3d_[a-z0-9_]+)", out))
    missing = [n for n in header_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    for n in header_functions():
        assert hasattr(_lib.LIB, n)
    assert set(_lib.SIGNATURES) <= exported


def test_abi_version():
    assert _lib.LIB.lux3d_abi_version() == 2
    assert _lib.ABI_VERSION == 2


FAKE = 0x100000  # 16-byte aligned fake device address; never dereferenced


def T(shape, dtype=_lib.BF16, strides=None, data=FAKE):
    if strides is None:
        strides, acc = [], 1
        for n in reversed(shape):
            strides.insert(0, acc)
            acc *= n
    return ctypes.pointer(_lib.descriptor(data, dtype, shape, strides))


def status(name, *args):
    rc, msg = _lib.call_status(name, *args)
    return rc, msg


def test_layer_norm_argument_errors():
    x = T([4, 64])
    rc, msg = status("lux3d_layer_norm", None, None, None, 1e-5, x, None)
    assert rc == _lib.ERR_NULL and "`x` is NULL" in msg
    rc, msg = status("lux3d_layer_norm", x, T([32], _lib.F32), None, 1e-5, x, None)
    assert rc == _lib.ERR_SHAPE and "`w`" in msg
    rc, msg = status("lux3d_layer_norm", x, None, None, 1e-5, T([4, 64], _lib.F32), None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status("lux3d_layer_norm", x, None, None, 1e-5, T([4, 32]), None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_layer_norm", T([4, 64], strides=[64, 2]), None, None, 1e-5, x, None)
    assert rc == _lib.ERR_LAYOUT
    rc, msg = status("lux3d_layer_norm", T([4, 64], _lib.I32), None, None, 1e-5, x, None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status("lux3d_layer_norm", x, None, None, -1.0, x, None)
    assert rc == _lib.ERR_VALUE
    bad_rank = _lib.descriptor(FAKE, _lib.BF16, [4], [1])
    bad_rank.rank = 0
    rc, msg = status("lux3d_layer_norm", ctypes.pointer(bad_rank), None, None, 1e-5, x, None)
    assert rc == _lib.ERR_SHAPE
    # leading dims that do not form a uniform row stride
    rc, msg = status("lux3d_layer_norm", T([2, 3, 64], strides=[1000, 64, 1]), None, None, 1e-5, T([2, 3, 64]),
                     None)
    assert rc == _lib.ERR_LAYOUT


def test_residual_and_modulate_errors():
    x = T([8, 128])
    rc, msg = status("lux3d_residual_layer_norm", x, T([8, 64]), None, None, None, 1e-5, x, x, None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_adaln_modulate", x, None, None, None, T([2, 128], _lib.F32), None, None, None, 1e-6, x,
                     None)
    assert rc == _lib.ERR_NULL
    # 8 rows do not split into 3 equal segments without offsets
    sh = T([3, 128], _lib.F32)
    rc, msg = status("lux3d_adaln_modulate", x, None, sh, None, sh, None, None, None, 1e-6, x, None)
    assert rc == _lib.ERR_SHAPE and "seg_offsets" in msg
    # offsets must be int64 [S+1]
    rc, msg = status("lux3d_adaln_modulate", x, T([4], _lib.I32), sh, None, sh, None, None, None, 1e-6, x, None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status("lux3d_adaln_modulate", x, T([3], _lib.I64), sh, None, sh, None, None, None, 1e-6, x, None)
    assert rc == _lib.ERR_SHAPE
    # base without piece
    rc, msg = status("lux3d_gated_residual", x, x, None, None, T([128], _lib.F32), x, None)
    assert rc == _lib.ERR_NULL


def test_gated_residual_adaln_modulate_errors():
    fn = "lux3d_gated_residual_adaln_modulate"
    x = T([8, 128])
    x2 = T([8, 128], data=FAKE + 0x10000)
    y = T([8, 128], data=FAKE + 0x20000)
    sh = T([2, 128], _lib.F32)
    rc, msg = status(fn, x, x2, None, sh, None, None, None, sh, None, 1e-6, x, y, None)
    assert rc == _lib.ERR_NULL and "`shift` and `scale`" in msg
    # y may not alias x or x_out
    rc, msg = status(fn, x, x2, None, sh, None, sh, None, sh, None, 1e-6, x, x, None)
    assert rc == _lib.ERR_LAYOUT and "alias" in msg
    # pieces must share one segment count
    rc, msg = status(fn, x, x2, None, T([4, 128], _lib.F32), None, sh, None, sh, None, 1e-6, x, y, None)
    assert rc == _lib.ERR_SHAPE and "segment counts" in msg
    # h's shape and dtype follow x
    rc, msg = status(fn, x, T([8, 64]), None, sh, None, sh, None, sh, None, 1e-6, x, y, None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status(fn, x, T([8, 128], _lib.F32), None, sh, None, sh, None, sh, None, 1e-6, x, y, None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status(fn, x, x2, None, sh, None, sh, None, sh, None, -1.0, x, y, None)
    assert rc == _lib.ERR_VALUE
    # a base vector without its piece
    rc, msg = status(fn, x, x2, None, None, T([128], _lib.F32), sh, None, sh, None, 1e-6, x, y, None)
    assert rc == _lib.ERR_NULL


def test_head_op_errors():
    q = T([2, 16, 10, 64], strides=[10 * 3 * 16 * 64, 64, 3 * 16 * 64, 1])
    out = T([2, 16, 10, 64])
    tab = T([2, 10, 64], _lib.F32)
    # Rope2d needs a token_dim divisible by 4 (the reference's own check)
    tab30 = T([2, 10, 30], _lib.F32)
    rc, msg = status("lux3d_qk_layernorm_rope2d", T([2, 16, 10, 30]), None, None, None, None, None, 1e-5, tab30,
                     tab30, T([2, 16, 10, 30]), None, None)
    assert rc == _lib.ERR_SHAPE and "divisible by 4" in msg
    # wrong table shape
    rc, msg = status("lux3d_qk_layernorm_rope2d", q, None, None, None, None, None, 1e-5, T([2, 11, 64], _lib.F32),
                     tab, out, None, None)
    assert rc == _lib.ERR_SHAPE
    # a LayerNorm bias without its weight (a weight without bias is a bias-free LayerNorm)
    rc, msg = status("lux3d_qk_layernorm_rope2d", q, None, T([64], _lib.F32), None, None, None, 1e-5, tab, tab, out,
                     None, None)
    assert rc == _lib.ERR_NULL and "bias given without a weight" in msg
    # q normalised, k not
    k = T([2, 16, 10, 64], strides=[10 * 3 * 16 * 64, 64, 3 * 16 * 64, 1], data=FAKE + 128)
    rc, msg = status("lux3d_qk_layernorm_rope2d", q, T([64], _lib.F32), None, k, None, None, 1e-5, tab, tab, out,
                     out, None)
    assert rc == _lib.ERR_NULL and "both be normalised" in msg
    # a non-unit innermost stride
    rc, msg = status("lux3d_qk_layernorm_rope2d", T([2, 16, 10, 64], strides=[20480, 1280, 128, 2]), None, None,
                     None, None, None, 1e-5, tab, tab, out, None, None)
    assert rc == _lib.ERR_LAYOUT
    # positions-based rotation holds at most 64 frequencies per axis half
    big = T([2, 16, 10, 512])
    rc, msg = status("lux3d_qk_layernorm_rope2d_pos", big, None, None, None, None, None, 1e-5,
                     T([2, 10, 2], _lib.I32), 100.0, big, None, None)
    assert rc == _lib.ERR_SHAPE
    # positions must be [B, N, 2] int
    rc, msg = status("lux3d_qk_layernorm_rope2d_pos", q, None, None, None, None, None, 1e-5,
                     T([2, 10, 2], _lib.F32), 100.0, out, None, None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status("lux3d_qk_layernorm_rope2d_pos", q, None, None, None, None, None, 1e-5,
                     T([2, 10, 2], _lib.I32), -1.0, out, None, None)
    assert rc == _lib.ERR_VALUE
    # rope3d: tables and coords together are ambiguous
    x = T([1, 10, 12, 128])
    rc, msg = status("lux3d_qk_l2norm_rope3d", x, None, None, None, T([10, 64], _lib.F32), T([10, 64], _lib.F32),
                     T([10, 3], _lib.I32), 10000.0, x, None, None)
    assert rc == _lib.ERR_VALUE
    rc, msg = status("lux3d_qk_l2norm_rope3d", x, T([12, 64], _lib.F32), None, None, None, None, None, 10000.0, x,
                     None, None)
    assert rc == _lib.ERR_SHAPE   # gamma must be [H, D] = 12*128 elements
    # rotating (re, im) pairs needs an even head dim; coords give 1..64 frequencies per axis
    odd = T([1, 10, 2, 7])
    rc, msg = status("lux3d_qk_l2norm_rope3d", odd, None, None, None, None, None, T([10, 3], _lib.I32), 10000.0,
                     odd, None, None)
    assert rc == _lib.ERR_SHAPE and "even" in msg
    wide = T([1, 10, 2, 1024])
    rc, msg = status("lux3d_qk_l2norm_rope3d", wide, None, None, None, None, None, T([10, 3], _lib.I32), 10000.0,
                     wide, None, None)
    assert rc == _lib.ERR_SHAPE and "frequencies" in msg
    # dinov3: prefix larger than the sequence
    y = T([1, 16, 9, 64])
    rc, msg = status("lux3d_dinov3_rope", y, None, T([4, 64], _lib.F32), T([4, 64], _lib.F32), 10, y, None, None)
    assert rc == _lib.ERR_VALUE


def test_pointwise_errors():
    x = T([100])
    rc, msg = status("lux3d_gelu_tanh", x, T([99]), None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_silu", x, T([100], _lib.F32), None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status("lux3d_gelu_erf", T([10, 10], strides=[20, 1]), T([10, 10]), None)
    assert rc == _lib.ERR_LAYOUT
    rc, msg = status("lux3d_timestep_embedding", T([2], _lib.F32), None, 255, 0, T([2, 255], _lib.F32), None)
    assert rc == _lib.ERR_VALUE     # sin-first needs an even dim
    rc, msg = status("lux3d_timestep_embedding", T([2], _lib.F32), T([100], _lib.F32), 256, 1,
                     T([2, 256], _lib.F32), None)
    assert rc == _lib.ERR_SHAPE     # freqs must hold dim/2 values
    rc, msg = status("lux3d_dequant_q8_0", T([35], _lib.U8), T([32]), None)
    assert rc == _lib.ERR_SHAPE and "34-byte" in msg
    rc, msg = status("lux3d_dequant_q8_0", T([68], _lib.U8), T([32]), None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_dequant_q8_0", T([34], _lib.U8, data=FAKE + 1), T([32]), None)
    assert rc == _lib.ERR_LAYOUT
    rc, msg = status("lux3d_dequant_q8_0", T([34], _lib.F32), T([32]), None)
    assert rc == _lib.ERR_DTYPE


def test_python_mirror_raises_lux3d_error():
    from lux3d_fused import Lux3dError
    with pytest.raises(Lux3dError) as e:
        _lib.call("lux3d_layer_norm", None, None, None, 1e-5, None, None)
    assert e.value.code == _lib.ERR_NULL


def test_q8_0_linear_argument_errors():
    n, k = 64, 96
    blocks = T([n * k // 32 * 34], _lib.U8)
    qs, scales = T([n, k], _lib.I8), T([n, k // 32], _lib.F32)
    # repack: k must be a multiple of 32, the byte count must match, qs int8
    rc, msg = status("lux3d_q8_0_repack", blocks, n, 100, qs, scales, None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_q8_0_repack", T([n * k // 32 * 34 - 34], _lib.U8), n, k, qs, scales, None)
    assert rc == _lib.ERR_SHAPE and "bytes of blocks" in msg
    rc, msg = status("lux3d_q8_0_repack", blocks, n, k, T([n, k], _lib.U8), scales, None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status("lux3d_q8_0_repack", blocks, n, k, T([n, k], _lib.I8, data=FAKE + 8), scales, None)
    assert rc == _lib.ERR_LAYOUT
    # linear: x bf16 (or f32 with k % 64 == 0) with k features, rows 16-byte
    # aligned; y [rows, n]
    x, y = T([10, k]), T([10, n])
    rc, msg = status("lux3d_q8_0_linear", T([10, k], _lib.F16), qs, scales, None, y, None)
    assert rc == _lib.ERR_DTYPE and "bf16 or f32" in msg
    rc, msg = status("lux3d_q8_0_linear", T([10, k], _lib.F32), qs, scales, None, y, None)
    assert rc == _lib.ERR_SHAPE and "multiple of 64" in msg
    rc, msg = status("lux3d_q8_0_linear", T([10, k + 32]), qs, scales, None, y, None)
    assert rc == _lib.ERR_SHAPE and "features" in msg
    rc, msg = status("lux3d_q8_0_linear", x, qs, scales, None, T([10, n + 1]), None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_q8_0_linear", x, qs, T([n, k // 32 + 1], _lib.F32), None, y, None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_q8_0_linear", x, qs, scales, T([n + 1], _lib.F32), y, None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_q8_0_linear", T([10, k], data=FAKE + 2), qs, scales, None, y, None)
    assert rc == _lib.ERR_LAYOUT


def test_sdpa_argument_errors():
    q, k, v, o = T([2, 4, 33, 64]), T([2, 4, 50, 64]), T([2, 4, 50, 64]), T([2, 4, 33, 64])
    rc, msg = status("lux3d_sdpa", T([8, 33, 64]), k, v, 0.125, o, None)
    assert rc == _lib.ERR_SHAPE and "[B, H, L, D]" in msg
    rc, msg = status("lux3d_sdpa", q, T([2, 4, 50, 64], _lib.F32), v, 0.125, o, None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status("lux3d_sdpa", q, T([2, 3, 50, 64]), v, 0.125, o, None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_sdpa", q, k, T([2, 4, 49, 64]), 0.125, o, None)
    assert rc == _lib.ERR_SHAPE and "shape of k" in msg
    rc, msg = status("lux3d_sdpa", q, k, v, 0.125, T([2, 4, 32, 64]), None)
    assert rc == _lib.ERR_SHAPE and "shape of q" in msg
    rc, msg = status("lux3d_sdpa", q, T([2, 4, 0, 64]), T([2, 4, 0, 64]), 0.125, o, None)
    assert rc == _lib.ERR_SHAPE and "no tokens" in msg
    rc, msg = status("lux3d_sdpa", q, k, v, 0.0, o, None)
    assert rc == _lib.ERR_VALUE
    rc, msg = status("lux3d_sdpa", q, k, v, float("nan"), o, None)
    assert rc == _lib.ERR_VALUE
    big = [1, 1, 4, 1024]
    rc, msg = status("lux3d_sdpa", T(big), T(big), T(big), 0.1, T(big), None)
    assert rc == _lib.ERR_SHAPE and "head dim" in msg
    strided = T([2, 4, 33, 64], strides=[4 * 33 * 128, 33 * 128, 128, 2])
    rc, msg = status("lux3d_sdpa", strided, k, v, 0.125, o, None)
    assert rc == _lib.ERR_LAYOUT
    rc, msg = status("lux3d_sdpa", None, k, v, 0.125, o, None)
    assert rc == _lib.ERR_NULL
    # exact_sdpa_heads: out has q's dtype or is f32; q, k, v share one dtype
    rc, msg = status("lux3d_sdpa", q, k, v, 0.125, T([2, 4, 33, 64], _lib.F32), None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status("lux3d_sdpa_heads_f32", q, k, v, 0.125, T([2, 4, 33, 64], _lib.F16), None)
    assert rc == _lib.ERR_DTYPE and "out has it or is f32" in msg
    rc, msg = status("lux3d_sdpa_heads_f32", q, T([2, 4, 50, 64], _lib.F32), v, 0.125, T([2, 4, 33, 64], _lib.F32),
                     None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status("lux3d_sdpa_heads_f32", q, k, v, -1.0, o, None)
    assert rc == _lib.ERR_VALUE


def test_sparse_argument_errors():
    co, nbr = T([100, 3], _lib.I32), T([100, 27], _lib.I32)
    rc, msg = status("lux3d_sparse_neighbors", co, T([128], _lib.I64), T([128], _lib.I32), nbr, None, None)
    assert rc == _lib.ERR_SHAPE and "power-of-two" in msg        # 128 < 2 N
    rc, msg = status("lux3d_sparse_neighbors", co, T([256], _lib.I64), T([255], _lib.I32), nbr, None, None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_sparse_neighbors", co, T([256], _lib.I32), T([256], _lib.I32), nbr, None, None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status("lux3d_sparse_neighbors", co, T([256], _lib.I64), T([256], _lib.I32), nbr, T([1], _lib.F32), None)
    assert rc == _lib.ERR_DTYPE and "bad_coords" in msg
    # the allocation-free variant: same shapes, and at most 2^20 voxels
    big = (1 << 20) + 1
    rc, msg = status("lux3d_sparse_neighbors_noalloc", T([big, 3], _lib.I32), T([big, 27], _lib.I32), None, None)
    assert rc == _lib.ERR_SHAPE and "limit of 1048576" in msg
    rc, msg = status("lux3d_sparse_neighbors_noalloc", co, T([100, 26], _lib.I32), None, None)
    assert rc == _lib.ERR_SHAPE and "[100, 27]" in msg
    rc, msg = status("lux3d_sparse_neighbors_noalloc", co, nbr, T([1], _lib.F32), None)
    assert rc == _lib.ERR_DTYPE and "bad_coords" in msg
    rc, msg = status("lux3d_sparse_neighbors_noalloc", T([100, 3], _lib.I64), nbr, None, None)
    assert rc == _lib.ERR_DTYPE
    x, w, out = T([100, 64], _lib.F32), T([27, 32, 64], _lib.F32), T([100, 32], _lib.F32)
    rc, msg = status("lux3d_sparse_conv3d", x, nbr, T([27, 32, 48], _lib.F32), None, out, None)
    assert rc == _lib.ERR_SHAPE and "SparseConv3d expects" in msg
    rc, msg = status("lux3d_sparse_conv3d", T([100, 64]), nbr, w, None, out, None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status("lux3d_sparse_conv3d", x, nbr, w, T([31], _lib.F32), out, None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_index_select_rows", T([10, 4]), T([5], _lib.F32), T([5, 4]), None, None)
    assert rc == _lib.ERR_DTYPE
    rc, msg = status("lux3d_index_select_rows", T([10, 4]), T([5], _lib.I32), T([5, 3]), None, None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_index_select_rows", T([10, 4]), T([5], _lib.I32), T([5, 4]), T([0], _lib.I32), None)
    assert rc == _lib.ERR_SHAPE and "bad_ids" in msg
    f, lg = T([100, 12], _lib.F32), T([100, 8], _lib.F32)
    args = [T([108], _lib.I32), T([800, 3], _lib.I32), T([800], _lib.I32), T([800, 1], _lib.F32),
            T([100, 8], _lib.F32), T([1], _lib.I32), None]
    rc, msg = status("lux3d_channel_to_spatial", co, f, lg, *args)
    assert rc == _lib.ERR_SHAPE and "divisible by 8" in msg
    rc, msg = status("lux3d_channel_to_spatial", co, T([100, 16], _lib.F32), T([100, 7], _lib.F32),
                     T([108], _lib.I32), T([800, 3], _lib.I32), T([800], _lib.I32), T([800, 2], _lib.F32),
                     T([100, 8], _lib.F32), T([1], _lib.I32), None)
    assert rc == _lib.ERR_SHAPE and "subdivision logits must be" in msg


def test_sdpa_layernorm_rope2d_argument_errors():
    q, k, v, o = T([2, 4, 33, 64]), T([2, 4, 50, 64]), T([2, 4, 50, 64]), T([2, 4, 33, 64])
    w, b = T([64], _lib.F32), T([64], _lib.F32)
    cs, sn = T([2, 33, 64], _lib.F32), T([2, 33, 64], _lib.F32)
    rc, msg = status("lux3d_sdpa_layernorm_rope2d", q, None, b, 1e-5, cs, sn, k, v, 0.125, o, None)
    assert rc == _lib.ERR_NULL and "needs a weight" in msg
    rc, msg = status("lux3d_sdpa_layernorm_rope2d", q, T([63], _lib.F32), b, 1e-5, cs, sn, k, v, 0.125, o, None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_sdpa_layernorm_rope2d", q, w, b, 1e-5, T([2, 34, 64], _lib.F32), sn, k, v, 0.125, o, None)
    assert rc == _lib.ERR_SHAPE and "cos_full" in msg
    rc, msg = status("lux3d_sdpa_layernorm_rope2d", q, w, b, -1.0, cs, sn, k, v, 0.125, o, None)
    assert rc == _lib.ERR_VALUE
    rc, msg = status("lux3d_sdpa_layernorm_rope2d", q, w, b, 1e-5, cs, sn, k, v, 0.0, o, None)
    assert rc == _lib.ERR_VALUE


def test_fused_model_attention_argument_errors():
    """The TripoSG / TRELLIS.2 / DINOv3 entries that take q's norm / rotation
    into the attention reject bad parameters and tables on the host (before
    choosing between the fused kernel and the two launches)."""
    q, k, v, o = T([1, 2, 40, 128]), T([1, 2, 40, 128]), T([1, 2, 40, 128]), T([1, 2, 40, 128])
    w = T([128], _lib.F32)
    rc, msg = status("lux3d_sdpa_rms_norm_heads", q, None, 1e-6, k, v, 0.1, o, None)
    assert rc == _lib.ERR_NULL and "q_w" in msg
    rc, msg = status("lux3d_sdpa_rms_norm_heads", q, T([64], _lib.F32), 1e-6, k, v, 0.1, o, None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_sdpa_rms_norm_heads", q, w, -1.0, k, v, 0.1, o, None)
    assert rc == _lib.ERR_VALUE
    rc, msg = status("lux3d_sdpa_rms_norm_heads", q, w, 1e-6, k, v, 0.1, T([1, 2, 39, 128]), None)
    assert rc == _lib.ERR_SHAPE
    gam, cs, sn = T([2, 128], _lib.F32), T([40, 64], _lib.F32), T([40, 64], _lib.F32)
    rc, msg = status("lux3d_sdpa_l2norm_rope3d", q, None, cs, sn, k, v, 0.1, o, None)
    assert rc == _lib.ERR_NULL and "q_gamma" in msg
    rc, msg = status("lux3d_sdpa_l2norm_rope3d", q, T([128], _lib.F32), cs, sn, k, v, 0.1, o, None)
    assert rc == _lib.ERR_SHAPE
    rc, msg = status("lux3d_sdpa_l2norm_rope3d", q, gam, T([40, 128], _lib.F32), sn, k, v, 0.1, o, None)
    assert rc == _lib.ERR_SHAPE and "[L, D/2]" in msg
    rc, msg = status("lux3d_sdpa_l2norm_rope3d", q, gam, cs, T([40, 64], _lib.BF16), k, v, 0.1, o, None)
    assert rc == _lib.ERR_LAYOUT
    rc, msg = status("lux3d_sdpa_l2norm_rope3d", q, gam, cs, None, k, v, 0.1, o, None)
    assert rc == _lib.ERR_NULL
    q3, k3, v3, o3 = T([1, 2, 40, 64], _lib.F32), T([1, 2, 40, 64], _lib.F32), T([1, 2, 40, 64], _lib.F32), \
        T([1, 2, 40, 64], _lib.F32)
    c3, s3 = T([35, 64], _lib.F32), T([35, 64], _lib.F32)
    rc, msg = status("lux3d_sdpa_dinov3_rope", q3, c3, s3, 41, k3, v3, 0.125, o3, None)
    assert rc == _lib.ERR_VALUE and "num_prefix" in msg
    rc, msg = status("lux3d_sdpa_dinov3_rope", q3, c3, s3, 4, k3, v3, 0.125, o3, None)
    assert rc == _lib.ERR_SHAPE and "[S - num_prefix, D]" in msg
    rc, msg = status("lux3d_sdpa_dinov3_rope", q3, c3, s3, 5, k3, v3, 0.125, T([1, 2, 40, 64]), None)
    assert rc == _lib.ERR_DTYPE


def test_integration_ffi_block_lists_every_entry():
    """The Rust extern blocks of the integration guide at the repository root
    declare exactly the functions of include/lux3d_fused.h and
    include/lux3d_weights.h, each with the header's parameter count."""
    def header_sigs(path):
        text = re.sub(r"/\*.*?\*/", "", open(path).read(), flags=re.S)
        out = {}
        for name, args in re.findall(r"\b(lux3d_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text):
            a = " ".join(args.split())
            out[name] = 0 if a in ("", "void") else a.count(",") + 1
        return out
    want = header_sigs(HEADER)
    want.update(header_sigs(os.path.join(ROOT, "include", "lux3d_weights.h")))
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    got = {}
    for name, args in re.findall(r"pub fn (lux3d_[a-z0-9_]+)\(([^;]*?)\)\s*(?:->[^;]*)?;", doc, flags=re.S):
        a = " ".join(args.split())
        got[name] = 0 if not a else a.count(",") + 1
    assert got == want
