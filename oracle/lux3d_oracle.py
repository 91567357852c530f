"""ctypes binding of the CPU oracle (liblux3d_oracle.so, built from
lux3d_oracle.c by oracle/Makefile).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker. The product library never uses
it. Arrays are numpy; bf16/f16 data travels as raw uint16 bits.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblux3d_oracle.so")

F32, BF16, F16 = 0, 1, 2

_P = ctypes.c_void_p
_I = ctypes.c_int64
_F = ctypes.c_float
_SIG = {
    "or_set_threads": ([ctypes.c_int], None),
    "or_get_threads": ([], ctypes.c_int),
    "or_f32_to_bf16": ([_F], ctypes.c_uint16),
    "or_bf16_to_f32": ([ctypes.c_uint16], _F),
    "or_f32_to_f16": ([_F], ctypes.c_uint16),
    "or_f16_to_f32": ([ctypes.c_uint16], _F),
    "or_convert": ([ctypes.c_int, _P, ctypes.c_int, _P, _I], None),
    "or_layer_norm": ([ctypes.c_int, _P, _I, _I, _P, _P, _F, _P], None),
    "or_layer_norm_slow": ([ctypes.c_int, _P, _I, _I, _P, _P, _F, _P], None),
    "or_layer_norm_no_affine": ([ctypes.c_int, _P, _I, _I, _F, _P], None),
    "or_residual_layer_norm": ([ctypes.c_int, _P, _P, _P, _I, _I, _P, _P, _F, _P, _P], None),
    "or_adaln_modulate": ([ctypes.c_int, _P, _I, _I, _P, _I, _P, _I, _P, _P, _I, _P, _P, _I, _P, _F, _P], None),
    "or_gated_residual": ([ctypes.c_int, _P, _P, _I, _I, _P, _I, _P, _I, _P, _P], None),
    "or_gated_residual_modulate": ([ctypes.c_int, _P, _P, _I, _I, _P, _I, _P, _I, _P, _P, _I, _P, _P, _I, _P,
                                    _F, _P, _P], None),
    "or_rms_norm_heads": ([ctypes.c_int, _P, _I, _I, _P, _F, _P], None),
    "or_qk_l2norm": ([ctypes.c_int, _P, _I, _I, _I, _P, _P], None),
    "or_rope2d_tables": ([_P, _I, _I, _I, _F, _P, _P], None),
    "or_rope2d_apply": ([ctypes.c_int, _P, _I, _I, _I, _I, _P, _P, _P], None),
    "or_layernorm_rope2d": ([ctypes.c_int, _P, _I, _I, _I, _I, _P, _P, _F, _P, _P, _P], None),
    "or_rope3d_tables": ([_P, _I, _I, _F, _P, _P], None),
    "or_rope3d_apply": ([ctypes.c_int, _P, _I, _I, _I, _I, _P, _P, _P], None),
    "or_qk_l2norm_rope3d": ([ctypes.c_int, _P, _I, _I, _I, _P, _P, _P, _P], None),
    "or_dinov3_rope_tables": ([_I, _I, _I, _F, _P, _P], None),
    "or_dinov3_rope_apply": ([ctypes.c_int, _P, _I, _I, _I, _I, _I, _P, _P, _P], None),
    "or_gelu_erf": ([ctypes.c_int, _P, _I, _P], None),
    "or_gelu_tanh": ([ctypes.c_int, _P, _I, _P], None),
    "or_silu": ([ctypes.c_int, _P, _I, _P], None),
    "or_timestep_embedding_sin_first": ([_P, _I, _I, _P], None),
    "or_timestep_embedding_cos_first": ([_P, _I, _I, _P], None),
    "or_timestep_embedding_freqs": ([_P, _I, _P, _I, ctypes.c_int, _P], None),
    "or_dequant_q8_0": ([_P, _I, ctypes.c_int, _P], None),
    "or_q8_0_linear": ([_P, _I, _I, _P, _I, _P, ctypes.c_int, _P, _P], None),
    "or_q8_0_linear_f32": ([_P, _I, _I, _P, _I, _P, ctypes.c_int, _P, _P], None),
    "or_quantize_q8_0": ([_P, _I, _P], None),
    "or_q8_0_linear_int8": ([_P, _I, _I, _P, _I, _P, _P], None),
    "or_sparse_neighbors": ([_P, _I, _P], None),
    "or_sparse_conv3d": ([_P, _I, _I, _P, _P, _P, _I, _P, _P], None),
    "or_channel_to_spatial": ([_P, _I, _P, _I, _P, _P, _P, _P, _P], ctypes.c_int64),
    "or_sdpa": ([ctypes.c_int, _P, _P, _P, _I, _I, _I, _I, ctypes.c_double, ctypes.c_int, _P, _P], None),
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run `make -C oracle`")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in _SIG.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


LIB = _load()


def set_threads(n: int) -> None:
    LIB.or_set_threads(int(n))


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def dt_of(a: np.ndarray, dt: int | None = None) -> int:
    if dt is not None:
        return dt
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    raise TypeError("pass dt=BF16 for uint16 bf16 bits")


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _like(a):
    return np.empty(a.shape, dtype=a.dtype)


# ---- conversions -----------------------------------------------------------

def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits (RNE, half-crate NaN rule)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    LIB.or_convert(F32, _ptr(x), BF16, _ptr(out), x.size)
    return out


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


# ---- ops (dt: dtype code of the activation arrays) ------------------------

def layer_norm(x, w, b, eps, dt=None, slow=False):
    dt = dt_of(x, dt)
    y = _like(x)
    d = x.shape[-1]
    fn = LIB.or_layer_norm_slow if slow else LIB.or_layer_norm
    w, b = _f32(w), _f32(b)
    fn(dt, _ptr(x), x.size // d, d, _ptr(w), _ptr(b), eps, _ptr(y))
    return y


def layer_norm_no_affine(x, eps, dt=None):
    dt = dt_of(x, dt)
    y = _like(x)
    d = x.shape[-1]
    LIB.or_layer_norm_no_affine(dt, _ptr(x), x.size // d, d, eps, _ptr(y))
    return y


def residual_layer_norm(x, a, gamma, w, b, eps, dt=None):
    dt = dt_of(x, dt)
    h, y = _like(x), _like(x)
    d = x.shape[-1]
    gamma, w, b = _f32(gamma), _f32(w), _f32(b)
    LIB.or_residual_layer_norm(dt, _ptr(x), _ptr(a), _ptr(gamma), x.size // d, d, _ptr(w), _ptr(b), eps,
                               _ptr(h), _ptr(y))
    return h, y


def _piece(p):
    if p is None:
        return None, 0
    p = _f32(p)
    if p.ndim == 1:
        return p, 0
    return p, p.shape[-1]


def adaln_modulate(x, seg_off, shift, scale, gate=None, shift_base=None, scale_base=None, gate_base=None,
                   eps=1e-6, dt=None):
    """Pieces are [S, C] f32 arrays (contiguous); seg_off int64 [S+1]."""
    dt = dt_of(x, dt)
    y = _like(x)
    d = x.shape[-1]
    rows = x.size // d
    seg_off = np.ascontiguousarray(seg_off, dtype=np.int64)
    sh, ldsh = _piece(shift)
    sc, ldsc = _piece(scale)
    g, ldg = _piece(gate)
    LIB.or_adaln_modulate(dt, _ptr(x), rows, d, _ptr(seg_off), seg_off.size - 1, _ptr(sh), ldsh,
                          _ptr(_f32(shift_base)), _ptr(sc), ldsc, _ptr(_f32(scale_base)), _ptr(g), ldg,
                          _ptr(_f32(gate_base)), eps, _ptr(y))
    return y


def gated_residual(x, h, seg_off, gate, gate_base=None, dt=None):
    dt = dt_of(x, dt)
    out = _like(x)
    d = x.shape[-1]
    seg_off = np.ascontiguousarray(seg_off, dtype=np.int64)
    g, ldg = _piece(gate)
    LIB.or_gated_residual(dt, _ptr(x), _ptr(h), x.size // d, d, _ptr(seg_off), seg_off.size - 1, _ptr(g), ldg,
                          _ptr(_f32(gate_base)), _ptr(out))
    return out


def gated_residual_modulate(x, h, seg_off, gate, shift, scale, gate_base=None, shift_base=None, scale_base=None,
                            eps=1e-6, dt=None):
    """x_out = x + h*gate (gate None: x + h), y = L3(x_out)*(scale+1) + shift.
    Pieces are [S, C] f32 arrays; seg_off int64 [S+1]. Returns (x_out, y)."""
    dt = dt_of(x, dt)
    xo, y = _like(x), _like(x)
    d = x.shape[-1]
    seg_off = np.ascontiguousarray(seg_off, dtype=np.int64)
    g, ldg = _piece(gate)
    sh, ldsh = _piece(shift)
    sc, ldsc = _piece(scale)
    LIB.or_gated_residual_modulate(dt, _ptr(x), _ptr(h), x.size // d, d, _ptr(seg_off), seg_off.size - 1, _ptr(g),
                                   ldg, _ptr(_f32(gate_base)), _ptr(sh), ldsh, _ptr(_f32(shift_base)), _ptr(sc),
                                   ldsc, _ptr(_f32(scale_base)), eps, _ptr(xo), _ptr(y))
    return xo, y


def rms_norm_heads(x, w, eps, dt=None):
    dt = dt_of(x, dt)
    y = _like(x)
    d = x.shape[-1]
    LIB.or_rms_norm_heads(dt, _ptr(x), x.size // d, d, _ptr(_f32(w)), eps, _ptr(y))
    return y


def qk_l2norm(x, gamma, dt=None):
    """x [..., H, D], gamma [H, D]."""
    dt = dt_of(x, dt)
    y = _like(x)
    h, d = x.shape[-2], x.shape[-1]
    LIB.or_qk_l2norm(dt, _ptr(x), x.size // (h * d), h, d, _ptr(_f32(gamma)), _ptr(y))
    return y


def rope2d_tables(pos, d, base):
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    b, n, _ = pos.shape
    c = np.empty((b, n, d), dtype=np.float32)
    s = np.empty((b, n, d), dtype=np.float32)
    LIB.or_rope2d_tables(_ptr(pos), b, n, d, base, _ptr(c), _ptr(s))
    return c, s


def rope2d_apply(t, cos_full, sin_alt, dt=None):
    """t [b, h, n, d]; tables [b, n, d]."""
    dt = dt_of(t, dt)
    y = _like(t)
    b, h, n, d = t.shape
    LIB.or_rope2d_apply(dt, _ptr(t), b, h, n, d, _ptr(_f32(cos_full)), _ptr(_f32(sin_alt)), _ptr(y))
    return y


def layernorm_rope2d(q, w, bias, eps, cos_full, sin_alt, dt=None):
    dt = dt_of(q, dt)
    y = _like(q)
    b, h, n, d = q.shape
    LIB.or_layernorm_rope2d(dt, _ptr(q), b, h, n, d, _ptr(_f32(w)), _ptr(_f32(bias)), eps, _ptr(_f32(cos_full)),
                            _ptr(_f32(sin_alt)), _ptr(y))
    return y


def rope3d_tables(coords, head_dim, base=10000.0):
    coords = np.ascontiguousarray(coords, dtype=np.int32)
    n = coords.shape[0]
    c = np.empty((n, head_dim // 2), dtype=np.float32)
    s = np.empty((n, head_dim // 2), dtype=np.float32)
    LIB.or_rope3d_tables(_ptr(coords), n, head_dim, base, _ptr(c), _ptr(s))
    return c, s


def rope3d_apply(x, cos, sin, dt=None):
    """x [b, l, h, d]; tables [l, d/2]."""
    dt = dt_of(x, dt)
    y = _like(x)
    b, l, h, d = x.shape
    LIB.or_rope3d_apply(dt, _ptr(x), b, l, h, d, _ptr(_f32(cos)), _ptr(_f32(sin)), _ptr(y))
    return y


def qk_l2norm_rope3d(x, gamma, cos, sin, dt=None):
    """x [rows, H, D] (rows = tokens); tables [rows, D/2]."""
    dt = dt_of(x, dt)
    y = _like(x)
    h, d = x.shape[-2], x.shape[-1]
    LIB.or_qk_l2norm_rope3d(dt, _ptr(x), x.size // (h * d), h, d, _ptr(_f32(gamma)), _ptr(_f32(cos)),
                            _ptr(_f32(sin)), _ptr(y))
    return y


def dinov3_rope_tables(grid_h, grid_w, head_dim, theta=100.0):
    p = grid_h * grid_w
    c = np.empty((p, head_dim), dtype=np.float32)
    s = np.empty((p, head_dim), dtype=np.float32)
    LIB.or_dinov3_rope_tables(grid_h, grid_w, head_dim, theta, _ptr(c), _ptr(s))
    return c, s


def dinov3_rope_apply(x, num_prefix, cos, sin, dt=None):
    """x [b, h, s, d]; tables [s - num_prefix, d]."""
    dt = dt_of(x, dt)
    y = _like(x)
    b, h, s, d = x.shape
    LIB.or_dinov3_rope_apply(dt, _ptr(x), b, h, s, d, num_prefix, _ptr(_f32(cos)), _ptr(_f32(sin)), _ptr(y))
    return y


def _act(fn, x, dt):
    dt = dt_of(x, dt)
    y = _like(x)
    fn(dt, _ptr(x), x.size, _ptr(y))
    return y


def gelu_erf(x, dt=None):
    return _act(LIB.or_gelu_erf, x, dt)


def gelu_tanh(x, dt=None):
    return _act(LIB.or_gelu_tanh, x, dt)


def silu(x, dt=None):
    return _act(LIB.or_silu, x, dt)


def timestep_embedding(t, dim, cos_first=True, freqs=None):
    """T1 / T2 with the frequencies the reference's host loop computes
    (libm expf), or from a given frequency vector `freqs` [dim // 2]."""
    t = _f32(t).reshape(-1)
    out = np.empty((t.size, dim), dtype=np.float32)
    if freqs is not None:
        f = _f32(freqs).reshape(-1)
        assert f.size == dim // 2
        LIB.or_timestep_embedding_freqs(_ptr(t), t.size, _ptr(f), dim, 1 if cos_first else 0, _ptr(out))
        return out
    fn = LIB.or_timestep_embedding_cos_first if cos_first else LIB.or_timestep_embedding_sin_first
    fn(_ptr(t), t.size, dim, _ptr(out))
    return out


def timestep_freqs_rounded_once(dim):
    """exp(x) evaluated in f64 and rounded once to f32, for the reference's
    f32 argument x = (nlp * i) / half, nlp = f32(-ln 10000)
    (trellis2_blocks.rs:189-194; triposg_dit.rs:286-291): the correctly
    rounded frequency wherever the f64 exp is within half an f32 ulp's
    margin, which tests/test_oracle_pins.py checks against exact values."""
    import math
    half = dim // 2
    nlp = np.float32(-math.log(10000.0))
    x = (nlp * np.arange(half, dtype=np.float32)) / np.float32(half)
    return np.exp(x.astype(np.float64)).astype(np.float32)


def dequant_q8_0(blocks, out_dt=BF16):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    nb = blocks.size // 34
    out = np.empty(nb * 32, dtype=np.float32 if out_dt == F32 else np.uint16)
    LIB.or_dequant_q8_0(_ptr(blocks), nb, out_dt, _ptr(out))
    return out


def quantize_q8_0(x):
    """BlockQ8_0::from_float of f32 x [..., K] (K % 32 == 0): u8 blocks [rows * K/32 * 34]."""
    x = _f32(x).reshape(-1)
    out = np.empty(x.size // 32 * 34, dtype=np.uint8)
    LIB.or_quantize_q8_0(_ptr(x), x.size, _ptr(out))
    return out


def q8_0_linear_int8(x, blocks, n, bias=None):
    """candle's CPU QMatMul for a Q8_0 weight (+ bias): f32 x [M, K], weight
    blocks of [n, K] -> f32 [M, n]."""
    x = _f32(x)
    M, K = x.shape
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    assert blocks.size == n * (K // 32) * 34
    y = np.empty((M, n), dtype=np.float32)
    b = _f32(bias) if bias is not None else None
    LIB.or_q8_0_linear_int8(_ptr(x), M, K, _ptr(blocks), n, _ptr(b) if b is not None else None, _ptr(y))
    return y


def q8_0_linear(x_bits, blocks, n, bias=None, out_dt=BF16, with_abs=False):
    """x: bf16 bits [M, K] (uint16), or f32 [M, K] for the f32-activation
    form (weights dequantized exactly to f32); blocks: Q8_0 bytes of the
    weight [n, K]. Returns y [M, n] (uint16 bits for bf16 / f16, f32
    otherwise) and, with_abs, sum_k |x * w| as f32 [M, n]."""
    f32x = np.asarray(x_bits).dtype == np.float32
    x_bits = np.ascontiguousarray(x_bits, dtype=np.float32 if f32x else np.uint16)
    m, k = x_bits.shape
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    assert blocks.size == n * (k // 32) * 34
    y = np.empty((m, n), dtype=np.float32 if out_dt == F32 else np.uint16)
    a = np.empty((m, n), dtype=np.float32) if with_abs else None
    fn = LIB.or_q8_0_linear_f32 if f32x else LIB.or_q8_0_linear
    fn(_ptr(x_bits), m, k, _ptr(blocks), n, _ptr(_f32(bias)), out_dt, _ptr(y), _ptr(a))
    return (y, a) if with_abs else y


def sdpa(q, k, v, scale, dt=None, out_dt=None, with_abs=False):
    """Attention over q [..., Lq, D], k and v [..., Lk, D] (same leading dims;
    f32, f16, or bf16 bits as uint16 with dt=BF16). Returns softmax(q k^T *
    scale) v as [..., Lq, D] in out_dt (default: the input dtype) and, with
    with_abs, sum_j p_j |v_j| / sum_j p_j as f32."""
    dt = dt_of(q, dt)
    out_dt = dt if out_dt is None else out_dt
    q, k, v = (np.ascontiguousarray(a) for a in (q, k, v))
    *lead, lq, d = q.shape
    lk = k.shape[-2]
    assert k.shape == v.shape and k.shape[-1] == d and tuple(k.shape[:-2]) == tuple(lead)
    bh = int(np.prod(lead)) if lead else 1
    out = np.empty(q.shape, dtype=np.float32 if out_dt == F32 else (np.float16 if out_dt == F16 else np.uint16))
    a = np.empty(q.shape, dtype=np.float32) if with_abs else None
    LIB.or_sdpa(dt, _ptr(q), _ptr(k), _ptr(v), bh, lq, lk, d, float(scale), out_dt, _ptr(out), _ptr(a))
    return (out, a) if with_abs else out


def sparse_neighbors(coords):
    """coords int32 [N, 3] -> neighbour rows int32 [N, 27] (-1: missing)."""
    coords = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 3)
    nbr = np.empty((coords.shape[0], 27), dtype=np.int32)
    LIB.or_sparse_neighbors(_ptr(coords), coords.shape[0], _ptr(nbr))
    return nbr


def sparse_conv3d(x, nbr, w27, bias=None, with_abs=False):
    """x f32 [R, Cin], nbr [N, 27] (rows of x), w27 f32 [27, Cout, Cin] ->
    f32 [N, Cout] (N may be a subset of the rows: the output rows follow nbr)."""
    x = _f32(x)
    cin = x.shape[1]
    w27 = _f32(w27)
    cout = w27.shape[1]
    nbr = np.ascontiguousarray(nbr, dtype=np.int32)
    n = nbr.shape[0]
    out = np.empty((n, cout), dtype=np.float32)
    a = np.empty((n, cout), dtype=np.float32) if with_abs else None
    LIB.or_sparse_conv3d(_ptr(x), n, cin, _ptr(nbr), _ptr(w27), _ptr(_f32(bias)), cout, _ptr(out), _ptr(a))
    return (out, a) if with_abs else out


def channel_to_spatial(coords, feats, logits):
    """Returns (child coords [M, 3], child feats [M, C/8], src rows [M], sub [N, 8])."""
    coords = np.ascontiguousarray(coords, dtype=np.int32).reshape(-1, 3)
    feats, logits = _f32(feats), _f32(logits)
    n, c = feats.shape
    oc = np.empty((8 * n, 3), dtype=np.int32)
    of = np.empty((8 * n, c // 8), dtype=np.float32)
    src = np.empty(8 * n, dtype=np.int32)
    sub = np.empty((n, 8), dtype=np.float32)
    m = LIB.or_channel_to_spatial(_ptr(coords), n, _ptr(feats), c, _ptr(logits), _ptr(oc), _ptr(of), _ptr(src),
                                  _ptr(sub))
    return oc[:m].copy(), of[:m].copy(), src[:m].copy(), sub
