"""Tensor-level mirror of candle-3d's operator surface on the fused HIP ops.

Each function keeps the name, argument meaning and error behaviour of the
reference helper or candle op it replaces (cited per function; paths are
relative to crates/lux3d-core/src/ of the candle-3d tree). Like a candle
CustomOp, every op borrows its inputs and allocates its outputs; torch tensors
on a ROCm device are used only as device memory and streams. All arithmetic
happens in liblux3d_fused.so; invalid arguments raise Lux3dError, exactly as
the reference's `candle_core::bail!` sites return an error.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16,
       torch.int32: _lib.I32, torch.int64: _lib.I64, torch.uint8: _lib.U8, torch.int8: _lib.I8}


def desc(t: Optional[torch.Tensor]):
    """lux3d_tensor_t pointer for a torch tensor (None -> NULL)."""
    if t is None:
        return None
    if t.dtype not in _DT:
        raise TypeError(f"unsupported dtype {t.dtype}")
    if t.dim() == 0:
        t = t.reshape(1)
    d = _lib.descriptor(t.data_ptr(), _DT[t.dtype], list(t.shape), list(t.stride()))
    return ctypes.pointer(d)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _keep(*ts):
    """Descriptors hold raw pointers: keep the tensors alive for the call."""
    return ts


# ---------------------------------------------------------------------------
# Row family
# ---------------------------------------------------------------------------

def layer_norm(x: torch.Tensor, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor],
               eps: float) -> torch.Tensor:
    """candle_nn::ops::layer_norm(x, w, b, eps) (upstream candle-nn), the op
    behind every `layer_norm(dim, eps, vb)` LayerNorm::forward in the
    reference (e.g. runtime/pi3_encoder.rs:67, runtime/vggt.rs:104)."""
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _lib.call("lux3d_layer_norm", desc(x), desc(weight), desc(bias), eps, desc(y), _stream(x))
    return y


def layer_norm_no_affine(xs: torch.Tensor, eps: float) -> torch.Tensor:
    """layer_norm_no_affine (runtime/trellis2_blocks.rs:280-286)."""
    return layer_norm(xs, None, None, eps)


def residual_layer_norm(x: torch.Tensor, a: torch.Tensor, ls_gamma: Optional[torch.Tensor],
                        weight: Optional[torch.Tensor], bias: Optional[torch.Tensor], eps: float,
                        h_out: Optional[torch.Tensor] = None):
    """`h = x + ls(a)`, `y = norm(h)`: LayerScale::forward
    (runtime/nn_blocks.rs:210-214) + residual + LayerNorm::forward as in
    VggtBlock::forward (runtime/vggt.rs:113-124). Returns (h, y)."""
    h = torch.empty(x.shape, dtype=x.dtype, device=x.device) if h_out is None else h_out
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _lib.call("lux3d_residual_layer_norm", desc(x), desc(a), desc(ls_gamma), desc(weight), desc(bias),
              eps, desc(h), desc(y), _stream(x))
    return h, y


def adaln_modulate(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor,
                   gate: Optional[torch.Tensor] = None, *, shift_base=None, scale_base=None,
                   gate_base=None, seg_offsets: Optional[torch.Tensor] = None,
                   eps: float = 1e-6) -> torch.Tensor:
    """`layer_norm_no_affine(x)*(1 + scale) + shift` (optionally
    `gate*(...) + x`), per batch element or ragged segment:
    runtime/trellis2_blocks.rs:617-630 (with `modulation + t_emb` via the
    *_base vectors) and runtime/vggt.rs:399-405 (gate variant)."""
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _lib.call("lux3d_adaln_modulate", desc(x), desc(seg_offsets), desc(shift), desc(shift_base),
              desc(scale), desc(scale_base), desc(gate), desc(gate_base), eps, desc(y), _stream(x))
    return y


def gated_residual(x: torch.Tensor, h: torch.Tensor, gate: torch.Tensor, *, gate_base=None,
                   seg_offsets: Optional[torch.Tensor] = None,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """`xs.add(h.broadcast_mul(gate))` (runtime/trellis2_blocks.rs:632-633)."""
    o = torch.empty(x.shape, dtype=x.dtype, device=x.device) if out is None else out
    _lib.call("lux3d_gated_residual", desc(x), desc(h), desc(seg_offsets), desc(gate), desc(gate_base),
              desc(o), _stream(x))
    return o


def gated_residual_adaln_modulate(x: torch.Tensor, h: torch.Tensor, gate: Optional[torch.Tensor],
                                  shift: torch.Tensor, scale: torch.Tensor, *, gate_base=None,
                                  shift_base=None, scale_base=None,
                                  seg_offsets: Optional[torch.Tensor] = None, eps: float = 1e-6,
                                  x_out: Optional[torch.Tensor] = None):
    """One pass of `xs = xs.add(h.broadcast_mul(gate))` (gate None: `xs.add(h)`)
    followed by `layer_norm_no_affine(xs)*(1 + scale) + shift`
    (runtime/trellis2_blocks.rs:708-713 sparse block, :637-642 dense block).
    Returns (x_out, y); x_out may be x (in-place residual update)."""
    xo = torch.empty(x.shape, dtype=x.dtype, device=x.device) if x_out is None else x_out
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _lib.call("lux3d_gated_residual_adaln_modulate", desc(x), desc(h), desc(seg_offsets), desc(gate),
              desc(gate_base), desc(shift), desc(shift_base), desc(scale), desc(scale_base), eps, desc(xo),
              desc(y), _stream(x))
    return xo, y


def chunk_modulation(mod_vec: torch.Tensor):
    """chunk_modulation (runtime/trellis2_blocks.rs:264-277): six [B, 1, C]
    views (shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp)
    of a [B, 6C] vector, without copies (the fused ops read the views)."""
    b, c6 = mod_vec.shape
    if c6 % 6:
        raise ValueError("adaLN modulation must chunk into 6")
    return [p.unsqueeze(1) for p in mod_vec.chunk(6, dim=-1)]


# ---------------------------------------------------------------------------
# VGGT / Pi3 2D RoPE (attention_math.rs)
# ---------------------------------------------------------------------------

@dataclass
class RopeEmbeddings:
    """RopeEmbeddings (runtime/attention_math.rs:88-95): cos_full and
    sin_alt_full, each [b, 1, n, token_dim] f32."""

    cos_full: torch.Tensor
    sin_alt_full: torch.Tensor


class Rope2d:
    """Rope2d (runtime/attention_math.rs:4-86)."""

    def __init__(self, base: float):
        self.base = float(base)

    def embeddings(self, positions: torch.Tensor, token_dim: int) -> RopeEmbeddings:
        half = token_dim // 2
        if half % 2 != 0:
            raise _lib.Lux3dError("Rope2d::embeddings", _lib.ERR_VALUE,
                                  f"rope token_dim must be divisible by 4, got {token_dim}")
        b, n, _ = positions.shape
        cos = torch.empty((b, 1, n, token_dim), dtype=torch.float32, device=positions.device)
        sin = torch.empty_like(cos)
        _lib.call("lux3d_rope2d_tables", desc(positions), self.base, desc(cos), desc(sin), _stream(cos))
        return RopeEmbeddings(cos, sin)


def _heads_out(q: torch.Tensor) -> torch.Tensor:
    return torch.empty(q.shape, dtype=q.dtype, device=q.device)


def layernorm_rope_fused(q: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float,
                         cos_full: torch.Tensor, sin_alt_full: torch.Tensor) -> torch.Tensor:
    """candle_nn::ops::layernorm_rope_fused (the fork's CustomOp3, routed at
    runtime/attention_math.rs:139-146): LN(64)+affine then 2D RoPE on a
    (possibly strided) [b, h, n, d] head view; contiguous output."""
    out = _heads_out(q)
    _lib.call("lux3d_qk_layernorm_rope2d", desc(q), desc(weight), desc(bias), None, None, None, eps,
              desc(cos_full), desc(sin_alt_full), desc(out), None, _stream(q))
    return out


def rope_fused(x: torch.Tensor, cos_full: torch.Tensor, sin_alt_full: torch.Tensor) -> torch.Tensor:
    """candle_nn::ops::rope_fused (runtime/attention_math.rs:162)."""
    out = _heads_out(x)
    _lib.call("lux3d_qk_layernorm_rope2d", desc(x), None, None, None, None, None, 0.0,
              desc(cos_full), desc(sin_alt_full), desc(out), None, _stream(x))
    return out


def apply_layernorm_rope(q: torch.Tensor, q_norm, embeddings: RopeEmbeddings) -> torch.Tensor:
    """apply_layernorm_rope (runtime/attention_math.rs:127-150); q_norm is
    (weight, bias, eps)."""
    w, b, eps = q_norm
    return layernorm_rope_fused(q, w, b, eps, embeddings.cos_full, embeddings.sin_alt_full)


def apply_rope(tokens: torch.Tensor, embeddings: RopeEmbeddings) -> torch.Tensor:
    """apply_rope (runtime/attention_math.rs:155-165)."""
    return rope_fused(tokens, embeddings.cos_full, embeddings.sin_alt_full)


def qk_layernorm_rope2d(q: torch.Tensor, k: torch.Tensor, q_norm, k_norm,
                        embeddings: Optional[RopeEmbeddings] = None, *,
                        positions: Optional[torch.Tensor] = None, base: float = 100.0):
    """Both apply_layernorm_rope calls of VggtAttention::forward
    (runtime/vggt.rs:170-181) in one launch. Rotation from the tables, or,
    with `positions`, computed in-kernel (no table traffic)."""
    qw, qb, eps = q_norm
    kw, kb, _ = k_norm
    qo, ko = _heads_out(q), _heads_out(k)
    if positions is not None:
        _lib.call("lux3d_qk_layernorm_rope2d_pos", desc(q), desc(qw), desc(qb), desc(k), desc(kw), desc(kb),
                  eps, desc(positions), base, desc(qo), desc(ko), _stream(q))
    else:
        _lib.call("lux3d_qk_layernorm_rope2d", desc(q), desc(qw), desc(qb), desc(k), desc(kw), desc(kb),
                  eps, desc(embeddings.cos_full), desc(embeddings.sin_alt_full), desc(qo), desc(ko),
                  _stream(q))
    return qo, ko


# ---------------------------------------------------------------------------
# TripoSG
# ---------------------------------------------------------------------------

def rms_norm_heads(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                   k: Optional[torch.Tensor] = None, k_weight: Optional[torch.Tensor] = None):
    """RmsNormHeads::rms_norm_heads (runtime/triposg_dit.rs:509-522) on a
    [B, H, L, D] head view (strided views accepted: the transpose/contiguous
    before it is fused). With `k`, both norms run in one launch."""
    qo = _heads_out(x)
    ko = _heads_out(k) if k is not None else None
    _lib.call("lux3d_rms_norm_heads", desc(x), desc(weight), desc(k), desc(k_weight), eps, desc(qo),
              desc(ko), _stream(x))
    return qo if k is None else (qo, ko)


# ---------------------------------------------------------------------------
# TRELLIS.2
# ---------------------------------------------------------------------------

class Trellis2QkRmsNorm:
    """Trellis2QkRmsNorm (runtime/trellis2_blocks.rs:288-320)."""

    def __init__(self, gamma: torch.Tensor):
        self.gamma = gamma

    def forward(self, xs: torch.Tensor) -> torch.Tensor:
        out = _heads_out(xs)
        _lib.call("lux3d_qk_l2norm_rope3d", desc(xs), desc(self.gamma), None, None, None, None, None, 0.0,
                  desc(out), None, _stream(xs))
        return out


class Trellis2Rope3d:
    """Trellis2Rope3d (runtime/trellis2_blocks.rs:84-161)."""

    def __init__(self, head_dim: int, rope_base: float = 10000.0):
        self.head_dim = int(head_dim)
        self.rope_base = float(rope_base)

    def cos_sin(self, coords: torch.Tensor):
        """coords int32 [L, 3] on the device -> (cos, sin) [L, head_dim/2]."""
        n = coords.shape[0]
        cos = torch.empty((n, self.head_dim // 2), dtype=torch.float32, device=coords.device)
        sin = torch.empty_like(cos)
        _lib.call("lux3d_rope3d_tables", desc(coords), self.head_dim, self.rope_base, desc(cos), desc(sin),
                  _stream(cos))
        return cos, sin

    def apply(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        out = _heads_out(x)
        _lib.call("lux3d_qk_l2norm_rope3d", desc(x), None, None, None, desc(cos), desc(sin), None, 0.0,
                  desc(out), None, _stream(x))
        return out


def qk_l2norm_rope3d(q: torch.Tensor, k: torch.Tensor, q_gamma: Optional[torch.Tensor],
                     k_gamma: Optional[torch.Tensor], *, coords: Optional[torch.Tensor] = None,
                     cos: Optional[torch.Tensor] = None, sin: Optional[torch.Tensor] = None,
                     rope_base: float = 10000.0):
    """Trellis2SelfAttention::attention's q/k stage
    (runtime/trellis2_blocks.rs:423-430) on [B, L, H, D] views, one launch."""
    qo, ko = _heads_out(q), _heads_out(k)
    _lib.call("lux3d_qk_l2norm_rope3d", desc(q), desc(q_gamma), desc(k), desc(k_gamma), desc(cos), desc(sin),
              desc(coords), rope_base, desc(qo), desc(ko), _stream(q))
    return qo, ko


def apply_rotary_to_patches(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                            num_prefix: int):
    """apply_rotary_to_patches (runtime/trellis2_dino.rs:406-436)."""
    qo, ko = _heads_out(q), _heads_out(k)
    _lib.call("lux3d_dinov3_rope", desc(q), desc(k), desc(cos), desc(sin), int(num_prefix), desc(qo),
              desc(ko), _stream(q))
    return qo, ko


# ---------------------------------------------------------------------------
# Activations, timestep embedding, Q8_0
# ---------------------------------------------------------------------------

def _act(name: str, x: torch.Tensor, out: Optional[torch.Tensor]) -> torch.Tensor:
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device) if out is None else out
    _lib.call(name, desc(x), desc(y), _stream(x))
    return y


def gelu_erf(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Tensor::gelu_erf (runtime/nn_blocks.rs:233)."""
    return _act("lux3d_gelu_erf", x, out)


def gelu(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Tensor::gelu, the tanh approximation (runtime/trellis2_blocks.rs:560)."""
    return _act("lux3d_gelu_tanh", x, out)


def silu(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Tensor::silu (runtime/trellis2_blocks.rs:236,257)."""
    return _act("lux3d_silu", x, out)


_LIBM = ctypes.CDLL("libm.so.6")
_LIBM.expf.restype = ctypes.c_float
_LIBM.expf.argtypes = [ctypes.c_float]
_LIBM.logf.restype = ctypes.c_float
_LIBM.logf.argtypes = [ctypes.c_float]


def host_timestep_freqs(dim: int) -> list:
    """The frequency vector the reference builds on the host,
    exp(-ln(10000) * i / half) with f32 arithmetic and libm expf
    (runtime/trellis2_blocks.rs:190-194; runtime/triposg_dit.rs:288-291)."""
    half = dim // 2
    nlp = ctypes.c_float(-math.log(10000.0)).value
    out = []
    for i in range(half):
        x = ctypes.c_float(ctypes.c_float(nlp * float(i)).value / float(half)).value
        out.append(_LIBM.expf(x))
    return out


def timestep_embedding(t: torch.Tensor, dim: int, cos_first: bool = True,
                       freqs: Optional[torch.Tensor] = None) -> torch.Tensor:
    """timestep_embedding (runtime/trellis2_blocks.rs:184-204, cos first)
    or TripoSgDiT::timestep_embedding (runtime/triposg_dit.rs:280-297, sin
    first) for a batch of f32 timesteps t [n] -> [n, dim] f32."""
    out = torch.empty((t.numel(), dim), dtype=torch.float32, device=t.device)
    _lib.call("lux3d_timestep_embedding", desc(t.reshape(-1)), desc(freqs), int(dim), 1 if cos_first else 0,
              desc(out), _stream(t))
    return out


def dequantize_q8_0(blocks: torch.Tensor, shape, dtype=torch.bfloat16) -> torch.Tensor:
    """QTensor::dequantize for a GGML Q8_0 tensor (runtime/nn_blocks.rs:140):
    u8 blocks [nblocks*34] -> dtype tensor of `shape`, bit-exact."""
    y = torch.empty(tuple(shape), dtype=dtype, device=blocks.device)
    _lib.call("lux3d_dequant_q8_0", desc(blocks.reshape(-1)), desc(y), _stream(y))
    return y


# ---------------------------------------------------------------------------
# Q8_0 quantized linear
# ---------------------------------------------------------------------------

def q8_0_repack(blocks: torch.Tensor, n: int, k: int):
    """The load-time step of a Q8_0 quantized linear (QMatMul::from_qtensor,
    runtime/nn_blocks.rs:145-150): GGML blocks of the weight [n, k] ->
    (qs int8 [n, k], scales f32 [n, k/32]), exact."""
    qs = torch.empty((n, k), dtype=torch.int8, device=blocks.device)
    scales = torch.empty((n, k // 32), dtype=torch.float32, device=blocks.device)
    _lib.call("lux3d_q8_0_repack", desc(blocks.reshape(-1)), int(n), int(k), desc(qs), desc(scales),
              _stream(blocks))
    return qs, scales


def q8_0_linear(x: torch.Tensor, qs: torch.Tensor, scales: torch.Tensor, bias: Optional[torch.Tensor] = None,
                out_dtype=torch.bfloat16) -> torch.Tensor:
    """`Linear::forward` for a Q8_0 weight (runtime/nn_blocks.rs:83-93):
    y = x @ dequant(W)^T (+ bias), x bf16 or f32 [..., k] -> y [..., n]
    (f32 x: the weights dequantized exactly to f32, k a multiple of 64)."""
    n = qs.shape[0]
    y = torch.empty(tuple(x.shape[:-1]) + (n,), dtype=out_dtype, device=x.device)
    _lib.call("lux3d_q8_0_linear", desc(x), desc(qs), desc(scales), desc(bias), desc(y), _stream(x))
    return y


def q8_0_quantize(x: torch.Tensor):
    """BlockQ8_0::from_float of f32 x [..., k] rows (candle-core
    k_quants.rs, the first step of candle's CPU QMatMul): -> (xq int8
    [rows, k], xd f32 [rows, k/32], the f16 block scales widened; a view of
    the library's block-major workspace)."""
    k = x.shape[-1]
    rows = x.numel() // k
    xq, xd = _q8_workspace(rows, k, x.device)
    _lib.call("lux3d_q8_0_quantize", desc(x), desc(xq), desc(xd), _stream(x))
    return xq, xd[:, :rows].t()


def _q8_workspace(rows, k, device):
    """xq int8 [rows, k] and the block-major xd f32 [k/32, rows rounded up to 64]."""
    xq = torch.empty((rows, k), dtype=torch.int8, device=device)
    xd = torch.empty((k // 32, (rows + 63) // 64 * 64), dtype=torch.float32, device=device)
    return xq, xd


def q8_0_linear_int8(x: torch.Tensor, qs: torch.Tensor, scales: torch.Tensor,
                     bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """`Linear::forward` for a Q8_0 weight with candle's CPU arithmetic
    (runtime/nn_blocks.rs:83-93 -> QMatMul::forward on the CPU): x f32 rows
    quantized to Q8_0 blocks, integer block dots, f32 block-order sum, +
    bias; f32 [..., k] -> f32 [..., n]. The quantization workspace is
    allocated here."""
    n, k = qs.shape
    rows = x.numel() // k
    xq, xd = _q8_workspace(rows, k, x.device)
    y = torch.empty(tuple(x.shape[:-1]) + (n,), dtype=torch.float32, device=x.device)
    _lib.call("lux3d_q8_0_linear_int8", desc(x), desc(qs), desc(scales), desc(bias), desc(xq), desc(xd), desc(y),
              _stream(x))
    return y


class QMatMul:
    """QMatMul over a Q8_0 weight [n, k] (the reference keeps the packed
    QTensor; here the blocks are repacked once to int8 + f32 scales)."""

    def __init__(self, qs: torch.Tensor, scales: torch.Tensor):
        self.qs, self.scales = qs, scales

    @classmethod
    def from_q8_0(cls, blocks: torch.Tensor, n: int, k: int) -> "QMatMul":
        return cls(*q8_0_repack(blocks, n, k))

    def forward(self, xs: torch.Tensor, bias: Optional[torch.Tensor] = None, out_dtype=torch.bfloat16):
        return q8_0_linear(xs, self.qs, self.scales, bias, out_dtype)


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(q k^T * scale) v over [B, H, L, D] views, one kernel, no scores
    buffer (attention_math.rs:199-259). `out` (default: a new contiguous
    [B, H, Lq, D]) may be any view with a unit inner stride, e.g. the
    [B, Lq, H, D] layout the caller transposes to next."""
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    _lib.call("lux3d_sdpa", desc(q), desc(k), desc(v), float(scale), desc(out), _stream(q))
    return out


def sdpa_layernorm_rope2d(q_raw: torch.Tensor, q_norm, embeddings: "RopeEmbeddings", k: torch.Tensor,
                          v: torch.Tensor, scale: float, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """exact_query_chunked_sdpa(apply_layernorm_rope(q_raw, q_norm, rope), k, v,
    scale) (vggt.rs:170-183) with q's LayerNorm + 2D RoPE done in the
    attention kernel's Q load; q_norm is (weight, bias, eps); k already
    normalised and rotated."""
    w, b, eps = q_norm
    if out is None:
        out = torch.empty(q_raw.shape, dtype=q_raw.dtype, device=q_raw.device)
    _lib.call("lux3d_sdpa_layernorm_rope2d", desc(q_raw), desc(w), desc(b), float(eps), desc(embeddings.cos_full),
              desc(embeddings.sin_alt_full), desc(k), desc(v), float(scale), desc(out), _stream(q_raw))
    return out


def sdpa_rms_norm_heads(q_raw: torch.Tensor, q_w: torch.Tensor, eps: float, k: torch.Tensor, v: torch.Tensor,
                       scale: float, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """exact_query_chunked_sdpa(rms_norm_heads(q_raw, q_w), k, v, scale)
    (triposg_dit.rs:446-455) with q's per-head RMSNorm done in the attention
    kernel's Q load; k already normalised."""
    if out is None:
        out = torch.empty(q_raw.shape, dtype=q_raw.dtype, device=q_raw.device)
    _lib.call("lux3d_sdpa_rms_norm_heads", desc(q_raw), desc(q_w), float(eps), desc(k), desc(v), float(scale),
              desc(out), _stream(q_raw))
    return out


def sdpa_l2norm_rope3d(q_raw: torch.Tensor, q_gamma: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                       k: torch.Tensor, v: torch.Tensor, scale: float,
                       out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Trellis2SelfAttention::attention (trellis2_blocks.rs:417-436) on
    [B, H, L, D] views: exact_query_chunked_sdpa(rope(l2norm(q_raw)), k, v,
    scale) with q's L2 norm (gamma [H, D]) and 3D RoPE (tables [L, D/2]) done
    in the attention kernel's Q load; k already normalised and rotated."""
    if out is None:
        out = torch.empty(q_raw.shape, dtype=q_raw.dtype, device=q_raw.device)
    _lib.call("lux3d_sdpa_l2norm_rope3d", desc(q_raw), desc(q_gamma), desc(cos), desc(sin), desc(k), desc(v),
              float(scale), desc(out), _stream(q_raw))
    return out


def sdpa_dinov3_rope(q_raw: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, num_prefix: int, k: torch.Tensor,
                     v: torch.Tensor, scale: float, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """exact_sdpa_heads(apply_rotary_to_patches(q_raw), k, v, scale)
    (trellis2_dino.rs:385-393) with q's rotate_half RoPE done in the
    attention kernel's Q load; k already rotated."""
    if out is None:
        out = torch.empty(q_raw.shape, dtype=q_raw.dtype, device=q_raw.device)
    _lib.call("lux3d_sdpa_dinov3_rope", desc(q_raw), desc(cos), desc(sin), int(num_prefix), desc(k), desc(v),
              float(scale), desc(out), _stream(q_raw))
    return out


def exact_query_chunked_sdpa(q, k, v, scale: float, chunk_size: int = 0) -> torch.Tensor:
    """attention_math.rs:199-241. chunk_size only bounded the reference's
    scores buffer; this kernel keeps no such buffer, so it is ignored."""
    return sdpa(q, k, v, scale)


def exact_sdpa_heads(q, k, v, scale: float, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """attention_math.rs:244-259: f32 arithmetic whatever q's dtype, output
    in q's dtype (default) or in `out`, which may also be f32."""
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    _lib.call("lux3d_sdpa_heads_f32", desc(q), desc(k), desc(v), float(scale), desc(out), _stream(q))
    return out


# ---------------------------------------------------------------------------
# TRELLIS.2 sparse voxel ops (runtime/trellis2_sparse.rs)
# ---------------------------------------------------------------------------

def kernel_offset_delta(k: int):
    """trellis2_sparse.rs:83-91: k = kd*9 + kh*3 + kw -> (kd-1, kh-1, kw-1)."""
    return (k // 9 - 1, (k % 9) // 3 - 1, k % 3 - 1)


def sparse_neighbors(coords: torch.Tensor, bad_coords: Optional[torch.Tensor] = None) -> torch.Tensor:
    """CoordMap + per-offset lookups on the device: coords int32 [N, 3] ->
    nbr int32 [N, 27] (-1: missing). `bad_coords` (int32 [1]) receives the
    number of coordinates outside the table's [-2^20, 2^20 - 1) range."""
    n = coords.shape[0]
    cap = 16
    while cap < 2 * n:
        cap *= 2
    keys = torch.empty(cap, dtype=torch.int64, device=coords.device)
    vals = torch.empty(cap, dtype=torch.int32, device=coords.device)
    nbr = torch.empty((n, 27), dtype=torch.int32, device=coords.device)
    _lib.call("lux3d_sparse_neighbors", desc(coords), desc(keys), desc(vals), desc(nbr), desc(bad_coords),
              _stream(coords))
    return nbr


def sparse_neighbors_noalloc(coords: torch.Tensor, nbr: torch.Tensor,
                             bad_coords: Optional[torch.Tensor] = None) -> torch.Tensor:
    """sparse_neighbors into a caller-provided `nbr` (int32 [N, 27]) with the
    hash table in the library's per-device static array: the library
    allocates nothing. N <= 2^20; calls that overlap on one GPU race."""
    _lib.call("lux3d_sparse_neighbors_noalloc", desc(coords), desc(nbr), desc(bad_coords), _stream(coords))
    return nbr


class SparseConv3d:
    """Submanifold 3x3x3 sparse convolution (trellis2_sparse.rs:135-243).
    `weight` is the checkpoint's flex_gemm layout [Cout, 3, 3, 3, Cin] (or
    its flattened GGUF form); it is transposed once to [27, Cout, Cin] f32."""

    def __init__(self, weight: torch.Tensor, bias: Optional[torch.Tensor], in_channels: int, out_channels: int):
        w = weight.reshape(out_channels, 27, in_channels).to(torch.float32)
        self.weight27 = w.permute(1, 0, 2).contiguous()
        self.bias = None if bias is None else bias.to(torch.float32).contiguous()
        self.in_channels, self.out_channels = in_channels, out_channels

    def forward(self, coords_or_nbr, feats: torch.Tensor) -> torch.Tensor:
        """coords int32 [N, 3] (the neighbour table is built), a prebuilt nbr
        int32 [N, 27], or a SparseRulebook; feats f32 [N, Cin] -> [N, Cout]."""
        out = torch.empty((feats.shape[0], self.out_channels), dtype=torch.float32, device=feats.device)
        if isinstance(coords_or_nbr, SparseRulebook):
            rb = coords_or_nbr
            _lib.call("lux3d_sparse_conv3d_rulebook", desc(feats), desc(rb.pairs), desc(rb.counts),
                      desc(self.weight27), desc(self.bias), desc(out), _stream(feats))
            return out
        nbr = coords_or_nbr if coords_or_nbr.shape[-1] == 27 else sparse_neighbors(coords_or_nbr)
        _lib.call("lux3d_sparse_conv3d", desc(feats), desc(nbr), desc(self.weight27), desc(self.bias), desc(out),
                  _stream(feats))
        return out


class SparseRulebook:
    """Per-tap (dst, src) pair lists of a coordinate set, built once and reused
    by every convolution on it (lux3d_sparse_rulebook)."""

    def __init__(self, nbr: torch.Tensor):
        n = nbr.shape[0]
        self.nbr = nbr
        self.pairs = torch.empty((27, n, 2), dtype=torch.int32, device=nbr.device)
        self.counts = torch.empty(27, dtype=torch.int32, device=nbr.device)
        _lib.call("lux3d_sparse_rulebook", desc(nbr), desc(self.pairs), desc(self.counts), _stream(nbr))


def index_select_rows(feats: torch.Tensor, ids: torch.Tensor, bad_ids: Optional[torch.Tensor] = None) -> torch.Tensor:
    """index_select_rows (trellis2_sparse.rs:117-131): feats[ids] along dim 0.
    `bad_ids` (int32 [1]) receives the number of ids outside [0, rows)."""
    out = torch.empty((ids.shape[0],) + tuple(feats.shape[1:]), dtype=feats.dtype, device=feats.device)
    _lib.call("lux3d_index_select_rows", desc(feats), desc(ids), desc(out), desc(bad_ids), _stream(feats))
    return out


def channel_to_spatial(coords: torch.Tensor, feats: torch.Tensor, subdiv_logits: torch.Tensor):
    """channel_to_spatial (trellis2_sparse.rs:269-338) on the device. Returns
    (child coords int32 [M, 3], child feats [M, C/8], sub_binary f32 [N, 8])
    after one stream sync to read M."""
    n, c = feats.shape
    dev = feats.device
    ws = torch.empty(n + (n + 1023) // 1024, dtype=torch.int32, device=dev)
    oc = torch.empty((8 * n, 3), dtype=torch.int32, device=dev)
    src = torch.empty(8 * n, dtype=torch.int32, device=dev)
    of = torch.empty((8 * n, c // 8), dtype=feats.dtype, device=dev)
    sub = torch.empty((n, 8), dtype=torch.float32, device=dev)
    cnt = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.call("lux3d_channel_to_spatial", desc(coords), desc(feats), desc(subdiv_logits), desc(ws), desc(oc),
              desc(src), desc(of), desc(sub), desc(cnt), _stream(feats))
    m = int(cnt.item())
    return oc[:m], of[:m], sub
