/*
 * lux3d_fused.h -- C ABI of the MI355X (gfx950) fused transformer-layer ops
 * for candle-3d (Lux3D). This is the drop-in boundary: a Rust CustomOp (or any
 * FFI caller) passes borrowed device buffers described by lux3d_tensor_t and a
 * HIP stream; every entry point validates its arguments on the host, enqueues
 * its kernels on that stream (one for each fused transformer-layer entry; see
 * Launches below), never synchronises and never allocates.
 *
 * Each entry names the reference function(s) it replaces (paths relative to
 * crates/lux3d-core/src/ of the candle-3d tree; "candle" = the candle fork the
 * reference depends on, Cargo.toml:23-25).
 *
 * Conventions
 *  - Tensors: `data` points at the first element (candle's Layout start
 *    offset already applied); strides are in elements. All kernels require
 *    the innermost stride to be 1 unless stated otherwise.
 *  - Activations: f32, bf16 or f16. Per-channel parameters (LayerNorm w/b,
 *    LayerScale gamma, RMS weights, modulation vectors, RoPE tables): f32,
 *    bf16 or f16 (loaded and widened to f32). Outputs have the activation's
 *    dtype. All arithmetic is f32; bf16/f16 outputs are rounded once
 *    (round-to-nearest-even).
 *  - Return value: LUX3D_OK (0) or a negative lux3d_status; the message is
 *    available from lux3d_last_error() on the calling thread. Argument errors
 *    are detected before anything is enqueued.
 *  - Launches: the fused transformer-layer entries (LayerNorm to Q8_0
 *    dequant below) enqueue exactly one kernel. Some next-row entries
 *    enqueue a short fixed sequence on the same stream; each says so.
 *  - Device-side preconditions that only the data can violate (coordinates
 *    out of range, gather ids out of range) are counted into an optional
 *    int32 error counter the entry sets, since checking them on the host
 *    would need a device-to-host copy and a sync.
 *  - Thread safety: no global mutable state besides the thread-local error
 *    message; results are deterministic (no floating-point atomics, fixed
 *    reduction order; the error counters use integer atomics).
 */
#ifndef LUX3D_FUSED_H
#define LUX3D_FUSED_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LUX3D_ABI_VERSION 2
#define LUX3D_MAX_RANK 5

typedef enum {
  LUX3D_F32 = 0,
  LUX3D_BF16 = 1,
  LUX3D_F16 = 2,
  LUX3D_I32 = 3,
  LUX3D_I64 = 4,
  LUX3D_U8 = 5,
  LUX3D_I8 = 6
} lux3d_dtype;

typedef enum {
  LUX3D_OK = 0,
  LUX3D_ERR_NULL = -1,     /* a required pointer/descriptor is NULL */
  LUX3D_ERR_SHAPE = -2,    /* shapes disagree or are unsupported */
  LUX3D_ERR_DTYPE = -3,    /* unsupported dtype or dtype mismatch */
  LUX3D_ERR_LAYOUT = -4,   /* unsupported strides */
  LUX3D_ERR_HIP = -5,      /* the kernel launch failed */
  LUX3D_ERR_VALUE = -6     /* a scalar argument is out of range */
} lux3d_status;

/* A borrowed device tensor (candle Storage + Layout). */
typedef struct {
  void *data;
  int32_t dtype;  /* lux3d_dtype */
  int32_t rank;   /* 1..LUX3D_MAX_RANK */
  int64_t shape[LUX3D_MAX_RANK];
  int64_t stride[LUX3D_MAX_RANK];
} lux3d_tensor_t;

/* A hipStream_t; NULL is the null stream. */
typedef void *lux3d_stream_t;

int lux3d_abi_version(void);
const char *lux3d_last_error(void);

/* --------------------------------------------------------------------------
 * Row LayerNorm over the last dim (rows = all leading dims, which must form a
 * uniform row stride).
 *   w, b non-NULL: candle_nn::ops::layer_norm / LayerNorm::forward, reached
 *     from layer_norm(dim, eps, vb): runtime/pi3_encoder.rs:67,70,153;
 *     runtime/vggt.rs:104,107,346,356; runtime/triposg_dit.rs:323,332-336;
 *     runtime/triposg_dino.rs:208,211; runtime/trellis2_dino.rs:324,327;
 *     runtime/trellis2_blocks.rs:587.
 *   w = b = NULL: layer_norm_no_affine (runtime/trellis2_blocks.rs:280-286),
 *     adaln_norm (runtime/vggt.rs:432-437), non_affine_layer_norm
 *     (runtime/trellis2_dino.rs:448-454).
 *   y may alias x.                                                          */
int lux3d_layer_norm(const lux3d_tensor_t *x, const lux3d_tensor_t *w,
                     const lux3d_tensor_t *b, float eps,
                     const lux3d_tensor_t *y, lux3d_stream_t stream);

/* --------------------------------------------------------------------------
 * Fused LayerScale + residual + LayerNorm:
 *   h = x + a*ls_gamma (ls_gamma NULL: h = x + a), stored in h_out;
 *   y = LayerNorm(h; w, b, eps) computed from the stored (rounded) h.
 * Replaces LayerScale::forward (runtime/nn_blocks.rs:210-214) + the residual
 * add + the next norm in VggtBlock::forward (runtime/vggt.rs:113-124),
 * dinov2 Block::forward (runtime/pi3_encoder.rs:78-89), DinoLayer::forward
 * (runtime/trellis2_dino.rs:344-355, runtime/triposg_dino.rs:218-228) and
 * DiTBlock::forward (runtime/triposg_dit.rs:364-379). w/b may be NULL
 * (non-affine norm). h_out may alias x.                                     */
int lux3d_residual_layer_norm(const lux3d_tensor_t *x, const lux3d_tensor_t *a,
                              const lux3d_tensor_t *ls_gamma,
                              const lux3d_tensor_t *w, const lux3d_tensor_t *b,
                              float eps, const lux3d_tensor_t *h_out,
                              const lux3d_tensor_t *y, lux3d_stream_t stream);

/* --------------------------------------------------------------------------
 * AdaLN modulate on dense or ragged token rows:
 *   n = LayerNorm_no_affine(x, eps)
 *   y = n*(scale + 1) + shift                       (gate == NULL)
 *   y = gate*(n*(scale + 1) + shift) + x            (gate != NULL)
 * with every modulation piece p in {shift, scale, gate} read per segment s
 * as p[s, c] (+ p_base[c] when p_base is given: the block's `modulation`
 * parameter added to t_emb, runtime/trellis2_blocks.rs:617).
 *   x: [rows, C] (or [B, L, C]); p: [S, C] views (any row stride, so the
 *   chunks of a [S, 6C] modulation vector are passed without a copy);
 *   p_base: [C] or NULL.
 *   seg_offsets: int64 [S+1] device array of row offsets (ragged TRELLIS.2
 *   voxel batches); NULL means S equal segments of rows/S rows (x [B, L, C]
 *   with S = B). Rows past offsets[S] use segment S-1.
 * Replaces Trellis2DenseBlock/Trellis2SparseBlock modulate chains
 * (runtime/trellis2_blocks.rs:617-630, 639-642, 693-714; chunk order per
 * chunk_modulation :264-277) and the VGGT camera-head poseLN modulation
 * (runtime/vggt.rs:399-405, gate variant).                                  */
int lux3d_adaln_modulate(const lux3d_tensor_t *x, const lux3d_tensor_t *seg_offsets,
                         const lux3d_tensor_t *shift, const lux3d_tensor_t *shift_base,
                         const lux3d_tensor_t *scale, const lux3d_tensor_t *scale_base,
                         const lux3d_tensor_t *gate, const lux3d_tensor_t *gate_base,
                         float eps, const lux3d_tensor_t *y, lux3d_stream_t stream);

/* --------------------------------------------------------------------------
 * Gated residual: out = x + h*gate, gate per segment as in
 * lux3d_adaln_modulate. Replaces `h.broadcast_mul(gate)` + `xs.add(h)` at
 * runtime/trellis2_blocks.rs:632-633, 644-645, 708-717. out may alias x.     */
int lux3d_gated_residual(const lux3d_tensor_t *x, const lux3d_tensor_t *h,
                         const lux3d_tensor_t *seg_offsets,
                         const lux3d_tensor_t *gate, const lux3d_tensor_t *gate_base,
                         const lux3d_tensor_t *out, lux3d_stream_t stream);

/* --------------------------------------------------------------------------
 * Gated residual, then the next AdaLN modulate, in one pass over the rows:
 *   x_out = x + h*gate          (gate == NULL: x_out = x + h)
 *   y     = LayerNorm_no_affine(x_out, eps)*(scale + 1) + shift
 * with y computed from the stored (rounded) x_out. x_out is bit-identical to
 * lux3d_gated_residual's; y is lux3d_adaln_modulate's arithmetic on it (the
 * row statistics may be summed in another order). Reads x and h once and
 * writes x_out and y once: 4 row passes in one launch instead of 5 in two.
 * gate / shift / scale (+ *_base) and seg_offsets as in lux3d_adaln_modulate;
 * all pieces share one segment count. x_out may alias x (the residual
 * stream updated in place); y must not alias x or x_out.
 * Replaces the block-internal sequences
 *   h.broadcast_mul(gate_msa); xs.add(h); layer_norm_no_affine(xs, 1e-6);
 *   .broadcast_mul(scale_mlp.affine(1, 1)); .broadcast_add(shift_mlp)
 * of Trellis2SparseBlock::forward (runtime/trellis2_blocks.rs:708-713) and
 *   xs.add(h) (cross-attention output, no gate); layer_norm_no_affine;
 *   modulate by scale_mlp / shift_mlp
 * of Trellis2DenseBlock::forward (runtime/trellis2_blocks.rs:637-642).      */
int lux3d_gated_residual_adaln_modulate(const lux3d_tensor_t *x, const lux3d_tensor_t *h,
                                        const lux3d_tensor_t *seg_offsets,
                                        const lux3d_tensor_t *gate, const lux3d_tensor_t *gate_base,
                                        const lux3d_tensor_t *shift, const lux3d_tensor_t *shift_base,
                                        const lux3d_tensor_t *scale, const lux3d_tensor_t *scale_base,
                                        float eps, const lux3d_tensor_t *x_out,
                                        const lux3d_tensor_t *y, lux3d_stream_t stream);

/* --------------------------------------------------------------------------
 * VGGT/Pi3 2D RoPE (R1) on Q and K head views, optionally after a per-head
 * affine LayerNorm (the q_norm/k_norm of the attention).
 *   q, k: [B, H, N, D] views with any outer strides (e.g. the permuted
 *     [B, N, 3, H, D] qkv buffer), D a multiple of 4 (as Rope2d requires);
 *     k may be NULL. D = 64 or 128 with 16-byte aligned rows takes the
 *     vectorised kernel, other head dims and alignments a generic one.
 *   q_w/q_b (k_w/k_b): [D] LayerNorm affine, or all NULL for RoPE only; the
 *     bias may be NULL with the weight given (a LayerNorm without bias:
 *     out = n*w), a bias without its weight is rejected.
 *   cos_full, sin_alt_full: [B, N, D] or [B, 1, N, D] f32 tables as built by
 *     Rope2d::embeddings (sin table with the rotate-half negation folded in).
 *   q_out, k_out: contiguous [B, H, N, D].
 *   out[j] = y[j]*cos_full[j] + y[partner(j)]*sin_alt_full[j], partner =
 *   the other quarter of j's half.
 * Replaces candle_nn::ops::layernorm_rope_fused / rope_fused (the fork's
 * CustomOp3s routed at runtime/attention_math.rs:132-146, 156-162) and the
 * composed path they short-cut (LayerNorm::forward on the strided view +
 * .contiguous() + rope_apply, runtime/attention_math.rs:104-118,148-149).  */
int lux3d_qk_layernorm_rope2d(const lux3d_tensor_t *q, const lux3d_tensor_t *q_w,
                              const lux3d_tensor_t *q_b, const lux3d_tensor_t *k,
                              const lux3d_tensor_t *k_w, const lux3d_tensor_t *k_b,
                              float eps, const lux3d_tensor_t *cos_full,
                              const lux3d_tensor_t *sin_alt_full,
                              const lux3d_tensor_t *q_out, const lux3d_tensor_t *k_out,
                              lux3d_stream_t stream);

/* Same, with the rotation computed in-kernel from integer positions
 * [B, N, 2] (int32 or int64, (y, x) order; specials at (0, 0)) and `base`,
 * i.e. Rope2d::embeddings (runtime/attention_math.rs:14-58) fused into the
 * apply: no [B, N, D] tables are read and no device->host position max is
 * needed (attention_math.rs:24).                                           */
int lux3d_qk_layernorm_rope2d_pos(const lux3d_tensor_t *q, const lux3d_tensor_t *q_w,
                                  const lux3d_tensor_t *q_b, const lux3d_tensor_t *k,
                                  const lux3d_tensor_t *k_w, const lux3d_tensor_t *k_b,
                                  float eps, const lux3d_tensor_t *positions, float base,
                                  const lux3d_tensor_t *q_out, const lux3d_tensor_t *k_out,
                                  lux3d_stream_t stream);

/* Rope2d::embeddings (runtime/attention_math.rs:14-58) on the device:
 * positions [B, N, 2] int32/int64 -> cos_full, sin_alt_full contiguous
 * [B, N, D] f32 (D = token_dim, divisible by 4).                            */
int lux3d_rope2d_tables(const lux3d_tensor_t *positions, float base,
                        const lux3d_tensor_t *cos_full, const lux3d_tensor_t *sin_alt_full,
                        lux3d_stream_t stream);

/* --------------------------------------------------------------------------
 * TripoSG per-head RMSNorm (N1) on Q and K head views:
 *   y = x / sqrt(mean(x^2) + eps) * w      (w: [D])
 *   q, k: [B, H, L, D] views with any outer strides (the per-head thirds of
 *   TripoSGAttnProcessor's cat([q,k,v]) need no transpose/contiguous copy);
 *   k may be NULL; outputs contiguous [B, H, L, D].
 * Replaces RmsNormHeads::rms_norm_heads (runtime/triposg_dit.rs:509-522)
 * and the .transpose(1,2).contiguous() before it (:446-453, 478-497).      */
int lux3d_rms_norm_heads(const lux3d_tensor_t *q, const lux3d_tensor_t *q_w,
                         const lux3d_tensor_t *k, const lux3d_tensor_t *k_w,
                         float eps, const lux3d_tensor_t *q_out,
                         const lux3d_tensor_t *k_out, lux3d_stream_t stream);

/* --------------------------------------------------------------------------
 * TRELLIS.2 q/k L2 "RMS" norm (N2) and/or 3D RoPE (R2) on [B, L, H, D] head
 * views (any outer strides; any D, even when rotating), q and k in one launch:
 *   N2 (gamma [H, D] given): y = x / clamp(||x||, 1e-12, 1e30) * gamma * sqrt(D)
 *   R2 (phases given): pairs (y[2i], y[2i+1]) rotated by phase i of token l,
 *     from tables cos/sin [L, D/2] (Trellis2Rope3d::cos_sin layout) or
 *     computed in-kernel from int32 coords [L, 3] and `base`.
 *   Both NULL skips that stage; q_out/k_out contiguous [B, L, H, D].
 * Replaces Trellis2QkRmsNorm::forward (runtime/trellis2_blocks.rs:306-319),
 * Trellis2Rope3d::apply (:139-160) and their use in
 * Trellis2SelfAttention::attention (:423-430); coords as validated by
 * Trellis2SlatDit::prepare (runtime/trellis2_dit.rs:511-544).              */
int lux3d_qk_l2norm_rope3d(const lux3d_tensor_t *q, const lux3d_tensor_t *q_gamma,
                           const lux3d_tensor_t *k, const lux3d_tensor_t *k_gamma,
                           const lux3d_tensor_t *cos, const lux3d_tensor_t *sin,
                           const lux3d_tensor_t *coords, float base,
                           const lux3d_tensor_t *q_out, const lux3d_tensor_t *k_out,
                           lux3d_stream_t stream);

/* Trellis2Rope3d::cos_sin (runtime/trellis2_blocks.rs:106-134) on the
 * device: coords int32 [L, 3] -> cos, sin contiguous [L, head_dim/2] f32.   */
int lux3d_rope3d_tables(const lux3d_tensor_t *coords, int64_t head_dim, float base,
                        const lux3d_tensor_t *cos, const lux3d_tensor_t *sin,
                        lux3d_stream_t stream);

/* --------------------------------------------------------------------------
 * DINOv3 2D RoPE (R3) on Q and K [B, H, S, D] views: tokens s < num_prefix
 * pass through unchanged, token s >= num_prefix uses table row
 * s - num_prefix of cos/sin [S - num_prefix, D]:
 *   out = x*cos + rotate_half(x)*sin,  rotate_half(x) = cat(-x2, x1).
 * Replaces apply_rotary_to_patches + rotate_half
 * (runtime/trellis2_dino.rs:406-445); tables from
 * Trellis2DinoConfig::rope_cos_sin (:140-187). k may be NULL.               */
int lux3d_dinov3_rope(const lux3d_tensor_t *q, const lux3d_tensor_t *k,
                      const lux3d_tensor_t *cos, const lux3d_tensor_t *sin,
                      int64_t num_prefix, const lux3d_tensor_t *q_out,
                      const lux3d_tensor_t *k_out, lux3d_stream_t stream);

/* --------------------------------------------------------------------------
 * Activations on contiguous tensors (y may alias x):
 *   gelu_erf  = 0.5*x*(1 + erf(x/sqrt(2)))       Tensor::gelu_erf
 *     (runtime/nn_blocks.rs:233,252; vggt.rs:412; triposg_dit.rs:298,380;
 *      trellis2_dino.rs:353; triposg_dino.rs:225)
 *   gelu_tanh = 0.5*x*(1 + tanh(sqrt(2/pi)*x*(1 + 0.044715*x^2)))
 *     Tensor::gelu (runtime/trellis2_blocks.rs:558-561)
 *   silu      = x / (1 + exp(-x))                Tensor::silu
 *     (runtime/trellis2_blocks.rs:236,257; vggt.rs:393)                     */
int lux3d_gelu_erf(const lux3d_tensor_t *x, const lux3d_tensor_t *y, lux3d_stream_t stream);
int lux3d_gelu_tanh(const lux3d_tensor_t *x, const lux3d_tensor_t *y, lux3d_stream_t stream);
int lux3d_silu(const lux3d_tensor_t *x, const lux3d_tensor_t *y, lux3d_stream_t stream);

/* --------------------------------------------------------------------------
 * Sinusoidal timestep embedding, t: f32 [n] (device), out: f32 [n, dim]:
 *   f_i = exp(-ln(10000) * i / half), arg = t*f_i, half = dim/2
 *   cos_first = 1: [cos(arg), sin(arg)] (+ a zero for odd dim)
 *     timestep_embedding (runtime/trellis2_blocks.rs:184-204), dim 256
 *   cos_first = 0: [sin(arg), cos(arg)]
 *     TripoSgDiT::timestep_embedding (runtime/triposg_dit.rs:280-297),
 *     dim = width; dim must be even.
 * freqs: optional f32 [dim/2] device vector of the f_i. The reference builds
 * them on the host with libm expf (trellis2_blocks.rs:191-194,
 * triposg_dit.rs:289-291) and uploads them; passing those exact values makes
 * every argument t*f_i bit-identical to the reference. NULL computes f_i on
 * the device (f64 exp rounded once to f32, which can differ from a libm
 * expf result by 1 ulp).                                                    */
int lux3d_timestep_embedding(const lux3d_tensor_t *t, const lux3d_tensor_t *freqs,
                             int64_t dim, int32_t cos_first,
                             const lux3d_tensor_t *out, lux3d_stream_t stream);

/* --------------------------------------------------------------------------
 * GGML Q8_0 dequantisation: blocks u8 [nblocks*34] of {f16 d (LE); int8
 * qs[32]} -> y [nblocks*32] (f32, bf16 or f16, contiguous), y = f32(d)*qs
 * (exact in f32) rounded once to y's dtype: bit-exact.
 * Replaces QTensor::dequantize for Q8_0 weights (runtime/nn_blocks.rs:140,
 * examples/quant_probe.rs:84-89); the Q8_0 selection rule is
 * weights/quantize.rs:319-338 (rank 2, row length % 32 == 0).              */
int lux3d_dequant_q8_0(const lux3d_tensor_t *blocks, const lux3d_tensor_t *y,
                       lux3d_stream_t stream);

/* --------------------------------------------------------------------------
 * Q8_0 quantized linear (the "next" row of the path: the consumer of the
 * dequant above).
 *
 * lux3d_q8_0_repack: one-time, at weight load. A Q8_0 weight [n, k] stored
 * as GGML blocks (u8 [n*k/32*34], row-major over (n, k/32); k % 32 == 0) is
 * rewritten as qs int8 (LUX3D_I8) [n, k] and scales f32 [n, k/32], both
 * contiguous and 16-byte aligned, so the GEMM streams it with 16-byte loads.
 * Exact (the values and scales are copied / widened, not rounded).
 * The reference's load-time step for a quantized linear is
 * QMatMul::from_qtensor (runtime/nn_blocks.rs:145-150).
 *
 * lux3d_q8_0_linear: y = x * W^T (+ bias) for the LinearInner::Quant branch
 * of Linear::forward (runtime/nn_blocks.rs:83-93, QMatMul::forward then
 * broadcast_add(bias)).
 *   x: bf16 or f32 [..., k] rows with a unit inner stride, 16-byte aligned
 *      rows (f32 x: k % 64 == 0, else LUX3D_ERR_SHAPE);
 *   qs, scales: from lux3d_q8_0_repack for the weight [n, k];
 *   bias: f32 [n] or NULL;
 *   y: [..., n] rows, bf16 / f16 / f32.
 * Each weight is dequantized exactly as lux3d_dequant_q8_0 does, to x's
 * dtype (bf16: RNE of the exact product; f32: the exact product), products
 * accumulate in f32 on the matrix cores, the bias is added in f32 and y is
 * rounded once. For f32 x the sum of each Q8_0 block is formed from exactly
 * split bf16 terms of x times the exact int8 values and then scaled by the
 * block's d: the f32 arithmetic up to the order of the sums (a non-finite d
 * makes the output non-finite as in the reference, though it can be +-inf
 * where the reference's per-weight 0 * inf gives NaN).
 * This is the dequantize-then-matmul path of candle's GPU backends; candle's
 * CPU path instead quantizes x to Q8_0 blocks and takes integer dot
 * products.                                                                 */
int lux3d_q8_0_repack(const lux3d_tensor_t *blocks, int64_t n, int64_t k,
                      const lux3d_tensor_t *qs, const lux3d_tensor_t *scales,
                      lux3d_stream_t stream);
int lux3d_q8_0_linear(const lux3d_tensor_t *x, const lux3d_tensor_t *qs,
                      const lux3d_tensor_t *scales, const lux3d_tensor_t *bias,
                      const lux3d_tensor_t *y, lux3d_stream_t stream);

/* lux3d_q8_0_linear_int8: the same Linear::forward Quant branch with
 * candle's CPU arithmetic (QMatMul::forward on the CPU: the QTensor custom
 * op over upstream candle-core's k_quants::matmul), bit for bit: each f32 x
 * row is quantized to Q8_0 blocks (lux3d_q8_0_quantize below), each output is
 *   acc = 0; for each block b in order: acc += (f32)(sum_j w_q[j] x_q[j]) * w_d * x_d
 * (int32 block dots on the int8 matrix cores, then every f32 operation
 * rounded in that order), and y = acc + bias (broadcast_add).
 *   x: f32 [..., k] rows, 16-byte aligned; qs, scales: lux3d_q8_0_repack;
 *   bias: f32 [n] or NULL; y: f32 [..., n] rows;
 *   xq: int8 [rows, k] and xd: f32 [k/32, rows rounded up to 64]
 *   (block-major: a block's scales of consecutive rows are adjacent),
 *   contiguous and 16-byte aligned -- a workspace that receives x's
 *   quantized blocks.
 * Two kernels (quantize, then the GEMM).
 *
 * lux3d_q8_0_quantize: BlockQ8_0::from_float of every 32-value block of each
 * x row (candle-core k_quants.rs; the first step of the CPU QMatMul): amax =
 * max |x| (NaN ignored), d = amax / 127, q = round-half-away(x / d as
 * x * (1 / d)) saturated to int8 (NaN -> 0), d rounded to f16. xq receives
 * the int8 values, xd (block-major, as above) the f16 scale widened to f32
 * (exact). One kernel.                                                     */
int lux3d_q8_0_linear_int8(const lux3d_tensor_t *x, const lux3d_tensor_t *qs,
                           const lux3d_tensor_t *scales, const lux3d_tensor_t *bias,
                           const lux3d_tensor_t *xq, const lux3d_tensor_t *xd,
                           const lux3d_tensor_t *y, lux3d_stream_t stream);
int lux3d_q8_0_quantize(const lux3d_tensor_t *x, const lux3d_tensor_t *xq,
                        const lux3d_tensor_t *xd, lux3d_stream_t stream);

/* ---- TRELLIS.2 sparse voxel ops (runtime/trellis2_sparse.rs) ----------------
 * lux3d_sparse_neighbors: CoordMap::new + the per-offset lookups of
 * SparseConv3d::forward (trellis2_sparse.rs:62-91, 205-222), on the device;
 * three kernels (clear the table, insert, look up).
 *   coords: int32 [N, 3] contiguous (x, y, z), each in [-2^20, 2^20 - 1)
 *     (the packed hash key); a coordinate outside is neither inserted nor
 *     found, and is counted into bad_coords;
 *   bad_coords: int32 [1] or NULL: set to the number of such coordinates;
 *   keys: int64 [cap], vals: int32 [cap] -- a workspace, cap a power of two
 *         >= 2 N (the hash table; cleared here);
 *   nbr: int32 [N, 27] out: nbr[i][k] = row of coords[i] + (kd-1, kh-1, kw-1),
 *        k = kd*9 + kh*3 + kw, or -1. A repeated coordinate maps to its last
 *        row (HashMap::insert overwrites).
 *
 * lux3d_sparse_conv3d: SparseConv3d::forward (trellis2_sparse.rs:197-243),
 * submanifold 3x3x3, output rows = input rows:
 *   out[i, o] = bias[o] + sum_k sum_c W[k][o][c] * x[nbr[i][k], c]
 *   x: f32 [N, Cin], nbr: int32 [N, 27] (from lux3d_sparse_neighbors),
 *   weight: f32 [27, Cout, Cin] (the loader's transposed kernel, weight27),
 *   bias: f32 [Cout] or NULL, out: f32 [N, Cout]; all contiguous.
 * One output-stationary implicit GEMM on the bf16 matrix cores when
 * Cin % 16 == 0 and x, weight are 16-byte aligned (f32 arithmetic: operands
 * split exactly into three bf16 terms, the six significant cross products
 * per step, each product within one f32 ulp); otherwise a generic kernel.
 * f32 accumulation; no scatter.
 *
 * lux3d_index_select_rows: index_select_rows (trellis2_sparse.rs:117-131):
 *   out[m, ...] = src[ids[m], ...]; src [R, ...] and out [M, ...] contiguous,
 *   same dtype and row shape; ids int32 or int64 [M]. An id outside [0, R)
 *   gives a zero row and is counted: bad_ids (int32 [1] or NULL) is set to
 *   the number of such ids (candle's index_select errors on them; the C++
 *   mirror reads the count back and throws).
 *
 * lux3d_channel_to_spatial: channel_to_spatial (trellis2_sparse.rs:269-338):
 *   coords int32 [N, 3]; feats [N, C] (any dtype, C % 8 == 0, contiguous);
 *   logits [N, 8] (f32 / bf16 / f16, contiguous; leaf = logits > 0);
 *   workspace int32 [N + ceil(N / 1024)];
 *   out: out_coords int32 [8N, 3], src_rows int32 [8N], out_feats [8N, C/8]
 *   (feats' dtype), sub f32 [N, 8] (1 / 0; may be NULL), count int32 [1].
 *   The first M = *count rows of the outputs hold the children in the
 *   reference order (parent order, ascending subidx = dx + 2 dy + 4 dz); the
 *   count stays in device memory (read it after a stream sync).            */
int lux3d_sparse_neighbors(const lux3d_tensor_t *coords, const lux3d_tensor_t *keys,
                           const lux3d_tensor_t *vals, const lux3d_tensor_t *nbr,
                           const lux3d_tensor_t *bad_coords, lux3d_stream_t stream);
/* lux3d_sparse_neighbors_noalloc: lux3d_sparse_neighbors without the `keys` /
 * `vals` workspace and without any allocation. This entry has no counterpart
 * in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops). The hash table lives in
 * a per-device static array of the library (24 MiB, held until the process
 * ends), so N is limited to 2^20 voxels (LUX3D_ERR_SHAPE beyond). Every call
 * on a GPU uses that GPU's one table: calls that overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller. Same
 * kernels and outputs as lux3d_sparse_neighbors. The first call on a device
 * looks the table's address up (hipGetSymbolAddress, which may load the
 * library's code object on that device): make one call per device outside
 * graph capture before capturing calls of this entry.                      */
int lux3d_sparse_neighbors_noalloc(const lux3d_tensor_t *coords, const lux3d_tensor_t *nbr,
                                   const lux3d_tensor_t *bad_coords, lux3d_stream_t stream);
int lux3d_sparse_conv3d(const lux3d_tensor_t *x, const lux3d_tensor_t *nbr,
                        const lux3d_tensor_t *weight, const lux3d_tensor_t *bias,
                        const lux3d_tensor_t *out, lux3d_stream_t stream);
/* lux3d_sparse_rulebook + lux3d_sparse_conv3d_rulebook: the same convolution
 * computed the reference's way round, without its host work and scatter
 * kernels: per-tap pair lists (dst, src) built once per coordinate set
 * (pairs int32 [27, N, 2] and counts int32 [27], from nbr), then
 * out = 0; out[dst] += x[src] W_k^T for k = 0..26 in order; out += bias --
 * the zeros / index_add / broadcast_add sequence of SparseConv3d::forward
 * (trellis2_sparse.rs:205-242). Only present neighbours reach the matrix
 * cores (f32 arithmetic on the bf16 matrix cores, as lux3d_sparse_conv3d),
 * so sparse sets run several times faster than the output-stationary
 * kernel. Cin % 16 == 0 and 16-byte aligned x and weight
 * are required (else LUX3D_ERR_SHAPE / LUX3D_ERR_LAYOUT: use
 * lux3d_sparse_conv3d). */
int lux3d_sparse_rulebook(const lux3d_tensor_t *nbr, const lux3d_tensor_t *pairs,
                          const lux3d_tensor_t *counts, lux3d_stream_t stream);
int lux3d_sparse_conv3d_rulebook(const lux3d_tensor_t *x, const lux3d_tensor_t *pairs,
                                 const lux3d_tensor_t *counts, const lux3d_tensor_t *weight,
                                 const lux3d_tensor_t *bias, const lux3d_tensor_t *out,
                                 lux3d_stream_t stream);
int lux3d_index_select_rows(const lux3d_tensor_t *src, const lux3d_tensor_t *ids,
                            const lux3d_tensor_t *out, const lux3d_tensor_t *bad_ids,
                            lux3d_stream_t stream);
int lux3d_channel_to_spatial(const lux3d_tensor_t *coords, const lux3d_tensor_t *feats,
                             const lux3d_tensor_t *logits, const lux3d_tensor_t *workspace,
                             const lux3d_tensor_t *out_coords, const lux3d_tensor_t *src_rows,
                             const lux3d_tensor_t *out_feats, const lux3d_tensor_t *sub,
                             const lux3d_tensor_t *count, lux3d_stream_t stream);

/* ---- attention ------------------------------------------------------------
 * lux3d_sdpa: out = softmax(q k^T * scale) v, replacing
 * exact_query_chunked_sdpa (runtime/attention_math.rs:199-241; its
 * chunk_size only bounds the scores buffer, which this kernel never
 * materialises), and exact_sdpa_heads (attention_math.rs:244-259) for f32
 * inputs (for 2-byte inputs see lux3d_sdpa_heads_f32).
 *   q: [B, H, Lq, D]; k, v: [B, H, Lk, D]; out: [B, H, Lq, D];
 *   one dtype for all four (f32, bf16 or f16); any batch / head / token
 *   strides (the permuted views of a fused qkv buffer pass as they are),
 *   unit innermost stride; Lk >= 1; D <= 512; scale finite and > 0.
 * D = 64 or 128 with every row 16-byte aligned runs on the matrix cores:
 * bf16 / f16 with f32 scores, f32 softmax, the probabilities rounded to the
 * input type for P v (f32 accumulation) and one rounding of the output; f32
 * on the bf16 matrix cores with q, k, v and the probabilities split exactly
 * into three bf16 terms each and the six significant cross products per
 * step (each product within one f32 ulp), scores, probabilities and sums
 * in f32. Other cases run a generic kernel in f32 throughout. The f32 paths
 * are the arithmetic of exact_sdpa_heads up to the order of the sums (and,
 * on the matrix cores, that sub-ulp product truncation). out must not
 * overlap q, k or v.                                                         */
int lux3d_sdpa(const lux3d_tensor_t *q, const lux3d_tensor_t *k,
               const lux3d_tensor_t *v, float scale, const lux3d_tensor_t *out,
               lux3d_stream_t stream);

/* lux3d_sdpa_heads_f32: exact_sdpa_heads (attention_math.rs:244-259), which
 * widens q, k and v to f32, computes scores, softmax and P v in f32 and
 * narrows the result to the input dtype. Arguments as lux3d_sdpa, except that
 * out may be f32 as well as q's dtype (then the f32 result is stored, not
 * narrowed). f32 inputs run as lux3d_sdpa. bf16 with D 64 / 128 and 16-byte
 * aligned rows runs on the bf16 matrix cores: bf16 products are exact in f32,
 * and the f32 probabilities enter P v as three bf16 terms whose sum is the
 * f32 value exactly, so the arithmetic is f32 products with f32 accumulation.
 * Other 2-byte cases run the generic kernel (f32 throughout). out must not
 * overlap q, k or v.                                                          */
int lux3d_sdpa_heads_f32(const lux3d_tensor_t *q, const lux3d_tensor_t *k,
                         const lux3d_tensor_t *v, float scale, const lux3d_tensor_t *out,
                         lux3d_stream_t stream);

/* lux3d_sdpa_layernorm_rope2d: the VGGT / Pi3 attention of vggt.rs:170-183,
 * exact_query_chunked_sdpa(apply_layernorm_rope(q, q_norm, rope), k, v,
 * scale), with q's LayerNorm + 2D RoPE (attention_math.rs:127-150) applied
 * inside the attention kernel's Q load: the normalised q never goes through
 * HBM. q is the raw [B, H, N, D] head view (bf16 / f16); q_w, q_b the
 * LayerNorm affine ([D], any float dtype; q_b may be NULL); cos_full / sin_alt_full the Rope2d
 * tables as lux3d_qk_layernorm_rope2d takes them; k the already normalised
 * and rotated keys (lux3d_qk_layernorm_rope2d on k alone); v, scale and out
 * as lux3d_sdpa (out [B, H, N, D]; it may be the view the caller transposes
 * next). The normalised q equals lux3d_qk_layernorm_rope2d's bit for bit, so
 * the result equals that call followed by lux3d_sdpa. D = 64 / 128 with
 * 16-byte aligned rows, parameters and table rows runs fused; any other
 * layout runs exactly those two launches, with out as the intermediate q.   */
int lux3d_sdpa_layernorm_rope2d(const lux3d_tensor_t *q, const lux3d_tensor_t *q_w,
                                const lux3d_tensor_t *q_b, float eps,
                                const lux3d_tensor_t *cos_full,
                                const lux3d_tensor_t *sin_alt_full, const lux3d_tensor_t *k,
                                const lux3d_tensor_t *v, float scale, const lux3d_tensor_t *out,
                                lux3d_stream_t stream);

/* lux3d_sdpa_rms_norm_heads: the TripoSG self-attention of
 * triposg_dit.rs:446-455, exact_query_chunked_sdpa(rms_norm_heads(q, w), k,
 * v, scale), with q's per-head RMSNorm (y = x / sqrt(mean(x^2) + eps) * w,
 * RmsNormHeads::rms_norm_heads, triposg_dit.rs:509-522) applied inside the
 * attention kernel's Q load. q is the raw [B, H, L, D] head view (any outer
 * strides: the per-head third of cat([q, k, v]) passes as it is); q_w [D]
 * any float dtype; k the already normalised keys (lux3d_rms_norm_heads);
 * v, scale and out as lux3d_sdpa. The normalised q equals
 * lux3d_rms_norm_heads' bit for bit, so the result equals that call
 * followed by lux3d_sdpa. bf16 / f16, D = 64 / 128, 16-byte aligned rows
 * and weight run fused; any other case runs exactly those two launches,
 * with out as the intermediate q.                                             */
int lux3d_sdpa_rms_norm_heads(const lux3d_tensor_t *q, const lux3d_tensor_t *q_w, float eps,
                              const lux3d_tensor_t *k, const lux3d_tensor_t *v, float scale,
                              const lux3d_tensor_t *out, lux3d_stream_t stream);

/* lux3d_sdpa_l2norm_rope3d: the TRELLIS.2 self-attention of
 * trellis2_blocks.rs:417-436 (Trellis2SelfAttention::attention),
 * exact_query_chunked_sdpa(rope(l2norm(q)), k, v, scale), with q's L2 norm
 * (y = x / clamp(||x||, 1e-12, 1e30) * gamma * sqrt(D), Trellis2QkRmsNorm,
 * :306-319) and 3D RoPE pair rotation (Trellis2Rope3d::apply, :139-160)
 * applied inside the attention kernel's Q load. q, k, v, out are
 * [B, H, L, D] views (TRELLIS.2's [B, L, H, D] buffers pass as their
 * permuted views); q_gamma [H, D]; cos, sin [L, D/2] (Trellis2Rope3d::cos_sin
 * layout, any float dtype); k already normalised and rotated
 * (lux3d_qk_l2norm_rope3d). The rotated q equals lux3d_qk_l2norm_rope3d's bit
 * for bit, so the result equals that call followed by lux3d_sdpa. bf16 / f16,
 * D = 64 / 128, 16-byte aligned rows, gamma and table rows run fused; any
 * other case runs exactly those two launches, with out as the intermediate q.  */
int lux3d_sdpa_l2norm_rope3d(const lux3d_tensor_t *q, const lux3d_tensor_t *q_gamma,
                             const lux3d_tensor_t *cos, const lux3d_tensor_t *sin,
                             const lux3d_tensor_t *k, const lux3d_tensor_t *v, float scale,
                             const lux3d_tensor_t *out, lux3d_stream_t stream);

/* lux3d_sdpa_dinov3_rope: the DINOv3 attention of trellis2_dino.rs:385-393,
 * exact_sdpa_heads(apply_rotary_to_patches(q), k, v, scale), with q's
 * rotate_half RoPE (tokens s >= num_prefix use row s - num_prefix of cos / sin
 * [S - num_prefix, D]; earlier tokens pass through; :406-445) applied inside
 * the attention kernel's Q load. q, k, v, out [B, H, S, D] of one dtype (f32,
 * the reference's, or bf16); k already rotated (lux3d_dinov3_rope); the
 * attention is lux3d_sdpa_heads_f32's. The rotated q equals
 * lux3d_dinov3_rope's bit for bit, so the result equals that call followed by
 * lux3d_sdpa_heads_f32. f32 / bf16, D = 64 / 128, 16-byte aligned rows and
 * table rows run fused; any other case runs exactly those two launches,
 * with out as the intermediate q.                                             */
int lux3d_sdpa_dinov3_rope(const lux3d_tensor_t *q, const lux3d_tensor_t *cos,
                           const lux3d_tensor_t *sin, int64_t num_prefix,
                           const lux3d_tensor_t *k, const lux3d_tensor_t *v, float scale,
                           const lux3d_tensor_t *out, lux3d_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* LUX3D_FUSED_H */
