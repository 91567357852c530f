/*
 * lux3d_oracle.h -- CPU restatement of candle-3d's fused transformer-layer op
 * semantics. TEST INFRASTRUCTURE ONLY: the parity tests, the smoke check and
 * bench.py's cpu_baseline leg call it as the checker; the product library
 * (liblux3d_fused.so) never links, loads or calls it.
 *
 * Each function names the reference code (paths under the candle-3d tree,
 * crates/lux3d-core/...) whose arithmetic it restates. Where the arithmetic
 * lives in the un-vendored candle fork (FerrisMind/candle rev 9f6eed19,
 * candle-core/candle-nn 0.1.0, half 2.7.1), the published upstream candle
 * algorithm is restated and the reference call site is cited.
 *
 * Numeric model. Every op computes in IEEE f32 with the reference's operation
 * order (no FMA contraction: built with -ffp-contract=off), and rounds once to
 * the storage dtype (bf16/f16: round-to-nearest-even). Summations are
 * sequential f32. Transcendentals are glibc's sinf/cosf/expf/tanhf/powf/logf,
 * i.e. the libm that Rust's f32 methods call on Linux.
 *
 * dtype codes: 0 = f32, 1 = bf16, 2 = f16 (same codes as the product ABI).
 */
#ifndef LUX3D_ORACLE_H
#define LUX3D_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_F32 = 0, OR_BF16 = 1, OR_F16 = 2 };

/* ---- threading (rows are split over a pthread pool, like candle's rayon) - */
void or_set_threads(int n);
int or_get_threads(void);

/* ---- scalar conversions ------------------------------------------------- */
uint16_t or_f32_to_bf16(float v);   /* half::bf16::from_f32 (RNE, NaN kept quiet) */
float or_bf16_to_f32(uint16_t v);
uint16_t or_f32_to_f16(float v);    /* RNE, IEEE binary16 */
float or_f16_to_f32(uint16_t v);    /* exact */
void or_convert(int src_dt, const void *src, int dst_dt, void *dst, int64_t n);

/* ---- row normalisations ------------------------------------------------- */
/* L1: candle_nn::ops::layer_norm (contiguous fast path). w/b may be NULL. */
void or_layer_norm(int dt, const void *x, int64_t rows, int64_t d,
                   const float *w, const float *b, float eps, void *y);
/* L2: candle_nn::LayerNorm::forward composed path (strided input). */
void or_layer_norm_slow(int dt, const void *x, int64_t rows, int64_t d,
                        const float *w, const float *b, float eps, void *y);
/* L3: layer_norm_no_affine (trellis2_blocks.rs:280-286). */
void or_layer_norm_no_affine(int dt, const void *x, int64_t rows, int64_t d,
                             float eps, void *y);
/* F1/F3: h = x + a*gamma (gamma NULL -> h = x + a); y = L1(h). */
void or_residual_layer_norm(int dt, const void *x, const void *a,
                            const float *gamma, int64_t rows, int64_t d,
                            const float *w, const float *b, float eps,
                            void *h, void *y);
/* MV + L3 + M1 (+ M1' gate): per segment s (rows seg_off[s]..seg_off[s+1]),
 *   shift = shift_seg[s*ld_shift + c] (+ shift_base[c]) etc.
 *   y = L3(x)*(scale + 1) + shift                      (gate == NULL)
 *   y = gate*(L3(x)*(scale + 1) + shift) + x           (gate != NULL)      */
void or_adaln_modulate(int dt, const void *x, int64_t rows, int64_t d,
                       const int64_t *seg_off, int64_t nseg,
                       const float *shift, int64_t ld_shift, const float *shift_base,
                       const float *scale, int64_t ld_scale, const float *scale_base,
                       const float *gate, int64_t ld_gate, const float *gate_base,
                       float eps, void *y);
/* G1: out = x + h*gate (gate per segment, like the modulation pieces). */
void or_gated_residual(int dt, const void *x, const void *h, int64_t rows,
                       int64_t d, const int64_t *seg_off, int64_t nseg,
                       const float *gate, int64_t ld_gate, const float *gate_base,
                       void *out);
/* G1 then L3 + M1 on the stored result (trellis2_blocks.rs:708-713, and
 * :637-642 with gate == NULL, a plain residual add): x_out = x + h*gate,
 * y = L3(x_out)*(scale + 1) + shift. */
void or_gated_residual_modulate(int dt, const void *x, const void *h, int64_t rows, int64_t d,
                                const int64_t *seg_off, int64_t nseg,
                                const float *gate, int64_t ld_gate, const float *gate_base,
                                const float *shift, int64_t ld_shift, const float *shift_base,
                                const float *scale, int64_t ld_scale, const float *scale_base,
                                float eps, void *x_out, void *y);
/* N1: rms_norm_heads (triposg_dit.rs:515-521). */
void or_rms_norm_heads(int dt, const void *x, int64_t rows, int64_t d,
                       const float *w, float eps, void *y);
/* N2: Trellis2QkRmsNorm::forward (trellis2_blocks.rs:306-319); x [rows, H, D]. */
void or_qk_l2norm(int dt, const void *x, int64_t rows, int64_t heads,
                  int64_t d, const float *gamma, void *y);

/* ---- rotary embeddings -------------------------------------------------- */
/* R1 tables: Rope2d::embeddings (attention_math.rs:14-58). positions int32
 * [b, n, 2] (y, x). cos_full / sin_alt_full: [b, n, d] f32. */
void or_rope2d_tables(const int32_t *pos, int64_t b, int64_t n, int64_t d,
                      float base, float *cos_full, float *sin_alt_full);
/* R1 apply: rope_apply (attention_math.rs:104-118); t [b, h, n, d]. */
void or_rope2d_apply(int dt, const void *t, int64_t b, int64_t h, int64_t n,
                     int64_t d, const float *cos_full, const float *sin_alt_full,
                     void *y);
/* L2 + R1: apply_layernorm_rope (attention_math.rs:127-150). */
void or_layernorm_rope2d(int dt, const void *q, int64_t b, int64_t h, int64_t n,
                         int64_t d, const float *w, const float *bias, float eps,
                         const float *cos_full, const float *sin_alt_full, void *y);
/* R2 tables: Trellis2Rope3d::cos_sin (trellis2_blocks.rs:106-134).
 * coords int32 [n, 3]; cos/sin [n, head_dim/2]. */
void or_rope3d_tables(const int32_t *coords, int64_t n, int64_t head_dim,
                      float base, float *cos, float *sin);
/* R2 apply: Trellis2Rope3d::apply (trellis2_blocks.rs:139-160).
 * x [b, l, h, d]; tables [l, d/2]. */
void or_rope3d_apply(int dt, const void *x, int64_t b, int64_t l, int64_t h,
                     int64_t d, const float *cos, const float *sin, void *y);
/* N2 + R2 (trellis2_blocks.rs:423-430) on x [rows, H, D], tables [rows, D/2]. */
void or_qk_l2norm_rope3d(int dt, const void *x, int64_t rows, int64_t heads,
                         int64_t d, const float *gamma, const float *cos,
                         const float *sin, void *y);
/* R3 tables: Trellis2DinoConfig::rope_cos_sin (trellis2_dino.rs:140-187). */
void or_dinov3_rope_tables(int64_t grid_h, int64_t grid_w, int64_t head_dim,
                           float theta, float *cos, float *sin);
/* R3 apply: apply_rotary_to_patches (trellis2_dino.rs:406-445);
 * x [b, h, s, d]; tables [s - num_prefix, d]. */
void or_dinov3_rope_apply(int dt, const void *x, int64_t b, int64_t h, int64_t s,
                          int64_t d, int64_t num_prefix, const float *cos,
                          const float *sin, void *y);

/* ---- activations --------------------------------------------------------- */
void or_gelu_erf(int dt, const void *x, int64_t n, void *y);
void or_gelu_tanh(int dt, const void *x, int64_t n, void *y);
void or_silu(int dt, const void *x, int64_t n, void *y);

/* ---- timestep embeddings (f32 out [n, dim]) ----------------------------- */
/* T1: TripoSgDiT::timestep_embedding (triposg_dit.rs:280-297), sin first. */
void or_timestep_embedding_sin_first(const float *t, int64_t n, int64_t dim, float *out);
/* T2: timestep_embedding (trellis2_blocks.rs:184-204), cos first. */
void or_timestep_embedding_cos_first(const float *t, int64_t n, int64_t dim, float *out);
/* Either convention (cos_first: T2) from a given frequency vector freqs[dim / 2]. */
void or_timestep_embedding_freqs(const float *t, int64_t n, const float *freqs, int64_t dim, int cos_first,
                                 float *out);

/* ---- Q8_0 dequant -------------------------------------------------------- */
/* GGML block_q8_0 = {f16 d; int8 qs[32]} (34 bytes); w = f32(d)*qs. */
void or_dequant_q8_0(const uint8_t *blocks, int64_t nblocks, int out_dt, void *out);

/* ---- Q8_0 quantized linear (dequantize-then-matmul semantics) ------------- */
/* y[m][n] = sum_k x[m][k] * w[n][k] (+ bias[n]) in double, rounded once to
 * out_dt, with w = bf16(f32(q) * d) (the Q8_0 -> bf16 dequant above) and x
 * bf16 bits [M, K]; blocks hold the weight [N, K] row-major over (n, k/32).
 * abs_sum (optional, f32 [M, N]) receives sum_k |x * w|, the scale of the
 * f32 accumulation error. */
void or_q8_0_linear(const uint16_t *x, int64_t M, int64_t K, const uint8_t *blocks, int64_t N,
                    const float *bias, int out_dt, void *y, float *abs_sum);
/* The same with f32 x [M, K] and the exact f32 weights q * d. */
void or_q8_0_linear_f32(const float *x, int64_t M, int64_t K, const uint8_t *blocks, int64_t N,
                        const float *bias, int out_dt, void *y, float *abs_sum);

/* ---- Q8_0 quantized linear, candle's CPU semantics ------------------------- */
/* BlockQ8_0::from_float: f32 x [n] (n % 32 == 0) -> GGML Q8_0 blocks. */
void or_quantize_q8_0(const float *x, int64_t n, uint8_t *blocks);
/* QMatMul::forward on the CPU + bias: x f32 [M, K] quantized per row to Q8_0,
 * integer block dots with the weight blocks [N, K], scaled and summed in f32
 * block order; y f32 [M, N]. */
void or_q8_0_linear_int8(const float *x, int64_t M, int64_t K, const uint8_t *blocks, int64_t N, const float *bias,
                         float *y);

/* ---- TRELLIS.2 sparse ops (runtime/trellis2_sparse.rs) --------------------- */
/* CoordMap + kernel_offset_delta: nbr[i][k] = row of coords[i] + delta(k), or
 * -1 (k = kd*9 + kh*3 + kw, delta = (kd-1, kh-1, kw-1)); coords [n, 3]. */
void or_sparse_neighbors(const int32_t *coords, int64_t n, int32_t *nbr);
/* SparseConv3d::forward with the [27, Cout, Cin] kernel (f64 sums). */
void or_sparse_conv3d(const float *x, int64_t n, int64_t cin, const int32_t *nbr, const float *w, const float *bias,
                      int64_t cout, float *out, float *abs_sum);
/* channel_to_spatial; returns the child count. */
int64_t or_channel_to_spatial(const int32_t *coords, int64_t n, const float *feats, int64_t c, const float *logits,
                              int32_t *out_coords, float *out_feats, int32_t *src_rows, float *sub);

/* Scaled dot-product attention, exact_sdpa_heads (attention_math.rs:244-259):
 * q [BH, Lq, D], k and v [BH, Lk, D] contiguous in in_dt; out [BH, Lq, D] in
 * out_dt = softmax(q k^T * scale) v, summed in double and rounded once.
 * wabs (optional, f32 [BH, Lq, D]) receives sum_j p_j |v_j| / sum_j p_j, the
 * scale of the error of rounding the probabilities. */
void or_sdpa(int in_dt, const void *q, const void *k, const void *v, int64_t BH, int64_t Lq, int64_t Lk,
             int64_t D, double scale, int out_dt, void *out, float *wabs);

#ifdef __cplusplus
}
#endif
#endif
