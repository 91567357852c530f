/*
 * lux3d_oracle.c -- CPU restatement of candle-3d's fused transformer-layer op
 * arithmetic. TEST INFRASTRUCTURE ONLY (the checker; see lux3d_oracle.h).
 *
 * Build: gcc -O3 -march=x86-64-v3 -ffp-contract=off -fno-fast-math -fPIC -shared -pthread
 * (oracle/Makefile).
 * -ffp-contract=off keeps every a*b+c as two IEEE roundings, which is what the
 * reference's Rust (which never contracts) computes.
 *
 * Conventions restated from upstream candle (the un-vendored fork, rev
 * 9f6eed19): `Tensor / f64` and `Tensor + f64` are `affine(mul, add)` =
 * `v * (float)mul + (float)add`; `mean_keepdim` = `sum_keepdim * (1/n)`;
 * `clamp(lo, hi)` = `maximum(lo).minimum(hi)`.
 *
 * Parity status of each function (the test that pins it):
 *   or_layer_norm            torch F.layer_norm (f64) + invariants   tests/test_oracle_pins.py
 *   or_layer_norm_slow       torch F.layer_norm (f64) + invariants
 *   or_layer_norm_no_affine  torch F.layer_norm (f64) + invariants
 *   or_residual_layer_norm   f64 closed form + LayerScale=0 reduction
 *   or_adaln_modulate        chunk-order KAT (tests/trellis2_blocks.rs:205-225) + f64 form
 *   or_gated_residual        f64 closed form + gate=0 identity
 *   or_gated_residual_modulate  torch f64 closed form of the stored residual
 *                            and its modulated norm; gate = 0 / scale = shift
 *                            = 0 reductions; ungated add (tests/test_oracle_pins.py)
 *   or_rms_norm_heads        f64 closed form + scale invariance
 *   or_qk_l2norm             KAT tests/trellis2_blocks.rs:126-153
 *   or_rope2d_*              complex-rotation (f64) + identity at p=0 + norm preservation
 *   or_rope3d_*              KATs tests/trellis2_blocks.rs:43-111
 *   or_dinov3_rope_*         KATs runtime/trellis2_dino.rs:516-644
 *   or_gelu_*, or_silu       torch F.gelu / F.silu (f64)
 *   or_timestep_embedding_*  KAT tests/trellis2_blocks.rs:157-171 + f64 form
 *   or_dequant_q8_0          brute force over all int8 x f16 scale sweep
 *   or_q8_0_linear           numpy f64 matmul of the dequantized weight; identity
 *                            weight; tiny brute force (tests/test_oracle_pins.py)
 *   or_q8_0_linear_f32       numpy f64 matmul of the f32-dequantized weight; identity
 *                            weight returns x; tiny brute force
 *   or_quantize_q8_0         brute force per block against an independent Python
 *                            restatement; amax / round-half-away / saturation / NaN
 *                            special cases; a round trip within d / 2 per value
 *   or_q8_0_linear_int8      the integer block dot exact against numpy int64;
 *                            brute force on tiny shapes (Python loop in the same
 *                            f32 order); a one-block case in closed form
 *   or_sparse_neighbors      reference KATs (tests/trellis2_sparse.rs:67-93) + brute
 *                            force over all pairs
 *   or_sparse_conv3d         torch conv3d (f64) on the densified grid; the
 *                            reference's identity / shift kernels
 *                            (tests/trellis2_sparse.rs:164-237)
 *   or_channel_to_spatial    reference KAT (tests/trellis2_sparse.rs:274-318) +
 *                            S2C round trip
 *   or_sdpa                  scipy softmax + numpy f64 matmuls; closed forms
 *                            (identical keys -> mean of v, one key -> v, a
 *                            dominant key -> its v row); key-permutation
 *                            invariance (tests/test_oracle_pins.py)
 */
#include "lux3d_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* threading                                                                */
/* ------------------------------------------------------------------------ */

static int g_threads = 1;

void or_set_threads(int n) { g_threads = n < 1 ? 1 : (n > 256 ? 256 : n); }
int or_get_threads(void) { return g_threads; }

typedef void (*row_fn)(const void *ctx, int64_t r0, int64_t r1);

typedef struct {
  row_fn fn;
  const void *ctx;
  int64_t r0, r1;
} job_t;

static void *job_main(void *p) {
  job_t *j = (job_t *)p;
  j->fn(j->ctx, j->r0, j->r1);
  return NULL;
}

static void parallel_rows(int64_t rows, row_fn fn, const void *ctx) {
  int t = g_threads;
  if (t <= 1 || rows < 2 * (int64_t)t) {
    fn(ctx, 0, rows);
    return;
  }
  pthread_t th[256];
  job_t jobs[256];
  int64_t chunk = (rows + t - 1) / t;
  int started = 0;
  for (int i = 0; i < t; ++i) {
    int64_t r0 = (int64_t)i * chunk, r1 = r0 + chunk;
    if (r0 >= rows) break;
    if (r1 > rows) r1 = rows;
    jobs[i].fn = fn;
    jobs[i].ctx = ctx;
    jobs[i].r0 = r0;
    jobs[i].r1 = r1;
    if (pthread_create(&th[i], NULL, job_main, &jobs[i]) != 0) {
      fn(ctx, r0, r1); /* run inline if a thread cannot start */
      jobs[i].fn = NULL;
    }
    started = i + 1;
  }
  for (int i = 0; i < started; ++i)
    if (jobs[i].fn) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                       */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }
static inline float u2f(uint32_t u) { float v; memcpy(&v, &u, 4); return v; }

/* half 2.7.1 `f32_to_bf16`: NaN keeps its sign and top payload bits and is
 * forced quiet; otherwise round-to-nearest-even on bit 15. */
uint16_t or_f32_to_bf16(float v) {
  uint32_t x = f2u(v);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x0040u);
  const uint32_t round_bit = 0x8000u;
  if ((x & round_bit) && (x & (3u * round_bit - 1u))) return (uint16_t)((x >> 16) + 1u);
  return (uint16_t)(x >> 16);
}

float or_bf16_to_f32(uint16_t v) { return u2f((uint32_t)v << 16); }

/* IEEE binary16, round-to-nearest-even, overflow to +-inf, NaN quiet. */
uint16_t or_f32_to_f16(float v) {
  uint32_t x = f2u(v);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? (0x0200u | (man >> 13)) : 0u));
  int32_t e = (int32_t)exp - 127 + 15;
  if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    /* subnormal (or zero) result */
    if (e < -10) return (uint16_t)sign;
    uint32_t m = man | 0x800000u;
    uint32_t shift = (uint32_t)(14 - e);
    uint32_t half_m = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (half_m & 1u))) half_m += 1u;
    return (uint16_t)(sign | half_m);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* may carry into exp: correct */
  return (uint16_t)h;
}

float or_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
  uint32_t man = (uint32_t)h & 0x3FFu;
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    /* subnormal: man * 2^-24, exact in f32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 0x1F) return u2f(sign | 0x7F800000u | (man << 13));
  return u2f(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

/* Direct f64 -> bf16 rounding (half's bf16::from_f64), via the f32 value
 * with the double-rounding tie corrected. */
static uint16_t f64_to_bf16(double v) {
  float f = (float)v;
  uint32_t x = f2u(f);
  if ((x & 0x7FFFFFFFu) <= 0x7F800000u && (x & 0xFFFFu) == 0x8000u && (double)f != v) {
    /* f sits exactly on a bf16 tie but v does not: round by the side v is on */
    int away = fabs(v) > fabs((double)f);
    return (uint16_t)((x >> 16) + (away ? 1u : 0u));
  }
  return or_f32_to_bf16(f);
}

static inline float ld(int dt, const void *p, int64_t i) {
  switch (dt) {
    case OR_BF16: return or_bf16_to_f32(((const uint16_t *)p)[i]);
    case OR_F16: return or_f16_to_f32(((const uint16_t *)p)[i]);
    default: return ((const float *)p)[i];
  }
}

static inline void st(int dt, void *p, int64_t i, float v) {
  switch (dt) {
    case OR_BF16: ((uint16_t *)p)[i] = or_f32_to_bf16(v); break;
    case OR_F16: ((uint16_t *)p)[i] = or_f32_to_f16(v); break;
    default: ((float *)p)[i] = v;
  }
}

void or_convert(int src_dt, const void *src, int dst_dt, void *dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) st(dst_dt, dst, i, ld(src_dt, src, i));
}

/* `affine(mul, add)` of candle on an f32 value: v * mul + add. */
static inline float affine(float v, double mul, double add) {
  return v * (float)mul + (float)add;
}

/* ------------------------------------------------------------------------ */
/* L1: candle_nn::ops::layer_norm, CPU fast path (upstream candle-nn ops.rs  */
/* LayerNorm CustomOp3::cpu_fwd), reached from every `layer_norm(dim, eps,   */
/* vb)` + `LayerNorm::forward` on a contiguous input: pi3_encoder.rs:67,70, */
/* vggt.rs:104,107, trellis2_dino.rs:324,327, triposg_dit.rs:332-336.       */
/*   sum, sum2 sequential f32; mean = sum/d; var = sum2/d - mean^2;         */
/*   inv_std = 1/sqrt(var+eps); y = (x-mean)*inv_std*w + b (one rounding).  */
/* ------------------------------------------------------------------------ */

typedef struct {
  int dt;
  const void *x;
  int64_t d;
  const float *w, *b;
  float eps;
  void *y;
} ln_ctx;

static void ln_row(int dt, const void *x, int64_t base, int64_t d, const float *w,
                   const float *b, float eps, void *y, int64_t ybase) {
  float sum = 0.f, sum2 = 0.f;
  for (int64_t c = 0; c < d; ++c) {
    float v = ld(dt, x, base + c);
    sum += v;
    sum2 += v * v;
  }
  float mean = sum / (float)d;
  float var = sum2 / (float)d - mean * mean;
  float inv_std = 1.0f / sqrtf(var + eps);
  for (int64_t c = 0; c < d; ++c) {
    float alpha = w ? w[c] : 1.0f, beta = b ? b[c] : 0.0f;
    float v = ld(dt, x, base + c);
    st(dt, y, ybase + c, (v - mean) * inv_std * alpha + beta);
  }
}

static void ln_rows(const void *p, int64_t r0, int64_t r1) {
  const ln_ctx *c = (const ln_ctx *)p;
  for (int64_t r = r0; r < r1; ++r) ln_row(c->dt, c->x, r * c->d, c->d, c->w, c->b, c->eps, c->y, r * c->d);
}

void or_layer_norm(int dt, const void *x, int64_t rows, int64_t d, const float *w,
                   const float *b, float eps, void *y) {
  ln_ctx c = {dt, x, d, w, b, eps, y};
  parallel_rows(rows, ln_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* L2: candle_nn::LayerNorm::forward composed path (upstream candle-nn       */
/* layer_norm.rs), taken for the strided q/k head views at vggt.rs:170-181   */
/* via attention_math.rs:148:                                                */
/*   mean = sum*(1/d); c = x - mean; var = sum(c^2)*(1/d);                   */
/*   n = c / sqrt(var*1 + eps); y = n*w + b.                                 */
/* ------------------------------------------------------------------------ */

static float slow_ln_stats(int dt, const void *x, int64_t base, int64_t d, float eps,
                           float *mean_out) {
  float sum = 0.f;
  for (int64_t c = 0; c < d; ++c) sum += ld(dt, x, base + c);
  float mean = affine(sum, 1.0 / (double)d, 0.0);
  float s2 = 0.f;
  for (int64_t c = 0; c < d; ++c) {
    float cv = ld(dt, x, base + c) - mean;
    s2 += cv * cv;
  }
  float var = affine(s2, 1.0 / (double)d, 0.0);
  *mean_out = mean;
  return sqrtf(affine(var, 1.0, (double)eps));
}

static void slow_ln_rows(const void *p, int64_t r0, int64_t r1) {
  const ln_ctx *c = (const ln_ctx *)p;
  for (int64_t r = r0; r < r1; ++r) {
    int64_t base = r * c->d;
    float mean;
    float den = slow_ln_stats(c->dt, c->x, base, c->d, c->eps, &mean);
    for (int64_t k = 0; k < c->d; ++k) {
      float n = (ld(c->dt, c->x, base + k) - mean) / den;
      if (c->w) n = n * c->w[k];
      if (c->b) n = n + c->b[k];
      st(c->dt, c->y, base + k, n);
    }
  }
}

void or_layer_norm_slow(int dt, const void *x, int64_t rows, int64_t d, const float *w,
                        const float *b, float eps, void *y) {
  ln_ctx c = {dt, x, d, w, b, eps, y};
  parallel_rows(rows, slow_ln_rows, &c);
}

/* L3: layer_norm_no_affine (trellis2_blocks.rs:280-286) and adaln_norm
 * (vggt.rs:432-437): the same composed arithmetic without w/b. */
void or_layer_norm_no_affine(int dt, const void *x, int64_t rows, int64_t d, float eps,
                             void *y) {
  ln_ctx c = {dt, x, d, NULL, NULL, eps, y};
  parallel_rows(rows, slow_ln_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* F1 / F3: LayerScale + residual, then L1.                                 */
/*   LayerScale::forward = xs.broadcast_mul(gamma) (nn_blocks.rs:210-214);  */
/*   residual add (vggt.rs:115-118, pi3_encoder.rs:80-83,                   */
/*   trellis2_dino.rs:348, triposg_dit.rs:367): h = (a*gamma) + x, stored   */
/*   in the activation dtype; the next norm reads the stored h.             */
/* ------------------------------------------------------------------------ */

typedef struct {
  int dt;
  const void *x, *a;
  const float *gamma;
  int64_t d;
  const float *w, *b;
  float eps;
  void *h, *y;
} res_ctx;

static void res_rows(const void *p, int64_t r0, int64_t r1) {
  const res_ctx *c = (const res_ctx *)p;
  for (int64_t r = r0; r < r1; ++r) {
    int64_t base = r * c->d;
    for (int64_t k = 0; k < c->d; ++k) {
      float t = ld(c->dt, c->a, base + k);
      if (c->gamma) t = t * c->gamma[k];
      st(c->dt, c->h, base + k, t + ld(c->dt, c->x, base + k));
    }
    ln_row(c->dt, c->h, base, c->d, c->w, c->b, c->eps, c->y, base);
  }
}

void or_residual_layer_norm(int dt, const void *x, const void *a, const float *gamma,
                            int64_t rows, int64_t d, const float *w, const float *b,
                            float eps, void *h, void *y) {
  res_ctx c = {dt, x, a, gamma, d, w, b, eps, h, y};
  parallel_rows(rows, res_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* MV + L3 + M1 (Trellis2DenseBlock::forward trellis2_blocks.rs:617-630,    */
/* 639-642; Trellis2SparseBlock 693-706):                                   */
/*   mod_vec = modulation + t_emb            (broadcast_add, f32)           */
/*   y = L3(x) * (scale*1 + 1) + shift        (affine(1,1), mul, add)       */
/* M1' VGGT camera head (vggt.rs:399-405): y = gate*(...) + x.              */
/* ------------------------------------------------------------------------ */

static int64_t seg_of_row(const int64_t *seg_off, int64_t nseg, int64_t r) {
  int64_t lo = 0, hi = nseg - 1;
  while (lo < hi) {
    int64_t mid = (lo + hi + 1) / 2;
    if (seg_off[mid] <= r) lo = mid; else hi = mid - 1;
  }
  return lo;
}

static inline float mod_piece(const float *seg, int64_t ld_, const float *base, int64_t s,
                              int64_t c) {
  float v = seg[s * ld_ + c];
  return base ? base[c] + v : v;
}

typedef struct {
  int dt;
  const void *x;
  int64_t d;
  const int64_t *seg_off;
  int64_t nseg;
  const float *shift, *shift_base, *scale, *scale_base, *gate, *gate_base;
  int64_t ld_shift, ld_scale, ld_gate;
  float eps;
  void *y;
} mod_ctx;

static void mod_rows(const void *p, int64_t r0, int64_t r1) {
  const mod_ctx *c = (const mod_ctx *)p;
  for (int64_t r = r0; r < r1; ++r) {
    int64_t s = seg_of_row(c->seg_off, c->nseg, r);
    int64_t base = r * c->d;
    float mean;
    float den = slow_ln_stats(c->dt, c->x, base, c->d, c->eps, &mean);
    for (int64_t k = 0; k < c->d; ++k) {
      float xv = ld(c->dt, c->x, base + k);
      float n = (xv - mean) / den;
      float sc = mod_piece(c->scale, c->ld_scale, c->scale_base, s, k);
      float sh = mod_piece(c->shift, c->ld_shift, c->shift_base, s, k);
      float m = n * affine(sc, 1.0, 1.0) + sh;
      if (c->gate) m = mod_piece(c->gate, c->ld_gate, c->gate_base, s, k) * m + xv;
      st(c->dt, c->y, base + k, m);
    }
  }
}

void or_adaln_modulate(int dt, const void *x, int64_t rows, int64_t d,
                       const int64_t *seg_off, int64_t nseg, const float *shift,
                       int64_t ld_shift, const float *shift_base, const float *scale,
                       int64_t ld_scale, const float *scale_base, const float *gate,
                       int64_t ld_gate, const float *gate_base, float eps, void *y) {
  mod_ctx c = {dt, x, d, seg_off, nseg, shift, shift_base, scale, scale_base, gate,
               gate_base, ld_shift, ld_scale, ld_gate, eps, y};
  parallel_rows(rows, mod_rows, &c);
}

/* G1: gated residual (trellis2_blocks.rs:632-633, 644-645): x + (h*gate). */
typedef struct {
  int dt;
  const void *x, *h;
  int64_t d;
  const int64_t *seg_off;
  int64_t nseg;
  const float *gate;
  int64_t ld_gate;
  const float *gate_base;
  void *out;
} gate_ctx;

static void gate_rows(const void *p, int64_t r0, int64_t r1) {
  const gate_ctx *c = (const gate_ctx *)p;
  for (int64_t r = r0; r < r1; ++r) {
    int64_t s = seg_of_row(c->seg_off, c->nseg, r);
    int64_t base = r * c->d;
    for (int64_t k = 0; k < c->d; ++k) {
      float g = mod_piece(c->gate, c->ld_gate, c->gate_base, s, k);
      float hv = ld(c->dt, c->h, base + k) * g;
      st(c->dt, c->out, base + k, ld(c->dt, c->x, base + k) + hv);
    }
  }
}

void or_gated_residual(int dt, const void *x, const void *h, int64_t rows, int64_t d,
                       const int64_t *seg_off, int64_t nseg, const float *gate,
                       int64_t ld_gate, const float *gate_base, void *out) {
  gate_ctx c = {dt, x, h, d, seg_off, nseg, gate, ld_gate, gate_base, out};
  parallel_rows(rows, gate_rows, &c);
}

/* G1 followed by L3 + M1 on the stored residual stream:
 * Trellis2SparseBlock::forward (trellis2_blocks.rs:708-713):
 *   h = h.broadcast_mul(gate_msa); xs = xs.add(h);
 *   n = layer_norm_no_affine(xs, 1e-6);
 *   n.broadcast_mul(scale_mlp.affine(1, 1)).broadcast_add(shift_mlp)
 * and Trellis2DenseBlock::forward (:637-642), where the cross-attention
 * output is added without a gate (gate == NULL here: x + h). The norm reads
 * xs as stored in the activation dtype. */
typedef struct {
  int dt;
  const void *x, *h;
  int64_t d;
  const int64_t *seg_off;
  int64_t nseg;
  const float *gate, *gate_base, *shift, *shift_base, *scale, *scale_base;
  int64_t ld_gate, ld_shift, ld_scale;
  float eps;
  void *x_out, *y;
} gmod_ctx;

static void gmod_rows(const void *p, int64_t r0, int64_t r1) {
  const gmod_ctx *c = (const gmod_ctx *)p;
  for (int64_t r = r0; r < r1; ++r) {
    int64_t s = seg_of_row(c->seg_off, c->nseg, r);
    int64_t base = r * c->d;
    for (int64_t k = 0; k < c->d; ++k) {
      float hv = ld(c->dt, c->h, base + k);
      if (c->gate) hv = hv * mod_piece(c->gate, c->ld_gate, c->gate_base, s, k);
      st(c->dt, c->x_out, base + k, ld(c->dt, c->x, base + k) + hv);
    }
    float mean;
    float den = slow_ln_stats(c->dt, c->x_out, base, c->d, c->eps, &mean);
    for (int64_t k = 0; k < c->d; ++k) {
      float n = (ld(c->dt, c->x_out, base + k) - mean) / den;
      float sc = mod_piece(c->scale, c->ld_scale, c->scale_base, s, k);
      float sh = mod_piece(c->shift, c->ld_shift, c->shift_base, s, k);
      st(c->dt, c->y, base + k, n * affine(sc, 1.0, 1.0) + sh);
    }
  }
}

void or_gated_residual_modulate(int dt, const void *x, const void *h, int64_t rows, int64_t d,
                                const int64_t *seg_off, int64_t nseg, const float *gate,
                                int64_t ld_gate, const float *gate_base, const float *shift,
                                int64_t ld_shift, const float *shift_base, const float *scale,
                                int64_t ld_scale, const float *scale_base, float eps,
                                void *x_out, void *y) {
  gmod_ctx c = {dt, x, h, d, seg_off, nseg, gate, gate_base, shift, shift_base, scale,
                scale_base, ld_gate, ld_shift, ld_scale, eps, x_out, y};
  parallel_rows(rows, gmod_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* N1: RmsNormHeads::rms_norm_heads (triposg_dit.rs:515-521):                */
/*   var = sum(x^2)*(1/d); y = x / sqrt(var*1 + eps) * w.                   */
/* ------------------------------------------------------------------------ */

typedef struct {
  int dt;
  const void *x;
  int64_t d;
  const float *w;
  float eps;
  void *y;
} rms_ctx;

static void rms_rows(const void *p, int64_t r0, int64_t r1) {
  const rms_ctx *c = (const rms_ctx *)p;
  for (int64_t r = r0; r < r1; ++r) {
    int64_t base = r * c->d;
    float s2 = 0.f;
    for (int64_t k = 0; k < c->d; ++k) {
      float v = ld(c->dt, c->x, base + k);
      s2 += v * v;
    }
    float var = affine(s2, 1.0 / (double)c->d, 0.0);
    float den = sqrtf(affine(var, 1.0, (double)c->eps));
    for (int64_t k = 0; k < c->d; ++k)
      st(c->dt, c->y, base + k, (ld(c->dt, c->x, base + k) / den) * c->w[k]);
  }
}

void or_rms_norm_heads(int dt, const void *x, int64_t rows, int64_t d, const float *w,
                       float eps, void *y) {
  rms_ctx c = {dt, x, d, w, eps, y};
  parallel_rows(rows, rms_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* N2: Trellis2QkRmsNorm::forward (trellis2_blocks.rs:306-319):              */
/*   n = clamp(sqrt(sum x^2), 1e-12, 1e30); y = ((x/n)*gamma[h]) * sqrt(D). */
/* ------------------------------------------------------------------------ */

static void l2norm_head(int dt, const void *x, int64_t base, int64_t d, const float *g,
                        float *out) {
  float s2 = 0.f;
  for (int64_t k = 0; k < d; ++k) {
    float v = ld(dt, x, base + k);
    s2 += v * v;
  }
  float n = sqrtf(s2);
  n = fmaxf(n, 1e-12f);
  n = fminf(n, 1.0e30f);
  float scale = sqrtf((float)d);
  for (int64_t k = 0; k < d; ++k) out[k] = affine((ld(dt, x, base + k) / n) * g[k], scale, 0.0);
}

typedef struct {
  int dt;
  const void *x;
  int64_t heads, d;
  const float *gamma, *cos, *sin;
  void *y;
} l2_ctx;

static void l2_rows(const void *p, int64_t r0, int64_t r1) {
  const l2_ctx *c = (const l2_ctx *)p;
  float tmp[1024];
  for (int64_t r = r0; r < r1; ++r)
    for (int64_t h = 0; h < c->heads; ++h) {
      int64_t base = (r * c->heads + h) * c->d;
      l2norm_head(c->dt, c->x, base, c->d, c->gamma + h * c->d, tmp);
      if (c->cos) {
        /* R2 on the normalised f32 head (Trellis2Rope3d::apply arithmetic) */
        for (int64_t k = 0; k < c->d / 2; ++k) {
          float co = c->cos[r * (c->d / 2) + k], si = c->sin[r * (c->d / 2) + k];
          float re = tmp[2 * k], im = tmp[2 * k + 1];
          st(c->dt, c->y, base + 2 * k, re * co - im * si);
          st(c->dt, c->y, base + 2 * k + 1, re * si + im * co);
        }
      } else {
        for (int64_t k = 0; k < c->d; ++k) st(c->dt, c->y, base + k, tmp[k]);
      }
    }
}

void or_qk_l2norm(int dt, const void *x, int64_t rows, int64_t heads, int64_t d,
                  const float *gamma, void *y) {
  l2_ctx c = {dt, x, heads, d, gamma, NULL, NULL, y};
  parallel_rows(rows, l2_rows, &c);
}

void or_qk_l2norm_rope3d(int dt, const void *x, int64_t rows, int64_t heads, int64_t d,
                         const float *gamma, const float *cos, const float *sin, void *y) {
  l2_ctx c = {dt, x, heads, d, gamma, cos, sin, y};
  parallel_rows(rows, l2_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* R1: VGGT / Pi3 2D RoPE (attention_math.rs:14-118).                        */
/* ------------------------------------------------------------------------ */

/* Rope2d::cos_sin (attention_math.rs:60-76): inv_freq[k] = 1/base^((2k)/dim)
 * with dim = half; freqs = p*inv (a K=1 matmul: one exact f32 product);
 * table row = [freqs, freqs]. */
static void rope2d_half_row(float base, int64_t half, uint32_t p, float *cos_row,
                            float *sin_row) {
  int64_t nf = half / 2;
  for (int64_t k = 0; k < nf; ++k) {
    float inv = 1.0f / powf(base, (float)(2 * k) / (float)half);
    float ang = (float)p * inv;
    float co = cosf(ang), si = sinf(ang);
    cos_row[k] = co;
    cos_row[k + nf] = co;
    sin_row[k] = si;
    sin_row[k + nf] = si;
  }
}

void or_rope2d_tables(const int32_t *pos, int64_t b, int64_t n, int64_t d, float base,
                      float *cos_full, float *sin_alt_full) {
  int64_t half = d / 2, quarter = half / 2;
  float cy[512], sy[512];
  for (int64_t t = 0; t < b * n; ++t) {
    for (int64_t axis = 0; axis < 2; ++axis) {
      /* positions.to_dtype(U32) (attention_math.rs:19) */
      uint32_t p = (uint32_t)pos[t * 2 + axis];
      rope2d_half_row(base, half, p, cy, sy);
      for (int64_t j = 0; j < half; ++j) {
        cos_full[t * d + axis * half + j] = cy[j];
        /* sin_alt: first quarter negated via affine(-1, 0) (:36-49) */
        sin_alt_full[t * d + axis * half + j] = j < quarter ? affine(sy[j], -1.0, 0.0) : sy[j];
      }
    }
  }
}

typedef struct {
  int dt;
  const void *t;
  int64_t h, n, d;
  const float *w, *b;
  float eps;
  int norm;
  const float *cos, *sin;
  void *y;
} r1_ctx;

/* rows = (b, h, n) flattened; tables indexed by (b, n). */
static void r1_rows(const void *p, int64_t r0, int64_t r1) {
  const r1_ctx *c = (const r1_ctx *)p;
  int64_t d = c->d, half = d / 2, quarter = half / 2;
  float v[1024];
  for (int64_t r = r0; r < r1; ++r) {
    int64_t bi = r / (c->h * c->n), ni = r % c->n;
    int64_t base = r * d, tb = (bi * c->n + ni) * d;
    if (c->norm) {
      float mean;
      float den = slow_ln_stats(c->dt, c->t, base, d, c->eps, &mean);
      /* a LayerNorm without bias (candle_nn::LayerNorm, bias None) stops at n * w */
      for (int64_t k = 0; k < d; ++k) {
        v[k] = ((ld(c->dt, c->t, base + k) - mean) / den) * c->w[k];
        if (c->b) v[k] = v[k] + c->b[k];
      }
    } else {
      for (int64_t k = 0; k < d; ++k) v[k] = ld(c->dt, c->t, base + k);
    }
    for (int64_t j = 0; j < d; ++j) {
      /* pairs_rot = cat(y2, y1, x2, x1) (attention_math.rs:108-112) */
      int64_t jj = j % half;
      int64_t partner = (j - jj) + (jj < quarter ? jj + quarter : jj - quarter);
      st(c->dt, c->y, base + j, v[j] * c->cos[tb + j] + v[partner] * c->sin[tb + j]);
    }
  }
}

void or_rope2d_apply(int dt, const void *t, int64_t b, int64_t h, int64_t n, int64_t d,
                     const float *cos_full, const float *sin_alt_full, void *y) {
  r1_ctx c = {dt, t, h, n, d, NULL, NULL, 0.f, 0, cos_full, sin_alt_full, y};
  parallel_rows(b * h * n, r1_rows, &c);
}

void or_layernorm_rope2d(int dt, const void *q, int64_t b, int64_t h, int64_t n, int64_t d,
                         const float *w, const float *bias, float eps, const float *cos_full,
                         const float *sin_alt_full, void *y) {
  r1_ctx c = {dt, q, h, n, d, w, bias, eps, 1, cos_full, sin_alt_full, y};
  parallel_rows(b * h * n, r1_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* R2: TRELLIS.2 3D RoPE (trellis2_blocks.rs:57-160).                        */
/*   freq_dim = head_dim/2/3; f[i] = 1/base^(i/freq_dim);                   */
/*   ang[axis*freq_dim + i] = float(coord[axis]) * f[i]; pad angles 0.      */
/*   (re, im) -> (re*c - im*s, re*s + im*c)                                 */
/* ------------------------------------------------------------------------ */

void or_rope3d_tables(const int32_t *coords, int64_t n, int64_t head_dim, float base,
                      float *cos, float *sin) {
  int64_t fd = head_dim / 2 / 3, half = head_dim / 2;
  float f[512];
  for (int64_t i = 0; i < fd; ++i) f[i] = 1.0f / powf(base, (float)i / (float)fd);
  for (int64_t t = 0; t < n; ++t) {
    for (int64_t j = 0; j < half; ++j) {
      float ang = 0.f;
      if (j < 3 * fd) ang = (float)coords[t * 3 + j / fd] * f[j % fd];
      cos[t * half + j] = cosf(ang);
      sin[t * half + j] = sinf(ang);
    }
  }
}

typedef struct {
  int dt;
  const void *x;
  int64_t l, h, d;
  const float *cos, *sin;
  void *y;
} r2_ctx;

static void r2_rows(const void *p, int64_t r0, int64_t r1) {
  const r2_ctx *c = (const r2_ctx *)p;
  int64_t half = c->d / 2;
  for (int64_t r = r0; r < r1; ++r) { /* r = (b, l, h) */
    int64_t li = (r / c->h) % c->l;
    int64_t base = r * c->d;
    for (int64_t k = 0; k < half; ++k) {
      float co = c->cos[li * half + k], si = c->sin[li * half + k];
      float re = ld(c->dt, c->x, base + 2 * k), im = ld(c->dt, c->x, base + 2 * k + 1);
      st(c->dt, c->y, base + 2 * k, re * co - im * si);
      st(c->dt, c->y, base + 2 * k + 1, re * si + im * co);
    }
  }
}

void or_rope3d_apply(int dt, const void *x, int64_t b, int64_t l, int64_t h, int64_t d,
                     const float *cos, const float *sin, void *y) {
  r2_ctx c = {dt, x, l, h, d, cos, sin, y};
  parallel_rows(b * l * h, r2_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* R3: DINOv3 2D RoPE (trellis2_dino.rs:140-187, 406-445).                   */
/* ------------------------------------------------------------------------ */

void or_dinov3_rope_tables(int64_t grid_h, int64_t grid_w, int64_t head_dim, float theta,
                           float *cos, float *sin) {
  int64_t fc = head_dim / 4;
  float inv[256];
  for (int64_t i = 0; i < fc; ++i)
    inv[i] = 1.0f / powf(theta, (float)i * (4.0f / (float)head_dim));
  float two_pi = (float)(M_PI * 2.0);
  int64_t half_len = fc * 2;
  for (int64_t y = 0; y < grid_h; ++y) {
    float cy = 2.0f * (((float)y + 0.5f) / (float)grid_h) - 1.0f;
    for (int64_t x = 0; x < grid_w; ++x) {
      float cx = 2.0f * (((float)x + 0.5f) / (float)grid_w) - 1.0f;
      int64_t row = (y * grid_w + x) * head_dim;
      float coords[2] = {cy, cx};
      for (int64_t a = 0; a < 2; ++a) {
        float base = two_pi * coords[a];
        for (int64_t i = 0; i < fc; ++i) {
          float ang = base * inv[i];
          for (int64_t rep = 0; rep < 2; ++rep) {
            cos[row + rep * half_len + a * fc + i] = cosf(ang);
            sin[row + rep * half_len + a * fc + i] = sinf(ang);
          }
        }
      }
    }
  }
}

typedef struct {
  int dt;
  const void *x;
  int64_t s, d, np;
  const float *cos, *sin;
  void *y;
} r3_ctx;

static void r3_rows(const void *p, int64_t r0, int64_t r1) {
  const r3_ctx *c = (const r3_ctx *)p;
  int64_t d = c->d, half = d / 2;
  for (int64_t r = r0; r < r1; ++r) { /* r = (b, h, s) */
    int64_t si = r % c->s, base = r * d;
    if (si < c->np) {
      for (int64_t k = 0; k < d; ++k) st(c->dt, c->y, base + k, ld(c->dt, c->x, base + k));
      continue;
    }
    int64_t tb = (si - c->np) * d;
    for (int64_t k = 0; k < d; ++k) {
      /* rotate_half = cat(-x2, x1) (trellis2_dino.rs:439-445) */
      float rh = k < half ? -ld(c->dt, c->x, base + k + half) : ld(c->dt, c->x, base + k - half);
      float v = ld(c->dt, c->x, base + k);
      st(c->dt, c->y, base + k, v * c->cos[tb + k] + rh * c->sin[tb + k]);
    }
  }
}

void or_dinov3_rope_apply(int dt, const void *x, int64_t b, int64_t h, int64_t s, int64_t d,
                          int64_t num_prefix, const float *cos, const float *sin, void *y) {
  r3_ctx c = {dt, x, s, d, num_prefix, cos, sin, y};
  parallel_rows(b * h * s, r3_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* Activations (upstream candle-core op.rs unary ops; call sites             */
/* trellis2_blocks.rs:560 gelu, nn_blocks.rs:233 gelu_erf, :236 silu).       */
/* ------------------------------------------------------------------------ */

typedef struct {
  int dt, kind;
  const void *x;
  void *y;
} act_ctx;

static void act_rows(const void *p, int64_t r0, int64_t r1) {
  const act_ctx *c = (const act_ctx *)p;
  for (int64_t i = r0; i < r1; ++i) {
    float v = ld(c->dt, c->x, i);
    if (c->kind == 0) {
      /* GeluErf: computed in f64, (erf(v/sqrt2) + 1) * 0.5 * v, one rounding */
      double dv = (double)v;
      double r = (erf(dv / sqrt(2.0)) + 1.0) * 0.5 * dv;
      if (c->dt == OR_BF16) ((uint16_t *)c->y)[i] = f64_to_bf16(r);
      else st(c->dt, c->y, i, (float)r);
    } else if (c->kind == 1) {
      /* Gelu (tanh): 0.5*v*(1 + tanh(sqrt(2/pi)*v*(1 + 0.044715*v*v))) in f32 */
      float k0 = sqrtf(2.0f / (float)M_PI);
      float inner = k0 * v * (1.0f + 0.044715f * v * v);
      st(c->dt, c->y, i, 0.5f * v * (1.0f + tanhf(inner)));
    } else {
      /* Silu: v / (1 + exp(-v)) */
      st(c->dt, c->y, i, v / (1.0f + expf(-v)));
    }
  }
}

static void act_run(int dt, int kind, const void *x, int64_t n, void *y) {
  act_ctx c = {dt, kind, x, y};
  parallel_rows(n, act_rows, &c);
}

void or_gelu_erf(int dt, const void *x, int64_t n, void *y) { act_run(dt, 0, x, n, y); }
void or_gelu_tanh(int dt, const void *x, int64_t n, void *y) { act_run(dt, 1, x, n, y); }
void or_silu(int dt, const void *x, int64_t n, void *y) { act_run(dt, 2, x, n, y); }

/* ------------------------------------------------------------------------ */
/* Timestep embeddings.                                                      */
/* ------------------------------------------------------------------------ */

/* T1 (triposg_dit.rs:286-297): lmp = -ln(10000f32); f = exp(lmp*i/half);
 * emb = t*f; out = [sin(emb), cos(emb)]. */
void or_timestep_embedding_sin_first(const float *t, int64_t n, int64_t dim, float *out) {
  int64_t half = dim / 2;
  float lmp = -logf(10000.0f);
  for (int64_t r = 0; r < n; ++r)
    for (int64_t i = 0; i < half; ++i) {
      float f = expf(lmp * (float)i / (float)half);
      float e = t[r] * f;
      out[r * dim + i] = sinf(e);
      out[r * dim + half + i] = cosf(e);
    }
}

/* Either convention from a given frequency vector freqs[dim / 2] (the
 * reference's own host loop computes it; see or_timestep_embedding_*): the
 * argument t * f is one f32 product in both (T2's affine(f, t, 0) rounds the
 * exact f64 product once), then [sin, cos] (T1) or [cos, sin] + 0 pad (T2). */
void or_timestep_embedding_freqs(const float *t, int64_t n, const float *freqs, int64_t dim, int cos_first,
                                 float *out) {
  int64_t half = dim / 2;
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t i = 0; i < half; ++i) {
      float a = t[r] * freqs[i];
      out[r * dim + i] = cos_first ? cosf(a) : sinf(a);
      out[r * dim + half + i] = cos_first ? sinf(a) : cosf(a);
    }
    if (cos_first && dim % 2) out[r * dim + dim - 1] = 0.f;
  }
}

/* T2 (trellis2_blocks.rs:189-203): nlp = -(ln(10000) as f64) as f32;
 * f = exp(nlp*i/half); args = f*t + 0 (affine); out = [cos, sin] (+0 pad). */
void or_timestep_embedding_cos_first(const float *t, int64_t n, int64_t dim, float *out) {
  int64_t half = dim / 2;
  float nlp = (float)(-log(10000.0));
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t i = 0; i < half; ++i) {
      float f = expf(nlp * (float)i / (float)half);
      float a = affine(f, (double)t[r], 0.0);
      out[r * dim + i] = cosf(a);
      out[r * dim + half + i] = sinf(a);
    }
    if (dim % 2) out[r * dim + dim - 1] = 0.f;
  }
}

/* ------------------------------------------------------------------------ */
/* Q1: GGML Q8_0 dequant (QTensor::dequantize, nn_blocks.rs:140; block      */
/* layout block_q8_0 = {f16 d; int8 qs[32]}, little-endian).               */
/* ------------------------------------------------------------------------ */

typedef struct {
  const uint8_t *blk;
  int dt;
  void *out;
} q8_ctx;

static void q8_rows(const void *p, int64_t r0, int64_t r1) {
  const q8_ctx *c = (const q8_ctx *)p;
  for (int64_t b = r0; b < r1; ++b) {
    const uint8_t *q = c->blk + b * 34;
    float d = or_f16_to_f32((uint16_t)(q[0] | (q[1] << 8)));
    for (int j = 0; j < 32; ++j) st(c->dt, c->out, b * 32 + j, (float)(int8_t)q[2 + j] * d);
  }
}

void or_dequant_q8_0(const uint8_t *blocks, int64_t nblocks, int out_dt, void *out) {
  q8_ctx c = {blocks, out_dt, out};
  parallel_rows(nblocks, q8_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* Quantized linear: LinearInner::Quant forward (nn_blocks.rs:83-93) as     */
/* QMatMul::forward with the weight dequantized to bf16, then the bias add. */
/* ------------------------------------------------------------------------ */

typedef struct {
  const float *x, *w, *bias;
  int64_t K, N;
  int dt;
  void *y;
  float *abs_sum;
} ql_ctx;

static void ql_rows(const void *p, int64_t r0, int64_t r1) {
  const ql_ctx *c = (const ql_ctx *)p;
  for (int64_t m = r0; m < r1; ++m) {
    const float *xr = c->x + m * c->K;
    for (int64_t n = 0; n < c->N; ++n) {
      const float *wr = c->w + n * c->K;
      double acc = 0.0, aacc = 0.0;
      for (int64_t k = 0; k < c->K; ++k) {
        const double pr = (double)xr[k] * (double)wr[k];
        acc += pr;
        aacc += fabs(pr);
      }
      if (c->bias) acc += (double)c->bias[n];
      const int64_t o = m * c->N + n;
      if (c->dt == OR_BF16) ((uint16_t *)c->y)[o] = f64_to_bf16(acc);
      else st(c->dt, c->y, o, (float)acc);
      if (c->abs_sum) c->abs_sum[o] = (float)aacc;
    }
  }
}

void or_q8_0_linear(const uint16_t *x, int64_t M, int64_t K, const uint8_t *blocks, int64_t N,
                    const float *bias, int out_dt, void *y, float *abs_sum) {
  float *xf = (float *)malloc(sizeof(float) * (size_t)(M * K));
  float *wf = (float *)malloc(sizeof(float) * (size_t)(N * K));
  uint16_t *wb = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(N * K));
  if (!xf || !wf || !wb) {
    free(xf); free(wf); free(wb);
    return;
  }
  for (int64_t i = 0; i < M * K; ++i) xf[i] = or_bf16_to_f32(x[i]);
  or_dequant_q8_0(blocks, N * (K / 32), OR_BF16, wb);
  for (int64_t i = 0; i < N * K; ++i) wf[i] = or_bf16_to_f32(wb[i]);
  ql_ctx c = {xf, wf, bias, K, N, out_dt, y, abs_sum};
  parallel_rows(M, ql_rows, &c);
  free(xf); free(wf); free(wb);
}

/* The same with f32 activations: each weight is the exact f32 product q * d
 * (the reference's own Q8_0 dequant target, nn_blocks.rs:140), the sum of
 * the f32 products in f64, one rounding. */
void or_q8_0_linear_f32(const float *x, int64_t M, int64_t K, const uint8_t *blocks, int64_t N,
                        const float *bias, int out_dt, void *y, float *abs_sum) {
  float *wf = (float *)malloc(sizeof(float) * (size_t)(N * K));
  if (!wf) return;
  or_dequant_q8_0(blocks, N * (K / 32), OR_F32, wf);
  ql_ctx c = {x, wf, bias, K, N, out_dt, y, abs_sum};
  parallel_rows(M, ql_rows, &c);
  free(wf);
}

/* ---- candle's CPU QMatMul for a Q8_0 weight ------------------------------
 * Linear::forward's Quant branch (nn_blocks.rs:80-93) calls QMatMul::forward,
 * which on the CPU is the QTensor custom op (f32 x only) running
 * k_quants::matmul of the upstream candle-core crate (quantized/k_quants.rs
 * of the fork FerrisMind/candle 9f6eed1, not vendored in the reference): every
 * x row is first quantized to Q8_0 blocks (BlockQ8_0::from_float), then each
 * output is the weight row's vec_dot with them, block by block, and the
 * bias is broadcast-added. With no AVX target feature (the reference sets
 * none: no .cargo/config) vec_dot takes the generic vec_dot_unopt:
 *   sumf = 0; for each block b in order:
 *     sumf += (f32)(sum_j wq[j] * xq[j]) * f32(w.d) * f32(x.d)
 * the products left to right, each operation rounded in f32. */

/* BlockQ8_0::from_float: amax = max |x| (NaN ignored, f32::max), d = amax /
 * 127, id = d != 0 ? 1 / d : 0, q = round-half-away(x * id) saturated to
 * int8 (NaN -> 0, Rust's `as i8`), d stored as f16 (half's from_f32: RNE). */
void or_quantize_q8_0(const float *x, int64_t n, uint8_t *blocks) {
  for (int64_t b = 0; b < n / 32; ++b) {
    const float *xs = x + b * 32;
    float amax = 0.f;
    for (int j = 0; j < 32; ++j) {
      float a = fabsf(xs[j]);
      if (a > amax) amax = a; /* f32::max: a NaN operand yields the other (the compare is false) */
    }
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t dh = or_f32_to_f16(d);
    uint8_t *o = blocks + b * 34;
    o[0] = (uint8_t)(dh & 0xFF);
    o[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 32; ++j) {
      float r = roundf(xs[j] * id);
      int q = isnan(r) ? 0 : (r >= 127.0f ? 127 : (r <= -128.0f ? -128 : (int)r));
      o[2 + j] = (uint8_t)(int8_t)q;
    }
  }
}

typedef struct {
  const uint8_t *xb, *wb;
  const float *bias;
  int64_t nb, N;
  float *y;
} q8d_ctx;

static void q8d_rows(const void *vc, int64_t r0, int64_t r1) {
  const q8d_ctx *c = (const q8d_ctx *)vc;
  for (int64_t m = r0; m < r1; ++m) {
    const uint8_t *xr = c->xb + m * c->nb * 34;
    for (int64_t n = 0; n < c->N; ++n) {
      const uint8_t *wr = c->wb + n * c->nb * 34;
      float sumf = 0.f;
      for (int64_t b = 0; b < c->nb; ++b) {
        const uint8_t *wq = wr + b * 34, *xq = xr + b * 34;
        int32_t s = 0;
        for (int j = 0; j < 32; ++j) s += (int32_t)(int8_t)wq[2 + j] * (int32_t)(int8_t)xq[2 + j];
        const float wd = or_f16_to_f32((uint16_t)(wq[0] | (wq[1] << 8)));
        const float xd = or_f16_to_f32((uint16_t)(xq[0] | (xq[1] << 8)));
        /* each operation rounded (the oracle builds with -ffp-contract=off) */
        sumf = sumf + ((float)s * wd) * xd;
      }
      c->y[m * c->N + n] = c->bias ? sumf + c->bias[n] : sumf;
    }
  }
}

void or_q8_0_linear_int8(const float *x, int64_t M, int64_t K, const uint8_t *blocks, int64_t N, const float *bias,
                         float *y) {
  const int64_t nb = K / 32;
  uint8_t *xb = (uint8_t *)malloc((size_t)(M * nb * 34));
  if (!xb) return;
  for (int64_t m = 0; m < M; ++m) or_quantize_q8_0(x + m * K, K, xb + m * nb * 34);
  q8d_ctx c = {xb, blocks, bias, nb, N, y};
  parallel_rows(M, q8d_rows, &c);
  free(xb);
}

/* ------------------------------------------------------------------------ */
/* Attention: exact_sdpa_heads (attention_math.rs:244-259) -- widen q, k, v  */
/* to float, scores = q k^T * scale, softmax over the keys, attn v, one       */
/* rounding to the output dtype. exact_query_chunked_sdpa                     */
/* (attention_math.rs:199-241) computes the same function (its query chunks   */
/* only bound the scores buffer). Sums here run in double.                    */
/* ------------------------------------------------------------------------ */

typedef struct {
  int in_dt, out_dt;
  const void *q, *k, *v;
  int64_t Lq, Lk, D;
  double scale;
  void *out;
  float *wabs;
} sdpa_ctx;

static void sdpa_rows(const void *p, int64_t r0, int64_t r1) {
  const sdpa_ctx *c = (const sdpa_ctx *)p;
  const int64_t Lk = c->Lk, D = c->D;
  double *s = (double *)malloc(sizeof(double) * (size_t)(Lk + 2 * D));
  if (!s) return;
  double *acc = s + Lk, *aacc = acc + D;
  for (int64_t r = r0; r < r1; ++r) {  /* r = bh * Lq + i */
    const int64_t bh = r / c->Lq;
    const int64_t qo = r * D, ko = bh * Lk * D;
    double mx = -INFINITY;
    for (int64_t j = 0; j < Lk; ++j) {
      double dot = 0.0;
      for (int64_t d = 0; d < D; ++d)
        dot += (double)ld(c->in_dt, c->q, qo + d) * (double)ld(c->in_dt, c->k, ko + j * D + d);
      s[j] = dot * c->scale;
      if (s[j] > mx) mx = s[j];
    }
    double l = 0.0;
    for (int64_t j = 0; j < Lk; ++j) {
      s[j] = exp(s[j] - mx);
      l += s[j];
    }
    for (int64_t d = 0; d < D; ++d) acc[d] = aacc[d] = 0.0;
    for (int64_t j = 0; j < Lk; ++j)
      for (int64_t d = 0; d < D; ++d) {
        const double pv = s[j] * (double)ld(c->in_dt, c->v, ko + j * D + d);
        acc[d] += pv;
        aacc[d] += fabs(pv);
      }
    for (int64_t d = 0; d < D; ++d) {
      const double o = acc[d] / l;
      if (c->out_dt == OR_BF16) ((uint16_t *)c->out)[qo + d] = f64_to_bf16(o);
      else st(c->out_dt, c->out, qo + d, (float)o);
      if (c->wabs) c->wabs[qo + d] = (float)(aacc[d] / l);
    }
  }
  free(s);
}

void or_sdpa(int in_dt, const void *q, const void *k, const void *v, int64_t BH, int64_t Lq, int64_t Lk,
             int64_t D, double scale, int out_dt, void *out, float *wabs) {
  sdpa_ctx c = {in_dt, out_dt, q, k, v, Lq, Lk, D, scale, out, wabs};
  parallel_rows(BH * Lq, sdpa_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* TRELLIS.2 sparse ops (runtime/trellis2_sparse.rs)                        */
/* ------------------------------------------------------------------------ */

/* Open-addressing map (x, y, z) -> row; an insert of an existing key
 * overwrites, as HashMap::insert in CoordMap::new (trellis2_sparse.rs:72-79). */
typedef struct {
  int64_t cap;
  int64_t *keys;
  int32_t *vals;
} cmap_t;

static int64_t cmap_key(int32_t x, int32_t y, int32_t z) {
  return (((int64_t)x + (1 << 20)) << 42) | (((int64_t)y + (1 << 20)) << 21) | ((int64_t)z + (1 << 20));
}
static uint64_t cmap_hash(int64_t k) {
  uint64_t h = (uint64_t)k * 0x9E3779B97F4A7C15ull;
  return h ^ (h >> 29);
}
static int cmap_init(cmap_t *m, int64_t n) {
  m->cap = 16;
  while (m->cap < 2 * n) m->cap *= 2;
  m->keys = (int64_t *)malloc(sizeof(int64_t) * (size_t)m->cap);
  m->vals = (int32_t *)malloc(sizeof(int32_t) * (size_t)m->cap);
  if (!m->keys || !m->vals) return 0;
  for (int64_t i = 0; i < m->cap; ++i) m->keys[i] = -1;
  return 1;
}
static void cmap_free(cmap_t *m) { free(m->keys); free(m->vals); }
static void cmap_put(cmap_t *m, int64_t k, int32_t v) {
  uint64_t s = cmap_hash(k) & (uint64_t)(m->cap - 1);
  while (m->keys[s] != -1 && m->keys[s] != k) s = (s + 1) & (uint64_t)(m->cap - 1);
  m->keys[s] = k;
  m->vals[s] = v;
}
static int32_t cmap_get(const cmap_t *m, int64_t k) {
  uint64_t s = cmap_hash(k) & (uint64_t)(m->cap - 1);
  while (m->keys[s] != -1) {
    if (m->keys[s] == k) return m->vals[s];
    s = (s + 1) & (uint64_t)(m->cap - 1);
  }
  return -1;
}

/* kernel_offset_delta (trellis2_sparse.rs:83-91): k = kd*9 + kh*3 + kw. */
static void offset_delta(int k, int32_t d[3]) {
  d[0] = k / 9 - 1;
  d[1] = (k % 9) / 3 - 1;
  d[2] = k % 3 - 1;
}

void or_sparse_neighbors(const int32_t *coords, int64_t n, int32_t *nbr) {
  cmap_t m;
  if (!cmap_init(&m, n)) return;
  for (int64_t i = 0; i < n; ++i) cmap_put(&m, cmap_key(coords[3 * i], coords[3 * i + 1], coords[3 * i + 2]), (int32_t)i);
  for (int64_t i = 0; i < n; ++i)
    for (int k = 0; k < 27; ++k) {
      int32_t d[3];
      offset_delta(k, d);
      nbr[i * 27 + k] = cmap_get(&m, cmap_key(coords[3 * i] + d[0], coords[3 * i + 1] + d[1], coords[3 * i + 2] + d[2]));
    }
  cmap_free(&m);
}

/* SparseConv3d::forward (trellis2_sparse.rs:197-243): out[i, o] = bias[o] +
 * sum_k sum_c W[k][o][c] * x[nbr[i][k], c], missing neighbours contribute
 * zero; W is the [27, Cout, Cin] kernel. Sums in double, one rounding to f32;
 * abs_sum (optional) receives sum |W x|. */
typedef struct {
  const float *x, *w, *bias;
  const int32_t *nbr;
  int64_t cin, cout;
  float *out, *abs_sum;
} conv_ctx;

static void conv_rows(const void *p, int64_t r0, int64_t r1) {
  const conv_ctx *c = (const conv_ctx *)p;
  for (int64_t i = r0; i < r1; ++i)
    for (int64_t o = 0; o < c->cout; ++o) {
      double acc = c->bias ? (double)c->bias[o] : 0.0, aacc = 0.0;
      for (int k = 0; k < 27; ++k) {
        const int32_t s = c->nbr[i * 27 + k];
        if (s < 0) continue;
        const float *xr = c->x + (int64_t)s * c->cin, *wr = c->w + ((int64_t)k * c->cout + o) * c->cin;
        for (int64_t ch = 0; ch < c->cin; ++ch) {
          const double pr = (double)wr[ch] * (double)xr[ch];
          acc += pr;
          aacc += fabs(pr);
        }
      }
      c->out[i * c->cout + o] = (float)acc;
      if (c->abs_sum) c->abs_sum[i * c->cout + o] = (float)aacc;
    }
}

void or_sparse_conv3d(const float *x, int64_t n, int64_t cin, const int32_t *nbr, const float *w, const float *bias,
                      int64_t cout, float *out, float *abs_sum) {
  conv_ctx c = {x, w, bias, nbr, cin, cout, out, abs_sum};
  parallel_rows(n, conv_rows, &c);
}

/* channel_to_spatial (trellis2_sparse.rs:269-338): leaf = logits > 0 per
 * parent; children in parent order, ascending subidx = dx + 2 dy + 4 dz; child
 * coord = 2 parent + (dx, dy, dz); child features = row parent * 8 + subidx of
 * feats viewed as [N * 8, C / 8]. Returns the child count M; out_coords
 * [M, 3], out_feats [M, C / 8], src_rows [M] (optional), sub [N, 8] (1 / 0). */
int64_t or_channel_to_spatial(const int32_t *coords, int64_t n, const float *feats, int64_t c, const float *logits,
                              int32_t *out_coords, float *out_feats, int32_t *src_rows, float *sub) {
  const int64_t cc = c / 8;
  int64_t m = 0;
  for (int64_t p = 0; p < n; ++p)
    for (int s = 0; s < 8; ++s) {
      const int leaf = logits[p * 8 + s] > 0.0f;
      if (sub) sub[p * 8 + s] = leaf ? 1.0f : 0.0f;
      if (!leaf) continue;
      out_coords[3 * m] = coords[3 * p] * 2 + (s % 2);
      out_coords[3 * m + 1] = coords[3 * p + 1] * 2 + (s / 2) % 2;
      out_coords[3 * m + 2] = coords[3 * p + 2] * 2 + s / 4;
      memcpy(out_feats + m * cc, feats + (p * 8 + s) * cc, sizeof(float) * (size_t)cc);
      if (src_rows) src_rows[m] = (int32_t)(p * 8 + s);
      ++m;
    }
  return m;
}
