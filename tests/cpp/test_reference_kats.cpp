// The reference's own known-answer tests for this path, restated against the
// C++ mirror (candle-3d_amd/host/lux3d_candle.hpp) and run on the GPU:
//   tests/trellis2_blocks.rs:43-171, 205-225   (crates/lux3d-core)
//   src/runtime/trellis2_dino.rs:516-644        (DINOv3 RoPE unit tests)
// plus the reference's error behaviour for the same functions and a few
// closed-form checks of the other mirrored ops.
//
// Usage: test_reference_kats [--cpu]
//   --cpu runs only the checks that fail before any device work (argument
//   validation), for a machine without a GPU. Exit status 0 when all pass.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "lux3d_candle.hpp"

using namespace lux3d::candle;

namespace {

int g_failures = 0;

#define CHECK(cond)                                                                    \
  do {                                                                                 \
    if (!(cond)) {                                                                     \
      std::printf("    CHECK failed at %s:%d: %s\n", __FILE__, __LINE__, #cond);       \
      ++g_failures;                                                                    \
      return;                                                                          \
    }                                                                                  \
  } while (0)

#define CHECK_NEAR(a, b, tol)                                                          \
  do {                                                                                 \
    const double a_ = (a), b_ = (b);                                                   \
    if (!(std::fabs(a_ - b_) < (tol))) {                                               \
      std::printf("    CHECK_NEAR failed at %s:%d: %s = %.9g, %s = %.9g (tol %g)\n",   \
                  __FILE__, __LINE__, #a, a_, #b, b_, (double)(tol));                 \
      ++g_failures;                                                                    \
      return;                                                                          \
    }                                                                                  \
  } while (0)

// The reference bails with these messages; the mirror throws Error with them.
template <typename F>
bool throws_with(F &&f, const char *needle) {
  try {
    f();
  } catch (const Error &e) {
    if (std::strstr(e.what(), needle)) return true;
    std::printf("    threw a different message: %s\n", e.what());
    return false;
  }
  return false;
}

std::vector<float> iota_f(size_t n, float start, float step) {
  std::vector<float> v(n);
  for (size_t i = 0; i < n; ++i) v[i] = start + step * (float)i;
  return v;
}

// ---------------------------------------------------------------------------
// tests/trellis2_blocks.rs
// ---------------------------------------------------------------------------

// rope_tables_match_reference_formula (:43-74): head_dim 12 -> freq_dim 2 per
// axis, freqs = [1, 10000^-0.5], axis-major angles, pad pair at angle 0.
void rope_tables_match_reference_formula(const Device &dev) {
  Trellis2Rope3d rope(12);
  const std::vector<int64_t> coords{1, 0, 0, 0, 1, 0};
  auto [cos, sin] = rope.cos_sin(coords, dev);
  CHECK((cos.dims() == Shape{2, 6}));
  const std::vector<float> c = cos.to_vec_f32(), s = sin.to_vec_f32();
  const float freq2 = 1.0f / std::pow(10000.0f, 0.5f);
  for (int token = 0; token < 2; ++token) {
    const int64_t *cd = &coords[token * 3];
    const float angles[6] = {(float)cd[0] * 1.0f, (float)cd[0] * freq2, (float)cd[1] * 1.0f,
                             (float)cd[1] * freq2, (float)cd[2] * 1.0f, (float)cd[2] * freq2};
    for (int j = 0; j < 6; ++j) {
      CHECK_NEAR(c[token * 6 + j], std::cos(angles[j]), 1e-6);
      CHECK_NEAR(s[token * 6 + j], std::sin(angles[j]), 1e-6);
    }
  }
}

// rope_apply_matches_complex_product_and_preserves_norm (:79-111).
void rope_apply_matches_complex_product_and_preserves_norm(const Device &dev) {
  Trellis2Rope3d rope(12);
  auto [cos, sin] = rope.cos_sin({1, 0, 0}, dev);
  const std::vector<float> x{1.0f, 0.0f, 2.0f, 3.0f, 5.0f, 0.0f, 7.0f, 1.0f, 0.0f, 2.0f, 4.0f, 4.0f};
  const Tensor xs = Tensor::from_f32(x, {1, 1, 1, 12}, DType::F32, dev);
  const Tensor out_t = rope.apply(xs, cos, sin);
  CHECK((out_t.dims() == Shape{1, 1, 1, 12}));
  const std::vector<float> out = out_t.to_vec_f32();
  const float freq2 = 1.0f / std::pow(10000.0f, 0.5f);
  const float phases[3][2] = {{1.0f, 1.0f}, {freq2, freq2}, {0.0f, 0.0f}};
  for (int pair = 0; pair < 6; ++pair) {
    float ac = 1.0f, as = 0.0f;  // z coordinate zero + pad pair: angle 0
    if (pair < 2) {
      ac = std::cos(phases[pair][0]);
      as = std::sin(phases[pair][1]);
    }
    const float re = x[2 * pair], im = x[2 * pair + 1];
    CHECK_NEAR(out[2 * pair], re * ac - im * as, 1e-5);
    CHECK_NEAR(out[2 * pair + 1], re * as + im * ac, 1e-5);
  }
  float e_in = 0.f, e_out = 0.f;
  for (int i = 0; i < 12; ++i) {
    e_in += x[i] * x[i];
    e_out += out[i] * out[i];
  }
  CHECK_NEAR(e_in, e_out, 1e-4);
}

// qk_rms_norm_matches_reference (:126-153).
void qk_rms_norm_matches_reference(const Device &dev) {
  const Tensor xs = Tensor::from_f32({3.0f, 4.0f, 0.0f, 0.0f}, {1, 1, 1, 4}, DType::F32, dev);
  const float gammas[2] = {1.0f, 2.0f};
  const float want[2][4] = {{0.6f * 2.0f, 0.8f * 2.0f, 0.0f, 0.0f}, {2.4f, 3.2f, 0.0f, 0.0f}};
  for (int g = 0; g < 2; ++g) {
    Trellis2QkRmsNorm norm(Tensor::from_f32(std::vector<float>(4, gammas[g]), {1, 4}, DType::F32, dev));
    const std::vector<float> out = norm.forward(xs).to_vec_f32();
    for (int i = 0; i < 4; ++i) CHECK_NEAR(out[i], want[g][i], 1e-6);
  }
}

// timestep_embedding_matches_reference (:157-171).
void timestep_embedding_matches_reference(const Device &dev) {
  const Tensor emb = timestep_embedding(500.0f, 4, dev);
  CHECK((emb.dims() == Shape{4}));
  const std::vector<float> v = emb.to_vec_f32();
  const float freq1 = (float)std::exp(-std::log(10000.0) / 2.0);
  const float expected[4] = {std::cos(500.0f), std::cos(500.0f * freq1), std::sin(500.0f), std::sin(500.0f * freq1)};
  for (int i = 0; i < 4; ++i) CHECK_NEAR(v[i], expected[i], 1e-5);
}

// ada_ln_modulation_chunks_in_reference_order (:205-225).
void ada_ln_modulation_chunks_in_reference_order(const Device &dev) {
  const Tensor mod_vec = Tensor::from_f32(iota_f(12, 1.0f, 1.0f), {1, 12}, DType::F32, dev);
  const std::array<Tensor, 6> chunks = chunk_modulation(mod_vec);
  for (int i = 0; i < 6; ++i) {
    CHECK((chunks[i].dims() == Shape{1, 1, 2}));
    const std::vector<float> v = chunks[i].to_vec_f32();
    CHECK(v[0] == (float)(2 * i + 1) && v[1] == (float)(2 * i + 2));
  }
}

// The sparse block's gated residual + MLP modulate (trellis2_blocks.rs:708-713)
// in one launch, on exact small-integer inputs: gate 0.5 with h = 2 adds 1 to
// every element of x; a row [a, a+1, ..., a+7] then normalises to the
// standard scores of 0..7, so y = z * (1 + scale) + shift with z known in
// closed form. Without a gate (the dense block's cross-attention add,
// :637-642) x_out = x + h exactly.
void gated_residual_modulate_closed_form(const Device &dev) {
  std::vector<float> xv(2 * 8), hv(2 * 8, 2.0f);
  for (int r = 0; r < 2; ++r)
    for (int c = 0; c < 8; ++c) xv[r * 8 + c] = (float)(10 * r + c);
  const Tensor x = Tensor::from_f32(xv, {2, 8}, DType::F32, dev);
  const Tensor h = Tensor::from_f32(hv, {2, 8}, DType::F32, dev);
  const Tensor gate = Tensor::from_f32(std::vector<float>(8, 0.5f), {1, 8}, DType::F32, dev);
  Modulation next{Tensor::from_f32(std::vector<float>(8, 0.25f), {1, 8}, DType::F32, dev),
                  Tensor::from_f32(std::vector<float>(8, 1.0f), {1, 8}, DType::F32, dev)};
  auto [xo, y] = gated_residual_adaln_modulate(x, h, gate, std::nullopt, next, 0.0);
  const std::vector<float> xs = xo.to_vec_f32(), ys = y.to_vec_f32();
  const double sd = std::sqrt(5.25);  // population std of 0..7
  for (int r = 0; r < 2; ++r)
    for (int c = 0; c < 8; ++c) {
      CHECK(xs[r * 8 + c] == xv[r * 8 + c] + 1.0f);
      CHECK_NEAR(ys[r * 8 + c], (c - 3.5) / sd * 2.0 + 0.25, 2e-6);
    }
  auto [xo2, y2] = gated_residual_adaln_modulate(x, h, std::nullopt, std::nullopt, next, 0.0);
  const std::vector<float> xs2 = xo2.to_vec_f32();
  for (size_t i = 0; i < xs2.size(); ++i) CHECK(xs2[i] == xv[i] + 2.0f);
  Modulation gated = next;
  gated.gate = gate;
  CHECK(throws_with([&] { gated_residual_adaln_modulate(x, h, gate, std::nullopt, gated, 0.0); }, "no output gate"));
}

// ---------------------------------------------------------------------------
// src/runtime/trellis2_dino.rs tests
// ---------------------------------------------------------------------------

// rope_tables_match_hand_computed_cos_sin (:516-565): head_dim 8, theta 100,
// 2x2 grid -> inv_freq [1, 0.1], [y freqs, x freqs] tiled twice.
void dinov3_rope_tables_match_hand_computed_cos_sin(const Device &dev) {
  const size_t grid = 2;
  auto [cos, sin] = dinov3_rope_cos_sin(8, 100.0f, grid, grid, dev);
  CHECK((cos.dims() == Shape{4, 8}) && (sin.dims() == Shape{4, 8}));
  const std::vector<float> c = cos.to_vec_f32(), s = sin.to_vec_f32();
  const float inv_freq[2] = {1.0f, 1.0f / std::pow(100.0f, 0.5f)};
  const float two_pi = (float)(M_PI * 2.0);
  int row = 0;
  for (size_t y = 0; y < grid; ++y) {
    const float cy = 2.0f * (((float)y + 0.5f) / (float)grid) - 1.0f;
    for (size_t x = 0; x < grid; ++x, ++row) {
      const float cx = 2.0f * (((float)x + 0.5f) / (float)grid) - 1.0f;
      std::vector<float> half;
      for (float coord : {cy, cx})
        for (float f : inv_freq) half.push_back(two_pi * coord * f);
      for (int j = 0; j < 8; ++j) {
        const float want = half[j % 4];
        CHECK_NEAR(c[row * 8 + j], std::cos(want), 1e-6);
        CHECK_NEAR(s[row * 8 + j], std::sin(want), 1e-6);
      }
    }
  }
}

// rope_applies_to_patches_only_and_prefix_tokens_pass_through (:583-643).
void dinov3_rope_applies_to_patches_only(const Device &dev) {
  const size_t head_dim = 8, num_prefix = 3, patches = 2, seq = num_prefix + patches;
  std::vector<float> qv(seq * head_dim);
  for (size_t i = 0; i < qv.size(); ++i) qv[i] = 0.1f * ((float)i + 1.0f);
  const Tensor q = Tensor::from_f32(qv, {1, 1, (int64_t)seq, (int64_t)head_dim}, DType::F32, dev);
  const Tensor k = Tensor::from_f32(qv, {1, 1, (int64_t)seq, (int64_t)head_dim}, DType::F32, dev);
  const float c = 0.5f, s = std::sqrt(0.5f);
  const Tensor cos = Tensor::from_f32(std::vector<float>(patches * head_dim, c),
                                      {(int64_t)patches, (int64_t)head_dim}, DType::F32, dev);
  const Tensor sin = Tensor::from_f32(std::vector<float>(patches * head_dim, s),
                                      {(int64_t)patches, (int64_t)head_dim}, DType::F32, dev);
  auto [q_rot, k_rot] = apply_rotary_to_patches(q, k, cos, sin, num_prefix);
  const std::vector<float> r = q_rot.to_vec_f32();
  for (size_t token = 0; token < num_prefix; ++token)
    for (size_t d = 0; d < head_dim; ++d) CHECK_NEAR(r[token * head_dim + d], 0.1f * ((float)(token * head_dim + d) + 1.0f), 1e-6);
  const float base = 0.1f * (float)(num_prefix * head_dim + 1);
  std::vector<float> qp(head_dim);
  for (size_t i = 0; i < head_dim; ++i) qp[i] = base + 0.1f * (float)i;
  for (size_t d = 0; d < head_dim; ++d) {
    const float partner = d < head_dim / 2 ? -qp[d + head_dim / 2] : qp[d - head_dim / 2];
    CHECK_NEAR(r[num_prefix * head_dim + d], qp[d] * c + partner * s, 1e-5);
  }
}

// ---------------------------------------------------------------------------
// Closed-form checks of the other mirrored ops (small hand-checkable inputs)
// ---------------------------------------------------------------------------

// VGGT block residual: h = x + a*gamma exactly (f32, one rounding each), y = LN(h).
void residual_layer_norm_closed_form(const Device &dev) {
  const int64_t d = 8;
  const std::vector<float> x = iota_f(d, -1.0f, 0.25f), a = iota_f(d, 2.0f, -0.5f), g(d, 0.5f);
  const LayerNorm norm(Tensor::from_f32(std::vector<float>(d, 1.0f), {d}, DType::F32, dev),
                       Tensor::from_f32(std::vector<float>(d, 0.0f), {d}, DType::F32, dev), 1e-5);
  const LayerScale ls(Tensor::from_f32(g, {d}, DType::F32, dev));
  auto [h, y] = residual_layer_norm(Tensor::from_f32(x, {1, d}, DType::F32, dev),
                                    Tensor::from_f32(a, {1, d}, DType::F32, dev), &ls, norm);
  const std::vector<float> hv = h.to_vec_f32(), yv = y.to_vec_f32();
  double mean = 0, var = 0;
  for (int64_t i = 0; i < d; ++i) {
    CHECK(hv[i] == x[i] + a[i] * 0.5f);
    mean += hv[i];
  }
  mean /= d;
  for (int64_t i = 0; i < d; ++i) var += (hv[i] - mean) * (hv[i] - mean);
  var /= d;
  for (int64_t i = 0; i < d; ++i) CHECK_NEAR(yv[i], (hv[i] - mean) / std::sqrt(var + 1e-5), 1e-5);
}

// VGGT QK LN + 2D RoPE on a strided qkv view: position (0, 0) is the
// identity rotation, so the special tokens equal the plain LayerNorm.
void vggt_qk_layernorm_rope_specials_are_plain_layernorm(const Device &dev) {
  const int64_t B = 1, N = 3, H = 2, D = 8;
  std::vector<float> qkv((size_t)(B * N * 3 * H * D));
  for (size_t i = 0; i < qkv.size(); ++i) qkv[i] = std::sin(0.37f * (float)i) * 2.0f;
  const Tensor t = Tensor::from_f32(qkv, {B, N, 3, H, D}, DType::F32, dev);
  const Tensor perm = t.permute({2, 0, 3, 1, 4});  // [3, B, H, N, D]
  const Tensor q = perm.get(0), k = perm.get(1);
  const LayerNorm ln(Tensor::from_f32(std::vector<float>(D, 1.0f), {D}, DType::F32, dev),
                     Tensor::from_f32(std::vector<float>(D, 0.0f), {D}, DType::F32, dev), 1e-5);
  const Tensor pos = Tensor::from_i32({0, 0, 1, 2, 2, 1}, {B, N, 2}, dev);
  auto [qo, ko] = qk_layernorm_rope2d(q, k, ln, ln, pos, 100.0f);
  const RopeEmbeddings emb = Rope2d(100.0f).embeddings(pos, (size_t)D);
  const Tensor q_tab = apply_layernorm_rope(q, ln, emb);
  const std::vector<float> a = qo.to_vec_f32(), b = q_tab.to_vec_f32();
  CHECK(ko.dims() == qo.dims());
  // positions and tables paths agree
  for (size_t i = 0; i < a.size(); ++i) CHECK_NEAR(a[i], b[i], 1e-5);
  // token 0 of every head is the plain LayerNorm of its row
  const std::vector<float> qin = q.to_vec_f32();
  for (int64_t h = 0; h < H; ++h) {
    const float *row = &qin[(size_t)((h * N + 0) * D)];
    double mean = 0, var = 0;
    for (int64_t j = 0; j < D; ++j) mean += row[j];
    mean /= D;
    for (int64_t j = 0; j < D; ++j) var += (row[j] - mean) * (row[j] - mean);
    var /= D;
    for (int64_t j = 0; j < D; ++j) CHECK_NEAR(a[(size_t)((h * N) * D + j)], (row[j] - mean) / std::sqrt(var + 1e-5), 1e-5);
  }
}

// VGGT attention (vggt.rs:170-183) with q's LayerNorm + RoPE fused into the
// attention kernel equals apply_layernorm_rope followed by
// exact_query_chunked_sdpa bit for bit.
void vggt_attention_fused_equals_two_calls(const Device &dev) {
  const int64_t B = 2, N = 300, H = 3, D = 64;
  std::vector<float> qkv((size_t)(B * N * 3 * H * D));
  for (size_t i = 0; i < qkv.size(); ++i) qkv[i] = std::sin(0.013f * (float)i) * 2.0f + 0.3f;
  const Tensor perm = Tensor::from_f32(qkv, {B, N, 3, H, D}, DType::BF16, dev).permute({2, 0, 3, 1, 4});
  std::vector<float> w(D), bias(D);
  for (int64_t j = 0; j < D; ++j) w[j] = 1.0f + 0.01f * (float)(j % 7), bias[j] = 0.02f * (float)(j % 5) - 0.04f;
  const LayerNorm ln(Tensor::from_f32(w, {D}, DType::F32, dev), Tensor::from_f32(bias, {D}, DType::F32, dev), 1e-6);
  std::vector<int32_t> pos((size_t)(B * N * 2));
  for (int64_t i = 0; i < B * N; ++i) pos[2 * i] = (int32_t)((i % N) / 17), pos[2 * i + 1] = (int32_t)((i % N) % 17);
  const RopeEmbeddings emb = Rope2d(100.0f).embeddings(Tensor::from_i32(pos, {B, N, 2}, dev), (size_t)D);
  const Tensor k = apply_layernorm_rope(perm.get(1), ln, emb);
  const Tensor fused = sdpa_layernorm_rope(perm.get(0), ln, emb, k, perm.get(2), 0.125f);
  const Tensor two = exact_query_chunked_sdpa(apply_layernorm_rope(perm.get(0), ln, emb), k, perm.get(2), 0.125f);
  CHECK(fused.to_vec_u16() == two.to_vec_u16());
}

// TripoSG (triposg_dit.rs:446-455), TRELLIS.2 (trellis2_blocks.rs:417-436)
// and DINOv3 (trellis2_dino.rs:385-393) attention with q's head norm /
// rotation fused into the attention kernel equal the head op followed by the
// attention bit for bit.
void model_attentions_fused_equal_two_calls(const Device &dev) {
  const int64_t B = 1, N = 200, H = 2, D = 128;
  std::vector<float> x((size_t)(B * N * H * 3 * D));
  for (size_t i = 0; i < x.size(); ++i) x[i] = std::sin(0.017f * (float)i) * 1.5f + 0.2f;
  std::vector<float> w(D), g(H * D);
  for (int64_t j = 0; j < D; ++j) w[j] = 1.0f + 0.01f * (float)(j % 9);
  for (int64_t j = 0; j < H * D; ++j) g[j] = 1.0f - 0.005f * (float)(j % 11);
  // TripoSG: per-head thirds of cat([q, k, v]) as [B, L, H, 3D], heads-first views
  const Tensor qkv = Tensor::from_f32(x, {B, N, H, 3 * D}, DType::BF16, dev);
  const Tensor q = qkv.narrow(3, 0, D).transpose(1, 2), k = qkv.narrow(3, D, D).transpose(1, 2);
  const Tensor v = qkv.narrow(3, 2 * D, D).transpose(1, 2);
  const Tensor qw = Tensor::from_f32(w, {D}, DType::F32, dev);
  const Tensor kn = rms_norm_heads(k, qw);
  const Tensor f1 = sdpa_rms_norm_heads(q, qw, kn, v, 0.088f);
  const Tensor t1 = exact_query_chunked_sdpa(rms_norm_heads(q, qw), kn, v, 0.088f);
  CHECK(f1.to_vec_u16() == t1.to_vec_u16());
  // TRELLIS.2: [B, L, H, D] buffers, L2 norm + 3D RoPE from voxel coords
  const Tensor buf = Tensor::from_f32(x, {B, N, 3, H, D}, DType::BF16, dev);
  std::vector<int64_t> coords((size_t)(N * 3));
  for (int64_t i = 0; i < N * 3; ++i) coords[(size_t)i] = (i * 7) % 23;
  const Trellis2Rope3d rope((size_t)D);
  auto [cos, sin] = rope.cos_sin(coords, dev);
  const Tensor gamma = Tensor::from_f32(g, {H, D}, DType::F32, dev);
  const Tensor bq = buf.permute({2, 0, 1, 3, 4}).get(0), bk = buf.permute({2, 0, 1, 3, 4}).get(1);
  const Tensor bv = buf.permute({2, 0, 1, 3, 4}).get(2);  // [B, L, H, D] views
  // the two launches: the L2 norm + rotation head op (one rounding), then attention
  const Tensor qn = Tensor::empty(bq.dims(), DType::BF16, dev), kr = Tensor::empty(bk.dims(), DType::BF16, dev);
  const lux3d_tensor_t dbq = bq.desc(), dbk = bk.desc(), dg = gamma.desc(), dcos = cos.desc(), dsin = sin.desc();
  const lux3d_tensor_t dqn = qn.desc(), dkr = kr.desc();
  CHECK(lux3d_qk_l2norm_rope3d(&dbq, &dg, &dbk, &dg, &dcos, &dsin, nullptr, 0.f, &dqn, &dkr, dev.stream()) == 0);
  const Tensor f2 = sdpa_l2norm_rope3d(bq.transpose(1, 2), gamma, cos, sin, kr.transpose(1, 2), bv.transpose(1, 2),
                                       0.088f);
  const Tensor t2 = exact_query_chunked_sdpa(qn.transpose(1, 2), kr.transpose(1, 2), bv.transpose(1, 2), 0.088f);
  CHECK(f2.to_vec_u16() == t2.to_vec_u16());
  // DINOv3 (f32, the reference's precision): 4 + 14 x 14 tokens, 4 prefix
  const int64_t S = 4 + 14 * 14, DH = 64;
  std::vector<float> xd((size_t)(3 * S * DH * H));
  for (size_t i = 0; i < xd.size(); ++i) xd[i] = std::cos(0.011f * (float)i);
  const Tensor dq = Tensor::from_f32(xd, {3, B, S, H, DH}, DType::F32, dev);
  auto [dc, ds] = dinov3_rope_cos_sin((size_t)DH, 100.0f, 14, 14, dev);
  const Tensor q3 = dq.get(0).transpose(1, 2), k3 = dq.get(1).transpose(1, 2), v3 = dq.get(2).transpose(1, 2);
  auto [qr, kr3] = apply_rotary_to_patches(q3, k3, dc, ds, 4);
  const Tensor f3 = sdpa_dinov3_rope(q3, dc, ds, 4, kr3, v3, 0.125f);
  const Tensor t3 = exact_sdpa_heads(qr, kr3, v3, 0.125f);
  CHECK(f3.to_vec_f32() == t3.to_vec_f32());
}

// Q8_0: w = f16(d) * int8(q), exact.
void dequantize_q8_0_exact(const Device &dev) {
  std::vector<uint8_t> blk(34);
  const uint16_t d_half = 0x3800;  // 0.5
  std::memcpy(blk.data(), &d_half, 2);
  for (int i = 0; i < 32; ++i) blk[2 + i] = (uint8_t)(int8_t)(i - 16);
  const Tensor w = dequantize_q8_0(Tensor::from_u8(blk, {34}, dev), {32}, DType::F32);
  const std::vector<float> v = w.to_vec_f32();
  for (int i = 0; i < 32; ++i) CHECK(v[i] == 0.5f * (float)(i - 16));
}

// Quantized linear: W = d * q with d = 0.5 (f16 0x3800) and q[n][k] = (n + k) % 7 - 3;
// y = x @ W^T + bias, checked against a double-precision host sum (every
// product here is exact in bf16 x bf16 and the sums are small integers / 2).
void q8_0_linear_closed_form(const Device &dev) {
  const int64_t m = 3, k = 64, n = 5;
  std::vector<uint8_t> blocks;
  for (int64_t r = 0; r < n; ++r)
    for (int64_t b = 0; b < k / 32; ++b) {
      blocks.push_back(0x00);
      blocks.push_back(0x38);
      for (int j = 0; j < 32; ++j) blocks.push_back((uint8_t)(int8_t)((r + b * 32 + j) % 7 - 3));
    }
  const QMatMul mm = QMatMul::from_q8_0(Tensor::from_u8(blocks, {(int64_t)blocks.size()}, dev), n, k);
  std::vector<float> x(m * k), bias(n);
  for (int64_t i = 0; i < m * k; ++i) x[i] = (float)((i * 5) % 9 - 4);
  for (int64_t j = 0; j < n; ++j) bias[j] = 0.25f * (float)j;
  const Tensor y = mm.forward(Tensor::from_f32(x, {m, k}, DType::BF16, dev),
                              Tensor::from_f32(bias, {n}, DType::F32, dev), DType::F32);
  CHECK((y.dims() == Shape{m, n}));
  const std::vector<float> v = y.to_vec_f32();
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      double acc = bias[j];
      for (int64_t t = 0; t < k; ++t) acc += (double)x[i * k + t] * 0.5 * (double)((j + t) % 7 - 3);
      CHECK(v[i * n + j] == (float)acc);
    }
}

// tests/trellis2_sparse.rs:471-623: exact self / cross attention (H = 2,
// head_dim 8, pattern_f32 inputs) against naive per-head softmax attention,
// max |diff| < 1e-5.
float pattern_f32(size_t index) { return ((float)(index % 23) - 11.0f) * 0.1f; }

std::vector<float> naive_attention(const std::vector<float> &q, const std::vector<float> &k,
                                   const std::vector<float> &v, size_t heads, size_t tokens, size_t kv_tokens,
                                   size_t hd) {
  const float scale = 1.0f / std::sqrt((float)hd);
  std::vector<float> out(heads * tokens * hd, 0.0f);
  for (size_t h = 0; h < heads; ++h)
    for (size_t t = 0; t < tokens; ++t) {
      std::vector<float> sc(kv_tokens);
      float mx = -INFINITY;
      for (size_t j = 0; j < kv_tokens; ++j) {
        float dot = 0.0f;
        for (size_t d = 0; d < hd; ++d) dot += q[(h * tokens + t) * hd + d] * k[(h * kv_tokens + j) * hd + d];
        sc[j] = dot * scale;
        mx = std::max(mx, sc[j]);
      }
      float sum = 0.0f;
      for (float &x : sc) {
        x = std::exp(x - mx);
        sum += x;
      }
      for (size_t j = 0; j < kv_tokens; ++j)
        for (size_t d = 0; d < hd; ++d) out[(h * tokens + t) * hd + d] += sc[j] / sum * v[(h * kv_tokens + j) * hd + d];
    }
  return out;
}

void sparse_attention_matches_naive(const Device &dev) {
  const size_t H = 2, HD = 8;
  const size_t cases[2][5] = {{17, 17, 1, 2, 3}, {9, 7, 4, 5, 6}};
  for (const auto &c : cases) {
    const size_t T = c[0], TKV = c[1];
    auto pat = [&](size_t n, size_t seed) {
      std::vector<float> x(H * n * HD);
      for (size_t i = 0; i < x.size(); ++i) x[i] = pattern_f32(i * 7 + seed * 3);
      return x;
    };
    const std::vector<float> q = pat(T, c[2]), k = pat(TKV, c[3]), v = pat(TKV, c[4]);
    const Tensor out = exact_query_chunked_sdpa(Tensor::from_f32(q, {1, (int64_t)H, (int64_t)T, (int64_t)HD}, DType::F32, dev),
                                                Tensor::from_f32(k, {1, (int64_t)H, (int64_t)TKV, (int64_t)HD}, DType::F32, dev),
                                                Tensor::from_f32(v, {1, (int64_t)H, (int64_t)TKV, (int64_t)HD}, DType::F32, dev),
                                                1.0f / std::sqrt((float)HD), 5);
    const std::vector<float> got = out.to_vec_f32(), want = naive_attention(q, k, v, H, T, TKV, HD);
    float md = 0.0f;
    for (size_t i = 0; i < got.size(); ++i) md = std::max(md, std::fabs(got[i] - want[i]));
    CHECK(md < 1e-5f);
  }
}

// exact_sdpa_heads (attention_math.rs:244-259) on bf16 q, k, v: f32
// arithmetic, the result narrowed to bf16 once. Against the naive f32
// attention of the same (bf16-valued) inputs, each output is within one half
// bf16 unit of the f32 value plus the f32 error of the naive sums. D 64 with
// 16-byte rows runs the matrix-core kernel.
void exact_sdpa_heads_bf16_is_f32_arithmetic(const Device &dev) {
  const size_t H = 2, T = 70, TKV = 130, HD = 64;
  auto pat = [&](size_t n, size_t seed) {
    std::vector<float> x(H * n * HD);
    for (size_t i = 0; i < x.size(); ++i) x[i] = pattern_f32(i * 7 + seed * 3) * 3.0f;
    return x;
  };
  const Tensor q = Tensor::from_f32(pat(T, 1), {1, (int64_t)H, (int64_t)T, (int64_t)HD}, DType::BF16, dev);
  const Tensor k = Tensor::from_f32(pat(TKV, 2), {1, (int64_t)H, (int64_t)TKV, (int64_t)HD}, DType::BF16, dev);
  const Tensor v = Tensor::from_f32(pat(TKV, 3), {1, (int64_t)H, (int64_t)TKV, (int64_t)HD}, DType::BF16, dev);
  const Tensor out = exact_sdpa_heads(q, k, v, 1.0f / std::sqrt((float)HD));
  CHECK(out.dtype() == DType::BF16);
  const std::vector<float> got = out.to_vec_f32();
  const std::vector<float> want = naive_attention(q.to_vec_f32(), k.to_vec_f32(), v.to_vec_f32(), H, T, TKV, HD);
  size_t bad = 0;
  for (size_t i = 0; i < got.size(); ++i)
    if (std::fabs(got[i] - want[i]) > std::ldexp(std::fabs(want[i]), -8) + 1e-5f) ++bad;
  CHECK(bad == 0);
}

// tests/trellis2_sparse.rs: kernel offsets, the coordinate map, the sparse
// conv against a dense loop reference, identity / shift kernels, the loader
// transpose and the C2S order.
void kernel_offset_deltas_cover_the_3x3x3_kernel(const Device &) {
  CHECK((kernel_offset_delta(0) == Coord{-1, -1, -1}));
  CHECK((kernel_offset_delta(13) == Coord{0, 0, 0}));
  CHECK((kernel_offset_delta(26) == Coord{1, 1, 1}));
  CHECK((kernel_offset_delta(5) == Coord{-1, 0, 1}));
  for (size_t k = 0; k < 27; ++k) {
    const Coord d = kernel_offset_delta(k);
    CHECK((size_t)((d[0] + 1) * 9 + (d[1] + 1) * 3 + (d[2] + 1)) == k);
  }
}

void coord_map_builds_and_looks_up(const Device &dev) {
  const std::vector<Coord> coords = {{0, 0, 0}, {1, 0, 3}, {7, 2, 5}};
  const std::vector<int32_t> nbr = sparse_neighbors(coords, dev).to_vec_i32();
  for (int i = 0; i < 3; ++i) CHECK(nbr[i * 27 + 13] == i);
  int found = 0;
  for (int32_t v : nbr) found += v >= 0;
  CHECK(found == 3);
}

std::vector<Coord> grid_with_holes() {
  std::vector<Coord> c;
  for (int x = 0; x < 4; ++x)
    for (int y = 0; y < 4; ++y)
      for (int z = 0; z < 4; ++z)
        if ((x * 16 + y * 4 + z) % 5 != 0) c.push_back({x, y, z});
  return c;
}

void sparse_conv_matches_dense_reference(const Device &dev) {
  const size_t CIN = 3, COUT = 5;
  const std::vector<Coord> coords = grid_with_holes();
  CHECK(coords.size() == 64 - 13);
  std::vector<float> feats(coords.size() * CIN), ck(COUT * 27 * CIN), bias(COUT);
  for (size_t i = 0; i < coords.size(); ++i)
    for (size_t c = 0; c < CIN; ++c) feats[i * CIN + c] = pattern_f32(i * 13 + c * 7);
  for (size_t o = 0; o < COUT; ++o)
    for (size_t k = 0; k < 27; ++k)
      for (size_t c = 0; c < CIN; ++c) ck[(o * 27 + k) * CIN + c] = pattern_f32(o * 31 + k * 5 + c * 3) * 0.5f;
  for (size_t o = 0; o < COUT; ++o) bias[o] = (float)((o * 3) % 7) * 0.02f - 0.06f;
  const SparseConv3d conv = SparseConv3d::load(Tensor::from_f32(ck, {(int64_t)COUT, 3, 3, 3, (int64_t)CIN}, DType::F32, dev),
                                               Tensor::from_f32(bias, {(int64_t)COUT}, DType::F32, dev), CIN, COUT);
  const std::vector<float> out =
      conv.forward(coords, Tensor::from_f32(feats, {(int64_t)coords.size(), (int64_t)CIN}, DType::F32, dev)).to_vec_f32();
  float md = 0.f;
  for (size_t i = 0; i < coords.size(); ++i)
    for (size_t o = 0; o < COUT; ++o) {
      float acc = bias[o];
      for (size_t k = 0; k < 27; ++k) {
        const Coord d = kernel_offset_delta(k);
        for (size_t j = 0; j < coords.size(); ++j)
          if (coords[j][0] == coords[i][0] + d[0] && coords[j][1] == coords[i][1] + d[1] &&
              coords[j][2] == coords[i][2] + d[2])
            for (size_t c = 0; c < CIN; ++c) acc += ck[(o * 27 + k) * CIN + c] * feats[j * CIN + c];
      }
      md = std::max(md, std::fabs(out[i * COUT + o] - acc));
    }
  CHECK(md < 1e-4f);
}

void sparse_conv_hand_picked_kernels(const Device &dev) {
  const std::vector<Coord> coords = {{0, 0, 0}, {1, 0, 0}, {1, 1, 0}, {3, 0, 0}};
  std::vector<float> x(8);
  for (size_t i = 0; i < 8; ++i) x[i] = pattern_f32(i);
  const Tensor feats = Tensor::from_f32(x, {4, 2}, DType::F32, dev);
  for (int k : {13, 22}) {
    std::vector<float> w(2 * 27 * 2, 0.f);
    for (int c = 0; c < 2; ++c) w[(c * 27 + k) * 2 + c] = 1.f;
    const SparseConv3d conv = SparseConv3d::load(Tensor::from_f32(w, {2, 3, 3, 3, 2}, DType::F32, dev), std::nullopt, 2, 2);
    const std::vector<float> out = conv.forward(coords, feats).to_vec_f32();
    for (int i = 0; i < 4; ++i)
      for (int c = 0; c < 2; ++c) {
        const float want = k == 13 ? x[i * 2 + c] : (i == 0 ? x[2 + c] : 0.f);  // +x neighbour of row 0 is row 1
        CHECK(std::fabs(out[i * 2 + c] - want) < 1e-6f);
      }
  }
}

// The identity and +x shift kernels again with 16 channels, which takes the
// rulebook path (per-tap pair lists, tap-ordered accumulation).
void sparse_conv_rulebook_identity_and_shift(const Device &dev) {
  const int C = 16;
  const std::vector<Coord> coords = {{0, 0, 0}, {1, 0, 0}, {1, 1, 0}, {3, 0, 0}, {2, 0, 0}};
  std::vector<float> x(coords.size() * C);
  for (size_t i = 0; i < x.size(); ++i) x[i] = pattern_f32(i * 3);
  const Tensor feats = Tensor::from_f32(x, {(int64_t)coords.size(), C}, DType::F32, dev);
  for (int k : {13, 22}) {
    std::vector<float> w(C * 27 * C, 0.f);
    for (int c = 0; c < C; ++c) w[(c * 27 + k) * C + c] = 1.f;
    const SparseConv3d conv = SparseConv3d::load(Tensor::from_f32(w, {C, 3, 3, 3, C}, DType::F32, dev), std::nullopt, C, C);
    const std::vector<float> out = conv.forward(coords, feats).to_vec_f32();
    // +x neighbours: row 0 -> row 1, row 1 -> row 4, row 4 -> row 3
    const int plus_x[5] = {1, 4, -1, -1, 3};
    for (size_t i = 0; i < coords.size(); ++i)
      for (int c = 0; c < C; ++c) {
        const int src = k == 13 ? (int)i : plus_x[i];
        CHECK(out[i * C + c] == (src < 0 ? 0.f : x[src * C + c]));
      }
  }
}

void sparse_conv_loader_transposes_flex_gemm_layout(const Device &dev) {
  const int CIN = 2, COUT = 3;
  std::vector<float> v(COUT * 27 * CIN);
  for (size_t i = 0; i < v.size(); ++i) v[i] = ((float)i + 1.0f) / 100.0f;
  const SparseConv3d conv = SparseConv3d::load(Tensor::from_f32(v, {COUT, 3, 3, 3, CIN}, DType::F32, dev), std::nullopt, CIN, COUT);
  const std::vector<float> w27 = conv.weight27().to_vec_f32();
  for (int k = 0; k < 27; ++k)
    for (int o = 0; o < COUT; ++o)
      for (int c = 0; c < CIN; ++c) CHECK(w27[(k * COUT + o) * CIN + c] == v[(o * 27 + k) * CIN + c]);
}

void c2s_order_and_feature_selection(const Device &dev) {
  const std::vector<Coord> coords = {{0, 0, 0}, {1, 0, 0}, {0, 1, 1}};
  std::vector<float> f(48), lg(24, -1.f);
  for (int i = 0; i < 48; ++i) f[i] = (float)i / 10.0f;
  lg[0] = lg[3] = lg[5] = 1.f;  // parent 0: children 0, 3, 5
  lg[8 + 1] = 1.f;              // parent 1: child 1
  const Channel2SpatialOutput out = channel_to_spatial(coords, Tensor::from_f32(f, {3, 16}, DType::F32, dev),
                                                       Tensor::from_f32(lg, {3, 8}, DType::F32, dev));
  CHECK((out.coords == std::vector<Coord>{{0, 0, 0}, {1, 1, 0}, {1, 0, 1}, {3, 0, 0}}));
  const std::vector<float> sel = out.feats.to_vec_f32();
  const int rows[4] = {0, 3, 5, 9};
  CHECK(sel.size() == 8);
  for (int r = 0; r < 4; ++r)
    for (int c = 0; c < 2; ++c) CHECK(sel[r * 2 + c] == f[rows[r] * 2 + c]);
  const std::vector<float> sub = out.sub_binary.to_vec_f32();
  CHECK(sub.size() == 24 && sub[0] == 1.f && sub[1] == 0.f && sub[9] == 1.f);
}

// A GGUF container as the reference's quantizer lays it out
// (tests/golden/tiny_q8.gguf, written by tests/golden/make_gguf.py): the Q8_0
// weight becomes a QMatMul (VarBuilder::get_quantized + QMatMul::from_qtensor,
// nn_blocks.rs:107-150), the F16 bias is read through VarBuilder::get, and
// x @ W^T + b is exact for these small-integer values.
std::string g_fixture_dir;

void gguf_q8_linear_from_file(const Device &dev) {
  const GgufFile f = GgufFile::open(g_fixture_dir + "/tiny_q8.gguf");
  CHECK(f.metadata_string("lux3d.family") == std::optional<std::string>("trellis2"));
  CHECK(f.metadata_uint("lux3d.tensor_count") == std::optional<uint64_t>(3));
  CHECK(!f.metadata_string("lux3d.tensor_count"));
  const std::string wn = "blocks.0.mlp.fc1.weight", bn = "blocks.0.mlp.fc1.bias";
  const WeightInfo w = f.info(wn);
  CHECK((w.shape == Shape{8, 64}) && w.dtype == LUX3D_GGML_Q8_0 && w.nbytes == 8 * 2 * 34);
  // host decode of the blocks: d = f16 0.5, q int8
  const uint8_t *bytes = static_cast<const uint8_t *>(w.data);
  std::vector<double> wt(8 * 64);
  for (int r = 0; r < 8; ++r)
    for (int c = 0; c < 64; ++c) {
      const uint8_t *blk = bytes + (r * 2 + c / 32) * 34;
      CHECK(blk[0] == 0x00 && blk[1] == 0x38);
      wt[r * 64 + c] = 0.5 * (double)(int8_t)blk[2 + c % 32];
    }
  const std::vector<float> deq = f.get(wn, DType::F32, dev).to_vec_f32();
  for (int i = 0; i < 8 * 64; ++i) CHECK(deq[i] == (float)wt[i]);
  const QMatMul mm = f.get_qmatmul(wn, 8, 64, dev);
  const Tensor bias = f.get(bn, DType::F32, dev);
  std::vector<float> x(3 * 64);
  for (int i = 0; i < 3 * 64; ++i) x[i] = (float)((i * 11) % 7 - 3);
  const std::vector<float> y = mm.forward(Tensor::from_f32(x, {3, 64}, DType::BF16, dev), bias, DType::F32).to_vec_f32();
  for (int m = 0; m < 3; ++m)
    for (int r = 0; r < 8; ++r) {
      double acc = 0.25 * r - 1.0;
      for (int c = 0; c < 64; ++c) acc += (double)x[m * 64 + c] * wt[r * 64 + c];
      CHECK(y[m * 8 + r] == (float)acc);
    }
  const std::vector<float> nw = f.get(Shape{64}, "blocks.0.norm.weight", DType::F32, dev).to_vec_f32();
  for (int c = 0; c < 64; ++c) CHECK(nw[c] == 1.0f + (float)c / 64.0f);
  CHECK(throws_with([&] { f.get_qmatmul(wn, 64, 8, dev); }, "does not match expected (64, 8)"));
  CHECK(throws_with([&] { f.get(Shape{65}, "blocks.0.norm.weight", DType::F32, dev); }, "shape mismatch"));
  CHECK(throws_with([&] { f.get_qmatmul(bn, 8, 1, dev); }, "does not match expected"));
  CHECK(throws_with([&] { f.info("nope"); }, "cannot find tensor nope"));
}

// ---------------------------------------------------------------------------
// Error behaviour (the reference's bail! messages)
// ---------------------------------------------------------------------------

void errors_on_host(const Device &dev) {
  CHECK(throws_with([&] { Trellis2Rope3d(12).cos_sin({1, 2, 3, 4}, dev); },
                    "TRELLIS.2 RoPE coords must be [L, 3] flattened"));
  CHECK(throws_with([&] { Trellis2Rope3d(4).cos_sin({1, 2, 3}, dev); }, "is too small for 3-axis RoPE"));
  CHECK(throws_with([&] { Trellis2Rope3d(13).cos_sin({1, 2, 3}, dev); }, "must be divisible by 2"));
  CHECK(throws_with([&] { dinov3_rope_cos_sin(10, 100.0f, 2, 2, dev); }, "is not divisible by 4"));
  // Trellis2SlatDit::prepare's checks (trellis2_dit.rs:516-541), before any device work
  const Trellis2Rope3d rope128(128);
  CHECK(throws_with([&] { slat_prepare({2, 8}, 16, {{0, 0, 0}, {1, 2, 3}}, 64, rope128, dev); },
                    "SLAT DiT expects 16 token channels, got 8"));
  CHECK(throws_with([&] { slat_prepare({3, 8}, 8, {{0, 0, 0}, {1, 2, 3}}, 64, rope128, dev); },
                    "SLAT DiT coords/features mismatch: 2 coords vs 3 rows"));
  CHECK(throws_with([&] { slat_prepare({2, 8}, 8, {{0, 0, 0}, {1, 64, 3}}, 64, rope128, dev); },
                    "SLAT coord [1, 64, 3] outside the 0..64 grid"));
  CHECK(throws_with([&] { slat_prepare({1, 8}, 8, {{-1, 0, 0}}, 64, rope128, dev); }, "outside the 0..64 grid"));
  CHECK(throws_with([&] { sparse_neighbors({{0, 0, 0}, {1 << 20, 0, 0}}, dev); }, "outside the table's"));
  CHECK(throws_with([&] { QMatMul::from_q8_0(Tensor(), 4, 48); }, "needs k % 32 == 0"));
  CHECK(throws_with([&] { GgufFile::open(g_fixture_dir + "/missing.gguf"); }, "cannot open"));
  CHECK(throws_with([&] { SafetensorsFile::open(g_fixture_dir + "/tiny_q8.gguf"); }, "safetensors"));
  const GgufFile f = GgufFile::open(g_fixture_dir + "/tiny_q8.gguf");
  CHECK(f.version() == 3 && f.names().size() == 3 && f.contains("blocks.0.norm.weight"));
}

// slat_prepare on valid coords: the tables equal Trellis2Rope3d::cos_sin's and
// the device coords round-trip; index_select_rows throws on an id past the rows.
void slat_prepare_and_gather_checks(const Device &dev) {
  const Trellis2Rope3d rope(12);
  const std::vector<Coord> coords = {{0, 0, 0}, {3, 1, 2}, {63, 63, 63}};
  const SlatTokens t = slat_prepare({3, 4}, 4, coords, 64, rope, dev);
  auto [cos, sin] = rope.cos_sin({0, 0, 0, 3, 1, 2, 63, 63, 63}, dev);
  CHECK(t.cos.to_vec_f32() == cos.to_vec_f32() && t.sin.to_vec_f32() == sin.to_vec_f32());
  const std::vector<int32_t> c = t.coords.to_vec_i32();
  CHECK(c.size() == 9 && c[3] == 3 && c[4] == 1 && c[5] == 2 && c[8] == 63);
  const Tensor feats = Tensor::from_f32({1, 2, 3, 4, 5, 6}, {3, 2}, DType::F32, dev);
  const std::vector<float> g = index_select_rows(feats, Tensor::from_i32({2, 0}, {2}, dev)).to_vec_f32();
  CHECK(g == std::vector<float>({5, 6, 1, 2}));
  CHECK(throws_with([&] { index_select_rows(feats, Tensor::from_i32({2, 3, -1}, {3}, dev)); },
                    "index_select_rows: 2 of 3 ids outside 0..3"));
}

void errors_on_device(const Device &dev) {
  const Tensor pos = Tensor::from_i32({0, 0, 1, 1}, {1, 2, 2}, dev);
  CHECK(throws_with([&] { Rope2d(100.0f).embeddings(pos, 6); }, "rope token_dim must be divisible by 4"));
  Trellis2Rope3d rope(12);
  auto [cos, sin] = rope.cos_sin({1, 0, 0}, dev);
  const Tensor x2 = Tensor::zeros({1, 2, 1, 12}, DType::F32, dev);
  CHECK(throws_with([&] { rope.apply(x2, cos, sin); }, "RoPE tables must be [2, 6]"));
  // a C ABI check surfaces as Error with the library's status and message
  try {
    layer_norm(Tensor::zeros({4, 8}, DType::BF16, dev), Tensor::zeros({7}, DType::F32, dev),
               Tensor::zeros({8}, DType::F32, dev), 1e-5f);
    CHECK(false);
  } catch (const Error &e) {
    CHECK(e.status() == LUX3D_ERR_SHAPE);
  }
}

struct Case {
  const char *name;
  std::function<void(const Device &)> fn;
  bool needs_gpu;
};

}  // namespace

int main(int argc, char **argv) {
  const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
  {  // fixtures live in tests/golden, beside this binary's tests/cpp
    std::string self = argv[0];
    const size_t slash = self.find_last_of('/');
    g_fixture_dir = (slash == std::string::npos ? std::string(".") : self.substr(0, slash)) + "/../golden";
  }
  const std::vector<Case> cases = {
      {"errors_on_host", errors_on_host, false},
      {"rope_tables_match_reference_formula", rope_tables_match_reference_formula, true},
      {"rope_apply_matches_complex_product_and_preserves_norm", rope_apply_matches_complex_product_and_preserves_norm, true},
      {"qk_rms_norm_matches_reference", qk_rms_norm_matches_reference, true},
      {"timestep_embedding_matches_reference", timestep_embedding_matches_reference, true},
      {"ada_ln_modulation_chunks_in_reference_order", ada_ln_modulation_chunks_in_reference_order, true},
      {"gated_residual_modulate_closed_form", gated_residual_modulate_closed_form, true},
      {"dinov3_rope_tables_match_hand_computed_cos_sin", dinov3_rope_tables_match_hand_computed_cos_sin, true},
      {"dinov3_rope_applies_to_patches_only", dinov3_rope_applies_to_patches_only, true},
      {"residual_layer_norm_closed_form", residual_layer_norm_closed_form, true},
      {"vggt_qk_layernorm_rope_specials_are_plain_layernorm", vggt_qk_layernorm_rope_specials_are_plain_layernorm, true},
      {"dequantize_q8_0_exact", dequantize_q8_0_exact, true},
      {"q8_0_linear_closed_form", q8_0_linear_closed_form, true},
      {"sparse_attention_matches_naive", sparse_attention_matches_naive, true},
      {"exact_sdpa_heads_bf16_is_f32_arithmetic", exact_sdpa_heads_bf16_is_f32_arithmetic, true},
      {"vggt_attention_fused_equals_two_calls", vggt_attention_fused_equals_two_calls, true},
      {"model_attentions_fused_equal_two_calls", model_attentions_fused_equal_two_calls, true},
      {"gguf_q8_linear_from_file", gguf_q8_linear_from_file, true},
      {"kernel_offset_deltas_cover_the_3x3x3_kernel", kernel_offset_deltas_cover_the_3x3x3_kernel, false},
      {"coord_map_builds_and_looks_up", coord_map_builds_and_looks_up, true},
      {"sparse_conv_matches_dense_reference", sparse_conv_matches_dense_reference, true},
      {"sparse_conv_hand_picked_kernels", sparse_conv_hand_picked_kernels, true},
      {"sparse_conv_loader_transposes_flex_gemm_layout", sparse_conv_loader_transposes_flex_gemm_layout, true},
      {"sparse_conv_rulebook_identity_and_shift", sparse_conv_rulebook_identity_and_shift, true},
      {"c2s_order_and_feature_selection", c2s_order_and_feature_selection, true},
      {"slat_prepare_and_gather_checks", slat_prepare_and_gather_checks, true},
      {"errors_on_device", errors_on_device, true},
  };
  Device dev;  // ordinal 0, null stream; Device::hip() is only called when a GPU is needed
  if (!cpu_only) dev = Device::hip(0);
  int run = 0;
  for (const Case &c : cases) {
    if (cpu_only && c.needs_gpu) continue;
    const int before = g_failures;
    try {
      c.fn(dev);
    } catch (const std::exception &e) {
      std::printf("    unexpected exception: %s\n", e.what());
      ++g_failures;
    }
    std::printf("%s %s\n", g_failures == before ? "PASS" : "FAIL", c.name);
    std::fflush(stdout);
    ++run;
  }
  std::printf("%d cases, %d failures\n", run, g_failures);
  return g_failures == 0 ? 0 : 1;
}
