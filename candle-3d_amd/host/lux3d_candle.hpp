// lux3d_candle.hpp -- C++ mirror of candle-3d's Tensor-level interface for
// the fused transformer-layer path, built on the liblux3d_fused C ABI
// (lux3d_fused.h).
//
// The reference is Rust (crates/lux3d-core over a candle fork). This header
// keeps its names, argument meaning and error behaviour:
//   * a Tensor is device storage shared between views plus a layout (shape,
//     element strides, start offset), like candle's Arc<Storage> + Layout;
//     views (narrow / transpose / permute / get / chunk / unsqueeze) copy
//     nothing;
//   * ops allocate their outputs, as a candle CustomOp does, and enqueue one
//     kernel on the tensor's device stream; only the host transfers
//     (from_* / to_vec_*) synchronise;
//   * every failure the reference reports through `candle_core::Result` /
//     `bail!` is thrown here as lux3d::candle::Error, with the C ABI's status
//     and message (or the reference's own message where the check is the
//     reference's).
#pragma once

#include <hip/hip_runtime_api.h>

#include <array>
#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "lux3d_fused.h"
#include "lux3d_weights.h"

namespace lux3d::candle {

enum class DType : int32_t {
  F32 = LUX3D_F32,
  BF16 = LUX3D_BF16,
  F16 = LUX3D_F16,
  I32 = LUX3D_I32,
  I64 = LUX3D_I64,
  U8 = LUX3D_U8,
  I8 = LUX3D_I8,
};
size_t dtype_size(DType dt);

// candle_core::Error: status is a lux3d_status (LUX3D_ERR_*).
class Error : public std::runtime_error {
 public:
  Error(int status, const std::string &msg) : std::runtime_error(msg), status_(status) {}
  int status() const { return status_; }

 private:
  int status_;
};

// A HIP device and the stream every op on it is enqueued on (the null
// stream unless with_stream() names another).
class Device {
 public:
  static Device hip(int ordinal = 0);
  Device with_stream(hipStream_t s) const;
  int ordinal() const { return ordinal_; }
  hipStream_t stream() const { return stream_; }
  void synchronize() const;

 private:
  int ordinal_ = 0;
  hipStream_t stream_ = nullptr;
};

using Shape = std::vector<int64_t>;

class Tensor {
 public:
  Tensor() = default;
  // Device allocations (contents undefined / zero) and host uploads. f32
  // values are rounded to nearest even for bf16 / f16 (half-crate rules).
  static Tensor empty(const Shape &shape, DType dt, const Device &dev);
  static Tensor zeros(const Shape &shape, DType dt, const Device &dev);
  static Tensor from_f32(const std::vector<float> &v, const Shape &shape, DType dt, const Device &dev);
  static Tensor from_i32(const std::vector<int32_t> &v, const Shape &shape, const Device &dev);
  static Tensor from_i64(const std::vector<int64_t> &v, const Shape &shape, const Device &dev);
  static Tensor from_u8(const std::vector<uint8_t> &v, const Shape &shape, const Device &dev);

  const Shape &dims() const { return shape_; }
  int64_t dim(int i) const;
  size_t rank() const { return shape_.size(); }
  int64_t elem_count() const;
  const Shape &stride() const { return stride_; }
  DType dtype() const { return dtype_; }
  const Device &device() const { return device_; }
  bool is_contiguous() const;

  // Views (no copies).
  Tensor narrow(int dim, int64_t start, int64_t len) const;
  Tensor transpose(int d0, int d1) const;
  Tensor permute(const std::vector<int> &order) const;
  Tensor get(int64_t index) const;  // Tensor::i(index) on dim 0
  Tensor unsqueeze(int dim) const;
  Tensor reshape(const Shape &shape) const;  // contiguous tensors only
  std::vector<Tensor> chunk(int64_t n, int dim) const;

  // Device -> host in logical (row-major) order; synchronises the stream.
  std::vector<float> to_vec_f32() const;
  std::vector<uint16_t> to_vec_u16() const;  // raw bf16 / f16 bits
  std::vector<int32_t> to_vec_i32() const;   // int32 tensors

  // The C ABI descriptor of this view.
  lux3d_tensor_t desc() const;

 private:
  struct Storage;
  std::shared_ptr<Storage> storage_;
  int64_t offset_ = 0;  // elements
  Shape shape_, stride_;
  DType dtype_ = DType::F32;
  Device device_;
  static Tensor alloc(const Shape &shape, DType dt, const Device &dev);
  std::vector<uint8_t> gather_bytes() const;
};

// ---- LayerNorm family -----------------------------------------------------

// candle_nn::ops::layer_norm(x, alpha, beta, eps) over the last dim.
Tensor layer_norm(const Tensor &x, const Tensor &alpha, const Tensor &beta, float eps);

// candle_nn::LayerNorm as built by `layer_norm(dim, eps, vb)` (the affine
// LayerNorm of runtime/vggt.rs:104, runtime/pi3_encoder.rs:67, ...).
class LayerNorm {
 public:
  LayerNorm(Tensor weight, std::optional<Tensor> bias, double eps);
  Tensor forward(const Tensor &xs) const;
  const Tensor &weight() const { return weight_; }
  const std::optional<Tensor> &bias() const { return bias_; }
  double eps() const { return eps_; }

 private:
  Tensor weight_;
  std::optional<Tensor> bias_;
  double eps_;
};

// layer_norm_no_affine (runtime/trellis2_blocks.rs:280-286).
Tensor layer_norm_no_affine(const Tensor &xs, double eps);

// LayerScale (runtime/nn_blocks.rs:210-214): xs * gamma.
class LayerScale {
 public:
  explicit LayerScale(Tensor gamma) : gamma_(std::move(gamma)) {}
  const Tensor &gamma() const { return gamma_; }

 private:
  Tensor gamma_;
};

// `h = x + ls(a)` then `norm(h)` (VggtBlock::forward, runtime/vggt.rs:113-124;
// ls may be null for the plain residual of runtime/triposg_dit.rs:364-379).
// Returns (h, norm(h)).
std::pair<Tensor, Tensor> residual_layer_norm(const Tensor &x, const Tensor &a, const LayerScale *ls,
                                              const LayerNorm &norm);

// ---- AdaLN (TRELLIS.2) ----------------------------------------------------

// chunk_modulation (runtime/trellis2_blocks.rs:264-277): the six [B, 1, C]
// views (shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp).
std::array<Tensor, 6> chunk_modulation(const Tensor &mod_vec);

// `layer_norm_no_affine(x) * (1 + scale) + shift` (and `gate * (...) + x`
// when gate is given) with shift / scale / gate per batch element or per
// ragged segment (seg_offsets int64 [S+1]); `*_base` is the block's
// `modulation` vector added to each piece (runtime/trellis2_blocks.rs:617-630,
// 693-706; runtime/vggt.rs:399-405).
struct Modulation {
  Tensor shift, scale;
  std::optional<Tensor> gate, shift_base, scale_base, gate_base;
};
Tensor adaln_modulate(const Tensor &x, const Modulation &m, double eps,
                      const std::optional<Tensor> &seg_offsets = std::nullopt);

// `xs + h * gate` (runtime/trellis2_blocks.rs:632-633).
Tensor gated_residual(const Tensor &x, const Tensor &h, const Tensor &gate,
                      const std::optional<Tensor> &gate_base = std::nullopt,
                      const std::optional<Tensor> &seg_offsets = std::nullopt);

// `xs = xs + h * gate` (gate absent: `xs + h`) followed by the next
// `layer_norm_no_affine(xs) * (1 + scale) + shift`, one launch: the sparse
// block's MLP entry (runtime/trellis2_blocks.rs:708-713) and the dense
// block's cross-attention add + MLP modulate (:637-642). Returns (xs, y).
// `next` holds shift / scale (+ bases); its gate must be empty.
std::pair<Tensor, Tensor> gated_residual_adaln_modulate(const Tensor &x, const Tensor &h,
                                                        const std::optional<Tensor> &gate,
                                                        const std::optional<Tensor> &gate_base,
                                                        const Modulation &next, double eps,
                                                        const std::optional<Tensor> &seg_offsets = std::nullopt);

// ---- VGGT / Pi3 2D RoPE (runtime/attention_math.rs) -------------------------

struct RopeEmbeddings {
  Tensor cos_full, sin_alt_full;  // [b, 1, n, token_dim] f32
};

class Rope2d {
 public:
  explicit Rope2d(float base) : base_(base) {}
  // positions: int32 / int64 [b, n, 2] on the device.
  RopeEmbeddings embeddings(const Tensor &positions, size_t token_dim) const;
  float base() const { return base_; }

 private:
  float base_;
};

// apply_layernorm_rope (runtime/attention_math.rs:127-150) and apply_rope
// (:155-165) on [b, h, n, d] views (strided allowed, unit inner stride).
Tensor apply_layernorm_rope(const Tensor &q, const LayerNorm &q_norm, const RopeEmbeddings &embeddings);
Tensor apply_rope(const Tensor &tokens, const RopeEmbeddings &embeddings);

// Both calls of VggtAttention::forward (runtime/vggt.rs:170-181) in one
// launch, the rotation computed from the positions in-kernel.
std::pair<Tensor, Tensor> qk_layernorm_rope2d(const Tensor &q, const Tensor &k, const LayerNorm &q_norm,
                                              const LayerNorm &k_norm, const Tensor &positions, float base);

// ---- TripoSG --------------------------------------------------------------

// RmsNormHeads::rms_norm_heads (runtime/triposg_dit.rs:509-522), eps 1e-6.
Tensor rms_norm_heads(const Tensor &x, const Tensor &weight);

// TripoSgDiT::timestep_embedding (runtime/triposg_dit.rs:280-297):
// [sin(t*f), cos(t*f)] for t [n] -> [n, dim].
Tensor triposg_timestep_embedding(const Tensor &t, size_t dim);

// ---- TRELLIS.2 ------------------------------------------------------------

// Trellis2QkRmsNorm (runtime/trellis2_blocks.rs:288-320), gamma [heads, head_dim].
class Trellis2QkRmsNorm {
 public:
  explicit Trellis2QkRmsNorm(Tensor gamma) : gamma_(std::move(gamma)) {}
  Tensor forward(const Tensor &xs) const;  // xs [B, L, H, D]

 private:
  Tensor gamma_;
};

// Trellis2Rope3d (runtime/trellis2_blocks.rs:84-161).
class Trellis2Rope3d {
 public:
  explicit Trellis2Rope3d(size_t head_dim, float rope_base = 10000.0f) : head_dim_(head_dim), rope_base_(rope_base) {}
  size_t head_dim() const { return head_dim_; }
  // coords: [L, 3] flattened (x, y, z). Returns (cos, sin) [L, head_dim/2] f32.
  std::pair<Tensor, Tensor> cos_sin(const std::vector<int64_t> &coords, const Device &dev) const;
  // x [B, L, H, head_dim]
  Tensor apply(const Tensor &x, const Tensor &cos, const Tensor &sin) const;

 private:
  size_t head_dim_;
  float rope_base_;
};

// Both tensors' N2 then R2 (Trellis2SelfAttention::attention,
// runtime/trellis2_blocks.rs:423-430) in one launch from voxel coords.
std::pair<Tensor, Tensor> qk_l2norm_rope3d(const Tensor &q, const Tensor &k, const Tensor &q_gamma,
                                           const Tensor &k_gamma, const Tensor &coords, float rope_base = 10000.0f);

// timestep_embedding (runtime/trellis2_blocks.rs:184-204): [cos, sin], [dim].
Tensor timestep_embedding(float t, size_t dim, const Device &dev);

// Trellis2DinoConfig::rope_cos_sin (runtime/trellis2_dino.rs:140-187):
// (cos, sin) [grid_h * grid_w, head_dim], built on the host as the
// reference does.
std::pair<Tensor, Tensor> dinov3_rope_cos_sin(size_t head_dim, float rope_theta, size_t grid_h, size_t grid_w,
                                              const Device &dev);

// apply_rotary_to_patches (runtime/trellis2_dino.rs:406-436).
std::pair<Tensor, Tensor> apply_rotary_to_patches(const Tensor &q, const Tensor &k, const Tensor &cos,
                                                  const Tensor &sin, size_t num_prefix);

// ---- elementwise / quantised weights -----------------------------------------

Tensor gelu(const Tensor &x);      // Tensor::gelu (tanh approximation)
Tensor gelu_erf(const Tensor &x);  // Tensor::gelu_erf
Tensor silu(const Tensor &x);      // Tensor::silu

// QTensor::dequantize for GGML Q8_0 (runtime/nn_blocks.rs:140): `blocks`
// holds elem_count(shape)/32 records of 34 bytes; out dtype F32, BF16 or F16.
Tensor dequantize_q8_0(const Tensor &blocks, const Shape &shape, DType out);

// Attention over [B, H, L, D] views: softmax(q k^T * scale) v, one kernel,
// no scores buffer. exact_query_chunked_sdpa (attention_math.rs:199-241; the
// chunk size only bounded the reference's scores buffer and is ignored) and
// exact_sdpa_heads (attention_math.rs:244-259; f32 arithmetic whatever the
// input dtype, lux3d_sdpa_heads_f32). Both return a contiguous
// [B, H, Lq, D] tensor in q's dtype.
Tensor exact_query_chunked_sdpa(const Tensor &q, const Tensor &k, const Tensor &v, float scale,
                                size_t chunk_size = SIZE_MAX);
Tensor exact_sdpa_heads(const Tensor &q, const Tensor &k, const Tensor &v, float scale);
// exact_query_chunked_sdpa(apply_layernorm_rope(q, q_norm, embeddings), k, v,
// scale) (vggt.rs:170-183) with q's LayerNorm + 2D RoPE in the attention
// kernel's Q load; k already normalised and rotated. Bit-identical to the
// two calls.
Tensor sdpa_layernorm_rope(const Tensor &q, const class LayerNorm &q_norm, const struct RopeEmbeddings &embeddings,
                           const Tensor &k, const Tensor &v, float scale);
// exact_query_chunked_sdpa(rms_norm_heads(q, q_w), k, v, scale)
// (triposg_dit.rs:446-455) with q's per-head RMSNorm (eps 1e-6) in the Q
// load; k already normalised. Bit-identical to the two calls.
Tensor sdpa_rms_norm_heads(const Tensor &q, const Tensor &q_w, const Tensor &k, const Tensor &v, float scale);
// Trellis2SelfAttention::attention (trellis2_blocks.rs:417-436) on
// [B, H, L, D] views: exact_query_chunked_sdpa(rope(l2norm(q)), k, v, scale)
// with q's L2 norm (gamma [H, D]) and 3D RoPE (cos / sin [L, D/2]) in the Q
// load; k already normalised and rotated. Bit-identical to the two calls.
Tensor sdpa_l2norm_rope3d(const Tensor &q, const Tensor &q_gamma, const Tensor &cos, const Tensor &sin,
                          const Tensor &k, const Tensor &v, float scale);
// exact_sdpa_heads(apply_rotary_to_patches(q), k, v, scale)
// (trellis2_dino.rs:385-393) with q's rotate_half RoPE in the Q load; k
// already rotated. Bit-identical to the two calls.
Tensor sdpa_dinov3_rope(const Tensor &q, const Tensor &cos, const Tensor &sin, size_t num_prefix, const Tensor &k,
                        const Tensor &v, float scale);

// QMatMul over a Q8_0 weight [n, k] (QMatMul::from_qtensor and forward,
// runtime/nn_blocks.rs:83-93, 145-150). from_q8_0 repacks the GGML blocks
// once; forward(xs [..., k] bf16) = xs @ dequant(W)^T in f32 accumulation.
class GgufFile;

class QMatMul {
 public:
  static QMatMul from_q8_0(const Tensor &blocks, int64_t n, int64_t k);
  Tensor forward(const Tensor &xs, const std::optional<Tensor> &bias = std::nullopt, DType out = DType::BF16) const;
  int64_t out_dim() const { return qs_.dim(0); }
  int64_t in_dim() const { return qs_.dim(1); }

 private:
  Tensor qs_, scales_;
};

// ---------------------------------------------------------------------------
// TRELLIS.2 sparse voxel ops (runtime/trellis2_sparse.rs). Coordinates are
// host vectors as in the reference (Vec<[i32; 3]>); features live on the
// device.
// ---------------------------------------------------------------------------

using Coord = std::array<int32_t, 3>;

// kernel_offset_delta (trellis2_sparse.rs:83-91): k = kd*9 + kh*3 + kw
Coord kernel_offset_delta(size_t k);
// CoordMap + the per-offset lookups, on the device: nbr int32 [N, 27]
Tensor sparse_neighbors(const std::vector<Coord> &coords, const Device &dev);
// index_select_rows (trellis2_sparse.rs:117-131); throws, as candle's
// index_select does, when an id is outside the rows (counted on the device,
// read back after a stream sync)
Tensor index_select_rows(const Tensor &feats, const Tensor &ids);

// Trellis2SlatDit::prepare (runtime/trellis2_dit.rs:511-544): checks the
// token features (their dims, [rows, in_channels]) against the host coords
// ([rows] x (x, y, z), each coordinate within 0..resolution) with the
// reference's messages, then builds the RoPE tables. Also returns the coords
// as a device int32 [rows, 3] tensor: the source lux3d_qk_l2norm_rope3d can
// rotate from in-kernel instead of reading the tables.
struct SlatTokens {
  Tensor coords, cos, sin;
};
SlatTokens slat_prepare(const Shape &feats_dims, int64_t in_channels, const std::vector<Coord> &coords,
                        int64_t resolution, const Trellis2Rope3d &rope, const Device &dev);

class SparseConv3d {
 public:
  // SparseConv3d::load (trellis2_sparse.rs:147-180): `weight` in the
  // checkpoint's flex_gemm layout [Cout, 3, 3, 3, Cin] (or flattened), any
  // float dtype; kept as weight27 [27, Cout, Cin] f32.
  static SparseConv3d load(const Tensor &weight, const std::optional<Tensor> &bias, int64_t in_channels,
                           int64_t out_channels);
  int64_t in_channels() const { return in_; }
  int64_t out_channels() const { return out_; }
  const Tensor &weight27() const { return w27_; }
  // forward (trellis2_sparse.rs:197-243): feats f32 [N, Cin] -> [N, Cout] f32
  Tensor forward(const std::vector<Coord> &coords, const Tensor &feats) const;
  // the same with a neighbour table already built for these coordinates
  Tensor forward_nbr(const Tensor &nbr, const Tensor &feats) const;

 private:
  Tensor w27_;
  std::optional<Tensor> bias_;
  int64_t in_ = 0, out_ = 0;
};

// channel_to_spatial (trellis2_sparse.rs:249-338)
struct Channel2SpatialOutput {
  std::vector<Coord> coords;  // children: parent order, ascending subidx
  Tensor feats;               // [M, C / 8]
  Tensor sub_binary;          // [N, 8] f32
};
Channel2SpatialOutput channel_to_spatial(const std::vector<Coord> &coords, const Tensor &feats,
                                         const Tensor &subdiv_logits);

// ---------------------------------------------------------------------------
// Weight files (lux3d_weights.h underneath): VarBuilder::from_gguf and
// VarBuilder::from_mmaped_safetensors (weights/mod.rs:121-140). The files
// stay mapped while the object lives; get() uploads and converts on the
// device (Q8_0 through the dequant kernel).
// ---------------------------------------------------------------------------

struct WeightInfo {
  std::string name;
  int32_t dtype = 0;  // GGUF: ggml type id; safetensors: lux3d_dtype (-1: not one)
  Shape shape;
  uint64_t nbytes = 0;
  const void *data = nullptr;  // host bytes in the mapping
};

class GgufFile {
 public:
  static GgufFile open(const std::string &path);
  uint32_t version() const;
  std::vector<std::string> names() const;
  bool contains(const std::string &name) const;
  WeightInfo info(const std::string &name) const;
  // gguf_metadata_string (weights/mod.rs:656-661): a string value or nothing
  std::optional<std::string> metadata_string(const std::string &key) const;
  std::optional<uint64_t> metadata_uint(const std::string &key) const;
  // VarBuilder::get on a GGUF: the tensor in dtype `dt` on `dev` (Q8_0 is
  // dequantized exactly, F16 / BF16 / F32 converted with one RNE rounding)
  Tensor get(const std::string &name, DType dt, const Device &dev) const;
  // VarBuilder::get(shape, name): the same, with the reference's shape check
  Tensor get(const Shape &expected, const std::string &name, DType dt, const Device &dev) const;
  // VarBuilder::get_quantized + QMatMul::from_qtensor for a rank-2 Q8_0
  // weight (nn_blocks.rs:107-150); quantized_linear's shape check against
  // (out_dim, in_dim)
  QMatMul get_qmatmul(const std::string &name, int64_t out_dim, int64_t in_dim, const Device &dev) const;

 private:
  std::shared_ptr<lux3d_gguf_t> h_;
};

class SafetensorsFile {
 public:
  static SafetensorsFile open(const std::string &path);
  std::vector<std::string> names() const;
  bool contains(const std::string &name) const;
  WeightInfo info(const std::string &name) const;
  std::optional<std::string> metadata(const std::string &key) const;
  // VarBuilder::get: the tensor in `dt` on `dev` (float types converted with
  // one RNE rounding; integer types must match `dt`)
  Tensor get(const std::string &name, DType dt, const Device &dev) const;
  Tensor get(const Shape &expected, const std::string &name, DType dt, const Device &dev) const;

 private:
  std::shared_ptr<lux3d_safetensors_t> h_;
};

}  // namespace lux3d::candle
