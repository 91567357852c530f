// lux3d_candle.cpp -- the C++ mirror of candle-3d's Tensor-level interface
// (lux3d_candle.hpp) over the liblux3d_fused C ABI. Host code only: device
// memory through the HIP runtime, every op one C ABI call.
#include "lux3d_candle.hpp"

#include "lux3d_weights.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>

namespace lux3d::candle {

namespace {

[[noreturn]] void fail(int status, const std::string &msg) { throw Error(status, msg); }

void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess) fail(LUX3D_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

void abi_check(int status) {
  if (status != LUX3D_OK) fail(status, lux3d_last_error());
}

std::string dims_str(const Shape &s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

// ---- host conversions (half crate semantics: round to nearest even, NaN kept quiet) ----
uint16_t f32_to_bf16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
  return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xFFu, mant = x & 0x7FFFFFu;
  if (exp == 0xFFu) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u | (mant >> 13) : 0u));
  const int e = (int)exp - 127 + 15;
  if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    const uint32_t m = mant | 0x800000u;
    const int shift = 14 - e;
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
  const uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // a carry into the exponent rounds up correctly
  return (uint16_t)(sign | h);
}

float bf16_to_f32(uint16_t b) {
  const uint32_t x = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
  uint32_t x;
  if (exp == 0) {
    if (mant == 0) {
      x = sign;
    } else {  // subnormal: renormalise
      int e = -1;
      uint32_t m = mant;
      do {
        ++e;
        m <<= 1;
      } while (!(m & 0x400u));
      x = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3FFu) << 13);
    }
  } else if (exp == 0x1F) {
    x = sign | 0x7F800000u | (mant << 13);
  } else {
    x = sign | ((exp - 15 + 127) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

Shape row_major(const Shape &shape) {
  Shape st(shape.size());
  int64_t acc = 1;
  for (size_t i = shape.size(); i-- > 0;) {
    st[i] = acc;
    acc *= shape[i];
  }
  return st;
}

int norm_dim(int dim, size_t rank, const char *what) {
  const int r = (int)rank;
  if (dim < 0) dim += r;
  if (dim < 0 || dim >= r) fail(LUX3D_ERR_SHAPE, std::string(what) + ": dim out of range for rank " + std::to_string(r));
  return dim;
}

// Descriptor holder so optional operands can be passed as pointers.
struct Desc {
  lux3d_tensor_t t{};
  bool set = false;
  Desc() = default;
  explicit Desc(const Tensor &x) : t(x.desc()), set(true) {}
  explicit Desc(const std::optional<Tensor> &x) {
    if (x) {
      t = x->desc();
      set = true;
    }
  }
  const lux3d_tensor_t *p() const { return set ? &t : nullptr; }
};

Tensor empty_like(const Tensor &x) { return Tensor::empty(x.dims(), x.dtype(), x.device()); }

}  // namespace

size_t dtype_size(DType dt) {
  switch (dt) {
    case DType::F32: case DType::I32: return 4;
    case DType::BF16: case DType::F16: return 2;
    case DType::I64: return 8;
    case DType::U8: case DType::I8: return 1;
  }
  return 0;
}

// ---------------------------------------------------------------------------
// Device
// ---------------------------------------------------------------------------

Device Device::hip(int ordinal) {
  int n = 0;
  hip_check(hipGetDeviceCount(&n), "hipGetDeviceCount");
  if (ordinal < 0 || ordinal >= n) fail(LUX3D_ERR_VALUE, "no HIP device " + std::to_string(ordinal));
  Device d;
  d.ordinal_ = ordinal;
  return d;
}

Device Device::with_stream(hipStream_t s) const {
  Device d = *this;
  d.stream_ = s;
  return d;
}

void Device::synchronize() const {
  hip_check(hipSetDevice(ordinal_), "hipSetDevice");
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
}

// ---------------------------------------------------------------------------
// Tensor
// ---------------------------------------------------------------------------

struct Tensor::Storage {
  void *ptr = nullptr;
  size_t bytes = 0;
  int device = 0;
  ~Storage() {
    if (ptr) {
      (void)hipSetDevice(device);
      (void)hipFree(ptr);
    }
  }
};

Tensor Tensor::alloc(const Shape &shape, DType dt, const Device &dev) {
  for (int64_t n : shape)
    if (n < 0) fail(LUX3D_ERR_SHAPE, "negative dimension in " + dims_str(shape));
  if (shape.size() > LUX3D_MAX_RANK) fail(LUX3D_ERR_SHAPE, "rank above " + std::to_string(LUX3D_MAX_RANK));
  Tensor t;
  t.shape_ = shape;
  t.stride_ = row_major(shape);
  t.dtype_ = dt;
  t.device_ = dev;
  t.storage_ = std::make_shared<Storage>();
  t.storage_->device = dev.ordinal();
  t.storage_->bytes = (size_t)std::max<int64_t>(t.elem_count(), 1) * dtype_size(dt);
  hip_check(hipSetDevice(dev.ordinal()), "hipSetDevice");
  hip_check(hipMalloc(&t.storage_->ptr, t.storage_->bytes), "hipMalloc");
  return t;
}

Tensor Tensor::empty(const Shape &shape, DType dt, const Device &dev) { return alloc(shape, dt, dev); }

Tensor Tensor::zeros(const Shape &shape, DType dt, const Device &dev) {
  Tensor t = alloc(shape, dt, dev);
  hip_check(hipMemsetAsync(t.storage_->ptr, 0, t.storage_->bytes, dev.stream()), "hipMemsetAsync");
  return t;
}

namespace {
Tensor upload(Tensor t, const void *src, size_t bytes) {
  const Device &dev = t.device();
  lux3d_tensor_t d = t.desc();
  hip_check(hipMemcpyAsync(d.data, src, bytes, hipMemcpyHostToDevice, dev.stream()), "hipMemcpyAsync");
  hip_check(hipStreamSynchronize(dev.stream()), "hipStreamSynchronize");  // the host buffer may go away
  return t;
}

int64_t count(const Shape &s) { return std::accumulate(s.begin(), s.end(), (int64_t)1, std::multiplies<int64_t>()); }
}  // namespace

Tensor Tensor::from_f32(const std::vector<float> &v, const Shape &shape, DType dt, const Device &dev) {
  if ((int64_t)v.size() != count(shape))
    fail(LUX3D_ERR_SHAPE, "from_f32: " + std::to_string(v.size()) + " values for shape " + dims_str(shape));
  Tensor t = alloc(shape, dt, dev);
  if (dt == DType::F32) return upload(t, v.data(), v.size() * 4);
  if (dt != DType::BF16 && dt != DType::F16) fail(LUX3D_ERR_DTYPE, "from_f32: float dtype expected");
  std::vector<uint16_t> h(v.size());
  for (size_t i = 0; i < v.size(); ++i) h[i] = dt == DType::BF16 ? f32_to_bf16(v[i]) : f32_to_f16(v[i]);
  return upload(t, h.data(), h.size() * 2);
}

Tensor Tensor::from_i32(const std::vector<int32_t> &v, const Shape &shape, const Device &dev) {
  if ((int64_t)v.size() != count(shape)) fail(LUX3D_ERR_SHAPE, "from_i32: size does not match " + dims_str(shape));
  return upload(alloc(shape, DType::I32, dev), v.data(), v.size() * 4);
}

Tensor Tensor::from_i64(const std::vector<int64_t> &v, const Shape &shape, const Device &dev) {
  if ((int64_t)v.size() != count(shape)) fail(LUX3D_ERR_SHAPE, "from_i64: size does not match " + dims_str(shape));
  return upload(alloc(shape, DType::I64, dev), v.data(), v.size() * 8);
}

Tensor Tensor::from_u8(const std::vector<uint8_t> &v, const Shape &shape, const Device &dev) {
  if ((int64_t)v.size() != count(shape)) fail(LUX3D_ERR_SHAPE, "from_u8: size does not match " + dims_str(shape));
  return upload(alloc(shape, DType::U8, dev), v.data(), v.size());
}

int64_t Tensor::dim(int i) const { return shape_[norm_dim(i, shape_.size(), "dim")]; }

int64_t Tensor::elem_count() const { return count(shape_); }

bool Tensor::is_contiguous() const {
  int64_t acc = 1;
  for (size_t i = shape_.size(); i-- > 0;) {
    if (shape_[i] != 1 && stride_[i] != acc) return false;
    acc *= shape_[i];
  }
  return true;
}

Tensor Tensor::narrow(int dim, int64_t start, int64_t len) const {
  dim = norm_dim(dim, shape_.size(), "narrow");
  if (start < 0 || len < 0 || start + len > shape_[dim])
    fail(LUX3D_ERR_SHAPE, "narrow: [" + std::to_string(start) + ", +" + std::to_string(len) + ") outside dim " +
                              std::to_string(dim) + " of " + dims_str(shape_));
  Tensor t = *this;
  t.offset_ += start * stride_[dim];
  t.shape_[dim] = len;
  return t;
}

Tensor Tensor::transpose(int d0, int d1) const {
  d0 = norm_dim(d0, shape_.size(), "transpose");
  d1 = norm_dim(d1, shape_.size(), "transpose");
  Tensor t = *this;
  std::swap(t.shape_[d0], t.shape_[d1]);
  std::swap(t.stride_[d0], t.stride_[d1]);
  return t;
}

Tensor Tensor::permute(const std::vector<int> &order) const {
  if (order.size() != shape_.size()) fail(LUX3D_ERR_SHAPE, "permute: order has the wrong rank");
  std::vector<bool> seen(order.size(), false);
  Tensor t = *this;
  for (size_t i = 0; i < order.size(); ++i) {
    const int o = norm_dim(order[i], shape_.size(), "permute");
    if (seen[o]) fail(LUX3D_ERR_SHAPE, "permute: repeated dim");
    seen[o] = true;
    t.shape_[i] = shape_[o];
    t.stride_[i] = stride_[o];
  }
  return t;
}

Tensor Tensor::get(int64_t index) const {
  if (shape_.empty() || index < 0 || index >= shape_[0]) fail(LUX3D_ERR_SHAPE, "get: index out of range");
  Tensor t = *this;
  t.offset_ += index * stride_[0];
  t.shape_.erase(t.shape_.begin());
  t.stride_.erase(t.stride_.begin());
  return t;
}

Tensor Tensor::unsqueeze(int dim) const {
  const int r = (int)shape_.size();
  if (dim < 0) dim += r + 1;
  if (dim < 0 || dim > r) fail(LUX3D_ERR_SHAPE, "unsqueeze: dim out of range");
  Tensor t = *this;
  const int64_t st = dim < r ? stride_[dim] * shape_[dim] : 1;
  t.shape_.insert(t.shape_.begin() + dim, 1);
  t.stride_.insert(t.stride_.begin() + dim, st);
  return t;
}

Tensor Tensor::reshape(const Shape &shape) const {
  if (count(shape) != elem_count())
    fail(LUX3D_ERR_SHAPE, "reshape: " + dims_str(shape_) + " -> " + dims_str(shape) + " changes the element count");
  if (!is_contiguous()) fail(LUX3D_ERR_LAYOUT, "reshape: the tensor is not contiguous");
  Tensor t = *this;
  t.shape_ = shape;
  t.stride_ = row_major(shape);
  return t;
}

std::vector<Tensor> Tensor::chunk(int64_t n, int dim) const {
  dim = norm_dim(dim, shape_.size(), "chunk");
  if (n <= 0) fail(LUX3D_ERR_VALUE, "chunk: n must be positive");
  const int64_t size = shape_[dim], step = (size + n - 1) / n;
  std::vector<Tensor> out;
  for (int64_t s = 0; s < size; s += step) out.push_back(narrow(dim, s, std::min(step, size - s)));
  return out;
}

lux3d_tensor_t Tensor::desc() const {
  lux3d_tensor_t d{};
  if (!storage_) fail(LUX3D_ERR_NULL, "desc: empty tensor");
  if (shape_.size() > LUX3D_MAX_RANK) fail(LUX3D_ERR_SHAPE, "desc: rank above " + std::to_string(LUX3D_MAX_RANK));
  d.data = static_cast<char *>(storage_->ptr) + offset_ * (int64_t)dtype_size(dtype_);
  d.dtype = (int32_t)dtype_;
  d.rank = (int32_t)shape_.size();
  for (size_t i = 0; i < shape_.size(); ++i) {
    d.shape[i] = shape_[i];
    d.stride[i] = stride_[i];
  }
  return d;
}

std::vector<uint8_t> Tensor::gather_bytes() const {
  const size_t es = dtype_size(dtype_);
  const int64_t n = elem_count();
  std::vector<uint8_t> out((size_t)n * es);
  if (n == 0) return out;
  // the span of storage this view touches
  int64_t lo = offset_, hi = offset_;
  for (size_t i = 0; i < shape_.size(); ++i) {
    const int64_t ext = (shape_[i] - 1) * stride_[i];
    if (ext < 0) lo += ext; else hi += ext;
  }
  std::vector<uint8_t> span((size_t)(hi - lo + 1) * es);
  device_.synchronize();
  hip_check(hipMemcpy(span.data(), static_cast<char *>(storage_->ptr) + lo * (int64_t)es, span.size(),
                      hipMemcpyDeviceToHost),
            "hipMemcpy");
  std::vector<int64_t> idx(shape_.size(), 0);
  for (int64_t e = 0; e < n; ++e) {
    int64_t off = offset_ - lo;
    for (size_t i = 0; i < shape_.size(); ++i) off += idx[i] * stride_[i];
    std::memcpy(&out[(size_t)e * es], &span[(size_t)off * es], es);
    for (size_t i = shape_.size(); i-- > 0;) {
      if (++idx[i] < shape_[i]) break;
      idx[i] = 0;
    }
  }
  return out;
}

std::vector<float> Tensor::to_vec_f32() const {
  const std::vector<uint8_t> b = gather_bytes();
  const int64_t n = elem_count();
  std::vector<float> v((size_t)n);
  for (int64_t i = 0; i < n; ++i) {
    switch (dtype_) {
      case DType::F32: std::memcpy(&v[i], &b[i * 4], 4); break;
      case DType::BF16: { uint16_t h; std::memcpy(&h, &b[i * 2], 2); v[i] = bf16_to_f32(h); break; }
      case DType::F16: { uint16_t h; std::memcpy(&h, &b[i * 2], 2); v[i] = f16_to_f32(h); break; }
      case DType::I32: { int32_t q; std::memcpy(&q, &b[i * 4], 4); v[i] = (float)q; break; }
      case DType::I64: { int64_t q; std::memcpy(&q, &b[i * 8], 8); v[i] = (float)q; break; }
      case DType::U8: v[i] = (float)b[i]; break;
      case DType::I8: v[i] = (float)(int8_t)b[i]; break;
    }
  }
  return v;
}

std::vector<uint16_t> Tensor::to_vec_u16() const {
  if (dtype_ != DType::BF16 && dtype_ != DType::F16) fail(LUX3D_ERR_DTYPE, "to_vec_u16: bf16 / f16 tensor expected");
  const std::vector<uint8_t> b = gather_bytes();
  std::vector<uint16_t> v(b.size() / 2);
  std::memcpy(v.data(), b.data(), b.size());
  return v;
}

std::vector<int32_t> Tensor::to_vec_i32() const {
  if (dtype_ != DType::I32) fail(LUX3D_ERR_DTYPE, "to_vec_i32: int32 tensor expected");
  const std::vector<uint8_t> b = gather_bytes();
  std::vector<int32_t> v(b.size() / 4);
  std::memcpy(v.data(), b.data(), b.size());
  return v;
}

// ---------------------------------------------------------------------------
// LayerNorm family
// ---------------------------------------------------------------------------

Tensor layer_norm(const Tensor &x, const Tensor &alpha, const Tensor &beta, float eps) {
  Tensor y = empty_like(x);
  abi_check(lux3d_layer_norm(Desc(x).p(), Desc(alpha).p(), Desc(beta).p(), eps, Desc(y).p(), x.device().stream()));
  return y;
}

LayerNorm::LayerNorm(Tensor weight, std::optional<Tensor> bias, double eps)
    : weight_(std::move(weight)), bias_(std::move(bias)), eps_(eps) {}

Tensor LayerNorm::forward(const Tensor &xs) const {
  Tensor y = empty_like(xs);
  abi_check(lux3d_layer_norm(Desc(xs).p(), Desc(weight_).p(), Desc(bias_).p(), (float)eps_, Desc(y).p(),
                             xs.device().stream()));
  return y;
}

Tensor layer_norm_no_affine(const Tensor &xs, double eps) {
  Tensor y = empty_like(xs);
  abi_check(lux3d_layer_norm(Desc(xs).p(), nullptr, nullptr, (float)eps, Desc(y).p(), xs.device().stream()));
  return y;
}

std::pair<Tensor, Tensor> residual_layer_norm(const Tensor &x, const Tensor &a, const LayerScale *ls,
                                              const LayerNorm &norm) {
  Tensor h = empty_like(x), y = empty_like(x);
  Desc g = ls ? Desc(ls->gamma()) : Desc();
  abi_check(lux3d_residual_layer_norm(Desc(x).p(), Desc(a).p(), g.p(), Desc(norm.weight()).p(), Desc(norm.bias()).p(),
                                      (float)norm.eps(), Desc(h).p(), Desc(y).p(), x.device().stream()));
  return {h, y};
}

// ---------------------------------------------------------------------------
// AdaLN
// ---------------------------------------------------------------------------

std::array<Tensor, 6> chunk_modulation(const Tensor &mod_vec) {
  const std::vector<Tensor> parts = mod_vec.chunk(6, -1);
  if (parts.size() != 6) fail(LUX3D_ERR_SHAPE, "adaLN modulation must chunk into 6");
  std::array<Tensor, 6> out;
  for (int i = 0; i < 6; ++i) out[i] = parts[i].unsqueeze(1);
  return out;
}

Tensor adaln_modulate(const Tensor &x, const Modulation &m, double eps, const std::optional<Tensor> &seg_offsets) {
  Tensor y = empty_like(x);
  abi_check(lux3d_adaln_modulate(Desc(x).p(), Desc(seg_offsets).p(), Desc(m.shift).p(), Desc(m.shift_base).p(),
                                 Desc(m.scale).p(), Desc(m.scale_base).p(), Desc(m.gate).p(), Desc(m.gate_base).p(),
                                 (float)eps, Desc(y).p(), x.device().stream()));
  return y;
}

Tensor gated_residual(const Tensor &x, const Tensor &h, const Tensor &gate, const std::optional<Tensor> &gate_base,
                      const std::optional<Tensor> &seg_offsets) {
  Tensor out = empty_like(x);
  abi_check(lux3d_gated_residual(Desc(x).p(), Desc(h).p(), Desc(seg_offsets).p(), Desc(gate).p(),
                                 Desc(gate_base).p(), Desc(out).p(), x.device().stream()));
  return out;
}

std::pair<Tensor, Tensor> gated_residual_adaln_modulate(const Tensor &x, const Tensor &h,
                                                        const std::optional<Tensor> &gate,
                                                        const std::optional<Tensor> &gate_base,
                                                        const Modulation &next, double eps,
                                                        const std::optional<Tensor> &seg_offsets) {
  if (next.gate) fail(LUX3D_ERR_VALUE, "gated_residual_adaln_modulate: the next modulate takes no output gate");
  Tensor xo = empty_like(x), y = empty_like(x);
  abi_check(lux3d_gated_residual_adaln_modulate(
      Desc(x).p(), Desc(h).p(), Desc(seg_offsets).p(), Desc(gate).p(), Desc(gate_base).p(), Desc(next.shift).p(),
      Desc(next.shift_base).p(), Desc(next.scale).p(), Desc(next.scale_base).p(), (float)eps, Desc(xo).p(),
      Desc(y).p(), x.device().stream()));
  return {xo, y};
}

// ---------------------------------------------------------------------------
// VGGT / Pi3 2D RoPE
// ---------------------------------------------------------------------------

RopeEmbeddings Rope2d::embeddings(const Tensor &positions, size_t token_dim) const {
  const size_t half = token_dim / 2;
  if (half % 2 != 0) fail(LUX3D_ERR_SHAPE, "rope token_dim must be divisible by 4, got " + std::to_string(token_dim));
  if (positions.rank() != 3) fail(LUX3D_ERR_SHAPE, "Rope2d::embeddings: positions must be [b, n, 2]");
  const int64_t b = positions.dim(0), n = positions.dim(1), d = (int64_t)token_dim;
  RopeEmbeddings e{Tensor::empty({b, 1, n, d}, DType::F32, positions.device()),
                   Tensor::empty({b, 1, n, d}, DType::F32, positions.device())};
  abi_check(lux3d_rope2d_tables(Desc(positions).p(), base_, Desc(e.cos_full).p(), Desc(e.sin_alt_full).p(),
                                positions.device().stream()));
  return e;
}

Tensor apply_layernorm_rope(const Tensor &q, const LayerNorm &q_norm, const RopeEmbeddings &embeddings) {
  Tensor out = empty_like(q);
  abi_check(lux3d_qk_layernorm_rope2d(Desc(q).p(), Desc(q_norm.weight()).p(), Desc(q_norm.bias()).p(), nullptr,
                                      nullptr, nullptr,
                                      (float)q_norm.eps(), Desc(embeddings.cos_full).p(),
                                      Desc(embeddings.sin_alt_full).p(), Desc(out).p(), nullptr, q.device().stream()));
  return out;
}

Tensor apply_rope(const Tensor &tokens, const RopeEmbeddings &embeddings) {
  Tensor out = empty_like(tokens);
  abi_check(lux3d_qk_layernorm_rope2d(Desc(tokens).p(), nullptr, nullptr, nullptr, nullptr, nullptr, 0.f,
                                      Desc(embeddings.cos_full).p(), Desc(embeddings.sin_alt_full).p(), Desc(out).p(),
                                      nullptr, tokens.device().stream()));
  return out;
}

std::pair<Tensor, Tensor> qk_layernorm_rope2d(const Tensor &q, const Tensor &k, const LayerNorm &q_norm,
                                              const LayerNorm &k_norm, const Tensor &positions, float base) {
  Tensor qo = empty_like(q), ko = empty_like(k);
  abi_check(lux3d_qk_layernorm_rope2d_pos(Desc(q).p(), Desc(q_norm.weight()).p(), Desc(q_norm.bias()).p(),
                                          Desc(k).p(), Desc(k_norm.weight()).p(), Desc(k_norm.bias()).p(),
                                          (float)q_norm.eps(),
                                          Desc(positions).p(), base, Desc(qo).p(), Desc(ko).p(), q.device().stream()));
  return {qo, ko};
}

// ---------------------------------------------------------------------------
// TripoSG
// ---------------------------------------------------------------------------

Tensor rms_norm_heads(const Tensor &x, const Tensor &weight) {
  Tensor out = empty_like(x);
  abi_check(lux3d_rms_norm_heads(Desc(x).p(), Desc(weight).p(), nullptr, nullptr, 1e-6f, Desc(out).p(), nullptr,
                                 x.device().stream()));
  return out;
}

namespace {
// exp(-ln(10000) * i / half) with the reference's f32 steps and libm expf.
std::vector<float> timestep_freqs(size_t dim, float neg_log_period) {
  const size_t half = dim / 2;
  std::vector<float> f(half);
  for (size_t i = 0; i < half; ++i) f[i] = std::exp(neg_log_period * (float)i / (float)half);
  return f;
}
}  // namespace

Tensor triposg_timestep_embedding(const Tensor &t, size_t dim) {
  const Device &dev = t.device();
  const Tensor freqs =
      Tensor::from_f32(timestep_freqs(dim, -std::log(10000.0f)), {(int64_t)(dim / 2)}, DType::F32, dev);
  Tensor out = Tensor::empty({t.elem_count(), (int64_t)dim}, DType::F32, dev);
  abi_check(lux3d_timestep_embedding(Desc(t).p(), Desc(freqs).p(), (int64_t)dim, 0, Desc(out).p(), dev.stream()));
  return out;
}

// ---------------------------------------------------------------------------
// TRELLIS.2
// ---------------------------------------------------------------------------

Tensor Trellis2QkRmsNorm::forward(const Tensor &xs) const {
  Tensor out = empty_like(xs);
  abi_check(lux3d_qk_l2norm_rope3d(Desc(xs).p(), Desc(gamma_).p(), nullptr, nullptr, nullptr, nullptr, nullptr, 0.f,
                                   Desc(out).p(), nullptr, xs.device().stream()));
  return out;
}

std::pair<Tensor, Tensor> Trellis2Rope3d::cos_sin(const std::vector<int64_t> &coords, const Device &dev) const {
  if (coords.size() % 3 != 0)
    fail(LUX3D_ERR_SHAPE,
         "TRELLIS.2 RoPE coords must be [L, 3] flattened, got " + std::to_string(coords.size()) + " values");
  if (head_dim_ % 2 != 0)
    fail(LUX3D_ERR_SHAPE, "TRELLIS.2 RoPE head dim must be divisible by 2, got " + std::to_string(head_dim_));
  if (head_dim_ / 2 / 3 == 0)
    fail(LUX3D_ERR_SHAPE, "TRELLIS.2 head_dim " + std::to_string(head_dim_) + " is too small for 3-axis RoPE");
  std::vector<int32_t> c(coords.size());
  for (size_t i = 0; i < coords.size(); ++i) {
    if (coords[i] < INT32_MIN || coords[i] > INT32_MAX) fail(LUX3D_ERR_VALUE, "TRELLIS.2 RoPE coord out of int32 range");
    c[i] = (int32_t)coords[i];
  }
  const int64_t L = (int64_t)(coords.size() / 3), half = (int64_t)(head_dim_ / 2);
  const Tensor ct = Tensor::from_i32(c, {L, 3}, dev);
  Tensor cos = Tensor::empty({L, half}, DType::F32, dev), sin = Tensor::empty({L, half}, DType::F32, dev);
  abi_check(lux3d_rope3d_tables(Desc(ct).p(), (int64_t)head_dim_, rope_base_, Desc(cos).p(), Desc(sin).p(),
                                dev.stream()));
  return {cos, sin};
}

Tensor Trellis2Rope3d::apply(const Tensor &x, const Tensor &cos, const Tensor &sin) const {
  if (x.rank() != 4) fail(LUX3D_ERR_SHAPE, "Trellis2Rope3d::apply: x must be [B, L, H, D], got " + dims_str(x.dims()));
  const int64_t tokens = x.dim(1), half = x.dim(3) / 2;
  const Shape want{tokens, half};
  if (cos.dims() != want || sin.dims() != want)
    fail(LUX3D_ERR_SHAPE, "RoPE tables must be [" + std::to_string(tokens) + ", " + std::to_string(half) +
                              "], got cos " + dims_str(cos.dims()) + " sin " + dims_str(sin.dims()));
  Tensor out = empty_like(x);
  abi_check(lux3d_qk_l2norm_rope3d(Desc(x).p(), nullptr, nullptr, nullptr, Desc(cos).p(), Desc(sin).p(), nullptr, 0.f,
                                   Desc(out).p(), nullptr, x.device().stream()));
  return out;
}

std::pair<Tensor, Tensor> qk_l2norm_rope3d(const Tensor &q, const Tensor &k, const Tensor &q_gamma,
                                           const Tensor &k_gamma, const Tensor &coords, float rope_base) {
  Tensor qo = empty_like(q), ko = empty_like(k);
  abi_check(lux3d_qk_l2norm_rope3d(Desc(q).p(), Desc(q_gamma).p(), Desc(k).p(), Desc(k_gamma).p(), nullptr, nullptr,
                                   Desc(coords).p(), rope_base, Desc(qo).p(), Desc(ko).p(), q.device().stream()));
  return {qo, ko};
}

Tensor timestep_embedding(float t, size_t dim, const Device &dev) {
  const Tensor tt = Tensor::from_f32({t}, {1}, DType::F32, dev);
  const Tensor freqs =
      Tensor::from_f32(timestep_freqs(dim, (float)(-std::log(10000.0))), {(int64_t)(dim / 2)}, DType::F32, dev);
  Tensor out = Tensor::empty({1, (int64_t)dim}, DType::F32, dev);
  abi_check(lux3d_timestep_embedding(Desc(tt).p(), Desc(freqs).p(), (int64_t)dim, 1, Desc(out).p(), dev.stream()));
  return out.reshape({(int64_t)dim});
}

std::pair<Tensor, Tensor> dinov3_rope_cos_sin(size_t head_dim, float rope_theta, size_t grid_h, size_t grid_w,
                                              const Device &dev) {
  const size_t freq_count = head_dim / 4;
  if (freq_count * 4 != head_dim)
    fail(LUX3D_ERR_SHAPE,
         "DINOv3 head_dim " + std::to_string(head_dim) + " is not divisible by 4; RoPE layout undefined");
  std::vector<float> inv(freq_count);
  for (size_t i = 0; i < freq_count; ++i) inv[i] = 1.0f / std::pow(rope_theta, (float)i * (4.0f / (float)head_dim));
  const float two_pi = (float)(M_PI * 2.0);
  const size_t patches = grid_h * grid_w, half_len = freq_count * 2;
  std::vector<float> c(patches * head_dim), s(patches * head_dim);
  for (size_t y = 0; y < grid_h; ++y) {
    const float cy = 2.0f * (((float)y + 0.5f) / (float)grid_h) - 1.0f;
    for (size_t x = 0; x < grid_w; ++x) {
      const float cx = 2.0f * (((float)x + 0.5f) / (float)grid_w) - 1.0f;
      const size_t row = (y * grid_w + x) * head_dim;
      const float coord[2] = {cy, cx};
      for (size_t a = 0; a < 2; ++a)
        for (size_t i = 0; i < freq_count; ++i) {
          const float ang = (two_pi * coord[a]) * inv[i];
          for (size_t rep = 0; rep < 2; ++rep) {  // tile(2)
            c[row + rep * half_len + a * freq_count + i] = std::cos(ang);
            s[row + rep * half_len + a * freq_count + i] = std::sin(ang);
          }
        }
    }
  }
  const Shape shape{(int64_t)patches, (int64_t)head_dim};
  return {Tensor::from_f32(c, shape, DType::F32, dev), Tensor::from_f32(s, shape, DType::F32, dev)};
}

std::pair<Tensor, Tensor> apply_rotary_to_patches(const Tensor &q, const Tensor &k, const Tensor &cos,
                                                  const Tensor &sin, size_t num_prefix) {
  Tensor qo = empty_like(q), ko = empty_like(k);
  abi_check(lux3d_dinov3_rope(Desc(q).p(), Desc(k).p(), Desc(cos).p(), Desc(sin).p(), (int64_t)num_prefix,
                              Desc(qo).p(), Desc(ko).p(), q.device().stream()));
  return {qo, ko};
}

// ---------------------------------------------------------------------------
// Elementwise / Q8_0
// ---------------------------------------------------------------------------

namespace {
template <int (*F)(const lux3d_tensor_t *, const lux3d_tensor_t *, lux3d_stream_t)>
Tensor unary(const Tensor &x) {
  Tensor y = empty_like(x);
  abi_check(F(Desc(x).p(), Desc(y).p(), x.device().stream()));
  return y;
}
}  // namespace

Tensor gelu(const Tensor &x) { return unary<lux3d_gelu_tanh>(x); }
Tensor gelu_erf(const Tensor &x) { return unary<lux3d_gelu_erf>(x); }
Tensor silu(const Tensor &x) { return unary<lux3d_silu>(x); }

Tensor dequantize_q8_0(const Tensor &blocks, const Shape &shape, DType out) {
  Tensor y = Tensor::empty(shape, out, blocks.device());
  abi_check(lux3d_dequant_q8_0(Desc(blocks).p(), Desc(y).p(), blocks.device().stream()));
  return y;
}

Tensor exact_sdpa_heads(const Tensor &q, const Tensor &k, const Tensor &v, float scale) {
  if (q.rank() != 4) fail(LUX3D_ERR_SHAPE, "sdpa: q must be [B, H, L, D], got " + dims_str(q.dims()));
  Tensor out = Tensor::empty(q.dims(), q.dtype(), q.device());
  abi_check(lux3d_sdpa_heads_f32(Desc(q).p(), Desc(k).p(), Desc(v).p(), scale, Desc(out).p(), q.device().stream()));
  return out;
}

Tensor sdpa_layernorm_rope(const Tensor &q, const LayerNorm &q_norm, const RopeEmbeddings &embeddings,
                           const Tensor &k, const Tensor &v, float scale) {
  Tensor out = Tensor::empty(q.dims(), q.dtype(), q.device());
  abi_check(lux3d_sdpa_layernorm_rope2d(Desc(q).p(), Desc(q_norm.weight()).p(), Desc(q_norm.bias()).p(),
                                        (float)q_norm.eps(),
                                        Desc(embeddings.cos_full).p(), Desc(embeddings.sin_alt_full).p(), Desc(k).p(),
                                        Desc(v).p(), scale, Desc(out).p(), q.device().stream()));
  return out;
}

Tensor sdpa_rms_norm_heads(const Tensor &q, const Tensor &q_w, const Tensor &k, const Tensor &v, float scale) {
  Tensor out = Tensor::empty(q.dims(), q.dtype(), q.device());
  abi_check(lux3d_sdpa_rms_norm_heads(Desc(q).p(), Desc(q_w).p(), 1e-6f, Desc(k).p(), Desc(v).p(), scale,
                                      Desc(out).p(), q.device().stream()));
  return out;
}

Tensor sdpa_l2norm_rope3d(const Tensor &q, const Tensor &q_gamma, const Tensor &cos, const Tensor &sin,
                          const Tensor &k, const Tensor &v, float scale) {
  Tensor out = Tensor::empty(q.dims(), q.dtype(), q.device());
  abi_check(lux3d_sdpa_l2norm_rope3d(Desc(q).p(), Desc(q_gamma).p(), Desc(cos).p(), Desc(sin).p(), Desc(k).p(),
                                     Desc(v).p(), scale, Desc(out).p(), q.device().stream()));
  return out;
}

Tensor sdpa_dinov3_rope(const Tensor &q, const Tensor &cos, const Tensor &sin, size_t num_prefix, const Tensor &k,
                        const Tensor &v, float scale) {
  Tensor out = Tensor::empty(q.dims(), q.dtype(), q.device());
  abi_check(lux3d_sdpa_dinov3_rope(Desc(q).p(), Desc(cos).p(), Desc(sin).p(), (int64_t)num_prefix, Desc(k).p(),
                                   Desc(v).p(), scale, Desc(out).p(), q.device().stream()));
  return out;
}

Tensor exact_query_chunked_sdpa(const Tensor &q, const Tensor &k, const Tensor &v, float scale, size_t) {
  if (q.rank() != 4) fail(LUX3D_ERR_SHAPE, "sdpa: q must be [B, H, L, D], got " + dims_str(q.dims()));
  Tensor out = Tensor::empty(q.dims(), q.dtype(), q.device());
  abi_check(lux3d_sdpa(Desc(q).p(), Desc(k).p(), Desc(v).p(), scale, Desc(out).p(), q.device().stream()));
  return out;
}

QMatMul QMatMul::from_q8_0(const Tensor &blocks, int64_t n, int64_t k) {
  if (n < 0 || k <= 0 || k % 32)
    fail(LUX3D_ERR_SHAPE, "Q8_0 weight [" + std::to_string(n) + ", " + std::to_string(k) + "] needs k % 32 == 0");
  QMatMul m;
  m.qs_ = Tensor::empty({n, k}, DType::I8, blocks.device());
  m.scales_ = Tensor::empty({n, k / 32}, DType::F32, blocks.device());
  abi_check(lux3d_q8_0_repack(Desc(blocks).p(), n, k, Desc(m.qs_).p(), Desc(m.scales_).p(), blocks.device().stream()));
  return m;
}

Tensor QMatMul::forward(const Tensor &xs, const std::optional<Tensor> &bias, DType out) const {
  Shape shape = xs.dims();
  if (shape.empty()) fail(LUX3D_ERR_SHAPE, "QMatMul::forward: scalar input");
  shape.back() = out_dim();
  Tensor y = Tensor::empty(shape, out, xs.device());
  abi_check(lux3d_q8_0_linear(Desc(xs).p(), Desc(qs_).p(), Desc(scales_).p(), Desc(bias).p(), Desc(y).p(),
                              xs.device().stream()));
  return y;
}

// ---------------------------------------------------------------------------
// TRELLIS.2 sparse ops
// ---------------------------------------------------------------------------

Coord kernel_offset_delta(size_t k) {
  if (k >= 27) fail(LUX3D_ERR_VALUE, "kernel offset " + std::to_string(k) + " out of range");
  return {(int32_t)(k / 9) - 1, (int32_t)((k % 9) / 3) - 1, (int32_t)(k % 3) - 1};
}

namespace {
Tensor coords_tensor(const std::vector<Coord> &coords, const Device &dev) {
  std::vector<int32_t> flat(coords.size() * 3);
  for (size_t i = 0; i < coords.size(); ++i)
    for (int a = 0; a < 3; ++a) flat[3 * i + a] = coords[i][a];
  return Tensor::from_i32(flat, {(int64_t)coords.size(), 3}, dev);
}
}  // namespace

Tensor sparse_neighbors(const std::vector<Coord> &coords, const Device &dev) {
  // the coordinates are on the host here: check the hash key's range before any device work
  for (const Coord &c : coords)
    for (int a = 0; a < 3; ++a)
      if (c[a] < -(1 << 20) || c[a] >= (1 << 20) - 1)
        fail(LUX3D_ERR_VALUE, "sparse_neighbors: coord [" + std::to_string(c[0]) + ", " + std::to_string(c[1]) + ", " +
                                  std::to_string(c[2]) + "] outside the table's [-2^20, 2^20 - 1) range");
  const int64_t n = (int64_t)coords.size();
  int64_t cap = 16;
  while (cap < 2 * n) cap *= 2;
  const Tensor keys = Tensor::empty({cap}, DType::I64, dev), vals = Tensor::empty({cap}, DType::I32, dev);
  Tensor nbr = Tensor::empty({n, 27}, DType::I32, dev);
  abi_check(lux3d_sparse_neighbors(Desc(coords_tensor(coords, dev)).p(), Desc(keys).p(), Desc(vals).p(), Desc(nbr).p(),
                                   nullptr, dev.stream()));
  return nbr;
}

SlatTokens slat_prepare(const Shape &feats_dims, int64_t in_channels, const std::vector<Coord> &coords,
                        int64_t resolution, const Trellis2Rope3d &rope, const Device &dev) {
  if (feats_dims.size() != 2) fail(LUX3D_ERR_SHAPE, "SLAT DiT features must be [rows, channels], got " + dims_str(feats_dims));
  const int64_t rows = feats_dims[0], channels = feats_dims[1];
  if (channels != in_channels)
    fail(LUX3D_ERR_SHAPE, "SLAT DiT expects " + std::to_string(in_channels) + " token channels, got " +
                              std::to_string(channels));
  if (rows != (int64_t)coords.size())
    fail(LUX3D_ERR_SHAPE, "SLAT DiT coords/features mismatch: " + std::to_string(coords.size()) + " coords vs " +
                              std::to_string(rows) + " rows");
  std::vector<int64_t> flat;
  flat.reserve(coords.size() * 3);
  for (const Coord &c : coords)
    for (int a = 0; a < 3; ++a) {
      if (c[a] < 0 || c[a] >= resolution)
        fail(LUX3D_ERR_VALUE, "SLAT coord [" + std::to_string(c[0]) + ", " + std::to_string(c[1]) + ", " +
                                  std::to_string(c[2]) + "] outside the 0.." + std::to_string(resolution) + " grid");
      flat.push_back(c[a]);
    }
  auto [cos, sin] = rope.cos_sin(flat, dev);
  return {coords_tensor(coords, dev), cos, sin};
}

Tensor index_select_rows(const Tensor &feats, const Tensor &ids) {
  Shape shape = feats.dims();
  if (shape.empty()) fail(LUX3D_ERR_SHAPE, "index_select_rows: scalar input");
  shape[0] = ids.elem_count();
  Tensor out = Tensor::empty(shape, feats.dtype(), feats.device());
  // candle's index_select fails on an id outside the rows: count them on the
  // device and read the count back (this op returns after a stream sync)
  Tensor bad = Tensor::empty({1}, DType::I32, feats.device());
  abi_check(lux3d_index_select_rows(Desc(feats).p(), Desc(ids).p(), Desc(out).p(), Desc(bad).p(),
                                    feats.device().stream()));
  const int64_t nbad = bad.to_vec_i32()[0];
  if (nbad)
    fail(LUX3D_ERR_VALUE, "index_select_rows: " + std::to_string(nbad) + " of " + std::to_string(ids.elem_count()) +
                              " ids outside 0.." + std::to_string(feats.dim(0)));
  return out;
}

SparseConv3d SparseConv3d::load(const Tensor &weight, const std::optional<Tensor> &bias, int64_t in_channels,
                                int64_t out_channels) {
  if (weight.elem_count() != out_channels * 27 * in_channels)
    fail(LUX3D_ERR_SHAPE, "SparseConv3d weight " + dims_str(weight.dims()) + " is not [" + std::to_string(out_channels) +
                              ", 3, 3, 3, " + std::to_string(in_channels) + "]");
  // [Cout, 27, Cin] -> [27, Cout, Cin] (load time, on the host)
  const std::vector<float> w = weight.to_vec_f32();
  std::vector<float> t(w.size());
  for (int64_t o = 0; o < out_channels; ++o)
    for (int64_t k = 0; k < 27; ++k)
      std::memcpy(&t[(k * out_channels + o) * in_channels], &w[(o * 27 + k) * in_channels],
                  sizeof(float) * (size_t)in_channels);
  SparseConv3d c;
  c.w27_ = Tensor::from_f32(t, {27, out_channels, in_channels}, DType::F32, weight.device());
  if (bias) {
    if (bias->elem_count() != out_channels) fail(LUX3D_ERR_SHAPE, "SparseConv3d bias must have Cout elements");
    c.bias_ = Tensor::from_f32(bias->to_vec_f32(), {out_channels}, DType::F32, bias->device());
  }
  c.in_ = in_channels;
  c.out_ = out_channels;
  return c;
}

Tensor SparseConv3d::forward_nbr(const Tensor &nbr, const Tensor &feats) const {
  const Device &dev = feats.device();
  Tensor out = Tensor::empty({feats.dim(0), out_}, DType::F32, dev);
  if (in_ % 16 == 0 && feats.rank() == 2 && feats.dim(0) == nbr.dim(0)) {
    // per-tap pair lists, then the reference's tap-ordered accumulation
    const int64_t n = nbr.dim(0);
    const Tensor pairs = Tensor::empty({27, n, 2}, DType::I32, dev), counts = Tensor::empty({27}, DType::I32, dev);
    abi_check(lux3d_sparse_rulebook(Desc(nbr).p(), Desc(pairs).p(), Desc(counts).p(), dev.stream()));
    abi_check(lux3d_sparse_conv3d_rulebook(Desc(feats).p(), Desc(pairs).p(), Desc(counts).p(), Desc(w27_).p(),
                                           Desc(bias_).p(), Desc(out).p(), dev.stream()));
    return out;
  }
  abi_check(lux3d_sparse_conv3d(Desc(feats).p(), Desc(nbr).p(), Desc(w27_).p(), Desc(bias_).p(), Desc(out).p(),
                                dev.stream()));
  return out;
}

Tensor SparseConv3d::forward(const std::vector<Coord> &coords, const Tensor &feats) const {
  if (feats.rank() != 2 || feats.dim(0) != (int64_t)coords.size() || feats.dim(1) != in_)
    fail(LUX3D_ERR_SHAPE, "SparseConv3d expects [N, " + std::to_string(in_) + "] with N = " +
                              std::to_string(coords.size()) + " coords, got " + dims_str(feats.dims()));
  return forward_nbr(sparse_neighbors(coords, feats.device()), feats);
}

Channel2SpatialOutput channel_to_spatial(const std::vector<Coord> &coords, const Tensor &feats,
                                         const Tensor &subdiv_logits) {
  const Device &dev = feats.device();
  const int64_t n = (int64_t)coords.size();
  if (feats.rank() != 2 || feats.dim(0) != n)
    fail(LUX3D_ERR_SHAPE, "channel_to_spatial coords/features mismatch: " + std::to_string(n) + " coords vs " +
                              std::to_string(feats.rank() ? feats.dim(0) : 0) + " rows");
  const int64_t c = feats.dim(1);
  const Tensor ws = Tensor::empty({n + (n + 1023) / 1024}, DType::I32, dev);
  const Tensor oc = Tensor::empty({8 * n, 3}, DType::I32, dev), src = Tensor::empty({8 * n}, DType::I32, dev);
  const Tensor of = Tensor::empty({8 * n, c / 8}, feats.dtype(), dev);
  Tensor sub = Tensor::empty({n, 8}, DType::F32, dev);
  const Tensor cnt = Tensor::empty({1}, DType::I32, dev);
  abi_check(lux3d_channel_to_spatial(Desc(coords_tensor(coords, dev)).p(), Desc(feats).p(), Desc(subdiv_logits).p(),
                                     Desc(ws).p(), Desc(oc).p(), Desc(src).p(), Desc(of).p(), Desc(sub).p(),
                                     Desc(cnt).p(), dev.stream()));
  const int64_t m = cnt.to_vec_i32()[0];  // the host needs the child count (the reference's Vec length)
  Channel2SpatialOutput r;
  const std::vector<int32_t> flat = oc.to_vec_i32();
  r.coords.resize((size_t)m);
  for (int64_t j = 0; j < m; ++j) r.coords[(size_t)j] = {flat[3 * j], flat[3 * j + 1], flat[3 * j + 2]};
  r.feats = of.narrow(0, 0, m);
  r.sub_binary = sub;
  return r;
}

// ---------------------------------------------------------------------------
// Weight files
// ---------------------------------------------------------------------------

namespace {

WeightInfo to_info(const lux3d_weights_tensor_t &t) {
  WeightInfo w;
  w.name = t.name;
  w.dtype = t.dtype;
  w.shape.assign(t.shape, t.shape + t.rank);
  w.nbytes = t.nbytes;
  w.data = t.data;
  return w;
}

void weights_check(bool ok) {
  if (!ok) fail(LUX3D_ERR_VALUE, lux3d_weights_last_error());
}

float host_elem_f32(int src_dt, const uint8_t *b, size_t i) {
  switch (src_dt) {
    case LUX3D_F32: { float f; std::memcpy(&f, b + 4 * i, 4); return f; }
    case LUX3D_BF16: { uint16_t h; std::memcpy(&h, b + 2 * i, 2); return bf16_to_f32(h); }
    case LUX3D_F16: { uint16_t h; std::memcpy(&h, b + 2 * i, 2); return f16_to_f32(h); }
  }
  return 0.f;
}

// Host bytes of lux3d dtype `src_dt` -> a device tensor of dtype `dt`
// (float types: widened exactly, rounded once; other types must match).
Tensor upload_as(const void *src, int src_dt, uint64_t nbytes, const Shape &shape, DType dt, const Device &dev,
                 const std::string &name) {
  Tensor t = Tensor::empty(shape, dt, dev);
  if (src_dt == (int)dt) {
    if ((uint64_t)t.elem_count() * dtype_size(dt) != nbytes)
      fail(LUX3D_ERR_SHAPE, "tensor `" + name + "`: byte count does not match its shape");
    return upload(t, src, nbytes);
  }
  const bool fsrc = src_dt == LUX3D_F32 || src_dt == LUX3D_BF16 || src_dt == LUX3D_F16;
  const bool fdst = dt == DType::F32 || dt == DType::BF16 || dt == DType::F16;
  if (!fsrc || !fdst) fail(LUX3D_ERR_DTYPE, "tensor `" + name + "`: no conversion to the requested dtype");
  const size_t n = (size_t)t.elem_count();
  const uint8_t *b = static_cast<const uint8_t *>(src);
  if (dt == DType::F32) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = host_elem_f32(src_dt, b, i);
    return upload(t, v.data(), n * 4);
  }
  std::vector<uint16_t> v(n);
  for (size_t i = 0; i < n; ++i) {
    const float f = host_elem_f32(src_dt, b, i);
    v[i] = dt == DType::BF16 ? f32_to_bf16(f) : f32_to_f16(f);
  }
  return upload(t, v.data(), n * 2);
}

void check_shape(const Shape &expected, const Shape &got, const std::string &name) {
  if (expected != got)
    fail(LUX3D_ERR_SHAPE, "shape mismatch for " + name + ", expected " + dims_str(expected) + ", got " + dims_str(got));
}

}  // namespace

GgufFile GgufFile::open(const std::string &path) {
  lux3d_gguf_t *g = lux3d_gguf_open(path.c_str());
  weights_check(g != nullptr);
  GgufFile f;
  f.h_ = std::shared_ptr<lux3d_gguf_t>(g, lux3d_gguf_close);
  return f;
}

uint32_t GgufFile::version() const { return lux3d_gguf_version(h_.get()); }

std::vector<std::string> GgufFile::names() const {
  std::vector<std::string> r;
  lux3d_weights_tensor_t t;
  for (int64_t i = 0; i < lux3d_gguf_tensor_count(h_.get()); ++i)
    if (lux3d_gguf_tensor(h_.get(), i, &t) == LUX3D_OK) r.emplace_back(t.name);
  return r;
}

bool GgufFile::contains(const std::string &name) const { return lux3d_gguf_find(h_.get(), name.c_str()) >= 0; }

WeightInfo GgufFile::info(const std::string &name) const {
  const int64_t i = lux3d_gguf_find(h_.get(), name.c_str());
  if (i < 0) fail(LUX3D_ERR_VALUE, "cannot find tensor " + name);
  lux3d_weights_tensor_t t;
  weights_check(lux3d_gguf_tensor(h_.get(), i, &t) == LUX3D_OK);
  return to_info(t);
}

std::optional<std::string> GgufFile::metadata_string(const std::string &key) const {
  const int64_t i = lux3d_gguf_metadata_find(h_.get(), key.c_str());
  if (i < 0) return std::nullopt;
  int32_t type, et;
  const void *v;
  uint64_t n;
  weights_check(lux3d_gguf_metadata(h_.get(), i, nullptr, &type, &et, &v, &n) == LUX3D_OK);
  if (type != LUX3D_GGUF_STRING) return std::nullopt;
  return std::string(static_cast<const char *>(v), (size_t)n);
}

std::optional<uint64_t> GgufFile::metadata_uint(const std::string &key) const {
  const int64_t i = lux3d_gguf_metadata_find(h_.get(), key.c_str());
  if (i < 0) return std::nullopt;
  int32_t type, et;
  const void *v;
  uint64_t n;
  weights_check(lux3d_gguf_metadata(h_.get(), i, nullptr, &type, &et, &v, &n) == LUX3D_OK);
  const uint8_t *b = static_cast<const uint8_t *>(v);
  switch (type) {
    case LUX3D_GGUF_U8: return (uint64_t)b[0];
    case LUX3D_GGUF_U16: { uint16_t x; std::memcpy(&x, b, 2); return x; }
    case LUX3D_GGUF_U32: { uint32_t x; std::memcpy(&x, b, 4); return x; }
    case LUX3D_GGUF_U64: { uint64_t x; std::memcpy(&x, b, 8); return x; }
  }
  return std::nullopt;
}

Tensor GgufFile::get(const std::string &name, DType dt, const Device &dev) const {
  const WeightInfo w = info(name);
  switch (w.dtype) {
    case LUX3D_GGML_Q8_0: {
      const Tensor blocks = upload(Tensor::empty({(int64_t)w.nbytes}, DType::U8, dev), w.data, w.nbytes);
      return dequantize_q8_0(blocks, w.shape, dt);
    }
    case LUX3D_GGML_F32: return upload_as(w.data, LUX3D_F32, w.nbytes, w.shape, dt, dev, name);
    case LUX3D_GGML_F16: return upload_as(w.data, LUX3D_F16, w.nbytes, w.shape, dt, dev, name);
    case LUX3D_GGML_BF16: return upload_as(w.data, LUX3D_BF16, w.nbytes, w.shape, dt, dev, name);
  }
  fail(LUX3D_ERR_DTYPE, "tensor `" + name + "` has ggml type " + std::to_string(w.dtype) +
                            " (F32, F16, BF16 and Q8_0 are supported)");
}

Tensor GgufFile::get(const Shape &expected, const std::string &name, DType dt, const Device &dev) const {
  check_shape(expected, info(name).shape, name);
  return get(name, dt, dev);
}

QMatMul GgufFile::get_qmatmul(const std::string &name, int64_t out_dim, int64_t in_dim, const Device &dev) const {
  const WeightInfo w = info(name);
  if (w.shape != Shape{out_dim, in_dim})
    fail(LUX3D_ERR_SHAPE, "quantized linear weight shape " + dims_str(w.shape) + " does not match expected (" +
                              std::to_string(out_dim) + ", " + std::to_string(in_dim) + ")");
  if (w.dtype != LUX3D_GGML_Q8_0)
    fail(LUX3D_ERR_DTYPE, "tensor `" + name + "` is not Q8_0 (ggml type " + std::to_string(w.dtype) + ")");
  const Tensor blocks = upload(Tensor::empty({(int64_t)w.nbytes}, DType::U8, dev), w.data, w.nbytes);
  return QMatMul::from_q8_0(blocks, out_dim, in_dim);
}

SafetensorsFile SafetensorsFile::open(const std::string &path) {
  lux3d_safetensors_t *s = lux3d_safetensors_open(path.c_str());
  weights_check(s != nullptr);
  SafetensorsFile f;
  f.h_ = std::shared_ptr<lux3d_safetensors_t>(s, lux3d_safetensors_close);
  return f;
}

std::vector<std::string> SafetensorsFile::names() const {
  std::vector<std::string> r;
  lux3d_weights_tensor_t t;
  for (int64_t i = 0; i < lux3d_safetensors_tensor_count(h_.get()); ++i)
    if (lux3d_safetensors_tensor(h_.get(), i, &t) == LUX3D_OK) r.emplace_back(t.name);
  return r;
}

bool SafetensorsFile::contains(const std::string &name) const {
  return lux3d_safetensors_find(h_.get(), name.c_str()) >= 0;
}

WeightInfo SafetensorsFile::info(const std::string &name) const {
  const int64_t i = lux3d_safetensors_find(h_.get(), name.c_str());
  if (i < 0) fail(LUX3D_ERR_VALUE, "cannot find tensor " + name);
  lux3d_weights_tensor_t t;
  weights_check(lux3d_safetensors_tensor(h_.get(), i, &t) == LUX3D_OK);
  return to_info(t);
}

std::optional<std::string> SafetensorsFile::metadata(const std::string &key) const {
  const char *v = lux3d_safetensors_metadata(h_.get(), key.c_str());
  if (!v) return std::nullopt;
  return std::string(v);
}

Tensor SafetensorsFile::get(const std::string &name, DType dt, const Device &dev) const {
  const WeightInfo w = info(name);
  if (w.dtype < 0) fail(LUX3D_ERR_DTYPE, "tensor `" + name + "` has a dtype this reader does not convert");
  return upload_as(w.data, w.dtype, w.nbytes, w.shape, dt, dev, name);
}

Tensor SafetensorsFile::get(const Shape &expected, const std::string &name, DType dt, const Device &dev) const {
  check_shape(expected, info(name).shape, name);
  return get(name, dt, dev);
}

}  // namespace lux3d::candle
