// pointwise.hip -- streaming kernels for gfx950: GELU (erf / tanh), SiLU,
// sinusoidal timestep embeddings and the bit-exact GGML Q8_0 dequant.
//
// Activations are pure HBM streams (one read, one write per element). Each
// thread moves one 16-byte chunk of 8 elements (measured on MI355X: one chunk
// per thread streams at 6.0 TB/s for configs[2], 2 and 4 chunks per thread at
// 5.8 / 5.5 TB/s), consecutive lanes touch consecutive chunks, and the
// activations are loaded and stored non-temporally. The transcendental work is
// one exp2 + one reciprocal per element for the tanh GELU and SiLU (hardware
// v_exp_f32 / v_rcp_f32).
#include "common.hpp"
#include "kernels.hpp"

namespace lux3d {

namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 1;
// One-wavefront workgroups for the activation streams (configs[2] GELU-tanh:
// 21.5 us with 64-thread workgroups, 23.5 us with 256).
constexpr int kActBlock = 64;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// erfc(z) for z >= 0 in the form of Press, Teukolsky, Vetterling & Flannery,
// "Numerical Recipes in C" (2nd ed., section 6.2):
//   erfc(z) = t * exp(-z^2 + P(t)),  t = 1 / (1 + z/2),
// a relative error bound for every z >= 0 (so the GELU tail x*Phi(x) keeps
// its accuracy). DEG 9: their Chebyshev-fitted coefficients, fractional
// error below 1.2e-7 in exact arithmetic and 3.6e-7 evaluated as below with a
// two-part exponent argument (f32 outputs). DEG 7 / 5: lower-degree fits of the same
// form, made here by iteratively reweighted least squares on 20,001
// Chebyshev nodes of t in (0, 1] against P(t) = log(erfcx(z)) - log(t).
// Evaluated in f32 as below (the exponent argument rounded to f32 before
// v_exp_f32) they keep the relative error of erfc below 8.2e-6 (DEG 7) and
// 5.5e-5 (DEG 5) over z in [0, 9], against scipy's erfc: 1/60 and 1/35 of a
// half-ulp of f16 and bf16, the outputs they serve. One v_rcp_f32, DEG FMAs
// and one v_exp_f32 per element (DEG 9 adds the two-part argument).
template <int DEG>
__device__ __forceinline__ float erfc_nonneg(float z) {
  const float t = fast_rcp(fmaf(0.5f, z, 1.0f));
  float p;
  if constexpr (DEG == 9) {
    p = 0.17087277f;
    p = fmaf(p, t, -0.82215223f);
    p = fmaf(p, t, 1.48851587f);
    p = fmaf(p, t, -1.13520398f);
    p = fmaf(p, t, 0.27886807f);
    p = fmaf(p, t, -0.18628806f);
    p = fmaf(p, t, 0.09678418f);
    p = fmaf(p, t, 0.37409196f);
    p = fmaf(p, t, 1.00002368f);
    p = fmaf(p, t, -1.26551223f);
  } else if constexpr (DEG == 7) {
    p = -0.159051761f;
    p = fmaf(p, t, 0.644935787f);
    p = fmaf(p, t, -0.842238188f);
    p = fmaf(p, t, 0.228695139f);
    p = fmaf(p, t, 0.0103887105f);
    p = fmaf(p, t, 0.383123904f);
    p = fmaf(p, t, 0.999658525f);
    p = fmaf(p, t, -1.26550972f);
  } else {
    static_assert(DEG == 5, "fitted degrees");
    p = 0.179756626f;
    p = fmaf(p, t, -0.571638405f);
    p = fmaf(p, t, 0.331650406f);
    p = fmaf(p, t, 0.321651608f);
    p = fmaf(p, t, 1.00409198f);
    p = fmaf(p, t, -1.26556265f);
  }
  constexpr float log2e = 1.4426950408889634f;
  if constexpr (DEG == 9) {
    // f32 outputs: -z^2 + P and its product with log2(e) are carried in two
    // parts, because rounding an argument near -102 to f32 before the exp2
    // costs up to 7.5e-6 relative. z^2 = hi + lo exactly (FMA remainder); the
    // sum P - hi is split by TwoSum; n = rint(a * log2(e)) is taken out and
    // the small remainder r is formed with FMAs (log2(e) = L2E + L2E_LO), so
    // erfc = t * 2^r * 2^n keeps the fit's accuracy (3.6e-7).
    constexpr float L2E_LO = 1.925963033500011e-8f;  // log2(e) - L2E
    const float hi = z * z, lo = fmaf(z, z, -hi);
    const float a = p - hi;                          // TwoSum(p, -hi) = a + ae exactly
    const float bb = a - p;
    const float ae = (p - (a - bb)) + (-hi - bb);
    const float a_lo = ae - lo;
    const float n = __builtin_rintf(a * log2e);
    float r = fmaf(a, log2e, -n);
    r = fmaf(a, L2E_LO, r);
    r = fmaf(a_lo, log2e, r);
    return t * __builtin_ldexpf(fast_exp2(r), (int)n);
  }
  return t * fast_exp2(fmaf(-z, z, p) * log2e);
}

// erfc fit degree for an output dtype: exact to well below its half-ulp
template <typename T> constexpr int erfc_deg() { return T::code == LUX3D_F32 ? 9 : T::code == LUX3D_F16 ? 7 : 5; }

template <int ACT, int ERFC_DEG = 9> __device__ __forceinline__ float act(float x) {
  if constexpr (ACT == ACT_GELU_TANH) {
    // candle's f32 Gelu: 0.5*x*(1 + tanh(a)), a = sqrt(2/pi)*x*(1 + 0.044715*x^2).
    // tanh(a) = sign(a)*(1 - 2/(1 + exp(2|a|))): near |tanh| = 1 the f32
    // subtraction rounds exactly as the f32 tanh result does, so 1 + tanh(a)
    // cancels as the reference's does (to exactly 0 for a < -9.01) and the
    // negative tail matches the reference instead of the true (tiny) value.
    constexpr float k2 = 2.0f * 1.4426950408889634f;  // 2*log2(e)
    const float a = 0.7978845608028654f * x * (1.0f + 0.044715f * x * x);
    const float m = 1.0f - 2.0f * fast_rcp(1.0f + fast_exp2(k2 * fabsf(a)));  // tanh(|a|)
    return 0.5f * x * (1.0f + __builtin_copysignf(m, a));
  } else if constexpr (ACT == ACT_GELU_ERF) {
    // 0.5*x*(1 + erf(x/sqrt2)) through q = erfc(|x|/sqrt2). For x < 0 the
    // reference forms 1 + erf(z) in f64, where erf(z) = -1 + q is rounded to
    // the f64 grid near -1 (spacing 2^-53): 1 + erf(z) is q rounded to a
    // multiple of 2^-53 (a no-op for q >= 2^-30, exactly 0 below 2^-54), which
    // is applied here so the negative tail matches the reference.
    const float q = erfc_nonneg<ERFC_DEG>(fabsf(x) * 0.7071067811865476f);
    if (x >= 0.f) return x - 0.5f * x * q;
    return x * (__builtin_rintf(q * 0x1p53f) * 0x1p-54f);
  } else {
    constexpr float k = -1.4426950408889634f;  // -log2(e)
    return x * fast_rcp(1.0f + fast_exp2(k * x));
  }
}

template <typename T, int ACT, int U = kUnroll, int BLOCK = kBlock>
__global__ __launch_bounds__(BLOCK) void act_kernel(const void *x, void *y, int64_t nchunks) {
  constexpr int EB = T::bytes;
  const int64_t base = (int64_t)blockIdx.x * BLOCK * U + threadIdx.x;
  float v[U][8];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t c = base + u * BLOCK;
    if (c < nchunks) Chunk<T>::load(reinterpret_cast<const char *>(x) + c * 8 * EB, v[u]);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t c = base + u * BLOCK;
    if (c < nchunks) {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[u][k] = act<ACT, erfc_deg<T>()>(v[u][k]);
      Chunk<T>::store(reinterpret_cast<char *>(y) + c * 8 * EB, v[u]);
    }
  }
}

// Elements [first, n) one per thread (tails and unaligned tensors).
template <typename T, int ACT>
__global__ __launch_bounds__(kBlock) void act_kernel_any(const void *x, void *y, int64_t first,
                                                         int64_t n) {
  const int64_t i = first + (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) store1<T>(y, i, act<ACT, erfc_deg<T>()>(load1<T>(x, i)));
}

template <typename T, int ACT>
hipError_t launch_act_t(const void *x, void *y, int64_t n, bool vec, hipStream_t s) {
  int64_t first = 0;
  if (vec) {
    const int64_t nchunks = n / 8;
    if (nchunks > 0) {
      const int64_t per_block = (int64_t)kActBlock * kUnroll;
      hipLaunchKernelGGL((act_kernel<T, ACT, kUnroll, kActBlock>),
                         dim3((unsigned)((nchunks + per_block - 1) / per_block)), dim3(kActBlock), 0, s, x, y,
                         nchunks);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    first = nchunks * 8;
  }
  const int64_t rest = n - first;
  if (rest > 0) {
    hipLaunchKernelGGL((act_kernel_any<T, ACT>), dim3((unsigned)((rest + kBlock - 1) / kBlock)),
                       dim3(kBlock), 0, s, x, y, first, n);
    return hipGetLastError();
  }
  return hipSuccess;
}

template <typename T>
hipError_t launch_act_dt(int a, const void *x, void *y, int64_t n, bool vec, hipStream_t s) {
  switch (a) {
    case ACT_GELU_ERF: return launch_act_t<T, ACT_GELU_ERF>(x, y, n, vec, s);
    case ACT_GELU_TANH: return launch_act_t<T, ACT_GELU_TANH>(x, y, n, vec, s);
    case ACT_SILU: return launch_act_t<T, ACT_SILU>(x, y, n, vec, s);
  }
  return hipErrorInvalidValue;
}

// ---- timestep embedding ------------------------------------------------------

__global__ __launch_bounds__(kBlock) void timestep_kernel(const float *t, int64_t n,
                                                          const float *freqs, int64_t dim,
                                                          int cos_first, float neg_log_period,
                                                          float *out) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= n * dim) return;
  const int64_t r = e / dim, j = e % dim;
  const int64_t half = dim / 2;
  if (j >= 2 * half) {  // odd dim: zero pad (cos-first convention only)
    out[e] = 0.f;
    return;
  }
  const int64_t i = j < half ? j : j - half;
  float f;
  if (freqs) {
    f = freqs[i];
  } else {
    // exp(-ln(1e4)*i/half): the f32 argument is formed exactly as the
    // reference does; the exponential is evaluated in f64 and rounded once.
    const float x = neg_log_period * (float)i / (float)half;
    f = (float)exp((double)x);
  }
  const float arg = t[r] * f;
  float sv, cv;
  sincosf(arg, &sv, &cv);
  const bool first_half = j < half;
  out[e] = cos_first ? (first_half ? cv : sv) : (first_half ? sv : cv);
}

// ---- Q8_0 dequant ------------------------------------------------------------
// Thread g produces output chunk g (8 values): block g/4, quarter g%4. The
// 34-byte blocks are only 2-byte aligned, so the scale and the 8 quants are
// read as 16-bit words; the stores are 16-byte (bf16/f16) or 32-byte (f32).

__device__ __forceinline__ uint32_t f32_to_f16_bits_exact(float v) {
  // IEEE binary16 round-to-nearest-even; NaN quiet with its top payload.
  const uint32_t x = __float_as_uint(v);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xFFu;
  const uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFFu) return sign | 0x7C00u | (man ? (0x0200u | (man >> 13)) : 0u);
  const int e = (int)exp - 127 + 15;
  if (e >= 0x1F) return sign | 0x7C00u;
  if (e <= 0) {
    if (e < -10) return sign;
    const uint32_t m = man | 0x800000u;
    const uint32_t shift = (uint32_t)(14 - e);
    uint32_t hm = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (hm & 1u))) hm += 1u;
    return sign | hm;
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return h;
}

template <int OUT>
__global__ __launch_bounds__(kBlock) void dequant_q8_0_kernel(const uint8_t *blocks, int64_t nchunks,
                                                              void *y, int vec) {
  const int64_t g = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (g >= nchunks) return;
  const int64_t blk = g >> 2;
  const int q = (int)(g & 3);
  const uint16_t *w = reinterpret_cast<const uint16_t *>(blocks + blk * 34);
  const float d = f16_bits_to_f32(w[0]);
  float v[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint16_t pair = w[1 + q * 4 + k];
    v[2 * k] = (float)(int8_t)(pair & 0xFFu) * d;
    v[2 * k + 1] = (float)(int8_t)(pair >> 8) * d;
  }
  if constexpr (OUT == LUX3D_F32) {
    float *o = reinterpret_cast<float *>(y) + g * 8;
    if (vec) {
      Chunk<F32>::store(o, v);
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) o[k] = v[k];
    }
  } else {
    uint32_t hb[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      hb[k] = OUT == LUX3D_BF16 ? f32_to_bf16_bits_exact(v[k]) : f32_to_f16_bits_exact(v[k]);
    uint16_t *o = reinterpret_cast<uint16_t *>(y) + g * 8;
    if (vec) {
      uint4 u;
      u.x = hb[0] | (hb[1] << 16);
      u.y = hb[2] | (hb[3] << 16);
      u.z = hb[4] | (hb[5] << 16);
      u.w = hb[6] | (hb[7] << 16);
      *reinterpret_cast<uint4 *>(o) = u;
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) o[k] = (uint16_t)hb[k];
    }
  }
}

// Staged variant for 16-byte aligned block buffers: a workgroup's 64 blocks
// are one contiguous span of 2,176 bytes (136 x 16), loaded with 16-byte
// loads into LDS; each thread then converts its 8 values from there (the
// direct kernel issues five 2-byte loads per thread, because the 34-byte
// records are only 2-byte aligned). configs[4]: 4.11 us against 4.35 us.
// Output bit-identical to dequant_q8_0_kernel.
constexpr int kDqBlocksPerGroup = kBlock / 4;

template <int OUT>
__global__ __launch_bounds__(kBlock) void dequant_q8_0_staged(const uint8_t *blocks, int64_t nblocks, void *y) {
  constexpr int BYTES = kDqBlocksPerGroup * 34;
  static_assert(BYTES % 16 == 0, "the span must be whole 16-byte chunks");
  __shared__ __align__(16) uint8_t span[BYTES];
  const int64_t b0 = (int64_t)blockIdx.x * kDqBlocksPerGroup;
  const int64_t end = (nblocks - b0) * 34;  // bytes of this group's span that exist
  const uint8_t *src = blocks + b0 * 34;
  for (int c = threadIdx.x; c < BYTES / 16; c += kBlock) {
    const int64_t o = (int64_t)c * 16;
    if (o + 16 <= end) {
      *reinterpret_cast<uint4 *>(span + o) = ld16(src + o);
    } else {
      for (int k = 0; k < 16; k += 2)  // ragged tail: 2-byte pieces (records are 2-byte aligned)
        if (o + k < end) *reinterpret_cast<uint16_t *>(span + o + k) = *reinterpret_cast<const uint16_t *>(src + o + k);
    }
  }
  lds_barrier();
  const int lb = threadIdx.x >> 2, q = threadIdx.x & 3;
  const int64_t blk = b0 + lb;
  if (blk >= nblocks) return;
  const uint16_t *w = reinterpret_cast<const uint16_t *>(span + lb * 34);
  const float d = f16_bits_to_f32(w[0]);
  float v[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint16_t pair = w[1 + q * 4 + k];
    v[2 * k] = (float)(int8_t)(pair & 0xFFu) * d;
    v[2 * k + 1] = (float)(int8_t)(pair >> 8) * d;
  }
  const int64_t g = blk * 4 + q;
  if constexpr (OUT == LUX3D_F32) {
    Chunk<F32>::store(reinterpret_cast<float *>(y) + g * 8, v);
  } else {
    // q * d is exact in f32, so every product is finite while the scale is:
    // the hardware round-to-nearest-even converts (identical to the exact
    // conversion for non-NaN values) then give the exact result. A block
    // with an infinite or NaN scale (NaN products carry a payload) takes the
    // exact software conversion.
    uint4 u;
    if (__builtin_isfinite(d)) {
      if constexpr (OUT == LUX3D_BF16) {
        u.x = pack_bf16x2(v[0], v[1]); u.y = pack_bf16x2(v[2], v[3]);
        u.z = pack_bf16x2(v[4], v[5]); u.w = pack_bf16x2(v[6], v[7]);
      } else {
        u.x = pack_f16x2(v[0], v[1]); u.y = pack_f16x2(v[2], v[3]);
        u.z = pack_f16x2(v[4], v[5]); u.w = pack_f16x2(v[6], v[7]);
      }
    } else {
      uint32_t hb[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        hb[k] = OUT == LUX3D_BF16 ? f32_to_bf16_bits_exact(v[k]) : f32_to_f16_bits_exact(v[k]);
      u.x = hb[0] | (hb[1] << 16);
      u.y = hb[2] | (hb[3] << 16);
      u.z = hb[4] | (hb[5] << 16);
      u.w = hb[6] | (hb[7] << 16);
    }
    st16(reinterpret_cast<uint16_t *>(y) + g * 8, u);
  }
}

}  // namespace

hipError_t launch_act(int a, int dt, const void *x, void *y, int64_t n, bool vec, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  switch (dt) {
    case LUX3D_F32: return launch_act_dt<F32>(a, x, y, n, vec, s);
    case LUX3D_BF16: return launch_act_dt<BF16>(a, x, y, n, vec, s);
    case LUX3D_F16: return launch_act_dt<F16>(a, x, y, n, vec, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_timestep(const float *t, int64_t n, const float *freqs, int64_t dim, int cos_first,
                           float neg_log_period, float *out, hipStream_t s) {
  const int64_t total = n * dim;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(timestep_kernel, dim3((unsigned)((total + kBlock - 1) / kBlock)), dim3(kBlock), 0, s,
                     t, n, freqs, dim, cos_first, neg_log_period, out);
  return hipGetLastError();
}

hipError_t launch_dequant_q8_0(const uint8_t *blocks, int64_t nblocks, int out_dt, void *y, bool vec,
                               hipStream_t s) {
  const int64_t nchunks = nblocks * 4;
  if (nchunks <= 0) return hipSuccess;
  if (vec && (reinterpret_cast<uintptr_t>(blocks) & 15u) == 0) {
    const dim3 sgrid((unsigned)((nblocks + kDqBlocksPerGroup - 1) / kDqBlocksPerGroup));
    switch (out_dt) {
      case LUX3D_F32: hipLaunchKernelGGL(dequant_q8_0_staged<LUX3D_F32>, sgrid, dim3(kBlock), 0, s, blocks, nblocks, y); break;
      case LUX3D_BF16: hipLaunchKernelGGL(dequant_q8_0_staged<LUX3D_BF16>, sgrid, dim3(kBlock), 0, s, blocks, nblocks, y); break;
      case LUX3D_F16: hipLaunchKernelGGL(dequant_q8_0_staged<LUX3D_F16>, sgrid, dim3(kBlock), 0, s, blocks, nblocks, y); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const dim3 grid((unsigned)((nchunks + kBlock - 1) / kBlock));
  switch (out_dt) {
    case LUX3D_F32:
      hipLaunchKernelGGL(dequant_q8_0_kernel<LUX3D_F32>, grid, dim3(kBlock), 0, s, blocks, nchunks, y, (int)vec);
      break;
    case LUX3D_BF16:
      hipLaunchKernelGGL(dequant_q8_0_kernel<LUX3D_BF16>, grid, dim3(kBlock), 0, s, blocks, nchunks, y, (int)vec);
      break;
    case LUX3D_F16:
      hipLaunchKernelGGL(dequant_q8_0_kernel<LUX3D_F16>, grid, dim3(kBlock), 0, s, blocks, nchunks, y, (int)vec);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace lux3d
