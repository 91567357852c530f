// common.hpp -- device helpers shared by the gfx950 kernels of liblux3d_fused:
// dtype traits with 16-byte vector I/O, f32<->bf16/f16 conversions, and
// wavefront reductions built on DPP and the gfx950 permlane swaps.
//
// Element I/O model: every kernel moves "chunks" of 8 consecutive elements
// per lane (one 16-byte load for bf16/f16, two for f32), so a wavefront's
// load instruction covers a contiguous 1 KiB (2-byte types) or 2 KiB (f32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <cstdlib>

#include "lux3d_fused.h"

namespace lux3d {

// ---------------------------------------------------------------------------
// Scalar conversions
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t v) { return __uint_as_float(v << 16); }

// f32 -> bf16, round-to-nearest-even; NaN keeps sign and top payload bits and
// is forced quiet. Bit-identical to half::bf16::from_f32 (used where results
// must be bit-exact: Q8_0 dequant).
__device__ __forceinline__ uint32_t f32_to_bf16_bits_exact(float f) {
  uint32_t x = __float_as_uint(f);
  uint32_t r = (x + 0x7FFFu + ((x >> 16) & 1u)) >> 16;
  return ((x & 0x7FFFFFFFu) > 0x7F800000u) ? ((x >> 16) | 0x40u) : r;
}

// Two f32 -> packed bf16x2 with the gfx950 hardware convert (v_cvt_pk_bf16_f32,
// round-to-nearest-even). Identical to the exact conversion for every non-NaN
// input.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  f32x2_t v = {lo, hi};
  bf16x2_t r = __builtin_convertvector(v, bf16x2_t);
  return __builtin_bit_cast(uint32_t, r);
}

// Exact three-term bf16 split of two f32 values a, b (packed pairs, low half
// = a): a = a1 + a2 + a3. a has 24 significant bits; a1 = RNE_bf16(a) leaves
// a remainder of at most 16 significant bits, a2 = RNE_bf16 of that one of at
// most 8, which bf16 holds exactly (bf16 has f32's exponent range). Exact
// while a3 stays a normal number, i.e. for |a| above about 2^-110 (below, the
// lost part is under 2^-126 in absolute terms), and while a1 does not round
// to infinity, i.e. for |a| below 2^128 (1 - 2^-9) ~ 3.39e38. An infinite or
// NaN a gives NaN terms.
struct Split3 {
  uint32_t t1, t2, t3;
};
__device__ __forceinline__ Split3 split3_bf16(float a, float b) {
  Split3 r;
  r.t1 = pack_bf16x2(a, b);
  const float ra = a - __uint_as_float(r.t1 << 16), rb = b - __uint_as_float(r.t1 & 0xffff0000u);
  r.t2 = pack_bf16x2(ra, rb);
  r.t3 = pack_bf16x2(ra - __uint_as_float(r.t2 << 16), rb - __uint_as_float(r.t2 & 0xffff0000u));
  return r;
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  f32x2_t v = {lo, hi};
  f16x2_t r = __builtin_convertvector(v, f16x2_t);
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t v) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)v);
}

// ---------------------------------------------------------------------------
// Rounding control. HIP compiles with floating-point contraction on, so
// `a * b + c` (also when written with __fmul_rn / __fadd_rn, which are plain
// operators in this toolchain) may become one FMA with a single rounding.
// mul_rn / add_rn are never contracted: each is one IEEE f32 operation,
// rounded on its own, as the reference's Rust (which never contracts)
// computes. Used where a result must match the reference bit for bit (the
// residual streams).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
// One rotated element y*c + p*s (p: the element's rotation partner) as
// fma(y, c, p*s): one rounding fewer than the reference's separately rounded
// products and sum (at most 1 f32 ulp apart before the output rounding, well
// inside the parity tolerance), and one instruction fewer per element. Every
// kernel that rotates uses this form, so their results agree bit for bit.
__device__ __forceinline__ float rotate1(float y, float c, float p, float s) {
  return __builtin_fmaf(y, c, mul_rn(p, s));
}

// ---------------------------------------------------------------------------
// 16-byte streaming accesses. Activations are touched exactly once per op, so
// they are loaded and stored non-temporally (the "nt" cache policy: streamed
// through L2 / the Infinity Cache without displacing reused data such as the
// per-channel parameters). LUX3D_NT_STREAMS=0 selects plain accesses (used to
// measure the difference).
// ---------------------------------------------------------------------------
#ifndef LUX3D_NT_STREAMS
#define LUX3D_NT_STREAMS 1
#endif

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <bool NT = (LUX3D_NT_STREAMS != 0)>
__device__ __forceinline__ uint4 ld16(const void *p) {
  if constexpr (NT) {
    u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
  } else {
    return *reinterpret_cast<const uint4 *>(p);
  }
}

template <bool NT = (LUX3D_NT_STREAMS != 0)>
__device__ __forceinline__ void st16(void *p, uint4 v) {
  if constexpr (NT) {
    u32x4_t t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<u32x4_t *>(p));
  } else {
    *reinterpret_cast<uint4 *>(p) = v;
  }
}

// ---------------------------------------------------------------------------
// dtype tags and 8-element chunk I/O
// ---------------------------------------------------------------------------

struct F32 { static constexpr int code = LUX3D_F32; static constexpr int bytes = 4; };
struct BF16 { static constexpr int code = LUX3D_BF16; static constexpr int bytes = 2; };
struct F16 { static constexpr int code = LUX3D_F16; static constexpr int bytes = 2; };

template <typename T> struct Chunk;

template <> struct Chunk<BF16> {
  template <bool NT = (LUX3D_NT_STREAMS != 0)>
  __device__ __forceinline__ static void load(const void *p, float (&v)[8]) {
    uint4 u = ld16<NT>(p);
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  }
  __device__ __forceinline__ static void store(void *p, const float (&v)[8]) {
    uint4 u;
    u.x = pack_bf16x2(v[0], v[1]);
    u.y = pack_bf16x2(v[2], v[3]);
    u.z = pack_bf16x2(v[4], v[5]);
    u.w = pack_bf16x2(v[6], v[7]);
    st16(p, u);
  }
  // value as it reads back after a store (for outputs that are re-read)
  __device__ __forceinline__ static float round_trip(float f) {
    return __uint_as_float(pack_bf16x2(f, 0.f) << 16);
  }
};

template <> struct Chunk<F16> {
  template <bool NT = (LUX3D_NT_STREAMS != 0)>
  __device__ __forceinline__ static void load(const void *p, float (&v)[8]) {
    uint4 u = ld16<NT>(p);
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = f16_bits_to_f32(w[i] & 0xFFFFu);
      v[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
    }
  }
  __device__ __forceinline__ static void store(void *p, const float (&v)[8]) {
    uint4 u;
    u.x = pack_f16x2(v[0], v[1]);
    u.y = pack_f16x2(v[2], v[3]);
    u.z = pack_f16x2(v[4], v[5]);
    u.w = pack_f16x2(v[6], v[7]);
    st16(p, u);
  }
  __device__ __forceinline__ static float round_trip(float f) {
    return f16_bits_to_f32(pack_f16x2(f, 0.f) & 0xFFFFu);
  }
};

template <> struct Chunk<F32> {
  template <bool NT = (LUX3D_NT_STREAMS != 0)>
  __device__ __forceinline__ static void load(const void *p, float (&v)[8]) {
    const char *c = reinterpret_cast<const char *>(p);
    uint4 a = ld16<NT>(c), b = ld16<NT>(c + 16);
    v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
    v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y); v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
  }
  __device__ __forceinline__ static void store(void *p, const float (&v)[8]) {
    char *c = reinterpret_cast<char *>(p);
    st16(c, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])));
    st16(c + 16, make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])));
  }
  __device__ __forceinline__ static float round_trip(float f) { return f; }
};

// Scalar element access for the unaligned / odd-size fallback kernels.
template <typename T> __device__ __forceinline__ float load1(const void *p, int64_t i);
template <> __device__ __forceinline__ float load1<F32>(const void *p, int64_t i) {
  return reinterpret_cast<const float *>(p)[i];
}
template <> __device__ __forceinline__ float load1<BF16>(const void *p, int64_t i) {
  return bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
}
template <> __device__ __forceinline__ float load1<F16>(const void *p, int64_t i) {
  return f16_bits_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
}
template <typename T> __device__ __forceinline__ void store1(void *p, int64_t i, float v);
template <> __device__ __forceinline__ void store1<F32>(void *p, int64_t i, float v) {
  reinterpret_cast<float *>(p)[i] = v;
}
template <> __device__ __forceinline__ void store1<BF16>(void *p, int64_t i, float v) {
  reinterpret_cast<uint16_t *>(p)[i] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xFFFFu);
}
template <> __device__ __forceinline__ void store1<F16>(void *p, int64_t i, float v) {
  reinterpret_cast<uint16_t *>(p)[i] = (uint16_t)(pack_f16x2(v, 0.f) & 0xFFFFu);
}

// Per-channel parameters of any supported float dtype (runtime code, uniform
// across the wavefront). `dt < 0` means "absent" and yields `dflt`.
__device__ __forceinline__ float param1(const void *p, int dt, int64_t i, float dflt) {
  if (dt == LUX3D_F32) return reinterpret_cast<const float *>(p)[i];
  if (dt == LUX3D_BF16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
  if (dt == LUX3D_F16) return f16_bits_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
  return dflt;
}

// 8 consecutive parameters starting at element i (i a multiple of 8 and the
// base 16-byte aligned: checked on the host before a vector kernel is chosen).
__device__ __forceinline__ void param8(const void *p, int dt, int64_t i, float dflt, float (&v)[8]) {
  // parameters are re-read by every row: plain (cached) loads
  if (dt == LUX3D_F32) {
    Chunk<F32>::load<false>(reinterpret_cast<const float *>(p) + i, v);
  } else if (dt == LUX3D_BF16) {
    Chunk<BF16>::load<false>(reinterpret_cast<const uint16_t *>(p) + i, v);
  } else if (dt == LUX3D_F16) {
    Chunk<F16>::load<false>(reinterpret_cast<const uint16_t *>(p) + i, v);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = dflt;
  }
}

// 4 consecutive parameters starting at element i (i a multiple of 4, the
// base 16-byte aligned), cached loads, or dflt.
__device__ __forceinline__ void param4(const void *p, int dt, int64_t i, float dflt, float *v) {
  if (dt == LUX3D_F32) {
    const float4 a = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(p) + i);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  } else if (dt == LUX3D_BF16 || dt == LUX3D_F16) {
    const uint2 a = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(p) + i);
    const uint32_t w[2] = {a.x, a.y};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t h = (w[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
      v[k] = dt == LUX3D_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = dflt;
  }
}
// Compute units of the stream's device, looked up once per device (256 on
// MI355X, and the value used if the lookup fails).
inline int cu_count(hipStream_t s) {
  static std::atomic<int> cus[64];  // 0: not looked up yet
  const int dev = hipGetStreamDeviceId(s);
  if (dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}
// Dynamic LDS bytes for a launch whose kernel uses `used` bytes, raised so
// that at most `wg_per_cu` of its workgroups are resident on a CU (the extra
// bytes are a reservation the kernel never touches). Some streaming kernels
// run fastest with fewer resident workgroups than their registers allow:
// past that point more loads in flight only queue at the memory controllers
// (sweeps of the reservation in one process: configs[1] F1 18.04 -> 17.67 us
// at 6 workgroups of 256 threads per CU, configs[3] modulate 66.0 -> 64.4 us
// at 2 of 512; the launchers state each cap they set). The CU's LDS size comes
// from the device attribute, looked up once per device; if the lookup fails
// no reservation is added. LUX3D_OCCUPANCY_CAP=0 in the environment turns
// the reservations off (read at every launch, for A/B timing in one process).
inline size_t lds_for_occupancy(hipStream_t s, int wg_per_cu, size_t used) {
  static std::atomic<int> lds_per_cu[64];  // 0: not looked up yet, -1: unknown
  const char *off = getenv("LUX3D_OCCUPANCY_CAP");
  if (off && off[0] == '0') return used;
  int dev = hipGetStreamDeviceId(s);
  if (dev < 0 || dev >= 64) return used;
  int lds = lds_per_cu[dev].load(std::memory_order_relaxed);
  if (lds == 0) {
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess ||
        lds <= 0)
      lds = -1;
    lds_per_cu[dev].store(lds, std::memory_order_relaxed);
  }
  if (lds < 0 || wg_per_cu < 1) return used;
  const size_t want = (size_t)lds / (size_t)(wg_per_cu + 1) + 1;  // wg_per_cu + 1 of them do not fit
  return used > want ? used : want;
}

// Keeps the machine scheduler from moving instructions across this point:
// it orders loads for latency and register pressure, not for vmcnt, and so
// would sink a small early load (a position, a parameter) below the row
// loads that a wait for it must then also wait for.
__device__ __forceinline__ void issue_fence() { __builtin_amdgcn_sched_barrier(0); }

// Per-channel parameters in two steps, for the kernels whose activation
// loads must stay in flight. vmcnt counts loads and stores together in issue
// order, so a parameter load inside a branch on its dtype whose data the
// branch converts at once (param8) makes the wavefront wait there for every
// earlier load and store. `pissue` issues the raw bytes of 8 parameters --
// elements i..i+3 and j..j+3 -- with no branch on the dtype, through
// bounds-checked buffer loads (bytes past the vector read as 0, an absent
// vector has a zero-size descriptor and reads nothing), and `pdecode`
// converts them where they are used, after the kernel's one wait.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t param_rsrc(const void *p, int dt, int64_t n) {
  int64_t bytes = (dt < 0 || !p) ? 0 : n * (dt == LUX3D_F32 ? 4 : 2);
  if (bytes > 0x7FFFFFFF) bytes = 0x7FFFFFFF;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}
struct PRaw {
  u32x4_t a, b;
};
__device__ __forceinline__ PRaw pissue(rsrc_t r, int dt, int64_t i, int64_t j) {
  const int sh = dt == LUX3D_F32 ? 2 : 1;
  PRaw q;
  q.a = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(i << sh), 0, 0);
  q.b = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(j << sh), 0, 0);
  return q;
}
__device__ __forceinline__ void pdecode(const PRaw &q, int dt, float dflt, float (&v)[8]) {
  if (dt == LUX3D_F32) {
    v[0] = __uint_as_float(q.a.x); v[1] = __uint_as_float(q.a.y);
    v[2] = __uint_as_float(q.a.z); v[3] = __uint_as_float(q.a.w);
    v[4] = __uint_as_float(q.b.x); v[5] = __uint_as_float(q.b.y);
    v[6] = __uint_as_float(q.b.z); v[7] = __uint_as_float(q.b.w);
  } else if (dt == LUX3D_BF16 || dt == LUX3D_F16) {
    const uint32_t w[4] = {q.a.x, q.a.y, q.b.x, q.b.y};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t h = (w[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
      v[k] = dt == LUX3D_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = dflt;
  }
}

template <typename T> __device__ __forceinline__ const char *cptr(const void *p) {
  return reinterpret_cast<const char *>(p);
}

// ---------------------------------------------------------------------------
// Cross-lane exchange and reductions (wave64, gfx950)
// ---------------------------------------------------------------------------

// DPP controls: quad_perm [1,0,3,2] = xor 1, quad_perm [2,3,0,1] = xor 2,
// quad_perm [3,2,1,0] = xor 3, row_half_mirror (lane i of 8 <- 7-i = i^7),
// row_mirror (lane i of 16 <- 15-i = i^15).
enum : int { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_XOR3 = 0x1B, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140 };

template <int CTRL> __device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of 8 / 16 lanes. Every lane of a group ends with
// the bit-identical total (each step adds two equal-valued halves).
__device__ __forceinline__ float group8_sum(float v) {
  v += dpp<DPP_XOR1>(v);
  v += dpp<DPP_XOR2>(v);
  v += dpp<DPP_HALF_MIRROR>(v);
  return v;
}
__device__ __forceinline__ float group16_sum(float v) {
  v = group8_sum(v);
  v += dpp<DPP_MIRROR>(v);
  return v;
}
// Whole-wave sum: 16-lane rows are combined with v_permlane16_swap (rows
// 0<->1, 2<->3) and v_permlane32_swap (lanes 0-31 <-> 32-63).
__device__ __forceinline__ float wave_sum(float v) {
  v = group16_sum(v);
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(b[0]) + __uint_as_float(b[1]);
  return v;
}

template <int LANES> __device__ __forceinline__ float group_sum(float v) {
  static_assert(LANES == 8 || LANES == 16 || LANES == 64, "group size");
  if constexpr (LANES == 8) return group8_sum(v);
  else if constexpr (LANES == 16) return group16_sum(v);
  else return wave_sum(v);
}

// Value held by lane (lane ^ M). xor 4 = xor 3, then xor 7 (two DPP moves);
// xor 8 = xor 7, then xor 15.
template <int M> __device__ __forceinline__ float lane_xor(float v) {
  if constexpr (M == 1) return dpp<DPP_XOR1>(v);
  else if constexpr (M == 2) return dpp<DPP_XOR2>(v);
  else if constexpr (M == 4) return dpp<DPP_HALF_MIRROR>(dpp<DPP_XOR3>(v));
  else if constexpr (M == 8) return dpp<DPP_MIRROR>(dpp<DPP_HALF_MIRROR>(v));
  else return __shfl_xor(v, M, 64);
}

// LayerNorm over a head row held as 8-element chunks: the chunk sums and the
// affine step, shared by every kernel that normalises head rows so that they
// agree bit for bit (the row total is the pairwise tree of chunk sums
// ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)) for 8 chunks).
__device__ __forceinline__ float ln_chunk_sum(const float (&x)[8]) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s += x[k];
  return s;
}
__device__ __forceinline__ float ln_chunk_center_sq(float (&x)[8], float mean) {
  float s2 = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    x[k] -= mean;
    s2 += x[k] * x[k];
  }
  return s2;
}
__device__ __forceinline__ void ln_chunk_affine(float (&x)[8], float rstd, const float (&w)[8], const float (&b)[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) x[k] = x[k] * rstd * w[k] + b[k];
}
// Per-head norm scales from the hardware reciprocal square root (v_rsq_f32,
// within about 1 f32 ulp of 1 / sqrt): one instruction instead of the ~20 of
// a correctly rounded sqrt and divide, evaluated twice per thread in the
// head kernels (configs[1] QK LayerNorm + RoPE: 18.4 against 19.5 us). The
// reference divides by sqrt(var + eps); the difference is far below the
// parity tolerance of every output dtype.
__device__ __forceinline__ float rsqrt_f32(float v) { return __builtin_amdgcn_rsqf(v); }
__device__ __forceinline__ float ln_rstd(float sq_total, float inv_d, float eps) {
  return rsqrt_f32(sq_total * inv_d + eps);
}
// 1 / clamp(sqrt(s), 1e-12, 1e30) for a sum of squares s >= 0 (or NaN):
// rsqrt of max(s, 1e-24); s = inf gives 1e-30 (sqrt(inf) clamps to 1e30);
// a NaN s takes the lower clamp, as candle's maximum(NaN, lo) = lo does.
__device__ __forceinline__ float l2_rnorm(float s) {
  return __builtin_isinf(s) ? 1e-30f : rsqrt_f32(fmaxf(s, 1e-24f));
}
// Per-head RMSNorm and L2 norm of a head row held as 8-element chunks by
// LPR lanes, shared by the head kernels and the attention kernel's Q load so
// that the two agree bit for bit:
//   rms: x = (x * rsqrt(sum(x^2) / D + eps)) * w
//   l2:  x = ((x / clamp(||x||, 1e-12, 1e30)) * g) * sqrt(D)
template <int LPR, int D>
__device__ __forceinline__ void head_rms_chunk(float (&x)[8], const float (&w)[8], float eps) {
  float s2 = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s2 += x[k] * x[k];
  const float rr = rsqrt_f32(group_sum<LPR>(s2) * (1.0f / D) + eps);
#pragma unroll
  for (int k = 0; k < 8; ++k) x[k] = (x[k] * rr) * w[k];
}
template <int LPR, int D> __device__ __forceinline__ void head_l2_chunk(float (&x)[8], const float (&g)[8]) {
  float s2 = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s2 += x[k] * x[k];
  const float rr = l2_rnorm(group_sum<LPR>(s2));
  const float scale = sqrtf((float)D);
#pragma unroll
  for (int k = 0; k < 8; ++k) x[k] = ((x[k] * rr) * g[k]) * scale;
}

// Workgroup barrier that orders LDS only: the fences are scoped to the
// local (LDS) address space, so the wave waits for its own LDS accesses
// (lgkmcnt) but not for outstanding global loads or stores, which stay in
// flight across the barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ int64_t uniform(int64_t v) {
  uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)v);
  uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// x / d for x < 2^31 from the launcher's (m, s) = (ceil(2^s / d), 31 +
// ceil(log2 d)): x m / 2^s exceeds x / d by less than 2^31 / 2^s <= 1 / d,
// which cannot reach the next integer. Three instructions instead of the
// ~10 of a runtime 32-bit division.
__device__ __forceinline__ uint32_t fdiv(uint32_t x, uint32_t m, int s) {
  return (uint32_t)(((uint64_t)x * m) >> s);
}
inline void div_magic(int64_t d, uint32_t &m, int &s) {
  int l = 0;
  while ((int64_t(1) << l) < d) ++l;
  s = 31 + l;
  m = (uint32_t)(((uint64_t(1) << s) + (uint64_t)d - 1) / (uint64_t)d);
}

// Segment of dense row r (equal segments of rows_per_seg rows, magic (m, s)
// of rows_per_seg from div_magic) when every row index is below 2^31:
// three scalar instructions instead of a 64-bit division.
__device__ __forceinline__ int64_t segment_of_dense(uint32_t r, uint32_t m, int s, int64_t nseg) {
  const int64_t q = (int64_t)fdiv(r, m, s);
  return q < nseg ? q : nseg - 1;
}

// Segment of row r given int64 offsets [nseg+1] (largest s with off[s] <= r),
// or equal segments of `rows_per_seg` rows when `off` is NULL. Always returns
// a value in [0, nseg-1], whatever the offsets hold.
__device__ __forceinline__ int64_t segment_of(const int64_t *off, int64_t nseg, int64_t rows_per_seg,
                                              int64_t r) {
  if (!off) {
    int64_t s = r / rows_per_seg;
    return s < nseg ? s : nseg - 1;
  }
  // read through the constant address space: with r uniform over the
  // wavefront (every caller) these are scalar loads, counted by lgkmcnt, so
  // the search does not wait on the wavefront's outstanding vector loads
  typedef const __attribute__((address_space(4))) int64_t *coff_t;
  const coff_t c = (coff_t)off;
  int64_t lo = 0, hi = nseg - 1;
  while (lo < hi) {
    int64_t mid = (lo + hi + 1) >> 1;
    if (c[mid] <= r) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// Direct global -> LDS loads (buffer_load ... lds)
// ---------------------------------------------------------------------------

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// A raw buffer descriptor (no stride, num_records bytes from base) for the
// direct loads; the fields are wave-uniform, readfirstlane keeps them scalar.
__device__ __forceinline__ i32x4_t buffer_rsrc(const void *base, int64_t bytes) {
  const uint64_t b = (uint64_t)base;
  const int n = bytes > 0x7FFFFFFF ? 0x7FFFFFFF : (int)bytes;
  return i32x4_t{(int)__builtin_amdgcn_readfirstlane((uint32_t)b), (int)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)),
                 __builtin_amdgcn_readfirstlane(n), 0x00020000};
}
// Each lane reads 16 (4) bytes at voff + soff of the buffer; the wavefront
// writes them in lane order at LDS byte address lds. Inline assembly rather
// than the compiler's buffer-load-to-LDS builtin: with the builtin the
// compiler knows the LDS is written by a vector-memory load and, unable to
// tell the two buffers of a ring apart, waits for every such load
// (vmcnt(0)) right after issuing the next block's loads in the attention
// loop and after each barrier of the Q8_0 ring, which serialises both
// pipelines; here the callers place their waits themselves. hipcc warns that
// m0 is a reserved register in the clobber list: the statement overwrites
// m0 without the compiler knowing its old value, which is safe only while
// the compiler keeps nothing of its own in m0 in these kernels. The build
// verifies that for every translation unit that calls these (check_m0.py
// over its device assembly: no m0 use outside these pairs), and fails
// otherwise.
__device__ __forceinline__ void lds_load16(i32x4_t rs, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff), "s"(rs), "s"(soff)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_load4(i32x4_t rs, uint32_t voff, uint32_t soff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds" ::"s"(lds), "v"(voff), "s"(rs), "s"(soff)
               : "memory", "m0");
}
// s_waitcnt immediates (gfx9 layout): vmcnt(n) with lgkmcnt(0), and vmcnt(n) alone
constexpr int waitcnt_vm_lgkm0(int n) { return 0x0070 | (n & 15) | ((n >> 4) << 14); }
constexpr int waitcnt_vm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }

}  // namespace lux3d
