// q8_gemm.hip -- the Q8_0 quantized linear for gfx950: y = x * W^T (+ bias)
// with W stored as GGML Q8_0 (int8 values, one scale per 32 along K).
//
// Semantics: W is dequantized exactly as the Q8_0 -> bf16 op does it
// (w = RNE_bf16(f32(q) * d), the product q * d being exact in f32), x is
// bf16, products accumulate in f32 on the matrix cores
// (v_mfma_f32_32x32x16_bf16), the bias is added in f32 and the result is
// rounded once to y's dtype. That is candle's dequantize-then-matmul path
// with a bf16 dequant target.
//
// Weights are first repacked once (q8_0_repack_kernel, the load-time step
// the reference takes in QMatMul::from_qtensor) from 34-byte blocks, which
// are only 2-byte aligned, into int8 [N, K] row-major plus f32 scales
// [N, K/32], so the GEMM streams them with 16-byte loads.
//
// GEMM tiling: a 256-thread workgroup computes a 128 x 128 tile of y; its
// four wavefronts each own 64 x 64 (2 x 2 MFMA tiles of 32 x 32, 64 f32
// accumulators per lane). Per k-step of 32 (one Q8_0 block) the workgroup
// stages x[128 x 32] and the dequantised W[128 x 32] as bf16 in LDS
// (double-buffered, rows padded to 80 bytes against bank conflicts); the
// next k-step's global loads are issued before the current step's MFMAs, so
// one barrier per k-step suffices.
#include "common.hpp"
#include "kernels.hpp"

namespace lux3d {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128, kBK = 32;
constexpr int kLdsRow = kBK + 8;          // bf16 elements per LDS row (80 bytes)
constexpr int kGemmThreads = 256;

// ---- repack: GGML blocks -> int8 [N, K] + f32 scales [N, K/32] -------------

__global__ __launch_bounds__(256) void q8_0_repack_kernel(const uint8_t *blocks, int64_t nblocks, int8_t *qs,
                                                          float *scales) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;  // one thread per 8 values
  if (g >= nblocks * 4) return;
  const int64_t blk = g >> 2;
  const int q = (int)(g & 3);
  const uint16_t *w = reinterpret_cast<const uint16_t *>(blocks + blk * 34);
  uint32_t lo = (uint32_t)w[1 + q * 4] | ((uint32_t)w[2 + q * 4] << 16);
  uint32_t hi = (uint32_t)w[3 + q * 4] | ((uint32_t)w[4 + q * 4] << 16);
  // blocks are row-major over (n, k/32): block blk holds row n = blk / (K/32)
  // values k = (blk % (K/32)) * 32 + ...; so the int8 stream is contiguous
  *reinterpret_cast<uint2 *>(qs + g * 8) = make_uint2(lo, hi);
  if (q == 0) scales[blk] = f16_bits_to_f32(w[0]);
}

// ---- GEMM -------------------------------------------------------------------

template <typename OUT>
__global__ __launch_bounds__(kGemmThreads) void q8_0_gemm_kernel(Q8GemmParams p) {
  __shared__ __align__(16) __bf16 As[2][kBM * kLdsRow];
  __shared__ __align__(16) __bf16 Bs[2][kBN * kLdsRow];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * kBM, n0 = (int64_t)blockIdx.x * kBN;
  const int64_t nk = p.K / kBK;

  // global -> register staging assignments
  // A: 128 rows x 64 bytes = 512 chunks of 16 B; thread t takes chunks t, t + 256
  int64_t a_row[2];
  int a_part[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = t + i * kGemmThreads;
    const int64_t r = m0 + (c >> 2);
    a_row[i] = r < p.M ? r : p.M - 1;  // clamped rows are loaded and never stored
    a_part[i] = c & 3;
  }
  // B: 128 rows x 32 int8 = 256 chunks of 16 B; thread t takes chunk t
  const int b_r = t >> 1, b_part = t & 1;
  const int64_t b_row = n0 + b_r < p.N ? n0 + b_r : p.N - 1;

  const char *xbase = reinterpret_cast<const char *>(p.x);
  uint4 ra[2], rb;
  float rd;
  auto load_step = [&](int64_t kt) {
    const int64_t k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < 2; ++i) ra[i] = ld16(xbase + (a_row[i] * p.ldx + k0 + a_part[i] * 8) * 2);
    rb = ld16(p.qs + b_row * p.K + k0 + b_part * 16);
    rd = p.scales[b_row * nk + kt];
  };
  auto store_step = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = t + i * kGemmThreads;
      *reinterpret_cast<uint4 *>(&As[buf][(c >> 2) * kLdsRow + a_part[i] * 8]) = ra[i];
    }
    // dequant: 16 int8 -> bf16(f32(q) * d), RNE (q * d is exact in f32)
    const uint32_t w4[4] = {rb.x, rb.y, rb.z, rb.w};
    uint32_t pk[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t v = w4[j];
      const float f0 = (float)(int8_t)(v & 0xFFu) * rd, f1 = (float)(int8_t)((v >> 8) & 0xFFu) * rd;
      const float f2 = (float)(int8_t)((v >> 16) & 0xFFu) * rd, f3 = (float)(int8_t)(v >> 24) * rd;
      pk[2 * j] = pack_bf16x2(f0, f1);
      pk[2 * j + 1] = pack_bf16x2(f2, f3);
    }
    uint4 *dst = reinterpret_cast<uint4 *>(&Bs[buf][b_r * kLdsRow + b_part * 16]);
    dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
    dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16_t{};

  load_step(0);
  store_step(0);
  lds_barrier();

  const int lrow = lane & 31, lk = (lane >> 5) * 8;
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = (int)(kt & 1);
    if (kt + 1 < nk) load_step(kt + 1);
#pragma unroll
    for (int s = 0; s < kBK / 16; ++s) {
      bf16x8_t a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const bf16x8_t *>(&As[buf][(wm * 64 + i * 32 + lrow) * kLdsRow + s * 16 + lk]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const bf16x8_t *>(&Bs[buf][(wn * 64 + j * 32 + lrow) * kLdsRow + s * 16 + lk]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_step(buf ^ 1);
    lds_barrier();
  }

  // epilogue: lane holds C[8*(e/4) + 4*(lane/32) + e%4][lane%32] of each tile
  char *ybase = reinterpret_cast<char *>(p.y);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t col = n0 + wn * 64 + j * 32 + (lane & 31);
    if (col >= p.N) continue;
    const float bias = p.bias ? p.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (row >= p.M) continue;
        const float v = acc[i][j][e] + bias;
        if constexpr (OUT::code == LUX3D_F32) {
          reinterpret_cast<float *>(ybase)[row * p.ldy + col] = v;
        } else {
          store1<OUT>(ybase, row * p.ldy + col, v);
        }
      }
  }
}

}  // namespace

hipError_t launch_q8_0_repack(const uint8_t *blocks, int64_t nblocks, int8_t *qs, float *scales, hipStream_t s) {
  if (nblocks <= 0) return hipSuccess;
  const int64_t threads = nblocks * 4;
  hipLaunchKernelGGL(q8_0_repack_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, blocks, nblocks,
                     qs, scales);
  return hipGetLastError();
}

hipError_t launch_q8_0_gemm(int out_dt, const Q8GemmParams &p, hipStream_t s) {
  if (p.M <= 0 || p.N <= 0) return hipSuccess;
  if (p.K <= 0 || p.K % kBK) return hipErrorInvalidValue;
  const int64_t gx = (p.N + kBN - 1) / kBN, gy = (p.M + kBM - 1) / kBM;
  if (gx > INT32_MAX || gy > 65535) return hipErrorInvalidValue;
  const dim3 grid((unsigned)gx, (unsigned)gy), block(kGemmThreads);
  switch (out_dt) {
    case LUX3D_BF16: hipLaunchKernelGGL(q8_0_gemm_kernel<BF16>, grid, block, 0, s, p); break;
    case LUX3D_F16: hipLaunchKernelGGL(q8_0_gemm_kernel<F16>, grid, block, 0, s, p); break;
    case LUX3D_F32: hipLaunchKernelGGL(q8_0_gemm_kernel<F32>, grid, block, 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace lux3d
