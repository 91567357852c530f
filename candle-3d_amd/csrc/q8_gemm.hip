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
// GEMM tiling: a 256-thread workgroup computes a BM x BN tile of y; its four
// wavefronts each own (BM/2) x (BN/2) as 32 x 32 MFMA tiles with f32
// accumulators. Per k-step of BK (two Q8_0 blocks where k allows) the
// workgroup stages x[BM x BK] and the dequantised W[BN x BK] as bf16 in LDS
// (double-buffered, rows padded by 16 bytes against bank conflicts); the
// next k-step's global loads are issued before the current step's MFMAs, so
// one barrier per k-step suffices. Global loads go through the caches: every
// x tile is read by each column block and every weight tile by each row
// block, so L2 and the Infinity Cache serve most of them.
#include "common.hpp"
#include "kernels.hpp"

namespace lux3d {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBK = 32;                   // the k granularity (one Q8_0 block)
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

// Block tile BM x BN, k-step BK (one or two Q8_0 blocks); the four
// wavefronts form a 2 x 2 grid, each owning (BM/2) x (BN/2) = TM x TN MFMA
// tiles of 32 x 32. MINW is the minimum number of wavefronts per SIMD the
// register allocation must allow.
template <typename OUT, int BM, int BN, int BK, int MINW>
__global__ __launch_bounds__(kGemmThreads, MINW) void q8_0_gemm_kernel(Q8GemmParams p) {
  constexpr int TM = BM / 64, TN = BN / 64;
  constexpr int LDS_ROW = BK + 8;                    // bf16 per LDS row (odd multiple of 16 bytes)
  constexpr int A_CPR = BK / 8;                      // 16-byte chunks per x row per k-step
  constexpr int A_CHUNKS = BM * A_CPR / kGemmThreads;
  constexpr int B_CPR = BK / 16;                     // 16-int8 chunks per weight row per k-step
  constexpr int B_CHUNKS = BN * B_CPR / kGemmThreads;
  static_assert(A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile too small for 256 threads");
  static_assert(BK % 32 == 0, "k-steps are whole Q8_0 blocks");
  __shared__ __align__(16) __bf16 As[2][BM * LDS_ROW];
  __shared__ __align__(16) __bf16 Bs[2][BN * LDS_ROW];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t nblk = p.K / 32;  // Q8_0 blocks per weight row
  const int64_t nk = p.K / BK;

  // global -> register staging: x row chunks and weight row chunks. Rows past
  // M (N) are clamped to M - 1 (N - 1): loaded, computed, never stored.
  int64_t a_off[A_CHUNKS];
  int a_lds[A_CHUNKS];
#pragma unroll
  for (int i = 0; i < A_CHUNKS; ++i) {
    const int c = t + i * kGemmThreads, r = c / A_CPR, part = c % A_CPR;
    const int64_t gr = m0 + r < p.M ? m0 + r : p.M - 1;
    a_off[i] = (gr * p.ldx + part * 8) * 2;
    a_lds[i] = r * LDS_ROW + part * 8;
  }
  int64_t b_row[B_CHUNKS];
  int b_part[B_CHUNKS], b_lds[B_CHUNKS];
#pragma unroll
  for (int i = 0; i < B_CHUNKS; ++i) {
    const int c = t + i * kGemmThreads, r = c / B_CPR;
    b_part[i] = c % B_CPR;
    b_row[i] = n0 + r < p.N ? n0 + r : p.N - 1;
    b_lds[i] = r * LDS_ROW + b_part[i] * 16;
  }

  const char *xbase = reinterpret_cast<const char *>(p.x);
  uint4 ra[A_CHUNKS], rb[B_CHUNKS];
  float rd[B_CHUNKS];
  auto load_step = [&](int64_t kt) {
    const int64_t k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) ra[i] = ld16<false>(xbase + a_off[i] + k0 * 2);
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      rb[i] = ld16<false>(p.qs + b_row[i] * p.K + k0 + b_part[i] * 16);
      rd[i] = p.scales[b_row[i] * nblk + k0 / 32 + b_part[i] / 2];
    }
  };
  auto store_step = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) *reinterpret_cast<uint4 *>(&As[buf][a_lds[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      // dequant: 16 int8 -> bf16(f32(q) * d), RNE (q * d is exact in f32)
      const uint32_t w4[4] = {rb[i].x, rb[i].y, rb[i].z, rb[i].w};
      uint32_t pk[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t v = w4[j];
        const float f0 = (float)(int8_t)(v & 0xFFu) * rd[i], f1 = (float)(int8_t)((v >> 8) & 0xFFu) * rd[i];
        const float f2 = (float)(int8_t)((v >> 16) & 0xFFu) * rd[i], f3 = (float)(int8_t)(v >> 24) * rd[i];
        pk[2 * j] = pack_bf16x2(f0, f1);
        pk[2 * j + 1] = pack_bf16x2(f2, f3);
      }
      uint4 *dst = reinterpret_cast<uint4 *>(&Bs[buf][b_lds[i]]);
      dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
      dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
    }
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};

  load_step(0);
  store_step(0);
  lds_barrier();

  const int lrow = lane & 31, lk = (lane >> 5) * 8;
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = (int)(kt & 1);
    if (kt + 1 < nk) load_step(kt + 1);
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      bf16x8_t a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        a[i] = *reinterpret_cast<const bf16x8_t *>(&As[buf][(wm * (BM / 2) + i * 32 + lrow) * LDS_ROW + s * 16 + lk]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        b[j] = *reinterpret_cast<const bf16x8_t *>(&Bs[buf][(wn * (BN / 2) + j * 32 + lrow) * LDS_ROW + s * 16 + lk]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_step(buf ^ 1);
    lds_barrier();
  }

  // epilogue: lane holds C[8*(e/4) + 4*(lane/32) + e%4][lane%32] of each tile
  char *ybase = reinterpret_cast<char *>(p.y);
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t col = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
    if (col >= p.N) continue;
    const float bias = p.bias ? p.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * (BM / 2) + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
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

// Tile choice (measured on MI355X, TFLOP/s at 1029x1024x4096 /
// 4096x2048x8192): 128x128 tiles with 64-deep k-steps, cached global loads
// (each x tile is read by every column block, each weight tile by every row
// block) and two wavefronts per SIMD: 321 / 651. Non-temporal loads: 318 /
// 516; 256x128: 217 / 553; 256x256: 130 / 605; 128x128 with k-steps of 32:
// 277 / 519 (used when K is not a multiple of 64).
template <typename OUT>
hipError_t launch_tiles(const Q8GemmParams &p, hipStream_t s) {
  const dim3 block(kGemmThreads);
#define LUX3D_GEMM_TILE(BM_, BN_, BK_, W_)                                                              \
  {                                                                                                     \
    const dim3 grid((unsigned)((p.N + BN_ - 1) / BN_), (unsigned)((p.M + BM_ - 1) / BM_));              \
    hipLaunchKernelGGL((q8_0_gemm_kernel<OUT, BM_, BN_, BK_, W_>), grid, block, 0, s, p); \
    return hipGetLastError();                                                                           \
  }
  if (p.K % 64 == 0) LUX3D_GEMM_TILE(128, 128, 64, 2)
  LUX3D_GEMM_TILE(128, 128, 32, 1)
#undef LUX3D_GEMM_TILE
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
  if ((p.N + 127) / 128 > INT32_MAX || (p.M + 127) / 128 > 65535) return hipErrorInvalidValue;
  switch (out_dt) {
    case LUX3D_BF16: return launch_tiles<BF16>(p, s);
    case LUX3D_F16: return launch_tiles<F16>(p, s);
    case LUX3D_F32: return launch_tiles<F32>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace lux3d
