// q8_gemm.hip -- the Q8_0 quantized linear for gfx950: y = x * W^T (+ bias)
// with W stored as GGML Q8_0 (int8 values, one scale per 32 along K).
//
// Semantics (bf16 x): W is dequantized exactly as the Q8_0 -> bf16 op does
// it (w = RNE_bf16(f32(q) * d), the product q * d being exact in f32), x is
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
// Three GEMM kernels (each one rounding of the f32 sum per output):
// - q8_0_gemm_ring_kernel (K % 64 == 0, the common case): a workgroup of NW
//   wavefronts (8, or 4 for small shapes) computes a BM x 32 NW tile; x, the
//   int8 weights and the scales stream through a 3-stage LDS ring by direct
//   global->LDS loads; each wavefront dequantises its own 32 weight columns
//   once per k-step.
// - q8_0_gemm_kernel (K % 64 == 32): a 256-thread workgroup computes a
//   128 x 128 tile; x and the dequantised W are staged as bf16 in LDS,
//   double-buffered, through registers.
// - q8_0_gemm_x3_kernel (f32 x, K % 64 == 0): f32 arithmetic on the bf16
//   matrix cores, x split exactly into three bf16 terms, the int8 weights
//   exact in bf16 and each Q8_0 block's scale applied to its block sum.
// Within a k-step the kernels assign k to MFMA sub-steps differently, so
// their outputs can differ in the last bit of the f32 sum; each is
// deterministic.
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

// ---- GEMM through an LDS ring fed by direct loads ---------------------------
//
// One 512-thread workgroup per CU computes a BM x 256 tile of y (BM = 256,
// or 128 for problems too small to give every CU a 256-row tile). Its eight
// wavefronts each own 32 columns and all BM rows (BM / 32 MFMA tiles of
// 32 x 32), so every weight element is dequantised by exactly one wavefront
// and amortised over BM rows of x.
//
// Operands reach LDS by direct global->LDS loads (buffer_load ... lds, 16 or
// 4 bytes per lane, written in lane order at the address in M0) through a
// RING_STAGES-deep ring; no global load targets registers inside the k loop,
// so the loads of the next stages stay in flight across k-steps. One stage
// (k-step of 64) holds:
//   x       BM rows x 128 bytes, chunk c of row r in slot c ^ ((r >> 1) & 7)
//           (conflict-free fragment reads without padding);
//   weights per wavefront 2 KB: lane l's 16-byte half q (q = 0, 1) of the
//           32 int8 it needs at q * 1024 + l * 16;
//   scales  per wavefront 256 bytes: lane l's f32 scale at l * 4.
// k order: within a k-step, lane half h (lane / 32) of sub-step s holds
// k = 32 h + 8 s + e (e < 8) for both operands, so each lane's weight bytes
// for the step are 32 contiguous int8 of one Q8_0 block with one scale.
// The loads are inline assembly: the compiler then neither counts them nor
// inserts conservative waits for them, and the waits below are explicit
// (vmcnt counts a wavefront's own loads in issue order).
//
// Sub-steps are software-pipelined: the fragments and dequantised weights of
// sub-step s + 1 are produced while the MFMAs of s run; the barrier sits
// before the last sub-step's MFMAs, which then overlap the first reads of the
// next stage. The epilogue stages each wavefront's block through the ring
// (bias added, rounded once) and writes whole 16-byte row pieces.

constexpr int kRingStages = 3;
constexpr int kRingThreads = 512;

// 8 int8 (two dwords) -> bf16(f32(q) * d), RNE; q * d is exact in f32
__device__ __forceinline__ bf16x8_t dequant8(uint32_t lo, uint32_t hi, float d) {
  uint32_t pk[4];
  const uint32_t w2[2] = {lo, hi};
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t v = w2[j];
    const float f0 = (float)(int8_t)(v & 0xFFu) * d, f1 = (float)(int8_t)((v >> 8) & 0xFFu) * d;
    const float f2 = (float)(int8_t)((v >> 16) & 0xFFu) * d, f3 = (float)(int8_t)(v >> 24) * d;
    pk[2 * j] = pack_bf16x2(f0, f1);
    pk[2 * j + 1] = pack_bf16x2(f2, f3);
  }
  return __builtin_bit_cast(bf16x8_t, make_uint4(pk[0], pk[1], pk[2], pk[3]));
}

// Needs K % 64 == 0 and every descriptor extent below 2^31 bytes (checked by
// the dispatcher). Tile order: workgroup ids are dealt round-robin to the 8
// XCDs; they are renumbered so that each XCD takes a contiguous range, walked
// in groups of GM row tiles (columns fastest within a group), so the tiles
// running on one XCD share x rows and weight columns in its L2.
template <typename OUT, int GM, int BM, int NW = 8>
__global__ __launch_bounds__(64 * NW, 1) void q8_0_gemm_ring_kernel(Q8GemmParams p, int tiles_m, int tiles_n) {
  // NW wavefronts, each owning 32 columns: BN = 32 NW (256 or 128); BM a multiple of 32 up to 256
  constexpr int BN = 32 * NW, BK = 64, TM = BM / 32, NS = kRingStages;
  constexpr int RW = BN * 64, RS = BN * 8;          // weights and scales per stage
  constexpr int kRingA = BM * 128, kRingStage = kRingA + RW + RS;  // 51,200 / 34,816 / 25,600 bytes
  constexpr int SEGW = BM / (8 * NW);              // x segments (1 KB = 8 rows) per wavefront
  constexpr int kRingOps = SEGW + 2 + 1;           // direct loads per wavefront per stage
  static_assert(BM % 32 == 0 && BM <= 256 && BM % (8 * NW) == 0 && (NW == 4 || NW == 8) && SEGW >= 1,
                "tile shape");
  __shared__ __align__(16) char ring[NS * kRingStage];

  const int G = tiles_m * tiles_n, bid = (int)blockIdx.x;
  const int per = G / 8, rem = G % 8, xcd = bid % 8, pos = bid / 8;
  const int lid = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + pos;
  const int group = lid / (GM * tiles_n), first_m = group * GM;
  const int gsize = tiles_m - first_m < GM ? tiles_m - first_m : GM;
  const int in_group = lid - group * GM * tiles_n;
  const int tm = first_m + in_group % gsize, tn = in_group / gsize;

  const int t = threadIdx.x;
  const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5, lrow = lane & 31;
  const int64_t m0 = (int64_t)tm * BM, c0 = (int64_t)tn * BN;
  const int64_t ncol = c0 + wave * 32 + lrow, nc = ncol < p.N ? ncol : p.N - 1;  // past N: clamped, never stored
  const int64_t nblk = p.K / 32;
  const int nk = (int)(p.K / BK);

  // direct-load sources: descriptors on the tile's first row / column, a
  // fixed per-lane offset, the k-step advance in the scalar offset
  uint32_t xoff[SEGW];
#pragma unroll
  for (int i = 0; i < SEGW; ++i) {
    const int g = wave * SEGW + i;  // 1 KB segment = 8 rows
    const int r = 8 * g + (lane >> 3), c = (lane & 7) ^ ((r >> 1) & 7);
    const int64_t gr = m0 + r < p.M ? m0 + r : p.M - 1;  // rows past M: clamped, never stored
    xoff[i] = (uint32_t)(((gr - m0) * p.ldx + 8 * c) * 2);
  }
  // each descriptor spans just the tile's rows / columns
  const int64_t last_row = p.M - 1 - m0 < BM - 1 ? p.M - 1 - m0 : BM - 1;
  const int64_t ncols = p.N - c0 < BN ? p.N - c0 : BN;
  const i32x4_t xr = buffer_rsrc(reinterpret_cast<const char *>(p.x) + m0 * p.ldx * 2, (last_row * p.ldx + p.K) * 2);
  const i32x4_t wr = buffer_rsrc(p.qs + c0 * p.K, ncols * p.K);
  const i32x4_t sr = buffer_rsrc(p.scales + c0 * nblk, ncols * nblk * 4);
  const uint32_t woff = (uint32_t)((nc - c0) * p.K + 32 * h);
  const uint32_t soff = (uint32_t)(((nc - c0) * nblk + h) * 4);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)ring;
  auto issue = [&](int kt, int buf) {
    const uint32_t st = lds0 + buf * kRingStage;
#pragma unroll
    for (int i = 0; i < SEGW; ++i)
      lds_load16(xr, xoff[i], (uint32_t)kt * BK * 2, __builtin_amdgcn_readfirstlane(st + (wave * SEGW + i) * 1024));
    lds_load16(wr, woff, (uint32_t)kt * BK, __builtin_amdgcn_readfirstlane(st + kRingA + wave * 2048));
    lds_load16(wr, woff, (uint32_t)kt * BK + 16, __builtin_amdgcn_readfirstlane(st + kRingA + wave * 2048 + 1024));
    lds_load4(sr, soff, (uint32_t)kt * 8, __builtin_amdgcn_readfirstlane(st + kRingA + RW + wave * 256));
  };

  // fragment of M-tile i, sub-step s at fbase[s] + i * 4096 (the swizzle only
  // depends on the row within a 32-row tile)
  int fbase[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) fbase[s] = lrow * 128 + (((4 * h + s) ^ ((lrow >> 1) & 7)) << 4);
  uint4 w0, w1;
  float sc;
  auto read_w = [&](const char *st) {
    w0 = *reinterpret_cast<const uint4 *>(st + kRingA + wave * 2048 + lane * 16);
    w1 = *reinterpret_cast<const uint4 *>(st + kRingA + wave * 2048 + 1024 + lane * 16);
    sc = *reinterpret_cast<const float *>(st + kRingA + RW + wave * 256 + lane * 4);
  };
  auto make_b = [&](int s) {
    const uint4 &v = s < 2 ? w0 : w1;
    return (s & 1) ? dequant8(v.z, v.w, sc) : dequant8(v.x, v.y, sc);
  };
  auto read_a = [&](const char *st, int s, bf16x8_t (&a)[TM]) {
#pragma unroll
    for (int i = 0; i < TM; ++i) a[i] = *reinterpret_cast<const bf16x8_t *>(st + fbase[s] + i * 4096);
  };
  f32x16_t acc[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) acc[i] = f32x16_t{};
  auto mfmas = [&](const bf16x8_t (&a)[TM], bf16x8_t b) {
#pragma unroll
    for (int i = 0; i < TM; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b, acc[i], 0, 0, 0);
  };

  // Prologue: stages 0 .. NS-2. The loop body is branch-free: past the last
  // k-step it reloads the last stage (in bounds) into a slot that is not read
  // for data again, so the wait counts are the same every step.
#pragma unroll
  for (int st = 0; st < NS - 1; ++st) issue(st < nk ? st : nk - 1, st);
  __builtin_amdgcn_s_waitcnt(waitcnt_vm((NS - 2) * kRingOps));  // stage 0 landed
  __builtin_amdgcn_s_barrier();

  bf16x8_t a0[TM], a1[TM], b0, b1;
  read_w(ring);
  read_a(ring, 0, a0);
  b0 = make_b(0);
  for (int kt = 0; kt < nk; ++kt) {
    // the slot refilled here was last read in step kt - 1, before its barrier
    issue(kt + NS - 1 < nk ? kt + NS - 1 : nk - 1, (kt + NS - 1) % NS);
    __builtin_amdgcn_sched_barrier(0);
    const char *st = ring + (kt % NS) * kRingStage;
    read_a(st, 1, a1);
    b1 = make_b(1);
    mfmas(a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    read_a(st, 2, a0);
    b0 = make_b(2);
    mfmas(a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    read_a(st, 3, a1);
    b1 = make_b(3);
    mfmas(a0, b0);
    __builtin_amdgcn_sched_barrier(0);
    // stage kt + 1 landed (only the stages issued after it may be in flight)
    // and this wavefront's reads of stage kt are done; then every one's
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0((NS - 2) * kRingOps));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const char *nx = ring + ((kt + 1) % NS) * kRingStage;
    read_w(nx);
    read_a(nx, 0, a0);
    mfmas(a1, b1);
    b0 = make_b(0);
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));  // the trailing reloads and reads

  char *ybase = reinterpret_cast<char *>(p.y);
  const float bias = (p.bias && ncol < p.N) ? p.bias[ncol] : 0.f;
  constexpr int EB = OUT::code == LUX3D_F32 ? 4 : 2;
  if (((uintptr_t)p.y % 16 == 0) && ((p.ldy * EB) % 16 == 0)) {
    // stage the wavefront's BM x 32 block through the ring, RP rows per
    // pass (rows padded by 16 bytes), and store whole 16-byte row pieces
    constexpr int ROW_B = 32 * EB, LROW = ROW_B + 16, CPR = ROW_B / 16, EPC = 16 / EB;
    // RP rows per pass: a multiple of 32 that divides BM and fits the ring
    constexpr int CAP = NS * kRingStage;
    constexpr int RP = NW * BM * LROW <= CAP ? BM
                       : (BM % 128 == 0 && NW * 128 * LROW <= CAP) ? 128
                       : (BM % 64 == 0 && NW * 64 * LROW <= CAP) ? 64 : 32;
    constexpr int REGION = RP * LROW;
    static_assert(NW * REGION <= CAP && BM % RP == 0, "epilogue staging fits the ring");
    __builtin_amdgcn_s_barrier();  // every wavefront is done with the ring
    char *reg = ring + wave * REGION;
    const int64_t c0w = c0 + wave * 32;
#pragma unroll
    for (int pass = 0; pass < BM / RP; ++pass) {
#pragma unroll
      for (int ii = 0; ii < RP / 32; ++ii)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = ii * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
          const float v = acc[pass * (RP / 32) + ii][e] + bias;
          if constexpr (EB == 4) *reinterpret_cast<float *>(reg + r * LROW + lrow * 4) = v;
          else if constexpr (OUT::code == LUX3D_BF16)
            *reinterpret_cast<uint16_t *>(reg + r * LROW + lrow * 2) = (uint16_t)(pack_bf16x2(v, 0.f) & 0xFFFFu);
          else *reinterpret_cast<uint16_t *>(reg + r * LROW + lrow * 2) = (uint16_t)(pack_f16x2(v, 0.f) & 0xFFFFu);
        }
#pragma unroll
      for (int it = 0; it < RP * CPR / 64; ++it) {
        const int q = it * 64 + lane, r = q / CPR, part = q % CPR;
        const int64_t row = m0 + pass * RP + r, col = c0w + part * EPC;
        if (row >= p.M || col >= p.N) continue;
        const uint4 v = *reinterpret_cast<const uint4 *>(reg + r * LROW + part * 16);
        char *dst = ybase + (row * p.ldy + col) * EB;
        if (col + EPC <= p.N) {
          *reinterpret_cast<uint4 *>(dst) = v;
        } else {
          const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int k = 0; k < EPC; ++k)
            if (col + k < p.N) {
              if constexpr (EB == 4) reinterpret_cast<uint32_t *>(dst)[k] = w4[k];
              else reinterpret_cast<uint16_t *>(dst)[k] = (uint16_t)(w4[k >> 1] >> (16 * (k & 1)));
            }
        }
      }
    }
    return;
  }
  // y rows not 16-byte aligned: one element per store
  if (ncol < p.N) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row >= p.M) continue;
        store1<OUT>(ybase, row * p.ldy + ncol, acc[i][e] + bias);
      }
  }
}

// ---- f32 activations on the bf16 matrix cores -------------------------------------
//
// y = sum over Q8_0 blocks b of d_b * (sum_{k in b} x_k q_k): each int8 q is
// exact in bf16, each f32 x is split exactly into three bf16 terms (x = x1 +
// x2 + x3, split3_bf16), so x q = x1 q + x2 q + x3 q with every product
// exact in f32. A 32-deep block of a 32 x 32 tile is six bf16 MFMAs (three
// terms x two 16-deep sub-steps) into a zeroed f32 block sum, which one FMA
// per element scales by the column's d and adds to the accumulator. That is
// the reference's f32 dequantize-then-matmul (w = q d exact in f32, f32
// products and sums, nn_blocks.rs:140) up to the order of the sums, at 6/16
// of the matrix-core cycles of v_mfma_f32_32x32x2_f32 per block. It replaced
// a ring kernel on v_mfma_f32_32x32x2_f32 (4096 x 2048 -> 8192: 994 -> 430
// us, same-box A/B).
//
// 128 x 256 tiles, 8 wavefronts as 2 (rows) x 4 (columns), 64 x 64 each.
// 32-deep k-steps through a 4-stage LDS ring filled by direct global -> LDS
// loads: x (128 rows x 128 bytes, row-major), the int8 weights (32 columns x
// 32 bytes per 1 KB segment; lane l holds column l % 32, bytes 16 (l / 32)
// .. + 15) and the scales (32 columns per wavefront, both lane halves). Each
// step one cooperative pass splits the next stage's x into three bf16 planes
// (double-buffered; 64-byte rows, 16-byte chunk c of row r in slot c ^ ((r
// >> 2) & 3), so fragment reads are conflict-free). k order: in sub-step s,
// lane half h holds k = 16 h + 8 s + e on both operands. One barrier per
// step: wait for stage kt + 1, barrier, issue stage kt + 3, split stage
// kt + 1, compute stage kt.
constexpr int kX3Stages = 4, kX3Threads = 512;
constexpr int kX3XL = 128 * 128, kX3WB = 256 * 32, kX3SB = 8 * 256;
constexpr int kX3Stage = kX3XL + kX3WB + kX3SB;  // 26,624 bytes
constexpr int kX3Plane = 128 * 64;               // one bf16 plane of 128 rows x 32 k
constexpr int kX3Ops = 4;                        // direct loads per wavefront per stage

template <typename OUT, int GM>
__global__ __launch_bounds__(kX3Threads, 1) void q8_0_gemm_x3_kernel(Q8GemmParams p, int tiles_m, int tiles_n) {
  constexpr int BM = 128, BN = 256, BK = 32, NS = kX3Stages;
  __shared__ __align__(16) char lds[NS * kX3Stage + 2 * 3 * kX3Plane];
  char *const planes = lds + NS * kX3Stage;

  const int G = tiles_m * tiles_n, bid = (int)blockIdx.x;
  const int per = G / 8, rem = G % 8, xcd = bid % 8, pos = bid / 8;
  const int lid = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + pos;
  const int group = lid / (GM * tiles_n), first_m = group * GM;
  const int gsize = tiles_m - first_m < GM ? tiles_m - first_m : GM;
  const int in_group = lid - group * GM * tiles_n;
  const int tm = first_m + in_group % gsize, tn = in_group / gsize;

  const int t = threadIdx.x;
  const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5, l32 = lane & 31;
  const int wm = wave >> 2, wn = wave & 3;
  const int64_t m0 = (int64_t)tm * BM, c0 = (int64_t)tn * BN;
  const int64_t nblk = p.K / 32;
  const int nk = (int)nblk;

  // direct-load offsets (rows and columns past the matrix clamp to the last)
  uint32_t xoff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 8 * (2 * wave + i) + (lane >> 3);
    const int64_t gr = m0 + r < p.M ? m0 + r : p.M - 1;
    xoff[i] = (uint32_t)(((gr - m0) * p.ldx + 4 * (lane & 7)) * 4);
  }
  const int64_t last_row = p.M - 1 - m0 < BM - 1 ? p.M - 1 - m0 : BM - 1;
  const int64_t ncols = p.N - c0 < BN ? p.N - c0 : BN;
  const int64_t wcol = c0 + 32 * wave + l32, wc = wcol < p.N ? wcol : p.N - 1;
  const i32x4_t xr = buffer_rsrc(reinterpret_cast<const char *>(p.x) + m0 * p.ldx * 4, (last_row * p.ldx + p.K) * 4);
  const i32x4_t wr = buffer_rsrc(p.qs + c0 * p.K, ncols * p.K);
  const i32x4_t sr = buffer_rsrc(p.scales + c0 * nblk, ncols * nblk * 4);
  const uint32_t woff = (uint32_t)((wc - c0) * p.K + 16 * h);
  const uint32_t soff = (uint32_t)((wc - c0) * nblk * 4);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)lds;
  auto issue = [&](int kt, int slot) {
    const uint32_t st = lds0 + slot * kX3Stage;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      lds_load16(xr, xoff[i], (uint32_t)kt * BK * 4, __builtin_amdgcn_readfirstlane(st + (2 * wave + i) * 1024));
    lds_load16(wr, woff, (uint32_t)kt * BK, __builtin_amdgcn_readfirstlane(st + kX3XL + wave * 1024));
    lds_load4(sr, soff, (uint32_t)kt * 4, __builtin_amdgcn_readfirstlane(st + kX3XL + kX3WB + wave * 256));
  };
  // the split pass: thread t takes 16-byte chunks t and t + 512 of the stage's
  // x (row q / 8, k 4 (q % 8) .. + 3)
  auto split = [&](int slot, int pb) {
    const char *xs = lds + slot * kX3Stage;
    char *pl = planes + pb * 3 * kX3Plane;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = t + i * 512, r = q >> 3, c = q & 7;
      const float4 v = *reinterpret_cast<const float4 *>(xs + q * 16);
      const Split3 lo = split3_bf16(v.x, v.y), hi = split3_bf16(v.z, v.w);
      const int off = r * 64 + (((c >> 1) ^ ((r >> 2) & 3)) << 4) + (c & 1) * 8;
      *reinterpret_cast<uint2 *>(pl + off) = make_uint2(lo.t1, hi.t1);
      *reinterpret_cast<uint2 *>(pl + kX3Plane + off) = make_uint2(lo.t2, hi.t2);
      *reinterpret_cast<uint2 *>(pl + 2 * kX3Plane + off) = make_uint2(lo.t3, hi.t3);
    }
  };
  // fragment offsets: A rows wm * 64 + i * 32 + l32, chunk 2 h + s
  int aoff[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = wm * 64 + i * 32 + l32;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) aoff[i][s2] = r * 64 + (((2 * h + s2) ^ ((r >> 2) & 3)) << 4);
  }
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16_t{};
  auto compute = [&](int slot, int pb) {
    const char *st = lds + slot * kX3Stage;
    const char *pl = planes + pb * 3 * kX3Plane;
    // weights of columns wn * 64 + j * 32 + l32: 16 int8 -> two bf16x8 (sub-steps)
    bf16x8_t b[2][2];
    float d[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint4 w = *reinterpret_cast<const uint4 *>(st + kX3XL + (2 * wn + j) * 1024 + lane * 16);
      d[j] = *reinterpret_cast<const float *>(st + kX3XL + kX3WB + (2 * wn + j) * 256 + l32 * 4);
      const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        uint32_t pk[4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const uint32_t v = wv[2 * s2 + u];
          pk[2 * u] = pack_bf16x2((float)(int8_t)(v & 0xFFu), (float)(int8_t)((v >> 8) & 0xFFu));
          pk[2 * u + 1] = pack_bf16x2((float)(int8_t)((v >> 16) & 0xFFu), (float)(int8_t)(v >> 24));
        }
        b[j][s2] = __builtin_bit_cast(bf16x8_t, u32x4_t{pk[0], pk[1], pk[2], pk[3]});
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      bf16x8_t a[3][2];
#pragma unroll
      for (int q = 0; q < 3; ++q)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) a[q][s2] = *reinterpret_cast<const bf16x8_t *>(pl + q * kX3Plane + aoff[i][s2]);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        // block sum, smallest terms first, then scaled by the column's d
        f32x16_t blk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2][0], b[j][0], f32x16_t{}, 0, 0, 0);
        blk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2][1], b[j][1], blk, 0, 0, 0);
        blk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1][0], b[j][0], blk, 0, 0, 0);
        blk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1][1], b[j][1], blk, 0, 0, 0);
        blk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0][0], b[j][0], blk, 0, 0, 0);
        blk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0][1], b[j][1], blk, 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = __builtin_fmaf(blk[e], d[j], acc[i][j][e]);
      }
    }
  };

#pragma unroll
  for (int s2 = 0; s2 < NS - 1; ++s2) issue(s2 < nk ? s2 : nk - 1, s2);
  __builtin_amdgcn_s_waitcnt(waitcnt_vm((NS - 2) * kX3Ops));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  split(0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    // stage kt + 1 landed (kt + 2 may be in flight); every wavefront is done
    // with compute(kt - 1) and split(kt)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(kX3Ops));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(kt + NS - 1 < nk ? kt + NS - 1 : nk - 1, (kt + NS - 1) % NS);
    __builtin_amdgcn_sched_barrier(0);
    if (kt + 1 < nk) split((kt + 1) % NS, (kt + 1) & 1);
    compute(kt % NS, kt & 1);
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  __builtin_amdgcn_s_barrier();  // every wavefront is done with the ring and the planes

  // epilogue: each wavefront's 64 x 64 block through LDS, bias added, one
  // rounding, 16-byte row pieces
  char *ybase = reinterpret_cast<char *>(p.y);
  constexpr int EB = OUT::code == LUX3D_F32 ? 4 : 2;
  float bias[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t col = c0 + wn * 64 + j * 32 + l32;
    bias[j] = (p.bias && col < p.N) ? p.bias[col] : 0.f;
  }
  if (((uintptr_t)p.y % 16 == 0) && ((p.ldy * EB) % 16 == 0)) {
    constexpr int ROW_B = 64 * EB, LROW = ROW_B + 16, CPR = ROW_B / 16, EPC = 16 / EB;
    constexpr int REGION = 64 * LROW;
    static_assert(8 * REGION <= (int)sizeof(lds), "epilogue staging fits");
    char *reg = lds + wave * REGION;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = i * 32 + 8 * (e >> 2) + 4 * h + (e & 3), cl = j * 32 + l32;
          const float v = acc[i][j][e] + bias[j];
          if constexpr (EB == 4) *reinterpret_cast<float *>(reg + r * LROW + cl * 4) = v;
          else if constexpr (OUT::code == LUX3D_BF16)
            *reinterpret_cast<uint16_t *>(reg + r * LROW + cl * 2) = (uint16_t)(pack_bf16x2(v, 0.f) & 0xFFFFu);
          else *reinterpret_cast<uint16_t *>(reg + r * LROW + cl * 2) = (uint16_t)(pack_f16x2(v, 0.f) & 0xFFFFu);
        }
    const int64_t r0 = m0 + wm * 64, cw = c0 + wn * 64;
#pragma unroll
    for (int it = 0; it < 64 * CPR / 64; ++it) {
      const int q = it * 64 + lane, r = q / CPR, part = q % CPR;
      const int64_t row = r0 + r, col = cw + part * EPC;
      if (row >= p.M || col >= p.N) continue;
      const uint4 v = *reinterpret_cast<const uint4 *>(reg + r * LROW + part * 16);
      char *dst = ybase + (row * p.ldy + col) * EB;
      if (col + EPC <= p.N) {
        *reinterpret_cast<uint4 *>(dst) = v;
      } else {
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int kk = 0; kk < EPC; ++kk)
          if (col + kk < p.N) {
            if constexpr (EB == 4) reinterpret_cast<uint32_t *>(dst)[kk] = w4[kk];
            else reinterpret_cast<uint16_t *>(dst)[kk] = (uint16_t)(w4[kk >> 1] >> (16 * (kk & 1)));
          }
      }
    }
    return;
  }
  // y rows not 16-byte aligned: one element per store
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t col = c0 + wn * 64 + j * 32 + l32;
    if (col >= p.N) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row >= p.M) continue;
        store1<OUT>(ybase, row * p.ldy + col, acc[i][j][e] + bias[j]);
      }
  }
}

// The ring kernel's buffer descriptors span one tile (at most 256 rows of x,
// 256 weight rows and their scales) and must stay below 2^31 bytes; its
// per-lane offsets are 32-bit.
bool ring_fits(const Q8GemmParams &p) {
  const int64_t lim = 0x7FFFFFFF;
  return p.K % 64 == 0 && (255 * p.ldx + p.K) * 2 <= lim && 256 * p.K <= lim &&
         (p.M + 127) / 128 * ((p.N + 255) / 256) <= INT32_MAX;
}

// Kernel choice (measured on MI355X, graph-timed over rotating inputs):
// the ring kernel whenever K % 64 == 0 (every shape of the models): 256-row
// tiles when they cover every CU at least once (1,018 TFLOP/s at
// 4096x2048x8192, 512 tiles), else 128-row tiles of 8 wavefronts when those
// do, else tiles of 4 wavefronts: 160 x 128 when 128 x 128 ones would
// outnumber the CUs but 160-row ones do not (1029x1024x4096: 7 x 32 tiles in
// 19.2 us, against 23.5 us for 9 x 32 of 128 x 128, 26.8 us for 9 x 16 tiles
// of 8 wavefronts, 22.4 us for 5 x 32 of 256 x 128), else 128 x 128. The
// 128 x 128 kernel with 32-deep k-steps covers K % 64 == 32.
constexpr int64_t kRingMinTiles = 256;  // MI355X compute units

template <typename OUT>
hipError_t launch_tiles(const Q8GemmParams &p, hipStream_t s) {
  if (p.x_f32) {
    // f32 activations (K % 64 == 0, checked by the caller)
    const int64_t tiles_m = (p.M + 127) / 128, tiles_n = (p.N + 255) / 256;
    if (tiles_m * tiles_n > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL((q8_0_gemm_x3_kernel<OUT, 8>), dim3((unsigned)(tiles_m * tiles_n)), dim3(kX3Threads), 0, s, p,
                       (int)tiles_m, (int)tiles_n);
    return hipGetLastError();
  }
  if (ring_fits(p)) {
    const int64_t tiles_n = (p.N + 255) / 256, tiles_m256 = (p.M + 255) / 256;
    if (tiles_m256 * tiles_n >= kRingMinTiles) {
      hipLaunchKernelGGL((q8_0_gemm_ring_kernel<OUT, 8, 256>), dim3((unsigned)(tiles_m256 * tiles_n)), dim3(kRingThreads),
                         0, s, p, (int)tiles_m256, (int)tiles_n);
    } else if ((p.M + 127) / 128 * tiles_n >= kRingMinTiles) {
      const int64_t tiles_m = (p.M + 127) / 128;
      hipLaunchKernelGGL((q8_0_gemm_ring_kernel<OUT, 8, 128>), dim3((unsigned)(tiles_m * tiles_n)), dim3(kRingThreads), 0,
                         s, p, (int)tiles_m, (int)tiles_n);
    } else if ((p.M + 127) / 128 * ((p.N + 127) / 128) > kRingMinTiles &&
               (p.M + 159) / 160 * ((p.N + 127) / 128) <= kRingMinTiles) {
      // fewer 128 x 256 tiles than CUs, more 128 x 128 ones: 160 x 128 tiles
      // of four wavefronts, one per CU (the 128-row tiles would leave some CUs
      // two; 1029 x 1024 -> 4096: 7 x 32 tiles in 19.2 us against 9 x 32 in
      // 23.5 us)
      const int64_t tiles_m = (p.M + 159) / 160, tiles_n128 = (p.N + 127) / 128;
      hipLaunchKernelGGL((q8_0_gemm_ring_kernel<OUT, 8, 160, 4>), dim3((unsigned)(tiles_m * tiles_n128)), dim3(256), 0,
                         s, p, (int)tiles_m, (int)tiles_n128);
    } else {
      // fewer 128 x 256 tiles than CUs: 128 x 128 tiles of four wavefronts
      // (two workgroups per CU by LDS) spread the same wavefronts over more CUs
      const int64_t tiles_m = (p.M + 127) / 128, tiles_n128 = (p.N + 127) / 128;
      hipLaunchKernelGGL((q8_0_gemm_ring_kernel<OUT, 8, 128, 4>), dim3((unsigned)(tiles_m * tiles_n128)), dim3(256), 0,
                         s, p, (int)tiles_m, (int)tiles_n128);
    }
    return hipGetLastError();
  }
  const dim3 grid((unsigned)((p.N + 127) / 128), (unsigned)((p.M + 127) / 128));
  hipLaunchKernelGGL((q8_0_gemm_kernel<OUT, 128, 128, 32, 1>), grid, dim3(kGemmThreads), 0, s, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_q8_0_repack(const uint8_t *blocks, int64_t nblocks, int8_t *qs, float *scales, hipStream_t s) {
  if (nblocks <= 0) return hipSuccess;
  const int64_t threads = nblocks * 4;
  hipLaunchKernelGGL(q8_0_repack_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, blocks, nblocks,
                     qs, scales);
  return hipGetLastError();
}

// ---- integer-dot Q8_0 linear: candle's CPU QMatMul semantics ----------------
//
// The reference's quantized Linear::forward (runtime/nn_blocks.rs:80-93) on
// the CPU quantizes each x row to Q8_0 blocks and takes integer dot
// products with the weight blocks (candle-core quantized/k_quants.rs,
// BlockQ8_0::from_float and vec_dot). Here:
// - q8_0_quantize_rows_kernel: eight lanes per 32-value block (16 bytes
//   each): amax = max |x| (NaN ignored, at least 0), d = amax / 127, id =
//   d != 0 ? 1 / d : 0 (correctly rounded f32 divisions), q = round half
//   away from zero of x * id, saturated to int8 with NaN -> 0, and d rounded
//   to f16 (RNE) and widened back to f32;
// - q8_0_int8_gemm_kernel: one v_mfma_i32_32x32x32_i8 per 32 x 32 tile and
//   Q8_0 block gives that block's exact int32 dot products; each is then
//   folded into the f32 sum as candle's generic vec_dot does, in block
//   order: acc = acc + ((f32)isum * wd) * xd, every operation rounded
//   (mul_rn / add_rn: no contraction), and y = acc + bias. The result is
//   bit-identical to candle's CPU path. The f32 fold (4 VALU operations per
//   output and block) bounds the kernel, not the int8 matrix rate.

__global__ __launch_bounds__(256) void q8_0_quantize_rows_kernel(Q8IntParams p) {
  const int64_t nb = p.K / 32;
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t blk = g >> 3;
  const int part = (int)(g & 7);
  const bool live = blk < p.M * nb;
  const int64_t bc = live ? blk : 0;
  const int64_t m = bc / nb, b = bc - m * nb;
  const float4 v = *reinterpret_cast<const float4 *>(p.x + m * p.ldx + b * 32 + part * 4);
  const float xv[4] = {v.x, v.y, v.z, v.w};
  // f32::max ignores a NaN operand; fmaxf (IEEE maxNum) does the same
  float a = fmaxf(fmaxf(fabsf(xv[0]), fabsf(xv[1])), fmaxf(fabsf(xv[2]), fabsf(xv[3])));
  a = fmaxf(a, dpp<DPP_XOR1>(a));
  a = fmaxf(a, dpp<DPP_XOR2>(a));
  a = fmaxf(a, dpp<DPP_HALF_MIRROR>(a));  // the 8 lanes of the block
  const float amax = fmaxf(a, 0.0f);       // candle starts its maximum at 0
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  uint32_t packed = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float r = roundf(mul_rn(xv[k], id));
    const int q = r != r ? 0 : (r >= 127.0f ? 127 : (r <= -128.0f ? -128 : (int)r));
    packed |= ((uint32_t)(uint8_t)(int8_t)q) << (8 * k);
  }
  if (!live) return;
  *reinterpret_cast<uint32_t *>(p.xq + m * p.K + b * 32 + part * 4) = packed;
  if (part == 0) p.xd[b * p.ldxd + m] = (float)(_Float16)d;  // block-major
}

// 256 threads (2 x 2 wavefronts of 32 x 32 tiles) per 64 x 64 tile of y; a
// stage is two Q8_0 blocks (k-step 64), double-buffered through LDS: rows of
// 64 int8 at an 80-byte stride (conflict-free 16-byte fragment reads) and
// the stage's block scales of the tile's 64 x rows and 64 weight rows. The
// second block's MFMA is issued before the first block's f32 fold, so the
// matrix core runs beside the fold's VALU work. An odd last block is loaded
// twice and folded once.
constexpr int kI8Tile = 64, kI8Row = 80;
__global__ __launch_bounds__(256) void q8_0_int8_gemm_kernel(Q8IntParams p, int tiles_n) {
  typedef int i32x4_t_ __attribute__((ext_vector_type(4)));
  typedef int i32x16_t_ __attribute__((ext_vector_type(16)));
  __shared__ __align__(16) int8_t As[2][kI8Tile * kI8Row];
  __shared__ __align__(16) int8_t Bs[2][kI8Tile * kI8Row];
  __shared__ __align__(16) float Ad[2][2][kI8Tile];  // [buffer][block of the stage][row]
  __shared__ __align__(16) float Bd[2][2][kI8Tile];
  (void)tiles_n;
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), wm = wave >> 1,
            wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * kI8Tile, n0 = (int64_t)blockIdx.x * kI8Tile;
  const int64_t nb = p.K / 32, nst = (nb + 1) / 2;
  // loaders: thread t moves the 16 bytes (t & 3) of x row t / 4 and of weight
  // row t / 4 per stage (rows past M / N clamped: loaded, computed, never
  // stored); wavefronts 0-1 the x scales (block wave & 1 of the stage, row
  // lane), 2-3 the weight scales
  const int lr = t >> 2, lq = t & 3;
  const int64_t ra = m0 + lr < p.M ? m0 + lr : p.M - 1, rb = n0 + lr < p.N ? n0 + lr : p.N - 1;
  const int8_t *sa = p.xq + ra * p.K + lq * 16, *sb = p.qs + rb * p.K + lq * 16;
  const int so = lr * kI8Row + lq * 16;
  const int sr = lane, sbk = wave & 1;
  const bool sx = wave < 2;
  const int64_t swr = n0 + sr < p.N ? n0 + sr : p.N - 1;
  // the thread's scale column: x scales are block-major (stride ldxd per
  // block), weight scales row-major (stride 1); the stride is wave-uniform
  const float *sp = sx ? p.xd + m0 + sr : p.scales + swr * nb;
  const int64_t sstep = sx ? p.ldxd : 1;
  // an odd last stage holds block nb - 1 in both halves: threads of the
  // second half (lq 2, 3) read 32 bytes back, and both scale rows read it
  const int back = lq >= 2 ? 32 : 0;
  uint4 va, vb;
  float vs;
  auto load = [&](int64_t st) {
    int64_t o = st * 64, kb = 2 * st + sbk;
    if (2 * st + 1 == nb) {
      o -= back;
      kb = 2 * st;
    }
    va = *reinterpret_cast<const uint4 *>(sa + o);
    vb = *reinterpret_cast<const uint4 *>(sb + o);
    vs = sp[kb * sstep];
  };
  auto store = [&](int buf) {
    *reinterpret_cast<uint4 *>(&As[buf][so]) = va;
    *reinterpret_cast<uint4 *>(&Bs[buf][so]) = vb;
    (sx ? Ad[buf][sbk] : Bd[buf][sbk])[sr] = vs;
  };
  load(0);
  store(0);
  lds_barrier();

  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  const int fr = lane & 31, fk = (lane >> 5) * 16;
  auto fold = [&](const i32x16_t_ &c, int buf, int blk) {
    const float wd = Bd[buf][blk][wn * 32 + fr];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // rows 8q + 4 (lane / 32) + 0..3 of the wavefront's 32
      const float4 xd4 = *reinterpret_cast<const float4 *>(&Ad[buf][blk][wm * 32 + 8 * q + 4 * (lane >> 5)]);
      const float xd[4] = {xd4.x, xd4.y, xd4.z, xd4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 4 * q + i;
        acc[e] = add_rn(acc[e], mul_rn(mul_rn((float)c[e], wd), xd[i]));
      }
    }
  };
  // a wavefront whose 32 rows all lie past M (in the last row of tiles) only
  // loads and synchronises: its products would never be stored
  const bool rows_live = m0 + wm * 32 < p.M;  // wave-uniform
  for (int64_t st = 0; st < nst; ++st) {
    const int buf = (int)(st & 1);
    if (st + 1 < nst) load(st + 1);
    if (rows_live) {
      const int8_t *a = &As[buf][(wm * 32 + fr) * kI8Row + fk], *b = &Bs[buf][(wn * 32 + fr) * kI8Row + fk];
      const i32x16_t_ c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(*reinterpret_cast<const i32x4_t_ *>(a),
                                                                 *reinterpret_cast<const i32x4_t_ *>(b), i32x16_t_{},
                                                                 0, 0, 0);
      // an odd last stage holds block nb - 1 in both halves: its second
      // product is computed and not folded
      const i32x16_t_ c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(*reinterpret_cast<const i32x4_t_ *>(a + 32),
                                                                 *reinterpret_cast<const i32x4_t_ *>(b + 32),
                                                                 i32x16_t_{}, 0, 0, 0);
      fold(c0, buf, 0);
      if (2 * st + 1 < nb) fold(c1, buf, 1);
    }
    if (st + 1 < nst) store(buf ^ 1);
    lds_barrier();
  }
  // lane holds y[8 (e / 4) + 4 (lane / 32) + e % 4][lane % 32] of its 32 x 32 tile
  const int64_t col = n0 + wn * 32 + fr;
  if (col >= p.N) return;
  const float bias = p.bias ? p.bias[col] : 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int64_t row = m0 + wm * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
    if (row < p.M) p.y[row * p.ldy + col] = p.bias ? add_rn(acc[e], bias) : acc[e];
  }
}

hipError_t launch_q8_0_gemm(int out_dt, const Q8GemmParams &p, hipStream_t s) {
  if (p.M <= 0 || p.N <= 0) return hipSuccess;
  if (p.K <= 0 || p.K % kBK) return hipErrorInvalidValue;
  if (p.x_f32 && (p.K % 64 || (127 * p.ldx + p.K) * 4 > 0x7FFFFFFF || 256 * p.K > 0x7FFFFFFF))
    return hipErrorInvalidValue;
  if ((p.N + 127) / 128 > INT32_MAX || (p.M + 127) / 128 > 65535) return hipErrorInvalidValue;
  switch (out_dt) {
    case LUX3D_BF16: return launch_tiles<BF16>(p, s);
    case LUX3D_F16: return launch_tiles<F16>(p, s);
    case LUX3D_F32: return launch_tiles<F32>(p, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_q8_0_quantize_rows(const Q8IntParams &p, hipStream_t s) {
  if (p.M <= 0) return hipSuccess;
  if (p.K <= 0 || p.K % 32) return hipErrorInvalidValue;
  const int64_t lanes = p.M * (p.K / 32) * 8;
  if ((lanes + 255) / 256 > INT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(q8_0_quantize_rows_kernel, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_q8_0_int8_gemm(const Q8IntParams &p, hipStream_t s) {
  if (p.M <= 0 || p.N <= 0) return hipSuccess;
  if (p.K <= 0 || p.K % 32 || p.ldxd < (p.M + kI8Tile - 1) / kI8Tile * kI8Tile) return hipErrorInvalidValue;
  const int64_t tn = (p.N + kI8Tile - 1) / kI8Tile, tm = (p.M + kI8Tile - 1) / kI8Tile;
  if (tn > INT32_MAX || tm > 65535) return hipErrorInvalidValue;
  hipLaunchKernelGGL(q8_0_int8_gemm_kernel, dim3((unsigned)tn, (unsigned)tm), dim3(256), 0, s, p, (int)tn);
  return hipGetLastError();
}

}  // namespace lux3d
