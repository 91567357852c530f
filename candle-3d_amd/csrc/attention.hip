// attention.hip -- scaled dot-product attention for gfx950:
// out = softmax(q k^T * scale) v over [B, H, L, D] views, one launch, no
// scores buffer in HBM.
//
// Semantics: scores are exact f32 sums of the input products (matrix cores
// accumulate bf16 x bf16 / f16 x f16 products in f32), the softmax runs in
// f32 with a running maximum (exp2 of the log2e-scaled scores), the
// probabilities are rounded to the input type for the P v product, which
// again accumulates in f32, and the output is divided by the f32 sum of those
// same rounded probabilities and rounded once. That is the arithmetic of exact_sdpa_heads (f32 throughout)
// up to the rounding of the probabilities; exact_query_chunked_sdpa on bf16
// additionally rounds q * scale, the scores and the probabilities to bf16,
// which this kernel does not.
//
// Matrix-core kernel (attn_mfma_kernel). A workgroup of 4 wavefronts owns
// BQ = 128 * QT queries of one (batch, head); each wavefront keeps QT tiles
// of 32 queries. Per block of BKV keys:
//   S^T = K Q^T    A operand: K rows from LDS, B operand: Q held in registers.
//                  The 32 x 32 result leaves every lane with ONE query
//                  (lane % 32) and 16 keys, so the row max needs a single
//                  exchange with lane ^ 32 and no other cross-lane traffic.
//   O^T += V^T P^T A operand: V^T fragments read from V's [key][dim] rows in
//                  LDS by ds_read_b64_tr_b16 (the transpose happens in the
//                  LDS read), B operand: the probabilities exactly where the S^T
//                  accumulator left them (the key order inside a 16-key
//                  k-step is permuted identically on both operands, which a
//                  sum over keys does not see). O^T again gives each lane its
//                  own query, so the rescale by exp2(m_old - m_new) and the
//                  final 1/l are per-lane multiplies.
// K and V blocks are double-buffered in LDS; the next block's global loads
// are issued before the current block's math, one LDS barrier per block.
// Workgroups are numbered so that the query blocks of one head run on one
// XCD (hardware places workgroup i on XCD i % 8) and share its L2 copy of K
// and V.
//
// Exact-probability form (EXACTP, bf16 only; exact_sdpa_heads): the
// probabilities stay f32 and enter P v as three bf16 terms p = p1 + p2 + p3
// (p1 = bf16(p), p2 = bf16(p - p1), p3 = p - p1 - p2), which sum to the f32
// value exactly: p has 24 significant bits and each RNE step leaves a
// remainder of at most 16, then 8 of them. bf16 x bf16 products are exact in
// f32, so scores and P v are f32 products with f32 accumulation -- the
// reference's widen-to-f32 arithmetic up to the order of the sums -- on the
// bf16 matrix cores; the row sum adds the f32 probabilities. The output is
// rounded once, to bf16 or (p.out_f32) stored as f32.
//
// f32 inputs (attn_f32x3_kernel, D 64 / 128): the same scheme on the bf16
// matrix cores, with q, k, v and the probabilities split exactly into three
// bf16 terms each and the six significant cross products per MFMA step;
// f32-class arithmetic at 6 / 16 of the f32 MFMA's matrix-core cycles.
//
// Generic kernel (attn_generic_kernel): one wavefront per query row, f32
// arithmetic throughout (lanes over keys for the scores, over head dims for
// the output); any float dtype, any alignment, D <= 512.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace lux3d {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

template <typename T> struct Mma;
template <> struct Mma<BF16> {
  typedef bf16x8_t op_t;
  __device__ __forceinline__ static f32x16_t run(op_t a, op_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
  __device__ __forceinline__ static float sum2(uint32_t pair, float acc) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pair), one, acc, false);
  }
};
template <> struct Mma<F16> {
  typedef f16x8_t op_t;
  __device__ __forceinline__ static f32x16_t run(op_t a, op_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack(float lo, float hi) { return pack_f16x2(lo, hi); }
  __device__ __forceinline__ static float sum2(uint32_t pair, float acc) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, pair), one, acc, false);
  }
};

// the same into element e of three packed operand vectors
__device__ __forceinline__ void split3_into(float a, float b, u32x4_t &x1, u32x4_t &x2, u32x4_t &x3, int e) {
  const Split3 r = split3_bf16(a, b);
  x1[e] = r.t1;
  x2[e] = r.t2;
  x3[e] = r.t3;
}

// The value the partner lane (lane ^ 32) holds, paired with this lane's own:
// v_permlane32_swap exchanges the two 32-lane halves.
__device__ __forceinline__ float half_swap_max(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_swap_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Logical workgroup id for physical id `pid` of `n`: XCD x (pid % 8) gets the
// contiguous logical range [start_x, start_x + count_x).
__device__ __forceinline__ int64_t xcd_logical_id(int64_t pid, int64_t n) {
  const int64_t per = n / 8, rem = n % 8, xcd = pid % 8, idx = pid / 8;
  return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + idx;
}

// LAZY: the reference maximum m moves only when a block's maximum exceeds it
// by more than 8 (log2 units), so probabilities exp2(s - m) stay <= 2^8 and
// the O rescale (skipped by a wave-uniform test while every factor is 1) is
// rare after the first blocks. The final O / l is the same function.
// DOT: the row sum l adds the probabilities as rounded for the P v product
// (v_dot2 of a packed pair with (1, 1)), one instruction per pair.
// PHASED (QT == 2): P v of query tile 0 is issued before the softmax of
// tile 1, so the matrix cores and the VALU overlap inside one wavefront.
// Measured on MI355X (TFLOP/s, VGGT frame / global, D 64): LAZY + DOT +
// PHASED 617 / 795 against 579 / 700 without; D 128 (TripoSG / TRELLIS.2
// 16k) LAZY + DOT 718 / 877 against 679 / 827, PHASED by key tile no gain.
// QP (QP_*): q arrives raw; its head norm and rotation (the head kernels'
// arithmetic and lane mapping, bit for bit) are applied while the Q
// fragments are loaded, so the normalised q never goes through HBM.
// EXACTP: f32 probabilities as three bf16 terms (see the file header).
template <typename T, int D, int QT, int BKV, int MINW, bool LAZY, bool DOT, bool PHASED, int QP = QP_NONE,
          bool DMA = false, bool EXACTP = false, int KS = 1>
__global__ __launch_bounds__(256, MINW) void attn_mfma_kernel(AttnParams p, int64_t nqb, int64_t nwg) {
  static_assert(!EXACTP || (std::is_same<T, BF16>::value && !DOT), "exact probabilities: bf16, f32 sums");
  static_assert(KS == 1 || (!PHASED && (BKV / 32) % KS == 0), "key groups: whole 32-key tiles per wavefront");
  using M = Mma<T>;
  using op_t = typename M::op_t;
  constexpr int QG = 4 / KS;               // query groups per workgroup (KS wavefronts each)
  constexpr int BQ = QG * 32 * QT;
  // 2-byte elements per K / V row in LDS: padded by 16 bytes, or (DMA)
  // unpadded with 16-byte chunk c of row r in slot c ^ ((r & 7) * D / 64)
  constexpr int KROW = DMA ? D : D + 8;
  constexpr int KCH = BKV * D / 8 / 256;   // 16-byte K (and V) chunks per thread per block
  constexpr int NKT = BKV / 32 / KS;       // 32-key tiles of a block per wavefront
  constexpr int NDT = D / 32;              // 32-dim output tiles
  static_assert(KCH >= 1 && BKV % 32 == 0 && D % 32 == 0, "tile shape");
  __shared__ __align__(16) uint16_t smem[4 * BKV * KROW];
  uint16_t(*Ks)[BKV * KROW] = reinterpret_cast<uint16_t(*)[BKV * KROW]>(smem);
  uint16_t(*Vs)[BKV * KROW] = reinterpret_cast<uint16_t(*)[BKV * KROW]>(smem + 2 * BKV * KROW);

  const int64_t lid = xcd_logical_id(blockIdx.x, nwg);
  const int64_t bh = lid / nqb, qb = lid % nqb;
  const int64_t bi = bh / p.H, hi = bh % p.H;
  const char *qbase = reinterpret_cast<const char *>(p.q) + (bi * p.q_sb + hi * p.q_sh) * 2;
  const char *kbase = reinterpret_cast<const char *>(p.k) + (bi * p.k_sb + hi * p.k_sh) * 2;
  const char *vbase = reinterpret_cast<const char *>(p.v) + (bi * p.v_sb + hi * p.v_sh) * 2;
  const int ob = EXACTP && p.out_f32 ? 4 : 2;  // output element bytes
  char *obase = reinterpret_cast<char *>(p.o) + (bi * p.o_sb + hi * p.o_sh) * ob;

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  // KS > 1: the KS wavefronts of query group qg hold the same queries and
  // take key tiles kt0 .. kt0 + NKT - 1 of every block (key group kg)
  const int qg = wave / KS, kg = wave % KS, kt0 = kg * NKT;
  const int64_t Lq = p.Lq, Lk = p.Lk;

  // Q as the B operand: lane holds Q[query l32][c * 16 + 8 * hh + e].
  op_t qf[QT][D / 16];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    int64_t qr = qb * BQ + (qg * QT + qt) * 32 + l32;
    qr = qr < Lq ? qr : Lq - 1;
    if constexpr (QP == QP_NONE) {
#pragma unroll
      for (int c = 0; c < D / 16; ++c)
        qf[qt][c] = *reinterpret_cast<const op_t *>(qbase + (qr * p.q_st + c * 16 + 8 * hh) * 2);
    }
  }
  if constexpr (QP != QP_NONE) {
    // Head norm + rotation of the wavefront's query rows with the head
    // kernels' mapping (D / 8 lanes per row, 8 elements per lane, the same
    // DPP sums and partner exchange), written as bf16 / f16 into the K / V
    // staging area, which is not in use yet; then each lane reads its
    // fragments.
    static_assert(D == 64 || D == 128, "Q prologue head dims");
    constexpr int LPR = D / 8, RPP = 64 / LPR;  // lanes per row, rows per pass
    static_assert(4 * QT * 32 * D <= 4 * BKV * KROW, "Q staging fits the K / V buffers");
    uint16_t *qs = smem + wave * (QT * 32 * D);
    const int ch = lane % LPR;
    float w8[8], b8[8];
    if constexpr (QP == QP_LN_R1 || QP == QP_RMS) param8(p.qw, p.qw_dt, ch * 8, 1.f, w8);
    if constexpr (QP == QP_LN_R1) param8(p.qb, p.qb_dt, ch * 8, 0.f, b8);
    if constexpr (QP == QP_L2_R2) param8(p.qw, p.qw_dt, hi * D + ch * 8, 1.f, w8);  // gamma of head hi
    // Every pass's row, table and parameter loads are issued first (one
    // fence keeps the scheduler from sinking them behind the reductions),
    // so each wavefront waits on one memory round trip, not one per pass.
    static_assert((QT * 32) % RPP == 0, "whole passes");
    constexpr int NP = QT * 32 / RPP;                                   // passes
    constexpr int TW = QP == QP_L2_R2 ? 4 : (QP == QP_RMS ? 1 : 8);   // table values per lane and pass
    float xs[NP][8], tc[NP][TW], tsn[NP][TW];
    int64_t qrs[NP];
#pragma unroll
    for (int it = 0; it < NP; ++it) {
      const int row = lane / LPR + it * RPP;
      int64_t qr = qb * BQ + qg * QT * 32 + row;
      qr = qr < Lq ? qr : Lq - 1;
      qrs[it] = qr;
      Chunk<T>::template load<false>(qbase + (qr * p.q_st + ch * 8) * 2, xs[it]);
      if constexpr (QP == QP_LN_R1) {
        const int64_t toff = bi * p.tab_sB + qr * p.tab_sN + ch * 8;
        param8(p.tab_c, p.tab_dt, toff, 1.f, tc[it]);
        param8(p.tab_s, p.tab_dt, toff, 0.f, tsn[it]);
      } else if constexpr (QP == QP_L2_R2) {
        const int64_t toff = qr * p.tab_sN + ch * 4;
        param4(p.tab_c, p.tab_dt, toff, 1.f, tc[it]);
        param4(p.tab_s, p.tab_dt, toff, 0.f, tsn[it]);
      } else if constexpr (QP == QP_R3) {
        // tokens before the prefix read table row 0 (their rotation is discarded)
        const int64_t toff = (qr >= p.prefix ? qr - p.prefix : 0) * p.tab_sN + ch * 8;
        param8(p.tab_c, p.tab_dt, toff, 1.f, tc[it]);
        param8(p.tab_s, p.tab_dt, toff, 0.f, tsn[it]);
      }
    }
    issue_fence();
#pragma unroll
    for (int it = 0; it < NP; ++it) {
      const int row = lane / LPR + it * RPP;
      const int64_t qr = qrs[it];
      float(&x)[8] = xs[it];
      if constexpr (QP == QP_LN_R1) {
        const float mean = group_sum<LPR>(ln_chunk_sum(x)) * (1.0f / D);
        const float rstd = ln_rstd(group_sum<LPR>(ln_chunk_center_sq(x, mean)), 1.0f / D, p.eps);
        ln_chunk_affine(x, rstd, w8, b8);
      } else if constexpr (QP == QP_RMS) {
        head_rms_chunk<LPR, D>(x, w8, p.eps);
      } else if constexpr (QP == QP_L2_R2) {
        head_l2_chunk<LPR, D>(x, w8);
      }
      // out[j] = x[j] * C[j] + x[j ^ M] * S[j] (rotate1)
      float y[8];
      if constexpr (QP == QP_LN_R1) {
        // Rope2d: partner j ^ D/4, C / S the cos_full / sin_alt_full rows
        float pv[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) pv[k] = lane_xor<D / 32>(x[k]);  // element j ^ D/4
#pragma unroll
        for (int k = 0; k < 8; ++k) y[k] = rotate1(x[k], tc[it][k], pv[k], tsn[it][k]);
      } else if constexpr (QP == QP_L2_R2) {
        // TRELLIS.2 pairs (2a, 2a + 1) = (re, im): partner j ^ 1 in the lane,
        // C = cos[n][a], S = -sin[n][a] for the re element, +sin for im
#pragma unroll
        for (int k = 0; k < 8; ++k)
          y[k] = rotate1(x[k], tc[it][k >> 1], x[k ^ 1], (k & 1) ? tsn[it][k >> 1] : -tsn[it][k >> 1]);
      } else if constexpr (QP == QP_R3) {
        // DINOv3 rotate_half: partner j ^ D/2, S = -sin for j < D/2; tokens
        // before the prefix pass through
        float pv[8];
        const bool rot = qr >= p.prefix;
#pragma unroll
        for (int k = 0; k < 8; ++k) pv[k] = lane_xor<D / 16>(x[k]);  // element j ^ D/2
        const bool lo = ch * 8 < D / 2;
#pragma unroll
        for (int k = 0; k < 8; ++k) y[k] = rot ? rotate1(x[k], tc[it][k], pv[k], lo ? -tsn[it][k] : tsn[it][k]) : x[k];
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) y[k] = x[k];
      }
      u32x4_t pk;
#pragma unroll
      for (int e = 0; e < 4; ++e) pk[e] = M::pack(y[2 * e], y[2 * e + 1]);
      *reinterpret_cast<u32x4_t *>(qs + row * D + ch * 8) = pk;
    }
    lds_barrier();
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int c = 0; c < D / 16; ++c)
        qf[qt][c] = *reinterpret_cast<const op_t *>(qs + (qt * 32 + l32) * D + c * 16 + 8 * hh);
    lds_barrier();  // the staging area becomes the K / V buffers below
  }

  // Staging: K and V rows as 16-byte chunks, both in their [key][dim]
  // layout. Keys past Lk are clamped to Lk - 1 (finite data; their scores
  // are masked).
  int k_row[KCH], k_part[KCH];
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    const int c = t + i * 256;
    k_row[i] = c / (D / 8);
    k_part[i] = c % (D / 8);
  }
  // byte offsets of this thread's rows relative to a block's first key
  int64_t k_off[KCH], v_off[KCH];
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    k_off[i] = ((int64_t)k_row[i] * p.k_st + k_part[i] * 8) * 2;
    v_off[i] = ((int64_t)k_row[i] * p.v_st + k_part[i] * 8) * 2;
  }
  // DMA: load i of a wavefront fills LDS bytes [seg * 1024, + 1024) of a
  // buffer, seg = wave * KCH + i, in lane order; the lane loads the logical
  // chunk that its slot holds. Each block's descriptors start at the block's
  // first key and end at the head's last byte, and the per-lane offset (the
  // part of the address the hardware range-checks; the scalar offset is not
  // checked) carries the whole in-block offset: keys past Lk fall outside
  // and read as zeros (finite; their scores are masked).
  constexpr int SWZ = D / 64;
  uint32_t dk_off[KCH], dv_off[KCH];
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    const int byte = (wave * KCH + i) * 1024 + lane * 16, r = byte / (2 * D), sl = (byte % (2 * D)) / 16;
    const int c = sl ^ ((r & 7) * SWZ);
    dk_off[i] = (uint32_t)(r * p.k_st * 2 + c * 16);
    dv_off[i] = (uint32_t)(r * p.v_st * 2 + c * 16);
  }
  const int64_t kbytes = ((Lk - 1) * p.k_st + D) * 2, vbytes = ((Lk - 1) * p.v_st + D) * 2;
  const int64_t kstep = BKV * p.k_st * 2, vstep = BKV * p.v_st * 2;
  const uint32_t lds_k = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint16_t *)smem;
  const uint32_t lds_v = lds_k + 2 * BKV * KROW * 2;
  auto dma_kv = [&](int64_t j, int buf) {
    const i32x4_t krs = buffer_rsrc(kbase + j * kstep, kbytes - j * kstep);
    const i32x4_t vrs = buffer_rsrc(vbase + j * vstep, vbytes - j * vstep);
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const uint32_t off = (uint32_t)((wave * KCH + i) * 1024 + buf * BKV * KROW * 2);
      lds_load16(krs, dk_off[i], 0, __builtin_amdgcn_readfirstlane(lds_k + off));
      lds_load16(vrs, dv_off[i], 0, __builtin_amdgcn_readfirstlane(lds_v + off));
    }
  };
  uint4 rk[KCH], rv[KCH];
  // `clamp` (the tail block only): keys past Lk read row Lk - 1
  auto load_kv = [&](int64_t j, bool clamp) {
    if (!clamp) {
      const char *kb = kbase + j * kstep, *vb = vbase + j * vstep;
#pragma unroll
      for (int i = 0; i < KCH; ++i) rk[i] = ld16<false>(kb + k_off[i]);
#pragma unroll
      for (int i = 0; i < KCH; ++i) rv[i] = ld16<false>(vb + v_off[i]);
      return;
    }
    const int64_t key0 = j * BKV;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      int64_t key = key0 + k_row[i];
      key = key < Lk ? key : Lk - 1;
      rk[i] = ld16<false>(kbase + (key * p.k_st + k_part[i] * 8) * 2);
      rv[i] = ld16<false>(vbase + (key * p.v_st + k_part[i] * 8) * 2);
    }
  };
  auto store_kv = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      *reinterpret_cast<uint4 *>(&Ks[buf][k_row[i] * KROW + k_part[i] * 8]) = rk[i];
      *reinterpret_cast<uint4 *>(&Vs[buf][k_row[i] * KROW + k_part[i] * 8]) = rv[i];
    }
  };

  f32x16_t o[QT][NDT];
  float m[QT], l[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m[qt] = -INFINITY;
    l[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[qt][dt] = f32x16_t{};
  }
  const float c2 = p.scale * kLog2e;
  const int64_t nkv = (Lk + BKV - 1) / BKV;
  const bool tail = (Lk % BKV) != 0;

  if constexpr (DMA) {
    dma_kv(0, 0);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  } else {
    load_kv(0, nkv == 1 && tail);
    store_kv(0);
  }
  lds_barrier();

  // one block of keys; MASK (the partial tail block) sets scores past Lk to -inf
  auto step = [&](int64_t j, auto mask_c) {
    constexpr bool MASK = decltype(mask_c)::value;
    const int buf = (int)(j & 1);
    if constexpr (DMA) {
      if (j + 1 < nkv) dma_kv(j + 1, buf ^ 1);
    } else {
      if (j + 1 < nkv) load_kv(j + 1, tail && j + 2 == nkv);
    }

    // S^T = K Q^T: lane holds key 8 * (i / 4) + 4 * hh + i % 4 of each 32-key tile, query l32.
    f32x16_t s[QT][NKT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) s[qt][kt] = f32x16_t{};
    if constexpr (PHASED && QT == 2) {
      // query tile 0's scores complete before tile 1's (each K fragment read
      // twice), so its maximum overlaps tile 1's MFMAs: VGGT frame 86.6 ->
      // 85.8 us, global 558.0 -> 552.6 us (same-box A/B)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
          for (int c = 0; c < D / 16; ++c) {
            const int krow = (kt0 + kt) * 32 + l32, kch = DMA ? ((2 * c + hh) ^ ((krow & 7) * SWZ)) : 2 * c + hh;
            const op_t a = *reinterpret_cast<const op_t *>(&Ks[buf][krow * KROW + kch * 8]);
            s[qt][kt] = M::run(a, qf[qt][c], s[qt][kt]);
          }
    } else {
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          const int krow = (kt0 + kt) * 32 + l32, kch = DMA ? ((2 * c + hh) ^ ((krow & 7) * SWZ)) : 2 * c + hh;
          const op_t a = *reinterpret_cast<const op_t *>(&Ks[buf][krow * KROW + kch * 8]);
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) s[qt][kt] = M::run(a, qf[qt][c], s[qt][kt]);
        }
    }
    if constexpr (MASK) {
      const int lim = (int)(Lk - j * BKV) - 4 * hh;  // local key offsets >= lim + 4 hh are past Lk
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if ((kt0 + kt) * 32 + 8 * (i >> 2) + (i & 3) >= lim) {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) s[qt][kt][i] = -INFINITY;
          }
    }

    // online softmax of query tile qt in two parts. smax moves the reference
    // maximum; after it one wave-uniform branch rescales O (rescale_all);
    // sexp then forms the probabilities (P packed as the B operand of
    // O^T += V^T P^T). Issued after that branch, the exponentials share one
    // basic block with the P v MFMAs, so the two can interleave.
    op_t pf[QT][NKT * 2];
    float alpha_q[QT];
    auto smax = [&](int qt) {
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[qt][kt][i]);
      const float cand = half_swap_max(mx) * c2;
      // LAZY keeps the reference maximum until a score exceeds it by 2^8: the
      // probabilities stay <= 256 and most blocks need no rescale at all
      float mn = m[qt];
      if constexpr (LAZY) {
        if (cand > mn + 8.f) mn = cand;
      } else {
        mn = fmaxf(mn, cand);
      }
      alpha_q[qt] = __builtin_amdgcn_exp2f(m[qt] - mn);
      m[qt] = mn;
    };
    auto rescale = [&](int qt) {
      if (!LAZY || __builtin_amdgcn_ballot_w64(alpha_q[qt] != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[qt][dt] *= alpha_q[qt];
      }
    };
    auto rescale_all = [&]() {
      bool any = false;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) any = any || alpha_q[qt] != 1.f;
      if (!LAZY || __builtin_amdgcn_ballot_w64(any)) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) o[qt][dt] *= alpha_q[qt];
      }
    };
    auto sexp = [&](int qt) {
      const float mn = m[qt];
      float ls = 0.f;
      if constexpr (EXACTP) {
        // f32 probabilities stay in s; split into bf16 terms at the P v product
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
          for (int i = 0; i < 16; i += 2) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qt][kt][i], c2, -mn));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qt][kt][i + 1], c2, -mn));
            s[qt][kt][i] = p0;
            s[qt][kt][i + 1] = p1;
            ls += p0 + p1;
          }
        l[qt] = l[qt] * alpha_q[qt] + ls;
        return;
      }
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          u32x4_t pk;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qt][kt][8 * jj + 2 * e], c2, -mn));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qt][kt][8 * jj + 2 * e + 1], c2, -mn));
            pk[e] = M::pack(p0, p1);
            // DOT: sum the rounded probabilities the P v product uses
            if constexpr (DOT) ls = M::sum2(pk[e], ls);
            else ls += p0 + p1;
          }
          pf[qt][kt * 2 + jj] = __builtin_bit_cast(op_t, pk);
        }
      l[qt] = l[qt] * alpha_q[qt] + ls;
    };
    // A = V^T[dim dt * 32 + l32][keys 16 * jj + 4 * hh + {0..3, 8..11}] of
    // tile kt (the accumulator order of the probabilities), read from V's
    // [key][dim] rows: ds_read_b64_tr_b16 hands lane i of each 16-lane group
    // element i % 4 of the 8 bytes that lane 4 e + i / 4 addressed, e = 0..3.
    // Lanes 4 e .. 4 e + 3 of a group address key row 4 hh + e and dims
    // 16 * ((lane / 16) % 2) + 4 * (lane % 4) .. + 3, so lane i receives dim
    // lane % 32 of keys 4 hh + 0..3; the second read, of keys 8 on.
    typedef short s16x4_t __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
    auto vfrag = [&](int dt, int kt, int jj) {
      const int g16 = lane & 15;
      const int vrow = (kt0 + kt) * 32 + 16 * jj + 4 * hh + (g16 >> 2);
      const int vcol = dt * 32 + 16 * ((lane >> 4) & 1) + 4 * (g16 & 3);  // rows vrow and vrow + 8 swizzle alike
      const int vch = DMA ? ((vcol >> 3) ^ ((vrow & 7) * SWZ)) : vcol >> 3;
      const uint16_t *vr = &Vs[buf][vrow * KROW + vch * 8 + (vcol & 7)];
      const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)(vr));
      const s16x4_t hi2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)(vr + 8 * KROW));
      return __builtin_bit_cast(op_t, __builtin_shufflevector(lo, hi2, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    // EXACTP: O^T += V^T (P1 + P2 + P3)^T, the three bf16 terms of each f32
    // probability pair built per 16-key step (one A fragment per dim tile)
    auto pv_exact = [&](int qt) {
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          u32x4_t p1, p2, p3;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            split3_into(s[qt][kt][8 * jj + 2 * e], s[qt][kt][8 * jj + 2 * e + 1], p1, p2, p3, e);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const op_t a = vfrag(dt, kt, jj);
            o[qt][dt] = M::run(a, __builtin_bit_cast(op_t, p1), o[qt][dt]);
            o[qt][dt] = M::run(a, __builtin_bit_cast(op_t, p2), o[qt][dt]);
            o[qt][dt] = M::run(a, __builtin_bit_cast(op_t, p3), o[qt][dt]);
          }
        }
    };
    if constexpr (EXACTP) {
#pragma unroll
      // one query tile at a time: with both tiles' exponentials in one basic
      // block the two-tile kernel spills
      for (int qt = 0; qt < QT; ++qt) {
        smax(qt);
        rescale(qt);
        sexp(qt);
        pv_exact(qt);
      }
    } else if constexpr (PHASED && QT == 2) {
      // P v of query tile 0 has no dependence on the softmax of tile 1:
      // issued together, the matrix cores and the VALU overlap in one wavefront
      smax(0);
      smax(1);
      rescale_all();
      sexp(0);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) o[0][dt] = M::run(vfrag(dt, kt, jj), pf[0][kt * 2 + jj], o[0][dt]);
      sexp(1);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) o[1][dt] = M::run(vfrag(dt, kt, jj), pf[1][kt * 2 + jj], o[1][dt]);
    } else {
      // DMA (the D = 128 kernels): every V fragment of the block is read
      // before the softmax, so the LDS latency hides behind the VALU work
      // (TRELLIS.2 40k 10.42 -> 9.91 ms, TripoSG 83.0 -> 81.6 us; D = 64 and
      // the register-staged D = 128 kernel do not gain or would spill).
      constexpr int NVF = DMA ? NDT * NKT * 2 : 1;
      op_t vf[NVF];
      if constexpr (DMA) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) vf[(dt * NKT + kt) * 2 + jj] = vfrag(dt, kt, jj);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) smax(qt);
      rescale_all();
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) sexp(qt);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            const op_t a = DMA ? vf[(dt * NKT + kt) * 2 + jj] : vfrag(dt, kt, jj);
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) o[qt][dt] = M::run(a, pf[qt][kt * 2 + jj], o[qt][dt]);
          }
    }

    if constexpr (DMA) __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // this wavefront's block j + 1 landed
    else if (j + 1 < nkv) store_kv(buf ^ 1);
    lds_barrier();
  };
  const int64_t nfull = tail ? nkv - 1 : nkv;
  for (int64_t j = 0; j < nfull; ++j) step(j, std::false_type{});
  if (tail) step(nkv - 1, std::true_type{});

  if constexpr (KS > 1) {
    // The KS partial results of a query group -- O (unnormalised), the
    // reference maximum m (log2 units) and the row-sum part l of each lane --
    // go through LDS (the K / V buffers are free after the last block's
    // barrier) and are merged in key-group order: M = max m_s,
    // l = sum l_s 2^(m_s - M), O = sum O_s 2^(m_s - M). Wavefront kg of the
    // group then owns the output dim tiles dt with dt % KS == kg. Lane-minor
    // layout: each LDS access of a wavefront is 64 consecutive floats.
    constexpr int PW = QT * (NDT * 16 + 2) * 64;  // floats per wavefront
    static_assert(4 * PW * 4 <= (int)sizeof(smem), "partials fit the K / V buffers");
    float *part = reinterpret_cast<float *>(smem);
    float *mine = part + wave * PW;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) mine[((qt * NDT + dt) * 16 + i) * 64 + lane] = o[qt][dt][i];
      mine[(QT * NDT * 16 + 2 * qt) * 64 + lane] = m[qt];
      mine[(QT * NDT * 16 + 2 * qt + 1) * 64 + lane] = l[qt];
    }
    lds_barrier();
    const float *grp = part + qg * KS * PW;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float ms[KS], a[KS], mm = -INFINITY;
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2) {
        ms[s2] = grp[s2 * PW + (QT * NDT * 16 + 2 * qt) * 64 + lane];
        mm = fmaxf(mm, ms[s2]);
      }
      float lsum = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < KS; ++s2) {
        a[s2] = __builtin_amdgcn_exp2f(ms[s2] - mm);
        lsum = lsum + grp[s2 * PW + (QT * NDT * 16 + 2 * qt + 1) * 64 + lane] * a[s2];
      }
      l[qt] = lsum;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        if (dt % KS != kg) continue;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          float acc = 0.f;
#pragma unroll
          for (int s2 = 0; s2 < KS; ++s2) acc = acc + grp[s2 * PW + ((qt * NDT + dt) * 16 + i) * 64 + lane] * a[s2];
          o[qt][dt][i] = acc;
        }
      }
    }
  }

  // out[query][dim]: lane holds dims dt * 32 + 8 * g + 4 * hh + {0..3}, g = 0..3
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int64_t qr = qb * BQ + (qg * QT + qt) * 32 + l32;
    const float inv = 1.f / half_swap_sum(l[qt]);
    if (qr >= Lq) continue;
    char *orow = obase + qr * p.o_st * ob;
    if (EXACTP && p.out_f32) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        if (KS > 1 && dt % KS != kg) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<float4 *>(orow + (dt * 32 + 8 * g + 4 * hh) * 4) =
              make_float4(o[qt][dt][4 * g] * inv, o[qt][dt][4 * g + 1] * inv, o[qt][dt][4 * g + 2] * inv,
                          o[qt][dt][4 * g + 3] * inv);
      }
      continue;
    }
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (KS > 1 && dt % KS != kg) continue;
        const uint2 w = make_uint2(M::pack(o[qt][dt][4 * g] * inv, o[qt][dt][4 * g + 1] * inv),
                                   M::pack(o[qt][dt][4 * g + 2] * inv, o[qt][dt][4 * g + 3] * inv));
        *reinterpret_cast<uint2 *>(orow + (dt * 32 + 8 * g + 4 * hh) * 2) = w;
      }
  }
}

// ---- f32 inputs on the bf16 matrix cores (three-term split) --------------------
//
// f32 q, k and v are split exactly into three bf16 terms each (x = x1 + x2 +
// x3, split3_bf16). A product x y is then the sum of nine bf16 x bf16
// products, each exact in f32; with |x2| <= 2^-8 |x| and |x3| <= 2^-17 |x|
// the three smallest (x2 y3, x3 y2, x3 y3) together stay below 2^-24 |x y|,
// under one f32 ulp of the product, and are dropped. Each MFMA step of S = K Q^T and of O^T += V^T P^T becomes six
// bf16 MFMAs (smallest terms first) accumulating in f32; the probabilities
// are f32 and split the same way, the row sum adds them in f32. That is the
// f32 arithmetic of exact_sdpa_heads (attention_math.rs:244-259) up to the
// order of the sums and that sub-ulp truncation per product, at 6 / 16
// of the matrix-core cycles of v_mfma_f32_32x32x2_f32 (which runs at 1/16
// of the bf16 rate). Layout as attn_mfma_kernel with QT = 1: K and V blocks
// of BKV keys are loaded as f32 (keys past Lk clamped to Lk - 1, their scores
// masked), split in registers and stored as three bf16 planes each, [key][dim]
// rows padded by 16 bytes, double-buffered.
// R3: DINOv3's rotate_half rotation of q (QP_R3) applied in the Q load with
// the head kernel's per-element arithmetic (rotate1), bit for bit.
template <int D, int BKV, int MINW, bool R3 = false>
__global__ __launch_bounds__(256, MINW) void attn_f32x3_kernel(AttnParams p, int64_t nqb, int64_t nwg) {
  using op_t = bf16x8_t;
  using M = Mma<BF16>;
  constexpr int BQ = 128;
  constexpr int KROW = D + 8;              // bf16 per plane row
  constexpr int PL = BKV * KROW;           // one plane of one block
  constexpr int KCH = BKV * D / 4 / 256;   // 16-byte f32 chunks of K (and of V) per thread per block
  constexpr int NKT = BKV / 32, NDT = D / 32;
  static_assert(KCH >= 1 && BKV % 32 == 0 && D % 32 == 0, "tile shape");
  __shared__ __align__(16) uint16_t smem[2 * 6 * PL];  // [buffer][K planes 0..2, V planes 0..2]

  const int64_t lid = xcd_logical_id(blockIdx.x, nwg);
  const int64_t bh = lid / nqb, qb = lid % nqb;
  const int64_t bi = bh / p.H, hi = bh % p.H;
  const float *qbase = reinterpret_cast<const float *>(p.q) + bi * p.q_sb + hi * p.q_sh;
  const float *kbase = reinterpret_cast<const float *>(p.k) + bi * p.k_sb + hi * p.k_sh;
  const float *vbase = reinterpret_cast<const float *>(p.v) + bi * p.v_sb + hi * p.v_sh;
  float *obase = reinterpret_cast<float *>(p.o) + bi * p.o_sb + hi * p.o_sh;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int l32 = lane & 31, hh = lane >> 5;
  const int64_t Lq = p.Lq, Lk = p.Lk;

  // Q as the B operand, three terms: lane holds Q[query l32][c * 16 + 8 * hh + e]
  op_t q1[D / 16], q2[D / 16], q3[D / 16];
  {
    int64_t qr = qb * BQ + wave * 32 + l32;
    qr = qr < Lq ? qr : Lq - 1;
    const float *qrow = qbase + qr * p.q_st;
    float xq[D / 16][8];
#pragma unroll
    for (int c = 0; c < D / 16; ++c) Chunk<F32>::load<false>(qrow + c * 16 + 8 * hh, xq[c]);
    if constexpr (R3) {
      // element j = 16 c + 8 hh + e; its partner j ^ D/2 is element e of the
      // lane's own chunk c ^ D/32; S = -sin for j < D/2. Tokens before the
      // prefix pass through (table row clamped to 0, rotation discarded).
      const bool rot = qr >= p.prefix;
      const int64_t trow = (rot ? qr - p.prefix : 0) * p.tab_sN;
      float yq[D / 16][8];
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        float C8[8], S8[8];
        param8(p.tab_c, p.tab_dt, trow + c * 16 + 8 * hh, 1.f, C8);
        param8(p.tab_s, p.tab_dt, trow + c * 16 + 8 * hh, 0.f, S8);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          yq[c][e] = rot ? rotate1(xq[c][e], C8[e], xq[c ^ (D / 32)][e], c < D / 32 ? -S8[e] : S8[e]) : xq[c][e];
      }
#pragma unroll
      for (int c = 0; c < D / 16; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) xq[c][e] = yq[c][e];
    }
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      u32x4_t x1, x2, x3;
#pragma unroll
      for (int e = 0; e < 4; ++e) split3_into(xq[c][2 * e], xq[c][2 * e + 1], x1, x2, x3, e);
      q1[c] = __builtin_bit_cast(op_t, x1);
      q2[c] = __builtin_bit_cast(op_t, x2);
      q3[c] = __builtin_bit_cast(op_t, x3);
    }
  }
  // staging: chunk c = t + 256 i holds K / V row c / (D/4), floats 4 (c % (D/4)) ..
  int s_row[KCH], s_c4[KCH];
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    const int c = t + i * 256;
    s_row[i] = c / (D / 4);
    s_c4[i] = c % (D / 4);
  }
  float4 rk[KCH], rv[KCH];
  // element offsets of this thread's chunks from a block's first key
  int64_t k_off[KCH], v_off[KCH];
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    k_off[i] = (int64_t)s_row[i] * p.k_st + s_c4[i] * 4;
    v_off[i] = (int64_t)s_row[i] * p.v_st + s_c4[i] * 4;
  }
  // `clamp` (the tail block only): keys past Lk read row Lk - 1
  auto load_kv = [&](int64_t j, bool clamp) {
    if (!clamp) {
      const float *kb = kbase + j * BKV * p.k_st, *vb = vbase + j * BKV * p.v_st;
#pragma unroll
      for (int i = 0; i < KCH; ++i) rk[i] = *reinterpret_cast<const float4 *>(kb + k_off[i]);
#pragma unroll
      for (int i = 0; i < KCH; ++i) rv[i] = *reinterpret_cast<const float4 *>(vb + v_off[i]);
      return;
    }
    const int64_t key0 = j * BKV;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      int64_t key = key0 + s_row[i];
      key = key < Lk ? key : Lk - 1;
      rk[i] = *reinterpret_cast<const float4 *>(kbase + key * p.k_st + s_c4[i] * 4);
      rv[i] = *reinterpret_cast<const float4 *>(vbase + key * p.v_st + s_c4[i] * 4);
    }
  };
  auto store_kv = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int off = s_row[i] * KROW + s_c4[i] * 4;
      const Split3 ka = split3_bf16(rk[i].x, rk[i].y), kb = split3_bf16(rk[i].z, rk[i].w);
      *reinterpret_cast<uint2 *>(smem + (buf * 6 + 0) * PL + off) = make_uint2(ka.t1, kb.t1);
      *reinterpret_cast<uint2 *>(smem + (buf * 6 + 1) * PL + off) = make_uint2(ka.t2, kb.t2);
      *reinterpret_cast<uint2 *>(smem + (buf * 6 + 2) * PL + off) = make_uint2(ka.t3, kb.t3);
      const Split3 va = split3_bf16(rv[i].x, rv[i].y), vb = split3_bf16(rv[i].z, rv[i].w);
      *reinterpret_cast<uint2 *>(smem + (buf * 6 + 3) * PL + off) = make_uint2(va.t1, vb.t1);
      *reinterpret_cast<uint2 *>(smem + (buf * 6 + 4) * PL + off) = make_uint2(va.t2, vb.t2);
      *reinterpret_cast<uint2 *>(smem + (buf * 6 + 5) * PL + off) = make_uint2(va.t3, vb.t3);
    }
  };

  f32x16_t o[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x16_t{};
  float m = -INFINITY, l = 0.f;
  const float c2 = p.scale * kLog2e;
  const int64_t nkv = (Lk + BKV - 1) / BKV;
  const bool tail = (Lk % BKV) != 0;

  load_kv(0, nkv == 1 && tail);
  store_kv(0);
  lds_barrier();

  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
  auto step = [&](int64_t j, auto mask_c) {
    constexpr bool MASK = decltype(mask_c)::value;
    const int buf = (int)(j & 1);
    if (j + 1 < nkv) load_kv(j + 1, tail && j + 2 == nkv);
    const uint16_t *K1 = smem + (buf * 6 + 0) * PL, *K2 = smem + (buf * 6 + 1) * PL, *K3 = smem + (buf * 6 + 2) * PL;

    // S^T = K Q^T: lane holds key 8 * (i / 4) + 4 * hh + i % 4 of each 32-key tile, query l32
    f32x16_t s[NKT];
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
      s[kt] = f32x16_t{};
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        const int off = (kt * 32 + l32) * KROW + (2 * c + hh) * 8;
        const op_t a1 = *reinterpret_cast<const op_t *>(K1 + off);
        const op_t a2 = *reinterpret_cast<const op_t *>(K2 + off);
        const op_t a3 = *reinterpret_cast<const op_t *>(K3 + off);
        s[kt] = M::run(a3, q1[c], s[kt]);
        s[kt] = M::run(a2, q2[c], s[kt]);
        s[kt] = M::run(a1, q3[c], s[kt]);
        s[kt] = M::run(a2, q1[c], s[kt]);
        s[kt] = M::run(a1, q2[c], s[kt]);
        s[kt] = M::run(a1, q1[c], s[kt]);
      }
    }
    if constexpr (MASK) {
      const int lim = (int)(Lk - j * BKV) - 4 * hh;  // local key offsets >= lim + 4 hh are past Lk
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (kt * 32 + 8 * (i >> 2) + (i & 3) >= lim) s[kt][i] = -INFINITY;
    }
    // online softmax in f32; the reference maximum moves only when a block's
    // maximum exceeds it by 2^8 (probabilities stay <= 256)
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[kt][i]);
    const float cand = half_swap_max(mx) * c2;
    float mn = m;
    if (cand > mn + 8.f) mn = cand;
    const float alpha = __builtin_amdgcn_exp2f(m - mn);
    m = mn;
    float ls = 0.f;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][i], c2, -mn));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][i + 1], c2, -mn));
        s[kt][i] = p0;
        s[kt][i + 1] = p1;
        ls += p0 + p1;
      }
    l = l * alpha + ls;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
    }
    // O^T += V^T P^T with three-term V and P: A = V^T fragments of each plane
    // (ds_read_b64_tr_b16 from V's [key][dim] rows, as in attn_mfma_kernel)
    auto vfrag = [&](int pl, int dt, int kt, int jj) {
      const int g16 = lane & 15;
      const int vrow = kt * 32 + 16 * jj + 4 * hh + (g16 >> 2);
      const int vcol = dt * 32 + 16 * ((lane >> 4) & 1) + 4 * (g16 & 3);
      const uint16_t *vr = smem + (buf * 6 + 3 + pl) * PL + vrow * KROW + vcol;
      const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)(vr));
      const s16x4_t hi2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)(vr + 8 * KROW));
      return __builtin_bit_cast(op_t, __builtin_shufflevector(lo, hi2, 0, 1, 2, 3, 4, 5, 6, 7));
    };
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        u32x4_t x1, x2, x3;
#pragma unroll
        for (int e = 0; e < 4; ++e) split3_into(s[kt][8 * jj + 2 * e], s[kt][8 * jj + 2 * e + 1], x1, x2, x3, e);
        const op_t P1 = __builtin_bit_cast(op_t, x1), P2 = __builtin_bit_cast(op_t, x2);
        const op_t P3 = __builtin_bit_cast(op_t, x3);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const op_t v1 = vfrag(0, dt, kt, jj), v2 = vfrag(1, dt, kt, jj), v3 = vfrag(2, dt, kt, jj);
          o[dt] = M::run(v3, P1, o[dt]);
          o[dt] = M::run(v2, P2, o[dt]);
          o[dt] = M::run(v1, P3, o[dt]);
          o[dt] = M::run(v2, P1, o[dt]);
          o[dt] = M::run(v1, P2, o[dt]);
          o[dt] = M::run(v1, P1, o[dt]);
        }
      }
    if (j + 1 < nkv) store_kv(buf ^ 1);
    lds_barrier();
  };
  const int64_t nfull = tail ? nkv - 1 : nkv;
  for (int64_t j = 0; j < nfull; ++j) step(j, std::false_type{});
  if (tail) step(nkv - 1, std::true_type{});

  // out[query][dim] (f32): lane holds dims dt * 32 + 8 * g + 4 * hh + {0..3}, g = 0..3
  const int64_t qr = qb * BQ + wave * 32 + l32;
  const float inv = 1.f / half_swap_sum(l);
  if (qr < Lq) {
    float *orow = obase + qr * p.o_st;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4 *>(orow + dt * 32 + 8 * g + 4 * hh) =
            make_float4(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv);
  }
}

// ---- generic kernel ----------------------------------------------------------

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ float wave_sum_xor(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ float bcast(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// DPL = head dims per lane (D <= 64 * DPL).
template <typename T, int DPL>
__global__ __launch_bounds__(256) void attn_generic_kernel(AttnParams p, int64_t rows) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;  // whole wavefronts leave; no barrier below
  const int64_t bh = r / p.Lq, qi = r % p.Lq;
  const int64_t bi = bh / p.H, hi = bh % p.H;
  constexpr int EB = T::bytes;
  const char *qrow = reinterpret_cast<const char *>(p.q) + (bi * p.q_sb + hi * p.q_sh + qi * p.q_st) * EB;
  const char *kbase = reinterpret_cast<const char *>(p.k) + (bi * p.k_sb + hi * p.k_sh) * EB;
  const char *vbase = reinterpret_cast<const char *>(p.v) + (bi * p.v_sb + hi * p.v_sh) * EB;
  char *orow = reinterpret_cast<char *>(p.o) + (bi * p.o_sb + hi * p.o_sh + qi * p.o_st) * (p.out_f32 ? 4 : EB);
  const int64_t D = p.D, Lk = p.Lk;

  float qv[DPL], o[DPL];
#pragma unroll
  for (int u = 0; u < DPL; ++u) {
    const int64_t d = lane + 64 * u;
    qv[u] = d < D ? load1<T>(qrow, d) : 0.f;
    o[u] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  for (int64_t j0 = 0; j0 < Lk; j0 += 64) {
    const int64_t key = j0 + lane;
    const bool valid = key < Lk;
    const char *kr = kbase + (valid ? key : Lk - 1) * p.k_st * EB;
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < DPL; ++u)
      for (int e = 0; e < 64; ++e) {
        const int64_t d = 64 * u + e;
        if (d >= D) break;
        s += bcast(qv[u], e) * load1<T>(kr, d);
      }
    s = valid ? s * p.scale : -INFINITY;
    const float mn = fmaxf(m, wave_max(s));
    const float alpha = __expf(m - mn);
    const float pj = valid ? __expf(s - mn) : 0.f;
    l = l * alpha + wave_sum_xor(pj);
    m = mn;
#pragma unroll
    for (int u = 0; u < DPL; ++u) o[u] *= alpha;
    const int64_t nk = Lk - j0 < 64 ? Lk - j0 : 64;
    for (int kk = 0; kk < nk; ++kk) {
      const float pk = bcast(pj, kk);
      const char *vr = vbase + (j0 + kk) * p.v_st * EB;
#pragma unroll
      for (int u = 0; u < DPL; ++u) {
        const int64_t d = lane + 64 * u;
        if (d < D) o[u] += pk * load1<T>(vr, d);
      }
    }
  }
  const float inv = 1.f / l;
#pragma unroll
  for (int u = 0; u < DPL; ++u) {
    const int64_t d = lane + 64 * u;
    if (d < D) {
      if (p.out_f32) store1<F32>(orow, d, o[u] * inv);
      else store1<T>(orow, d, o[u] * inv);
    }
  }
}

template <typename T, int D, int QT, int BKV, int MINW, bool LAZY, bool DOT, bool PHASED, bool DMA,
          bool EXACTP = false, int KS = 1>
hipError_t launch_mfma(const AttnParams &p, hipStream_t s) {
  constexpr int BQ = 4 / KS * 32 * QT;
  const int64_t nqb = (p.Lq + BQ - 1) / BQ;
  const int64_t nwg = p.B * p.H * nqb;
  if (nwg > INT32_MAX) return hipErrorInvalidValue;
  const dim3 grid((unsigned)nwg), block(256);
  if constexpr (EXACTP) {
    // exact_sdpa_heads: q as it is, or DINOv3's rotation in the Q load
    if (p.qpro == QP_R3)
      hipLaunchKernelGGL((attn_mfma_kernel<T, D, QT, BKV, MINW, LAZY, false, PHASED, QP_R3, DMA, true, KS>), grid, block,
                         0, s, p, nqb, nwg);
    else
      hipLaunchKernelGGL((attn_mfma_kernel<T, D, QT, BKV, MINW, LAZY, false, PHASED, QP_NONE, DMA, true, KS>), grid,
                         block, 0, s, p, nqb, nwg);
  } else {
    switch (p.qpro) {
      case QP_LN_R1:
        hipLaunchKernelGGL((attn_mfma_kernel<T, D, QT, BKV, MINW, LAZY, DOT, PHASED, QP_LN_R1, DMA, false, KS>), grid, block, 0,
                           s, p, nqb, nwg);
        break;
      case QP_RMS:
        hipLaunchKernelGGL((attn_mfma_kernel<T, D, QT, BKV, MINW, LAZY, DOT, PHASED, QP_RMS, DMA, false, KS>), grid, block, 0, s,
                           p, nqb, nwg);
        break;
      case QP_L2_R2:
        hipLaunchKernelGGL((attn_mfma_kernel<T, D, QT, BKV, MINW, LAZY, DOT, PHASED, QP_L2_R2, DMA, false, KS>), grid, block, 0,
                           s, p, nqb, nwg);
        break;
      default:
        hipLaunchKernelGGL((attn_mfma_kernel<T, D, QT, BKV, MINW, LAZY, DOT, PHASED, QP_NONE, DMA, false, KS>), grid, block, 0,
                           s, p, nqb, nwg);
    }
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_generic(const AttnParams &p, hipStream_t s) {
  const int64_t rows = p.B * p.H * p.Lq;
  const int64_t groups = (rows + 3) / 4;
  if (groups > INT32_MAX) return hipErrorInvalidValue;
  const dim3 grid((unsigned)groups), block(256);
  if (p.D <= 64) hipLaunchKernelGGL((attn_generic_kernel<T, 1>), grid, block, 0, s, p, rows);
  else if (p.D <= 128) hipLaunchKernelGGL((attn_generic_kernel<T, 2>), grid, block, 0, s, p, rows);
  else if (p.D <= 256) hipLaunchKernelGGL((attn_generic_kernel<T, 4>), grid, block, 0, s, p, rows);
  else if (p.D <= 512) hipLaunchKernelGGL((attn_generic_kernel<T, 8>), grid, block, 0, s, p, rows);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

// Every key offset of a head (in bytes, elements of eb bytes) fits the
// 32-bit offsets of the direct loads
bool dma_fits(const AttnParams &p, int eb) {
  const int64_t st = p.k_st > p.v_st ? p.k_st : p.v_st;
  return p.k_st >= 0 && p.v_st >= 0 && ((p.Lk + 64) * st + p.D) * eb < (int64_t(1) << 31);
}

template <int D, int BKV, int MINW>
hipError_t launch_f32x3(const AttnParams &p, hipStream_t s) {
  const int64_t nqb = (p.Lq + 127) / 128;
  const int64_t nwg = p.B * p.H * nqb;
  if (nwg > INT32_MAX) return hipErrorInvalidValue;
  if (p.qpro == QP_R3)
    hipLaunchKernelGGL((attn_f32x3_kernel<D, BKV, MINW, true>), dim3((unsigned)nwg), dim3(256), 0, s, p, nqb, nwg);
  else
    hipLaunchKernelGGL((attn_f32x3_kernel<D, BKV, MINW>), dim3((unsigned)nwg), dim3(256), 0, s, p, nqb, nwg);
  return hipGetLastError();
}

// D 128: K / V as direct global -> LDS loads (DMA) when every key offset of
// a head fits the 32-bit buffer offsets (TripoSG 87.2 against 92.3 us,
// TRELLIS.2 40k voxels 10.3 against 11.2 ms, bit-identical). D 64 stays
// register-staged (with rotating inputs DMA gained nothing there):
// 128-query workgroups (three per CU) or 256-query ones (the phased form,
// two per CU), whichever leaves the busiest CU less work (below), also with
// q's LayerNorm fused (VGGT frame 92.8 against 96.0 us); the exact-
// probability kernel takes 128-query ones up to kShortQ queries.
constexpr int64_t kShortQ = 4096;
constexpr int64_t kCus = 256;  // MI355X

// Time of the busiest CU when nwg workgroups spread evenly over the CUs and
// per_cu of them run at once; t[k] is the time of k resident workgroups.
int64_t busiest_cu_time(int64_t nwg, int per_cu, const int *t) {
  const int64_t m = (nwg + kCus - 1) / kCus;
  return (m / per_cu) * t[per_cu] + t[m % per_cu];
}
// t: VGGT frames (1374 keys, D 64) timed with k workgroups resident per CU,
// in 0.1 us: 128-query 20.4 / 32.5 / 45.4 us (k = 1 / 2 / 3), 256-query
// 32.0 / 54.7 us (k = 1 / 2). The 256-query form must win by 3%; so set,
// the rule picks the faster form at each of 2 to 8 frames, 1 / 2 / 4 x 2048
// tokens and DINOv3's 1029 (both forms timed at each).
bool use_256_query(const AttnParams &p) {
  static const int t1[4] = {0, 204, 325, 454}, t2[3] = {0, 320, 547};
  const int64_t n1 = p.B * p.H * ((p.Lq + 127) / 128), n2 = p.B * p.H * ((p.Lq + 255) / 256);
  return 100 * busiest_cu_time(n2, 2, t2) < 97 * busiest_cu_time(n1, 3, t1);
}

// Key groups per query tile (KS, D 64): with few 128-query tiles (DINOv3:
// 16 heads x 9 tiles = 144 workgroups, one wavefront per SIMD on 144 of the
// 256 CUs) the four wavefronts of a workgroup share 128 / KS queries and
// split each key block KS ways, merging in LDS at the end: KS times the
// workgroups, each wavefront with 1 / KS of the keys. These kernels are
// VALU-bound (exact_sdpa_heads: about 370 VALU instructions per 64-key block
// and wavefront against 32 MFMAs), so the busiest SIMD's share sets the
// time; KS = 2 is taken while the doubled grid still fits three workgroups
// per CU. Measured (exact_sdpa_heads bf16, D 64, us, KS = 1 / 2 / 4):
// 16 heads x 1029 tokens 26.3 / 24.2 / 25.5, x 1024 22.6 / 17.3 / 16.4,
// 8 x 1029 23.9 / 17.3 / 16.7, 2 x 16 x 1029 37.0 / 32.2 / 38.1, 4 x 4096
// 78.3 / 55.0 / 50.5, 16 x 2048 45.7 / 43.2 / 50.9; KS = 4 (128-key blocks,
// two workgroups per CU) gains little more where it gains and loses
// elsewhere, so it is not chosen by default. Needs Lk >= the block (every
// key group sees keys in block 0). LUX3D_ATTN_KS=1 / 2 / 4 forces a choice
// (timing).
int key_groups(const AttnParams &p) {
  const int64_t tiles = p.B * p.H * ((p.Lq + 127) / 128);
  int ks = 2 * tiles <= 3 * kCus ? 2 : 1;
  if (const char *e = getenv("LUX3D_ATTN_KS")) ks = atoi(e);
  if (ks == 4 && p.Lk >= 128) return 4;
  if (ks == 2 && p.Lk >= 64) return 2;
  return 1;
}

template <typename T>
hipError_t launch_t(const AttnParams &p, hipStream_t s) {
  // a Q prologue runs on the matrix-core kernels only: 2-byte types (or f32
  // with DINOv3's rotation), D 64 / 128; exact_sdpa_heads takes QP_R3 only
  if (p.qpro != QP_NONE) {
    if (!p.mfma || (p.D != 64 && p.D != 128) || p.qpro < QP_LN_R1 || p.qpro > QP_R3) return hipErrorInvalidValue;
    if (T::code == LUX3D_F32 && p.qpro != QP_R3) return hipErrorInvalidValue;
    if ((p.qpro == QP_R3) != p.exact_p) return hipErrorInvalidValue;
    if (p.qpro == QP_R3 && T::code == LUX3D_F16) return hipErrorInvalidValue;
  }
  if (p.out_f32 && !p.exact_p && T::code != LUX3D_F32) return hipErrorInvalidValue;
  if (p.exact_p && T::code != LUX3D_F32) {
    // f32 probabilities: the bf16 matrix-core kernel with three-term P, else
    // the generic kernel (f32 throughout)
    if constexpr (T::code == LUX3D_BF16) {
      if (p.mfma && p.D == 64) {
        const int ks = key_groups(p);
        if (ks == 4) return launch_mfma<T, 64, 1, 128, 2, true, false, false, false, true, 4>(p, s);
        if (ks == 2) return launch_mfma<T, 64, 1, 64, 3, true, false, false, false, true, 2>(p, s);
        if (p.Lq <= kShortQ) return launch_mfma<T, 64, 1, 64, 3, true, false, false, false, true>(p, s);
        return launch_mfma<T, 64, 2, 64, 2, true, false, false, false, true>(p, s);
      }
      if (p.mfma && p.D == 128) {
        if (dma_fits(p, 2)) return launch_mfma<T, 128, 1, 64, 2, true, false, false, true, true>(p, s);
        return launch_mfma<T, 128, 1, 64, 2, true, false, false, false, true>(p, s);
      }
    }
    return launch_generic<T>(p, s);
  }
  if constexpr (T::code != LUX3D_F32) {
    if (p.mfma) {
      if (p.D == 64) {
        const int ks = key_groups(p);
        if (ks == 4) return launch_mfma<T, 64, 1, 128, 2, true, true, false, false, false, 4>(p, s);
        if (ks == 2) return launch_mfma<T, 64, 1, 64, 3, true, true, false, false, false, 2>(p, s);
        if (!use_256_query(p))
          return launch_mfma<T, 64, 1, 64, 3, true, true, false, false>(p, s);
        return launch_mfma<T, 64, 2, 64, 2, true, true, true, false>(p, s);
      }
      if (p.D == 128) {
        if (dma_fits(p, 2)) return launch_mfma<T, 128, 1, 64, 2, true, true, false, true>(p, s);
        return launch_mfma<T, 128, 1, 64, 2, true, true, false, false>(p, s);
      }
    }
  } else {
    if (p.mfma) {
      // f32 on the bf16 matrix cores (three-term splits), 32-key blocks: at
      // D 64 55 KB of LDS and 181 VGPRs, two workgroups per CU; at D 128
      // 104 KB, one. Against the f32 MFMA kernel this replaced (same box,
      // graph-timed): VGGT frame 342 against 541 us, TripoSG 401 against 523,
      // DINOv3 52.5 against 86.0
      if (p.D == 64) return launch_f32x3<64, 32, 2>(p, s);
      if (p.D == 128) return launch_f32x3<128, 32, 1>(p, s);
    }
  }
  return launch_generic<T>(p, s);
}

}  // namespace

hipError_t launch_attention(int dt, const AttnParams &p, hipStream_t s) {
  if (p.B <= 0 || p.H <= 0 || p.Lq <= 0) return hipSuccess;
  if (p.Lk <= 0 || p.D <= 0) return hipErrorInvalidValue;
  switch (dt) {
    case LUX3D_BF16: return launch_t<BF16>(p, s);
    case LUX3D_F16: return launch_t<F16>(p, s);
    case LUX3D_F32: return launch_t<F32>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace lux3d
