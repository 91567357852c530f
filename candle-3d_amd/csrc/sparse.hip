// sparse.hip -- TRELLIS.2 sparse voxel ops for gfx950 (runtime/trellis2_sparse.rs):
// the coordinate map and neighbour table, the submanifold 3x3x3 sparse
// convolution, row gathers and the channel-to-spatial (C2S) subdivision.
//
// Coordinate map: an open-addressing hash table in a caller workspace (keys
// packed as 3 x 21-bit biased coordinates, linear probing, 64-bit
// compare-and-swap inserts; a duplicate coordinate keeps the largest row,
// which is the reference HashMap's "later insert overwrites"). The
// neighbour table nbr[i][k] = row of coords[i] + delta(k) or -1, with
// k = kd*9 + kh*3 + kw and delta = (kd-1, kh-1, kw-1).
//
// Sparse convolution, output-stationary: out[i, :] = bias + sum_k W_k
// x[nbr[i][k], :] as ONE implicit GEMM [N, 27*Cin] x [27*Cin, Cout] whose A
// rows are gathered through the neighbour table (missing neighbours load
// zeros). The reference's 27 gather + GEMM + index_add passes become one
// kernel, and every output element is written once: no scatter, no atomics,
// a fixed summation order. f32 arithmetic, as the reference computes sparse
// features in F32, on the bf16 matrix cores: each staged f32 operand is split
// exactly into three bf16 terms and a product keeps the six largest of the
// nine term products (split3_bf16; the rulebook tap kernel below states the
// bound). Taps that no row of a tile uses are skipped.
//
// C2S: per parent the leaf mask (logits > 0) and its popcount, an exclusive
// scan of the counts (block scans + one scan of the block totals), then one
// thread per (parent, subidx) writes the child coordinate and source row in
// the reference order (parent order, ascending subidx), and a row gather
// copies the child features. The child count is written to device memory.
#include <mutex>

#include "common.hpp"
#include "kernels.hpp"

namespace lux3d {

// Coordinate hash table of the allocation-free neighbour entry
// (lux3d_sparse_neighbors_noalloc): keys u64 [kNoAllocCap] then vals int32
// [kNoAllocCap], one copy per device, held until the process ends. Device
// code only: host code uses the address hipGetSymbolAddress returns for the
// current device (noalloc_table below), never this name.
static __device__ __align__(256) unsigned char scratch[kNoAllocTableBytes];

namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr unsigned long long kEmptyKey = ~0ull;

__device__ __forceinline__ unsigned long long pack_coord(int32_t x, int32_t y, int32_t z) {
  return ((unsigned long long)(uint32_t)(x + (1 << 20)) << 42) | ((unsigned long long)(uint32_t)(y + (1 << 20)) << 21) |
         (unsigned long long)(uint32_t)(z + (1 << 20));
}
__device__ __forceinline__ bool coord_ok(int32_t x, int32_t y, int32_t z) {
  const int32_t lo = -(1 << 20), hi = (1 << 20) - 1;
  return x >= lo && x < hi && y >= lo && y < hi && z >= lo && z < hi;
}
__device__ __forceinline__ uint64_t hash_key(unsigned long long k) {
  uint64_t h = (uint64_t)k * 0x9E3779B97F4A7C15ull;
  return h ^ (h >> 29);
}

// bad (optional): the count of coordinates outside the packable range,
// zeroed here and incremented by map_insert_kernel (the next launch).
__global__ __launch_bounds__(256) void map_clear_kernel(unsigned long long *keys, int32_t *vals, int64_t cap,
                                                        int32_t *bad) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < cap) {
    keys[i] = kEmptyKey;
    vals[i] = -1;
  }
  if (bad && i == 0) *bad = 0;
}

__global__ __launch_bounds__(256) void map_insert_kernel(const int32_t *coords, int64_t n, unsigned long long *keys,
                                                         int32_t *vals, int64_t cap, int32_t *bad) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int32_t x = coords[3 * i], y = coords[3 * i + 1], z = coords[3 * i + 2];
  if (!coord_ok(x, y, z)) {  // neither inserted nor found: counted
    if (bad) atomicAdd(bad, 1);
    return;
  }
  const unsigned long long key = pack_coord(x, y, z);
  uint64_t slot = hash_key(key) & (uint64_t)(cap - 1);
  for (int64_t probe = 0; probe < cap; ++probe) {  // cap >= 2n: a free slot exists
    const unsigned long long prev = atomicCAS(&keys[slot], kEmptyKey, key);
    if (prev == kEmptyKey || prev == key) {
      atomicMax(&vals[slot], (int32_t)i);
      return;
    }
    slot = (slot + 1) & (uint64_t)(cap - 1);
  }
}

__global__ __launch_bounds__(256) void map_neighbors_kernel(const int32_t *coords, int64_t n,
                                                            const unsigned long long *keys, const int32_t *vals,
                                                            int64_t cap, int32_t *nbr) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= n * 27) return;
  const int64_t i = t / 27;
  const int k = (int)(t % 27);
  const int32_t x = coords[3 * i] + k / 9 - 1, y = coords[3 * i + 1] + (k % 9) / 3 - 1, z = coords[3 * i + 2] + k % 3 - 1;
  int32_t found = -1;
  if (coord_ok(x, y, z)) {
    const unsigned long long key = pack_coord(x, y, z);
    uint64_t slot = hash_key(key) & (uint64_t)(cap - 1);
    for (int64_t probe = 0; probe < cap; ++probe) {
      const unsigned long long kk = keys[slot];
      if (kk == key) {
        found = vals[slot];
        break;
      }
      if (kk == kEmptyKey) break;
      slot = (slot + 1) & (uint64_t)(cap - 1);
    }
  }
  nbr[t] = found;
}

// ---- sparse convolution -------------------------------------------------------

// A 256-thread workgroup computes BM rows x BN output channels; its 4
// wavefronts (2 x 2) each own (BM/2) x (BN/2) as 32 x 32 MFMA tiles. The K
// loop runs over the used taps and Cin in steps of BK = 16; each step stages
// x and W_k as three bf16 planes (the layout of sparse_tap_x3_kernel) and
// runs six bf16 MFMAs per tile.
template <int BM, int BN>
__global__ __launch_bounds__(256) void sparse_conv_x3_kernel(SparseConvParams p) {
  typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
  constexpr int BK = 16;
  constexpr int TM = BM / 64, TN = BN / 64;
  constexpr int ACH = BM * BK / 4 / 256, BCH = BN * BK / 4 / 256;  // float4 per thread per step
  static_assert(ACH >= 1 && BCH >= 1, "tile");
  constexpr int PA = BM * BK * 2, PB = BN * BK * 2;  // bytes of one bf16 plane
  constexpr int STAGE = 3 * (PA + PB);
  __shared__ __align__(16) char lds[2 * STAGE];
  __shared__ int32_t nb[BM * 27];
  __shared__ uint32_t tap_mask;

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  const int64_t N = p.n, Cin = p.cin, Cout = p.cout;

  if (t == 0) tap_mask = 0u;
  __syncthreads();
  uint32_t my_mask = 0;
  for (int e = t; e < BM * 27; e += 256) {
    const int r = e / 27, k = e % 27;
    int32_t s = m0 + r < N ? p.nbr[(m0 + r) * 27 + k] : -1;
    s = s < N ? s : -1;  // a table entry past the rows reads as a missing neighbour
    nb[e] = s;
    if (s >= 0) my_mask |= 1u << k;
  }
  if (my_mask) atomicOr(&tap_mask, my_mask);
  __syncthreads();
  const uint32_t mask = tap_mask;

  // staging: A = gathered x rows, B = W[k] rows (output channels past Cout clamp)
  int a_row[ACH], a_part[ACH], b_row[BCH], b_part[BCH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int c = t + i * 256;
    a_row[i] = c / (BK / 4);
    a_part[i] = c % (BK / 4);
  }
#pragma unroll
  for (int i = 0; i < BCH; ++i) {
    const int c = t + i * 256;
    b_row[i] = c / (BK / 4);
    b_part[i] = c % (BK / 4);
  }
  const int64_t csteps = Cin / BK;
  float4 ra[ACH], rb[BCH];
  bool aok[ACH];
  auto load_step = [&](int k, int64_t c0) {
    // a missing row loads row 0 and is zeroed when staged: a branch around
    // the load would make the compiler wait for it before the next load
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int32_t s = nb[a_row[i] * 27 + k];
      aok[i] = s >= 0;
      ra[i] = *reinterpret_cast<const float4 *>(p.x + (int64_t)(s >= 0 ? s : 0) * Cin + c0 + a_part[i] * 4);
    }
#pragma unroll
    for (int i = 0; i < BCH; ++i) {
      int64_t o = n0 + b_row[i];
      o = o < Cout ? o : Cout - 1;
      rb[i] = *reinterpret_cast<const float4 *>(p.w + ((int64_t)k * Cout + o) * Cin + c0 + b_part[i] * 4);
    }
  };
  auto put = [](char *plane0, int pbytes, int off, float4 v) {
    const Split3 lo = split3_bf16(v.x, v.y), hi = split3_bf16(v.z, v.w);
    *reinterpret_cast<uint2 *>(plane0 + off) = make_uint2(lo.t1, hi.t1);
    *reinterpret_cast<uint2 *>(plane0 + pbytes + off) = make_uint2(lo.t2, hi.t2);
    *reinterpret_cast<uint2 *>(plane0 + 2 * pbytes + off) = make_uint2(lo.t3, hi.t3);
  };
  auto store_step = [&](int buf) {
    char *st = lds + buf * STAGE;
#pragma unroll
    for (int i = 0; i < ACH; ++i)
      put(st, PA, a_row[i] * 32 + a_part[i] * 8, aok[i] ? ra[i] : make_float4(0.f, 0.f, 0.f, 0.f));
#pragma unroll
    for (int i = 0; i < BCH; ++i) put(st + 3 * PA, PB, b_row[i] * 32 + b_part[i] * 8, rb[i]);
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};

  // the step sequence: used taps in order, Cin chunks inside each
  const int ntaps = __builtin_popcount(mask);
  const int64_t nsteps = (int64_t)ntaps * csteps;
  auto step_at = [&](int64_t st, int &k, int64_t &c0) {
    const int64_t ti = st / csteps;
    c0 = (st % csteps) * BK;
    uint32_t mm = mask;
    for (int64_t q = 0; q < ti; ++q) mm &= mm - 1;  // drop the lowest ti set bits
    k = __builtin_ctz(mm);
  };
  if (nsteps > 0) {
    int k;
    int64_t c0;
    step_at(0, k, c0);
    load_step(k, c0);
    store_step(0);
  }
  lds_barrier();
  const int frag = (lane & 31) * 32 + (lane >> 5) * 16;
  int cur_k;
  int64_t cur_c0;
  if (nsteps > 0) step_at(0, cur_k, cur_c0);
  for (int64_t st = 0; st < nsteps; ++st) {
    const int buf = (int)(st & 1);
    int nk = cur_k;
    int64_t nc0 = cur_c0 + BK;
    if (nc0 >= Cin) {  // next used tap
      nc0 = 0;
      const uint32_t rest = mask & ~((2u << cur_k) - 1u);
      nk = rest ? __builtin_ctz(rest) : cur_k;
    }
    if (st + 1 < nsteps) load_step(nk, nc0);
    {
      const char *sa = lds + buf * STAGE, *sb = sa + 3 * PA;
      bf16x8_t a[3][TM], b[3][TN];
#pragma unroll
      for (int q = 0; q < 3; ++q) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
          a[q][i] = *reinterpret_cast<const bf16x8_t *>(sa + q * PA + (wm * (BM / 2) + i * 32) * 32 + frag);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          b[q][j] = *reinterpret_cast<const bf16x8_t *>(sb + q * PB + (wn * (BN / 2) + j * 32) * 32 + frag);
      }
      // smallest terms first: (x3 w1, x2 w2, x1 w3), (x2 w1, x1 w2), x1 w1
      constexpr int ta[6] = {2, 1, 0, 1, 0, 0}, tb[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll
      for (int u = 0; u < 6; ++u)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ta[u]][i], b[tb[u]][j], acc[i][j], 0, 0, 0);
    }
    if (st + 1 < nsteps) store_step(buf ^ 1);
    lds_barrier();
    cur_k = nk;
    cur_c0 = nc0;
  }

  // C[8 * (e / 4) + 4 * (lane / 32) + e % 4][lane % 32]: rows are voxels, columns output channels
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t col = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
    if (col >= Cout) continue;
    const float bias = p.bias ? p.bias[col] : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * (BM / 2) + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (row < N) p.out[row * Cout + col] = acc[i][j][e] + bias;
      }
  }
}

// ---- rulebook path: per-tap pair lists, one gather-GEMM-add pass per tap -------

__global__ __launch_bounds__(256) void rulebook_clear_kernel(int32_t *counts) {
  if (threadIdx.x < 27) counts[threadIdx.x] = 0;
}

// pairs[k][j] = (dst row i, src row nbr[i][k]) for every present neighbour.
// One thread per voxel; a workgroup reserves each tap's slots with a single
// global atomic (wave counts from ballots, summed in LDS) and places its pairs
// in voxel order within that range, so the atomics are 27 per 256 voxels
// instead of one per present neighbour. The order of the workgroups' ranges
// inside a tap is arbitrary (each dst row occurs once per tap).
__global__ __launch_bounds__(256) void rulebook_kernel(const int32_t *nbr, int64_t n, int32_t *pairs,
                                                       int32_t *counts) {
  __shared__ int32_t rows[256 * 27];
  __shared__ int32_t wcnt[27][4];
  __shared__ int32_t base[27];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t i0 = (int64_t)blockIdx.x * 256, i = i0 + t;
  const int64_t nrow = n - i0 < 256 ? n - i0 : 256;
  // the workgroup's rows of the neighbour table, read coalesced
  for (int e = t; e < nrow * 27; e += 256) rows[e] = nbr[i0 * 27 + e];
  __syncthreads();
  uint32_t present = 0;
#pragma unroll
  for (int k = 0; k < 27; ++k) {
    const int32_t sk = i < n ? rows[t * 27 + k] : -1;
    const bool pk = sk >= 0 && sk < n;
    present |= (uint32_t)pk << k;
    const uint64_t b = __builtin_amdgcn_ballot_w64(pk);
    if (lane == 0) wcnt[k][wave] = __builtin_popcountll(b);
  }
  __syncthreads();
  if (t < 27) {
    int32_t run = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int32_t c = wcnt[t][w];
      wcnt[t][w] = run;  // exclusive prefix over the waves
      run += c;
    }
    base[t] = run ? atomicAdd(&counts[t], run) : 0;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 27; ++k) {
    const bool pk = (present >> k) & 1u;
    const uint64_t b = __builtin_amdgcn_ballot_w64(pk);
    if (pk) {
      const int32_t below = (int32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0));
      const int64_t pos = (int64_t)k * n + base[k] + wcnt[k][wave] + below;
      pairs[pos * 2] = (int32_t)i;
      pairs[pos * 2 + 1] = rows[t * 27 + k];
    }
  }
}

__global__ __launch_bounds__(256) void fill_rows_kernel(float *out, int64_t n, int64_t cout, const float *bias,
                                                        bool add) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= n * cout) return;
  const float b = bias ? bias[t % cout] : 0.f;
  out[t] = add ? out[t] + b : b;
}

// out[dst[r], col] += acc for a tap tile. The rows of a tile are distinct
// destinations (each voxel occurs once per tap), so all of a lane's 16 reads
// are issued before its first write; rows without a destination read row 0
// and are not written. (Written as one read-add-write per element, the
// compiler must assume that rows may repeat and serializes 16 round trips.)
template <int BM, int BN, int TM, int TN>
__device__ __forceinline__ void tap_epilogue(float *out, int64_t Cout, int64_t n0, int wm, int wn, int lane,
                                             const int32_t *dst, const f32x16_t (&acc)[TM][TN]) {
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t col = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
    if (col >= Cout) continue;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      int32_t d[16];
      float old[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        d[e] = dst[wm * (BM / 2) + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)];
        old[e] = out[(int64_t)(d[e] >= 0 ? d[e] : 0) * Cout + col];
      }
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (d[e] >= 0) out[(int64_t)d[e] * Cout + col] = old[e] + acc[i][j][e];
    }
  }
}

// One tap: out[dst_j, :] += x[src_j, :] W_k^T for the count[k] pairs of tap
// k (rows of a tile are distinct destinations, so the read-modify-write
// needs no atomics), with f32 arithmetic on the bf16 matrix cores. Each staged f32
// value of x[src] and W_k is split exactly into three bf16 terms (split3_bf16:
// v = v1 + v2 + v3, |v2| <= 2^-8 |v|, |v3| <= 2^-17 |v|) and written to LDS as
// three planes; every 16-deep k-step of a 32 x 32 output tile then runs six
// bf16 MFMAs, x3 w1, x2 w2, x1 w3, x2 w1, x1 w2, x1 w1, accumulating in f32.
// The products dropped (x2 w3 + x3 w2 + x3 w3) stay below 2^-24 |x w|, under
// one f32 ulp of the product, so each tap is the f32 GEMM of the reference up
// to the order of the sums and that truncation, at 6/16 of the matrix-core
// cycles of v_mfma_f32_32x32x2_f32. Plane rows are 16 bf16 (32 bytes) with no
// padding: a fragment read (lane l: row l % 32, k half l / 32) covers 1 KB
// contiguously, and each thread's 8-byte plane writes of 4 consecutive k
// cover 512 contiguous bytes per wavefront (at 32-deep steps, rows of 64
// bytes, chunk c in slot c ^ ((r >> 2) & 3)). Two stages, one barrier per step;
// the next step's global loads are issued before the current step's MFMAs.
// This replaced a tap kernel on v_mfma_f32_32x32x2_f32 (64 x 64 tiles):
// 7.52 -> 5.13 ms (C 1024 over 24k voxels), 1.76 -> 1.54 ms (C 256 over
// 150k), same-box A/B.
template <int BM, int BN, int BK = 16>
__global__ __launch_bounds__(256) void sparse_tap_x3_kernel(SparseConvParams p, const int32_t *pairs,
                                                            const int32_t *counts, int k) {
  typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
  static_assert(BK == 16 || BK == 32, "k-step");
  constexpr int RB = 2 * BK;  // bytes of one plane row
  // 16-byte chunk c8 of plane row r: slot c8 at BK = 16 (a fragment read
  // covers 1 KB contiguously), c8 ^ ((r >> 2) & 3) at BK = 32
  auto slot = [](int c8, int r) { return BK == 16 ? c8 : c8 ^ ((r >> 2) & 3); };
  constexpr int TM = BM / 64, TN = BN / 64;
  constexpr int ACH = BM * BK / 4 / 256, BCH = BN * BK / 4 / 256;
  static_assert(ACH >= 1 && BCH >= 1, "tile");
  constexpr int PA = BM * BK * 2, PB = BN * BK * 2;  // bytes of one plane
  constexpr int STAGE = 3 * (PA + PB);
  __shared__ __align__(16) char lds[2 * STAGE];
  __shared__ int32_t src[BM], dst[BM];

  const int64_t cnt = counts[k] < p.n ? counts[k] : p.n;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
  if (m0 >= cnt) return;  // uniform: the whole workgroup leaves before any barrier
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t N = p.n, Cin = p.cin, Cout = p.cout;
  const int32_t *pk = pairs + (int64_t)k * N * 2;
  for (int r = t; r < BM; r += 256) {
    const bool ok = m0 + r < cnt;
    dst[r] = ok ? pk[(m0 + r) * 2] : -1;
    const int32_t s = ok ? pk[(m0 + r) * 2 + 1] : -1;
    src[r] = s >= 0 && s < N ? s : -1;
  }
  __syncthreads();

  // chunk c = 4 consecutive k of row c / (BK / 4) at k offset 4 (c % (BK / 4))
  const float *wk = p.w + (int64_t)k * Cout * Cin;
  // Rows without a source (past the tap's pairs) load row 0 and are zeroed
  // after the load: a branch around the load would make the compiler wait
  // for it before issuing the next one.
  const float *arow[ACH], *brow[BCH];
  int aoff[ACH], boff[BCH];
  bool aok[ACH];
#pragma unroll
  for (int i = 0; i < ACH; ++i) {
    const int c = t + i * 256, row = c / (BK / 4), part = c % (BK / 4);
    const int32_t s = src[row];
    aok[i] = s >= 0;
    arow[i] = p.x + (int64_t)(s >= 0 ? s : 0) * Cin + part * 4;
    aoff[i] = row * RB + slot(part >> 1, row) * 16 + (part & 1) * 8;
  }
#pragma unroll
  for (int i = 0; i < BCH; ++i) {
    const int c = t + i * 256, row = c / (BK / 4), part = c % (BK / 4);
    int64_t o = n0 + row;
    o = o < Cout ? o : Cout - 1;
    brow[i] = wk + o * Cin + part * 4;
    boff[i] = row * RB + slot(part >> 1, row) * 16 + (part & 1) * 8;
  }
  float4 ra[ACH], rb[BCH];
  auto load_step = [&](int64_t c0) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) ra[i] = *reinterpret_cast<const float4 *>(arow[i] + c0);
#pragma unroll
    for (int i = 0; i < BCH; ++i) rb[i] = *reinterpret_cast<const float4 *>(brow[i] + c0);
  };
  auto put = [](char *plane0, int pbytes, int off, float4 v) {
    const Split3 lo = split3_bf16(v.x, v.y), hi = split3_bf16(v.z, v.w);
    *reinterpret_cast<uint2 *>(plane0 + off) = make_uint2(lo.t1, hi.t1);
    *reinterpret_cast<uint2 *>(plane0 + pbytes + off) = make_uint2(lo.t2, hi.t2);
    *reinterpret_cast<uint2 *>(plane0 + 2 * pbytes + off) = make_uint2(lo.t3, hi.t3);
  };
  auto store_step = [&](int buf) {
    char *st = lds + buf * STAGE;
#pragma unroll
    for (int i = 0; i < ACH; ++i) put(st, PA, aoff[i], aok[i] ? ra[i] : make_float4(0.f, 0.f, 0.f, 0.f));
#pragma unroll
    for (int i = 0; i < BCH; ++i) put(st + 3 * PA, PB, boff[i], rb[i]);
  };
  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x16_t{};
  const int64_t nsteps = Cin / BK;
  load_step(0);
  store_step(0);
  lds_barrier();
  // fragment rows: row (lane % 32) of each 32-row tile, 16-byte chunk
  // 2 s + lane / 32 in sub-step s
  int afr[TM][BK / 16], bfr[TN][BK / 16];
#pragma unroll
  for (int s2 = 0; s2 < BK / 16; ++s2) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = wm * (BM / 2) + i * 32 + (lane & 31);
      afr[i][s2] = r * RB + slot(2 * s2 + (lane >> 5), r) * 16;
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int r = wn * (BN / 2) + j * 32 + (lane & 31);
      bfr[j][s2] = r * RB + slot(2 * s2 + (lane >> 5), r) * 16;
    }
  }
  for (int64_t st = 0; st < nsteps; ++st) {
    const int buf = (int)(st & 1);
    if (st + 1 < nsteps) load_step((st + 1) * BK);
    const char *sa = lds + buf * STAGE, *sb = sa + 3 * PA;
#pragma unroll
    for (int s2 = 0; s2 < BK / 16; ++s2) {
      bf16x8_t a[3][TM], b[3][TN];
#pragma unroll
      for (int q = 0; q < 3; ++q) {
#pragma unroll
        for (int i = 0; i < TM; ++i) a[q][i] = *reinterpret_cast<const bf16x8_t *>(sa + q * PA + afr[i][s2]);
#pragma unroll
        for (int j = 0; j < TN; ++j) b[q][j] = *reinterpret_cast<const bf16x8_t *>(sb + q * PB + bfr[j][s2]);
      }
      // smallest terms first: (x3 w1, x2 w2, x1 w3), (x2 w1, x1 w2), x1 w1
      constexpr int ta[6] = {2, 1, 0, 1, 0, 0}, tb[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll
      for (int u = 0; u < 6; ++u)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ta[u]][i], b[tb[u]][j], acc[i][j], 0, 0, 0);
    }
    if (st + 1 < nsteps) store_step(buf ^ 1);
    lds_barrier();
  }
  tap_epilogue<BM, BN, TM, TN>(p.out, Cout, n0, wm, wn, lane, dst, acc);
}


// Any Cin / Cout: one thread per output element, f32 sums in tap, channel order.
__global__ __launch_bounds__(256) void sparse_conv_generic_kernel(SparseConvParams p) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= p.n * p.cout) return;
  const int64_t i = t / p.cout, o = t % p.cout;
  float acc = 0.f;
  for (int k = 0; k < 27; ++k) {
    const int32_t s = p.nbr[i * 27 + k];
    if (s < 0 || s >= p.n) continue;
    const float *xr = p.x + (int64_t)s * p.cin, *wr = p.w + ((int64_t)k * p.cout + o) * p.cin;
    for (int64_t c = 0; c < p.cin; ++c) acc = __builtin_fmaf(wr[c], xr[c], acc);
  }
  p.out[t] = acc + (p.bias ? p.bias[o] : 0.f);
}

// ---- row gather -------------------------------------------------------------------

// out[m, :] = src[ids[m], :] for m < rows (rows read from `count` when given);
// ids out of range give zero rows. VEC: 16-byte aligned rows.
template <typename IDX, bool VEC>
// bad (optional): incremented once per id outside [0, nsrc) (its row is
// written as zeros); zeroed beforehand by zero_counter_kernel.
__global__ __launch_bounds__(256) void gather_rows_kernel(const char *src, int64_t nsrc, const IDX *ids, int64_t rows,
                                                          const int32_t *count, char *out, int64_t row_bytes,
                                                          int32_t *bad) {
  const int64_t lim = count ? (int64_t)*count : rows;
  const int64_t units = VEC ? row_bytes / 16 : row_bytes;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t m = t / units, u = t % units;
  if (m >= lim || m >= rows) return;
  const int64_t id = (int64_t)ids[m];
  if (bad && u == 0 && !(id >= 0 && id < nsrc)) atomicAdd(bad, 1);
  if (VEC) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (id >= 0 && id < nsrc) v = *reinterpret_cast<const uint4 *>(src + id * row_bytes + u * 16);
    *reinterpret_cast<uint4 *>(out + m * row_bytes + u * 16) = v;
  } else {
    out[m * row_bytes + u] = (id >= 0 && id < nsrc) ? src[id * row_bytes + u] : 0;
  }
}

// Rows of at least 512 bytes (16-byte aligned): one wavefront per row, four
// rows per workgroup; each lane keeps up to four 16-byte chunks in flight
// (4 KB of the row per pass) before storing them. The row count and the row
// id are read once per wavefront.
template <typename IDX>
__global__ __launch_bounds__(256) void gather_rows_wave_kernel(const char *src, int64_t nsrc, const IDX *ids,
                                                               int64_t rows, const int32_t *count, char *out,
                                                               int64_t row_bytes, int32_t *bad) {
  const int64_t lim = count ? (int64_t)*count : rows;
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= lim || m >= rows) return;  // wave-uniform
  const int64_t id = (int64_t)ids[m];
  const bool ok = id >= 0 && id < nsrc;
  if (bad && lane == 0 && !ok) atomicAdd(bad, 1);
  char *dr = out + m * row_bytes;
  const int64_t units = row_bytes / 16;
  if (!ok) {  // wave-uniform: the row is written as zeros, src is not read
    for (int64_t u = lane; u < units; u += 64) *reinterpret_cast<uint4 *>(dr + u * 16) = make_uint4(0, 0, 0, 0);
    return;
  }
  const char *sr = src + id * row_bytes;
  for (int64_t u0 = 0; u0 < units; u0 += 256) {
    uint4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t u = u0 + i * 64 + lane;
      v[i] = u < units ? *reinterpret_cast<const uint4 *>(sr + u * 16) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t u = u0 + i * 64 + lane;
      if (u < units) *reinterpret_cast<uint4 *>(dr + u * 16) = v[i];
    }
  }
}

__global__ __launch_bounds__(64) void zero_counter_kernel(int32_t *c) {
  if (threadIdx.x == 0) *c = 0;
}

// ---- C2S ----------------------------------------------------------------------------

constexpr int kScanBlock = 1024;  // parents per scan block (256 threads x 4)

template <typename T>
__global__ __launch_bounds__(256) void c2s_count_kernel(const void *logits, int64_t n, float *sub, int32_t *offs,
                                                        int32_t *block_sums) {
  __shared__ int32_t wsum[4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t p0 = (int64_t)blockIdx.x * kScanBlock + t * 4;
  int32_t c[4];
  int32_t tot = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t p = p0 + q;
    int32_t cnt = 0;
    if (p < n) {
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const bool leaf = load1<T>(logits, p * 8 + s) > 0.f;
        cnt += leaf;
        if (sub) sub[p * 8 + s] = leaf ? 1.f : 0.f;
      }
    }
    c[q] = cnt;
    tot += cnt;
  }
  // exclusive scan of the thread totals inside the wave, then across waves
  int32_t incl = tot;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int32_t v = __shfl_up(incl, d, 64);
    if (lane >= d) incl += v;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int32_t base = 0;
  for (int w = 0; w < wave; ++w) base += wsum[w];
  int32_t run = base + incl - tot;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (p0 + q < n) offs[p0 + q] = run;
    run += c[q];
  }
  if (t == 255) block_sums[blockIdx.x] = base + incl;
}

// exclusive scan of the block totals in place (one workgroup); total -> count
// The same counts and offsets with coalesced loads (logits, and sub when
// given, 16-byte aligned): the block's logits arrive as 16-byte chunks in
// lane order, their leaf flags go to LDS (and to sub), and each thread then
// counts its 4 parents from LDS.
template <typename T>
__global__ __launch_bounds__(256) void c2s_count_vec_kernel(const void *logits, int64_t n, float *sub,
                                                            int32_t *offs, int32_t *block_sums) {
  constexpr int PER = 16 / T::bytes;                // logits per 16-byte chunk
  constexpr int CHUNKS = kScanBlock * 8 / PER;      // chunks per workgroup
  __shared__ __align__(16) uint8_t leaf[kScanBlock * 8];
  __shared__ int32_t wsum[4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t l0 = (int64_t)blockIdx.x * kScanBlock * 8, nl = n * 8;
  for (int c = t; c < CHUNKS; c += 256) {
    const int64_t l = l0 + (int64_t)c * PER;
    if (l >= nl) break;  // n * 8 logits: a multiple of PER, so every chunk is whole
    const uint4 u = ld16<false>(reinterpret_cast<const char *>(logits) + l * T::bytes);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    float f[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      if constexpr (T::bytes == 4) f[e] = __uint_as_float(w[e]);
      else if constexpr (T::code == LUX3D_BF16) f[e] = __uint_as_float((e & 1) ? (w[e >> 1] & 0xFFFF0000u) : (w[e >> 1] << 16));
      else f[e] = f16_bits_to_f32((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xFFFFu));
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) leaf[c * PER + e] = f[e] > 0.f;
    if (sub) {
#pragma unroll
      for (int e = 0; e < PER; e += 4)
        *reinterpret_cast<float4 *>(sub + l + e) = make_float4(f[e] > 0.f ? 1.f : 0.f, f[e + 1] > 0.f ? 1.f : 0.f,
                                                               f[e + 2] > 0.f ? 1.f : 0.f, f[e + 3] > 0.f ? 1.f : 0.f);
    }
  }
  __syncthreads();
  const int64_t p0 = (int64_t)blockIdx.x * kScanBlock + t * 4;
  int32_t c[4];
  int32_t tot = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int32_t cnt = 0;
    if (p0 + q < n) {
      const uint2 b = *reinterpret_cast<const uint2 *>(&leaf[(t * 4 + q) * 8]);  // 8 flags of 0 / 1
      cnt = (int32_t)(__builtin_popcount(b.x) + __builtin_popcount(b.y));
    }
    c[q] = cnt;
    tot += cnt;
  }
  int32_t incl = tot;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int32_t v = __shfl_up(incl, d, 64);
    if (lane >= d) incl += v;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int32_t base = 0;
  for (int w = 0; w < wave; ++w) base += wsum[w];
  int32_t run = base + incl - tot;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (p0 + q < n) offs[p0 + q] = run;
    run += c[q];
  }
  if (t == 255) block_sums[blockIdx.x] = base + incl;
}

__global__ __launch_bounds__(256) void c2s_scan_kernel(int32_t *block_sums, int64_t nb, int32_t *count) {
  __shared__ int32_t wsum[4];
  __shared__ int32_t carry;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  if (t == 0) carry = 0;
  __syncthreads();
  for (int64_t b0 = 0; b0 < nb; b0 += 256) {
    const int64_t b = b0 + t;
    const int32_t v = b < nb ? block_sums[b] : 0;
    int32_t incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int32_t u = __shfl_up(incl, d, 64);
      if (lane >= d) incl += u;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int32_t base = carry;
    for (int w = 0; w < wave; ++w) base += wsum[w];
    if (b < nb) block_sums[b] = base + incl - v;
    __syncthreads();
    if (t == 255) carry = base + incl;
    __syncthreads();
  }
  if (t == 0) *count = carry;
}

template <typename T>
__global__ __launch_bounds__(256) void c2s_emit_kernel(const int32_t *coords, const void *logits, int64_t n,
                                                       const int32_t *offs, const int32_t *block_sums,
                                                       int32_t *out_coords, int32_t *src_rows) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= n * 8) return;
  const int64_t p = t / 8;
  const int s = (int)(t % 8);
  if (!(load1<T>(logits, t) > 0.f)) return;
  int32_t before = 0;
  for (int q = 0; q < s; ++q) before += load1<T>(logits, p * 8 + q) > 0.f;
  const int64_t j = (int64_t)offs[p] + block_sums[p / kScanBlock] + before;
  out_coords[3 * j] = coords[3 * p] * 2 + (s & 1);
  out_coords[3 * j + 1] = coords[3 * p + 1] * 2 + ((s >> 1) & 1);
  out_coords[3 * j + 2] = coords[3 * p + 2] * 2 + (s >> 2);
  src_rows[j] = (int32_t)(p * 8 + s);
}

unsigned grid_of(int64_t threads) { return (unsigned)((threads + 255) / 256); }

}  // namespace

namespace {
// Per-device address of `scratch`, looked up once per device (with that
// device current) on the first allocation-free call.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {};

hipError_t noalloc_table(void **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}
}  // namespace

hipError_t launch_sparse_map_noalloc(const int32_t *coords, int64_t n, int32_t *nbr, int32_t *bad, hipStream_t s) {
  if (n > kNoAllocMaxVoxels) return hipErrorInvalidValue;
  int64_t cap = 16;
  while (cap < 2 * n) cap *= 2;
  if (cap > kNoAllocCap) return hipErrorInvalidValue;  // the table's slots
  void *table = nullptr;
  const hipError_t e = noalloc_table(&table);
  if (e != hipSuccess) return e;
  // the table is cleared by the first kernel of the sequence (no memset)
  auto *keys = static_cast<unsigned long long *>(table);
  auto *vals = reinterpret_cast<int32_t *>(static_cast<unsigned char *>(table) + kNoAllocCap * sizeof(unsigned long long));
  return launch_sparse_map(coords, n, keys, vals, cap, nbr, bad, s);
}

hipError_t launch_sparse_map(const int32_t *coords, int64_t n, unsigned long long *keys, int32_t *vals, int64_t cap,
                             int32_t *nbr, int32_t *bad, hipStream_t s) {
  if (cap <= 0 || (cap & (cap - 1)) || cap < 2 * n) return hipErrorInvalidValue;
  if (grid_of(cap) == 0 || (cap + 255) / 256 > INT32_MAX || (n * 27 + 255) / 256 > INT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(map_clear_kernel, dim3(grid_of(cap)), dim3(256), 0, s, keys, vals, cap, bad);
  if (n == 0) return hipGetLastError();
  hipLaunchKernelGGL(map_insert_kernel, dim3(grid_of(n)), dim3(256), 0, s, coords, n, keys, vals, cap, bad);
  hipLaunchKernelGGL(map_neighbors_kernel, dim3(grid_of(n * 27)), dim3(256), 0, s, coords, n, keys, vals, cap, nbr);
  return hipGetLastError();
}

hipError_t launch_sparse_conv(const SparseConvParams &p, hipStream_t s) {
  if (p.n <= 0 || p.cout <= 0) return hipSuccess;
  if (p.mfma) {
    const int64_t gy = (p.n + 63) / 64;
    if (gy > 65535) {
      if ((p.n + 127) / 128 > 65535) return hipErrorInvalidValue;
      hipLaunchKernelGGL((sparse_conv_x3_kernel<128, 64>), dim3((unsigned)((p.cout + 63) / 64), (unsigned)((p.n + 127) / 128)),
                         dim3(256), 0, s, p);
      return hipGetLastError();
    }
    hipLaunchKernelGGL((sparse_conv_x3_kernel<64, 64>), dim3((unsigned)((p.cout + 63) / 64), (unsigned)gy), dim3(256), 0,
                       s, p);
    return hipGetLastError();
  }
  if ((p.n * p.cout + 255) / 256 > INT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sparse_conv_generic_kernel, dim3(grid_of(p.n * p.cout)), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_sparse_rulebook(const int32_t *nbr, int64_t n, int32_t *pairs, int32_t *counts, hipStream_t s) {
  if ((n * 27 + 255) / 256 > INT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rulebook_clear_kernel, dim3(1), dim3(256), 0, s, counts);
  if (n > 0) hipLaunchKernelGGL(rulebook_kernel, dim3(grid_of(n)), dim3(256), 0, s, nbr, n, pairs, counts);
  return hipGetLastError();
}

hipError_t launch_sparse_conv_rulebook(const SparseConvParams &p, const int32_t *pairs, const int32_t *counts,
                                       hipStream_t s) {
  if (p.n <= 0 || p.cout <= 0) return hipSuccess;
  if ((p.n * p.cout + 255) / 256 > INT32_MAX || (p.n + 63) / 64 > 65535) return hipErrorInvalidValue;
  // out = 0; out[dst] += x[src] W_k^T for k = 0..26 in order; out += bias:
  // the reference's zeros / index_add / broadcast_add sequence
  hipLaunchKernelGGL(fill_rows_kernel, dim3(grid_of(p.n * p.cout)), dim3(256), 0, s, p.out, p.n, p.cout,
                     (const float *)nullptr, false);
  // 128 x 128 tiles for wide convs (C 1024 -> 1024 over 24k voxels: 5.13
  // against 5.97 ms for 64 x 64), 64 x 64 below (C 256 over 150k voxels: 1.54
  // against 1.72 ms, where 128-row tiles leave CUs idle); same-box A/B.
  if (p.cin >= 512 && p.cout >= 512) {
    const dim3 grid((unsigned)((p.cout + 127) / 128), (unsigned)((p.n + 127) / 128));
    for (int k = 0; k < 27; ++k)
      hipLaunchKernelGGL((sparse_tap_x3_kernel<128, 128>), grid, dim3(256), 0, s, p, pairs, counts, k);
  } else {
    const dim3 grid((unsigned)((p.cout + 63) / 64), (unsigned)((p.n + 63) / 64));
    for (int k = 0; k < 27; ++k) {
      if (p.cin % 32 == 0)  // 32-deep steps: half the barriers (1.434 against 1.468 ms, C 256)
        hipLaunchKernelGGL((sparse_tap_x3_kernel<64, 64, 32>), grid, dim3(256), 0, s, p, pairs, counts, k);
      else
        hipLaunchKernelGGL((sparse_tap_x3_kernel<64, 64>), grid, dim3(256), 0, s, p, pairs, counts, k);
    }
  }
  if (p.bias)
    hipLaunchKernelGGL(fill_rows_kernel, dim3(grid_of(p.n * p.cout)), dim3(256), 0, s, p.out, p.n, p.cout, p.bias,
                       true);
  return hipGetLastError();
}

hipError_t launch_gather_rows(const void *src, int64_t nsrc, const void *ids, bool ids64, int64_t rows,
                              const int32_t *count, void *out, int64_t row_bytes, int32_t *bad, hipStream_t s) {
  if (bad) hipLaunchKernelGGL(zero_counter_kernel, dim3(1), dim3(64), 0, s, bad);
  if (rows <= 0 || row_bytes <= 0) return hipGetLastError();
  const bool vec = row_bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  const int64_t units = vec ? row_bytes / 16 : row_bytes;
  if ((rows * units + 255) / 256 > INT32_MAX) return hipErrorInvalidValue;
  const dim3 grid(grid_of(rows * units)), block(256);
  const char *sp = static_cast<const char *>(src);
  char *op = static_cast<char *>(out);
  if (vec && units >= 32) {  // configs[3] C2S (2 KB child rows): 90.0 against 91.8 us
    const dim3 wgrid((unsigned)((rows + 3) / 4));
    if ((rows + 3) / 4 > INT32_MAX) return hipErrorInvalidValue;
    if (ids64)
      hipLaunchKernelGGL((gather_rows_wave_kernel<int64_t>), wgrid, block, 0, s, sp, nsrc,
                         static_cast<const int64_t *>(ids), rows, count, op, row_bytes, bad);
    else
      hipLaunchKernelGGL((gather_rows_wave_kernel<int32_t>), wgrid, block, 0, s, sp, nsrc,
                         static_cast<const int32_t *>(ids), rows, count, op, row_bytes, bad);
    return hipGetLastError();
  }
  if (ids64) {
    if (vec) hipLaunchKernelGGL((gather_rows_kernel<int64_t, true>), grid, block, 0, s, sp, nsrc,
                                static_cast<const int64_t *>(ids), rows, count, op, row_bytes, bad);
    else hipLaunchKernelGGL((gather_rows_kernel<int64_t, false>), grid, block, 0, s, sp, nsrc,
                            static_cast<const int64_t *>(ids), rows, count, op, row_bytes, bad);
  } else {
    if (vec) hipLaunchKernelGGL((gather_rows_kernel<int32_t, true>), grid, block, 0, s, sp, nsrc,
                                static_cast<const int32_t *>(ids), rows, count, op, row_bytes, bad);
    else hipLaunchKernelGGL((gather_rows_kernel<int32_t, false>), grid, block, 0, s, sp, nsrc,
                            static_cast<const int32_t *>(ids), rows, count, op, row_bytes, bad);
  }
  return hipGetLastError();
}

hipError_t launch_c2s(const C2SParams &p, hipStream_t s) {
  const int64_t nb = (p.n + kScanBlock - 1) / kScanBlock;
  if (p.n < 0 || (p.n * 8 + 255) / 256 > INT32_MAX) return hipErrorInvalidValue;
  if (p.n == 0) {
    hipLaunchKernelGGL(c2s_scan_kernel, dim3(1), dim3(256), 0, s, p.block_sums, (int64_t)0, p.count);
    return hipGetLastError();
  }
  const bool vec = (uintptr_t)p.logits % 16 == 0 && (uintptr_t)p.sub % 16 == 0;
  switch (p.logits_dt) {
    case LUX3D_F32:
      if (vec)
        hipLaunchKernelGGL((c2s_count_vec_kernel<F32>), dim3((unsigned)nb), dim3(256), 0, s, p.logits, p.n, p.sub,
                           p.offs, p.block_sums);
      else
        hipLaunchKernelGGL((c2s_count_kernel<F32>), dim3((unsigned)nb), dim3(256), 0, s, p.logits, p.n, p.sub, p.offs,
                           p.block_sums);
      break;
    case LUX3D_BF16:
      if (vec)
        hipLaunchKernelGGL((c2s_count_vec_kernel<BF16>), dim3((unsigned)nb), dim3(256), 0, s, p.logits, p.n, p.sub,
                           p.offs, p.block_sums);
      else
        hipLaunchKernelGGL((c2s_count_kernel<BF16>), dim3((unsigned)nb), dim3(256), 0, s, p.logits, p.n, p.sub,
                           p.offs, p.block_sums);
      break;
    case LUX3D_F16:
      if (vec)
        hipLaunchKernelGGL((c2s_count_vec_kernel<F16>), dim3((unsigned)nb), dim3(256), 0, s, p.logits, p.n, p.sub,
                           p.offs, p.block_sums);
      else
        hipLaunchKernelGGL((c2s_count_kernel<F16>), dim3((unsigned)nb), dim3(256), 0, s, p.logits, p.n, p.sub,
                           p.offs, p.block_sums);
      break;
    default: return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL(c2s_scan_kernel, dim3(1), dim3(256), 0, s, p.block_sums, nb, p.count);
  switch (p.logits_dt) {
    case LUX3D_F32:
      hipLaunchKernelGGL((c2s_emit_kernel<F32>), dim3(grid_of(p.n * 8)), dim3(256), 0, s, p.coords, p.logits, p.n,
                         p.offs, p.block_sums, p.out_coords, p.src_rows);
      break;
    case LUX3D_BF16:
      hipLaunchKernelGGL((c2s_emit_kernel<BF16>), dim3(grid_of(p.n * 8)), dim3(256), 0, s, p.coords, p.logits, p.n,
                         p.offs, p.block_sums, p.out_coords, p.src_rows);
      break;
    default:
      hipLaunchKernelGGL((c2s_emit_kernel<F16>), dim3(grid_of(p.n * 8)), dim3(256), 0, s, p.coords, p.logits, p.n,
                         p.offs, p.block_sums, p.out_coords, p.src_rows);
      break;
  }
  // child features: rows src_rows[j] of feats viewed as [n * 8, C / 8]
  return launch_gather_rows(p.feats, p.n * 8, p.src_rows, false, p.n * 8, p.count, p.out_feats, p.child_row_bytes,
                            nullptr, s);
}

}  // namespace lux3d
