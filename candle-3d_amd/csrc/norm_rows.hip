// norm_rows.hip -- row-reduction kernels for gfx950: LayerNorm (affine or
// not), LayerScale + residual + LayerNorm, AdaLN modulate (dense or ragged
// segments), the gated residual, and the gated residual followed by the next
// AdaLN modulate in one pass.
//
// Mapping. A row of D elements is owned by TPR threads (one wavefront for
// TPR = 64, or 2 / 4 wavefronts reducing through LDS for short row counts).
// Thread t holds chunks c = 0..NC-1 of 8 elements: for 2-byte types the 8
// elements at (c*TPR + t)*8, for f32 the 4 at (2c*TPR + t)*4 and the 4 at
// ((2c+1)*TPR + t)*4 (chunk_at), so each 16-byte load or store instruction
// of a wavefront covers 1 KiB of contiguous row data. The whole row stays in registers:
// HBM traffic is exactly one read of every input and one write of every
// output. Statistics are two-pass over the registers (mean, then centred sum
// of squares), reduced with DPP + permlane swaps (no LDS for TPR = 64).
#include "common.hpp"
#include "kernels.hpp"

namespace lux3d {

namespace {

constexpr int kBlock = 256;
// Workgroup of the staged modulate rows (one row per wavefront): 8 rows
// share one staging of the segment pieces. Same-box A/B against 256 / 1024
// threads: configs[2] gated residual + modulate 12.9 against 13.9 / 13.0 us,
// configs[3] 135.1 against 138.5 / 141.4 us, configs[2] modulate 7.37
// against 7.46 / 7.45 us, configs[3] modulate 66.2 against 66.2 / 77.2 us
// (1024-thread workgroups straddle more segment boundaries).
constexpr int kStagedBlock = 512;

// Segment of row r: the launcher's magic division for dense segments, the
// scalar binary search over the offsets for ragged ones.
__device__ __forceinline__ int64_t row_segment(const RowParams &p, int64_t r) {
  if (p.rps_m) return segment_of_dense((uint32_t)r, p.rps_m, p.rps_s, p.nseg);
  return segment_of(p.seg_off, p.nseg, p.rows_per_seg, r);
}

template <int TPR, int BLOCK = kBlock>
__device__ __forceinline__ float row_total(float s, float *red) {
  s = wave_sum(s);
  if constexpr (TPR == 64) {
    return s;
  } else {
    constexpr int WPR = TPR / 64;
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = s;
    lds_barrier();  // the row's stores (e.g. the residual stream h) stay in flight
    const int w0 = (w / WPR) * WPR;
    float tot = red[w0];
#pragma unroll
    for (int k = 1; k < WPR; ++k) tot += red[w0 + k];
    return tot;
  }
}

__device__ __forceinline__ void mod8(const ModPiece &m, int64_t seg, int64_t idx, float dflt,
                                     float (&v)[8]) {
  param8(reinterpret_cast<const char *>(m.p) + 0, m.dt, seg * m.ld + idx, dflt, v);
  if (m.base_dt >= 0) {
    float b[8];
    param8(m.base, m.base_dt, idx, 0.f, b);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = b[k] + v[k];
  }
}

// Per-segment pieces (AdaLN shift / scale / gate, each optionally plus its
// base vector) are the same for every row of a segment. With STAGE, a
// workgroup whose rows all lie in one segment sums each piece once into LDS
// (dynamic shared memory, npieces * d floats) and every row reads it from
// there: re-reading the f32 pieces per row from the vector cache moved 2-4x
// the row's own bytes through it (configs[3] ragged modulate with base
// vectors: 92.6 us direct, 68.3 us staged). A workgroup that straddles a
// segment boundary reads them per row from global memory.
struct Staged {
  float *shift, *scale1, *gate;  // scale1 = scale + 1
};

template <int MODE, int BLOCK>
__device__ __forceinline__ void stage_pieces(const RowParams &p, int64_t seg, float *lds, Staged &st) {
  const int64_t d = p.d;
  const bool has_gate = MODE == ROW_GATE || p.gate.dt >= 0;
  float *q = lds;
  constexpr bool MOD = MODE == ROW_MODULATE || MODE == ROW_GATE_MOD;
  if constexpr (MOD) {
    st.shift = q; q += d;
    st.scale1 = q; q += d;
  }
  st.gate = has_gate ? q : nullptr;
  for (int64_t e = threadIdx.x; e < d / 8; e += BLOCK) {
    float a[8];
    if constexpr (MOD) {
      mod8(p.shift, seg, e * 8, 0.f, a);
#pragma unroll
      for (int k = 0; k < 8; ++k) st.shift[e * 8 + k] = a[k];
      mod8(p.scale, seg, e * 8, 0.f, a);
#pragma unroll
      for (int k = 0; k < 8; ++k) st.scale1[e * 8 + k] = a[k] + 1.0f;
    }
    if (has_gate) {
      mod8(p.gate, seg, e * 8, 1.f, a);
#pragma unroll
      for (int k = 0; k < 8; ++k) st.gate[e * 8 + k] = a[k];
    }
  }
  lds_barrier();
}

__device__ __forceinline__ void lds8(const float *src, int64_t idx, float (&v)[8]) {
  const float4 a = *reinterpret_cast<const float4 *>(src + idx);
  const float4 b = *reinterpret_cast<const float4 *>(src + idx + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Element offsets of chunk c of lane t in a row: its two 4-element halves.
// 2-byte types: 8 consecutive elements (one 16-byte access). f32: the halves
// lie TPR * 4 elements apart, so that every 16-byte access instruction of a
// wavefront covers 1 KiB of contiguous row (32 consecutive bytes per lane
// would make each instruction touch 2 KiB with half of it used; the copy
// of that layout measured 12-16% slower than the interleaved one at the
// configs' f32 rows). The row's statistics do not depend on which elements a
// lane holds, and every operand of an element uses the same offsets.
struct ChunkAt {
  int64_t o0, o1;
};
template <typename T, int TPR>
__device__ __forceinline__ ChunkAt chunk_at(int c, int t) {
  if constexpr (T::bytes == 4) return {(int64_t)(2 * c * TPR + t) * 4, (int64_t)((2 * c + 1) * TPR + t) * 4};
  else return {(int64_t)(c * TPR + t) * 8, (int64_t)(c * TPR + t) * 8 + 4};
}
template <typename T>
__device__ __forceinline__ void ld_row(const char *row, ChunkAt a, float (&v)[8]) {
  if constexpr (T::bytes == 4) {
    const uint4 x = ld16<LUX3D_NT_STREAMS != 0>(row + a.o0 * 4), y = ld16<LUX3D_NT_STREAMS != 0>(row + a.o1 * 4);
    v[0] = __uint_as_float(x.x); v[1] = __uint_as_float(x.y); v[2] = __uint_as_float(x.z); v[3] = __uint_as_float(x.w);
    v[4] = __uint_as_float(y.x); v[5] = __uint_as_float(y.y); v[6] = __uint_as_float(y.z); v[7] = __uint_as_float(y.w);
  } else {
    Chunk<T>::load(row + a.o0 * T::bytes, v);
  }
}
template <typename T>
__device__ __forceinline__ void st_row(char *row, ChunkAt a, const float (&v)[8]) {
  if constexpr (T::bytes == 4) {
    st16(row + a.o0 * 4, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                    __float_as_uint(v[3])));
    st16(row + a.o1 * 4, make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                                    __float_as_uint(v[7])));
  } else {
    Chunk<T>::store(row + a.o0 * T::bytes, v);
  }
}
// the parameters of chunk a (offset by off elements)
template <typename T>
__device__ __forceinline__ void param_at(const void *p, int dt, int64_t off, ChunkAt a, float dflt, float (&v)[8]) {
  if constexpr (T::bytes == 4) {
    param4(p, dt, off + a.o0, dflt, v);
    param4(p, dt, off + a.o1, dflt, v + 4);
  } else {
    param8(p, dt, off + a.o0, dflt, v);
  }
}
template <typename T>
__device__ __forceinline__ void mod_at(const ModPiece &m, int64_t seg, ChunkAt a, float dflt, float (&v)[8]) {
  param_at<T>(m.p, m.dt, seg * m.ld, a, dflt, v);
  if (m.base_dt >= 0) {
    float b[8];
    param_at<T>(m.base, m.base_dt, 0, a, 0.f, b);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = b[k] + v[k];
  }
}
__device__ __forceinline__ void lds_at(const float *src, ChunkAt a, float (&v)[8]) {
  const float4 x = *reinterpret_cast<const float4 *>(src + a.o0);
  const float4 y = *reinterpret_cast<const float4 *>(src + a.o1);
  v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
  v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
}

template <typename T, int TPR, int NC, int MODE, int BLOCK = kBlock, bool STAGE = false>
__global__ __launch_bounds__(BLOCK) void row_kernel(RowParams p) {
  static_assert(BLOCK % TPR == 0, "a block holds whole rows");
  static_assert(!STAGE || MODE == ROW_MODULATE || MODE == ROW_GATE || MODE == ROW_GATE_MOD,
                "only segment pieces are staged");
  constexpr bool SEGMENTED = MODE == ROW_MODULATE || MODE == ROW_GATE || MODE == ROW_GATE_MOD;
  constexpr int RPB = BLOCK / TPR;
  constexpr int EB = T::bytes;
  __shared__ float red_a[BLOCK / 64], red_b[BLOCK / 64];
  extern __shared__ __align__(16) float lds_pieces[];  // 16-byte aligned: read as float4

  const int t = threadIdx.x % TPR;
  const int64_t row0 = (int64_t)blockIdx.x * RPB;
  int64_t row = row0 + threadIdx.x / TPR;
  const bool live = row < p.rows;
  row = uniform(live ? row : p.rows - 1);

  float v[NC][8];
  const char *xr = reinterpret_cast<const char *>(p.x) + row * p.x_rs * EB;
#pragma unroll
  for (int c = 0; c < NC; ++c) ld_row<T>(xr, chunk_at<T, TPR>(c, t), v[c]);
  // LN (one stream in, one out): w and b are issued with the row as raw
  // bytes (pissue) and decoded after the statistics, so their latency hides
  // under the row's (configs[0]: 3.69 against 3.87 us, same-box A/B). The
  // other modes keep their parameters where they are used: issuing them all
  // with the rows measured slower for the two-stream rows (configs[1] F1
  // 18.7 against 18.5 us).
  constexpr bool LN_UPFRONT = MODE == ROW_LN && NC <= 2;
  PRaw q_w[LN_UPFRONT ? NC : 1], q_b[LN_UPFRONT ? NC : 1];
  if constexpr (LN_UPFRONT) {
    const rsrc_t r_w = param_rsrc(p.w, p.w_dt, p.d), r_b = param_rsrc(p.b, p.b_dt, p.d);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const ChunkAt at = chunk_at<T, TPR>(c, t);
      q_w[c] = pissue(r_w, p.w_dt, at.o0, at.o1);
      q_b[c] = pissue(r_b, p.b_dt, at.o0, at.o1);
    }
  }
  // GATE_MOD: the branch rows are loaded with x, ahead of the segment lookup
  // and the staging barrier, so both streams are in flight together
  float hb[MODE == ROW_GATE_MOD ? NC : 1][8];
  if constexpr (MODE == ROW_GATE_MOD) {
    const char *ar = reinterpret_cast<const char *>(p.a) + row * p.a_rs * EB;
#pragma unroll
    for (int c = 0; c < NC; ++c) ld_row<T>(ar, chunk_at<T, TPR>(c, t), hb[c]);
  }

  // segment of this row; with STAGE, whether the workgroup shares one
  bool staged = false;
  Staged st{};
  int64_t seg = 0;
  if constexpr (SEGMENTED) {
    if constexpr (STAGE) {
      const int64_t last = row0 + RPB - 1 < p.rows ? row0 + RPB - 1 : p.rows - 1;
      const int64_t seg0 = row_segment(p, row0);
      staged = row_segment(p, last) == seg0;  // uniform over the workgroup
      seg = seg0;
      if (staged) stage_pieces<MODE, BLOCK>(p, seg0, lds_pieces, st);
      else seg = row_segment(p, row);
    } else {
      seg = row_segment(p, row);
    }
  }

  if constexpr (MODE == ROW_GATE) {
    const char *ar = reinterpret_cast<const char *>(p.a) + row * p.a_rs * EB;
    char *yr = reinterpret_cast<char *>(p.y) + row * p.y_rs * EB;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const ChunkAt at = chunk_at<T, TPR>(c, t);
      float hv[8], g[8];
      ld_row<T>(ar, at, hv);
      if (staged) lds_at(st.gate, at, g);
      else mod_at<T>(p.gate, seg, at, 1.f, g);
#pragma unroll
      for (int k = 0; k < 8; ++k) v[c][k] = add_rn(v[c][k], mul_rn(hv[k], g[k]));
      if (live) st_row<T>(yr, at, v[c]);
    }
    return;
  }

  if constexpr (MODE == ROW_GATE_MOD) {
    // x' = x + h*gate (gate absent: 1, so x' = x + h exactly), two roundings
    // as broadcast_mul then add; the norm reads the stored x'
    // (no gate: nothing is staged for it and the factor is 1)
    char *hr = reinterpret_cast<char *>(p.h) + row * p.h_rs * EB;
    const bool gated = p.gate.dt >= 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const ChunkAt at = chunk_at<T, TPR>(c, t);
      float g[8];
      if (!gated) {
#pragma unroll
        for (int k = 0; k < 8; ++k) g[k] = 1.f;
      } else if (staged) {
        lds_at(st.gate, at, g);
      } else {
        mod_at<T>(p.gate, seg, at, 1.f, g);
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) v[c][k] = Chunk<T>::round_trip(add_rn(v[c][k], mul_rn(hb[c][k], g[k])));
      if (live) st_row<T>(hr, at, v[c]);
    }
  }

  // One row per workgroup (the short jobs, where a row's latency is the
  // job's): g arrives with the residual inputs as raw bytes, and w and b are
  // issued right after them, ahead of the h store, so that they arrive while
  // the statistics are reduced instead of after them. configs[4] F1 f32:
  // 4.19 against 4.44 us (same-box A/B). The long jobs measured slower in
  // this order (configs[1] F1 19.1 against 18.3 us) and load their
  // parameters where they are used. The h store stays conditional on `live`:
  // written unconditionally, the compiler dropped its non-temporal bit and
  // the job took 4.9 us.
  constexpr bool EARLY = MODE == ROW_RESID_LN && RPB == 1 && NC <= 2;
  PRaw e_g[EARLY ? NC : 1], e_w[EARLY ? NC : 1], e_b[EARLY ? NC : 1];
  if constexpr (EARLY) {
    const char *ar = reinterpret_cast<const char *>(p.a) + row * p.a_rs * EB;
    char *hr = reinterpret_cast<char *>(p.h) + row * p.h_rs * EB;
    float av[NC][8], g[NC][8];
    const rsrc_t r_g = param_rsrc(p.g, p.g_dt, p.d);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const ChunkAt at = chunk_at<T, TPR>(c, t);
      ld_row<T>(ar, at, av[c]);
      e_g[c] = pissue(r_g, p.g_dt, at.o0, at.o1);
    }
    issue_fence();
#pragma unroll
    for (int c = 0; c < NC; ++c) pdecode(e_g[c], p.g_dt, 1.f, g[c]);
    const rsrc_t r_w = param_rsrc(p.w, p.w_dt, p.d), r_b = param_rsrc(p.b, p.b_dt, p.d);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const ChunkAt at = chunk_at<T, TPR>(c, t);
      e_w[c] = pissue(r_w, p.w_dt, at.o0, at.o1);
      e_b[c] = pissue(r_b, p.b_dt, at.o0, at.o1);
    }
    issue_fence();
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float ls = p.g_dt >= 0 ? mul_rn(av[c][k], g[c][k]) : av[c][k];
        v[c][k] = Chunk<T>::round_trip(add_rn(ls, v[c][k]));  // the norm reads the stored h
      }
      if (live) st_row<T>(hr, chunk_at<T, TPR>(c, t), v[c]);
    }
  }

  if constexpr (MODE == ROW_RESID_LN && !EARLY) {
    const char *ar = reinterpret_cast<const char *>(p.a) + row * p.a_rs * EB;
    char *hr = reinterpret_cast<char *>(p.h) + row * p.h_rs * EB;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const ChunkAt at = chunk_at<T, TPR>(c, t);
      float av[8], g[8];
      ld_row<T>(ar, at, av);
      param_at<T>(p.g, p.g_dt, 0, at, 1.f, g);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        // LayerScale product and residual add as two roundings (no FMA
        // contraction), exactly broadcast_mul then add.
        const float ls = p.g_dt >= 0 ? mul_rn(av[k], g[k]) : av[k];
        v[c][k] = Chunk<T>::round_trip(add_rn(ls, v[c][k]));  // the norm reads the stored h
      }
      if (live) st_row<T>(hr, at, v[c]);
    }
  }

  // ---- statistics: mean, then centred second moment (from registers) ----
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int k = 0; k < 8; ++k) s += v[c][k];
  const float inv_d = 1.0f / (float)p.d;
  const float mean = row_total<TPR, BLOCK>(s, red_a) * inv_d;
  float s2 = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float dv = v[c][k] - mean;
      s2 += dv * dv;
    }
  const float var = row_total<TPR, BLOCK>(s2, red_b) * inv_d;
  const float rstd = 1.0f / sqrtf(var + p.eps);

  char *yr = reinterpret_cast<char *>(p.y) + row * p.y_rs * EB;
  if constexpr (MODE == ROW_MODULATE || MODE == ROW_GATE_MOD) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const ChunkAt at = chunk_at<T, TPR>(c, t);
      float sh[8], sc1[8], out[8];
      if (staged) {
        lds_at(st.shift, at, sh);
        lds_at(st.scale1, at, sc1);
      } else {
        mod_at<T>(p.shift, seg, at, 0.f, sh);
        mod_at<T>(p.scale, seg, at, 0.f, sc1);
#pragma unroll
        for (int k = 0; k < 8; ++k) sc1[k] = sc1[k] + 1.0f;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) out[k] = (v[c][k] - mean) * rstd * sc1[k] + sh[k];
      if (MODE == ROW_MODULATE && p.gate.dt >= 0) {  // M1' output gate (GATE_MOD's gate is the residual's)
        float g[8];
        if (staged) lds_at(st.gate, at, g);
        else mod_at<T>(p.gate, seg, at, 1.f, g);
#pragma unroll
        for (int k = 0; k < 8; ++k) out[k] = g[k] * out[k] + v[c][k];
      }
      if (live) st_row<T>(yr, at, out);
    }
  } else {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const ChunkAt at = chunk_at<T, TPR>(c, t);
      float w[8], b[8], out[8];
      if constexpr (LN_UPFRONT) {
        pdecode(q_w[c], p.w_dt, 1.f, w);
        pdecode(q_b[c], p.b_dt, 0.f, b);
      } else if constexpr (EARLY) {
        pdecode(e_w[c], p.w_dt, 1.f, w);
        pdecode(e_b[c], p.b_dt, 0.f, b);
      } else {
        param_at<T>(p.w, p.w_dt, 0, at, 1.f, w);
        param_at<T>(p.b, p.b_dt, 0, at, 0.f, b);
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) out[k] = (v[c][k] - mean) * rstd * w[k] + b[k];
      if (live) st_row<T>(yr, at, out);
    }
  }
}

// ---- persistent residual + LayerNorm (2-byte rows of 1024) ------------------
//
// The long F1 jobs (VGGT's [B * N, 1024] blocks in bf16 / f16). One
// 256-thread workgroup per CU; each wavefront owns a row at a time (lane l:
// the 8-element chunks at 8 l and 512 + 8 l) and walks rows with a grid
// stride, on its own: no LDS, no barrier.
// - γ, w and b are loaded once per thread, not once per row.
// - The next row is loaded before this row's arithmetic and stores, as raw
//   bytes through buffer loads on the (wave-uniform) row address, so no
//   per-lane address arithmetic sits between the rows; 32-bit scalar row
//   math (a 64-bit signed compare of scalars takes a VGPR, and the compiler
//   took one that a pending load also wrote: a wait).
// - Loads and stores are unconditional, so the compiler's vmcnt waits are
//   exact: a wavefront's last row re-reads its own data.
// - Two register sets alternate (the loop is unrolled by two, the first row
//   peeled so that the loop is entered as it is re-entered), and each row's
//   store data stays allocated until the next row's loads are issued (an
//   empty asm use): a load into a register that a pending store still reads
//   from waits for that store.
// - Statistics: each chunk is wave-summed on its own and the two totals are
//   added, chunk 0 first: chunk c of lane l is what lane l of wavefront c
//   holds in row_kernel<T, 128, 1, ROW_RESID_LN>, whose row total adds its
//   two wavefronts' sums in that order, so every output is bit-identical to
//   row_kernel's (and to the short jobs').
// configs[1] F1: 16.8 against 17.6-17.8 µs for two-wavefront rows walked the
// same way and 18.2 µs for row_kernel (same box, graph-timed, cold); two
// workgroups per CU or more, 64-thread workgroups, or loading two rows
// ahead: slower.
template <typename T> __device__ __forceinline__ void decode8(uint4 u, float (&v)[8]) {
  const uint32_t q[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (T::code == LUX3D_BF16) {
      v[2 * i] = __uint_as_float(q[i] << 16);
      v[2 * i + 1] = __uint_as_float(q[i] & 0xFFFF0000u);
    } else {
      v[2 * i] = f16_bits_to_f32(q[i] & 0xFFFFu);
      v[2 * i + 1] = f16_bits_to_f32(q[i] >> 16);
    }
  }
}
template <typename T> __device__ __forceinline__ u32x4_t encode8(const float (&v)[8]) {
  u32x4_t u;
  if constexpr (T::code == LUX3D_BF16) {
    u.x = pack_bf16x2(v[0], v[1]); u.y = pack_bf16x2(v[2], v[3]);
    u.z = pack_bf16x2(v[4], v[5]); u.w = pack_bf16x2(v[6], v[7]);
  } else {
    u.x = pack_f16x2(v[0], v[1]); u.y = pack_f16x2(v[2], v[3]);
    u.z = pack_f16x2(v[4], v[5]); u.w = pack_f16x2(v[6], v[7]);
  }
  return u;
}
// a 16-byte access of one row through a descriptor covering `bytes` of it
// (non-temporal: aux bit 1)
__device__ __forceinline__ rsrc_t row_rsrc(const void *row, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(row), (short)0, bytes, 0x00020000);
}

template <typename T>
__global__ __launch_bounds__(256) void resid_ln_persist_kernel(RowParams p, int rows) {
  static_assert(T::bytes == 2, "2-byte rows of 1024");
  constexpr int EB = T::bytes, NT = 2;
  const int lane = threadIdx.x & 63;
  const int wpb = (int)(blockDim.x >> 6);
  const int wv = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * wpb + (threadIdx.x >> 6)));
  const int nw = (int)gridDim.x * wpb;
  const ChunkAt a0 = chunk_at<T, 64>(0, lane), a1 = chunk_at<T, 64>(1, lane);
  const int off0 = (int)(a0.o0 * EB), off1 = (int)(a1.o0 * EB);
  float g[2][8], w[2][8], b[2][8];
  param_at<T>(p.g, p.g_dt, 0, a0, 1.f, g[0]);
  param_at<T>(p.g, p.g_dt, 0, a1, 1.f, g[1]);
  param_at<T>(p.w, p.w_dt, 0, a0, 1.f, w[0]);
  param_at<T>(p.w, p.w_dt, 0, a1, 1.f, w[1]);
  param_at<T>(p.b, p.b_dt, 0, a0, 0.f, b[0]);
  param_at<T>(p.b, p.b_dt, 0, a1, 0.f, b[1]);
  const float inv_d = 1.0f / (float)p.d;
  const bool has_g = p.g_dt >= 0;
  const int rbytes = (int)(p.d * EB);
  const char *xs = reinterpret_cast<const char *>(p.x), *as = reinterpret_cast<const char *>(p.a);
  char *hs = reinterpret_cast<char *>(p.h), *ys = reinterpret_cast<char *>(p.y);
  struct Raw {
    uint4 x0, x1, a0, a1;
  };
  struct Out {
    u32x4_t h0, h1, y0, y1;
  };
  auto ld = [&](const rsrc_t &r, int off) -> uint4 {
    const u32x4_t u = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, NT);
    return make_uint4(u.x, u.y, u.z, u.w);
  };
  auto ldrow = [&](int r) -> Raw {
    const rsrc_t rx = row_rsrc(xs + (int64_t)r * p.x_rs * EB, rbytes);
    const rsrc_t ra = row_rsrc(as + (int64_t)r * p.a_rs * EB, rbytes);
    return Raw{ld(rx, off0), ld(rx, off1), ld(ra, off0), ld(ra, off1)};
  };
  // one row: c holds it, the next row goes into n; po is the previous row's
  // store data, kept allocated until the loads are issued
  auto step = [&](int r, const Raw &c, Raw &n, Out &o, const Out &po) {
    n = ldrow(r + nw < rows ? r + nw : r);
    asm volatile("" ::"v"(po.h0), "v"(po.h1), "v"(po.y0), "v"(po.y1));
    issue_fence();  // the loads stay ahead of this row's arithmetic
    float v[2][8], av[2][8];
    decode8<T>(c.x0, v[0]);
    decode8<T>(c.x1, v[1]);
    decode8<T>(c.a0, av[0]);
    decode8<T>(c.a1, av[1]);
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        // LayerScale product and residual add as two roundings, as row_kernel
        const float ls = has_g ? mul_rn(av[cc][k], g[cc][k]) : av[cc][k];
        v[cc][k] = Chunk<T>::round_trip(add_rn(ls, v[cc][k]));
      }
    const rsrc_t rh = row_rsrc(hs + (int64_t)r * p.h_rs * EB, rbytes);
    const rsrc_t ry = row_rsrc(ys + (int64_t)r * p.y_rs * EB, rbytes);
    o.h0 = encode8<T>(v[0]);
    o.h1 = encode8<T>(v[1]);
    __builtin_amdgcn_raw_buffer_store_b128(o.h0, rh, off0, 0, NT);
    __builtin_amdgcn_raw_buffer_store_b128(o.h1, rh, off1, 0, NT);
    float s[2] = {0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int k = 0; k < 8; ++k) s[cc] += v[cc][k];
    const float mean = (wave_sum(s[0]) + wave_sum(s[1])) * inv_d;
    float q[2] = {0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float dv = v[cc][k] - mean;
        q[cc] += dv * dv;
      }
    const float var = (wave_sum(q[0]) + wave_sum(q[1])) * inv_d;
    const float rstd = 1.0f / sqrtf(var + p.eps);
    float out[2][8];
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int k = 0; k < 8; ++k) out[cc][k] = (v[cc][k] - mean) * rstd * w[cc][k] + b[cc][k];
    o.y0 = encode8<T>(out[0]);
    o.y1 = encode8<T>(out[1]);
    __builtin_amdgcn_raw_buffer_store_b128(o.y0, ry, off0, 0, NT);
    __builtin_amdgcn_raw_buffer_store_b128(o.y1, ry, off1, 0, NT);
  };
  int r = wv;
  if (r >= rows) return;  // wave-uniform; no barrier follows
  Raw c0 = ldrow(r), c1;
  Out o0 = {}, o1 = {};
  step(r, c0, c1, o0, o1);
  for (r += nw; r < rows; r += nw) {
    step(r, c1, c0, o1, o0);
    r += nw;
    if (r >= rows) break;
    step(r, c0, c1, o0, o1);
  }
}

// Fallback for any D and any alignment: one 256-thread block per row, three
// passes over the row (the second and third hit L2).
template <typename T, int MODE>
__global__ __launch_bounds__(kBlock) void row_kernel_any(RowParams p) {
  __shared__ float red_a[kBlock / 64], red_b[kBlock / 64];
  const int64_t row = blockIdx.x;
  const int64_t seg = row_segment(p, row);
  auto piece = [&](const ModPiece &m, int64_t c, float dflt) -> float {
    float v = param1(m.p, m.dt, seg * m.ld + c, dflt);
    return m.base_dt >= 0 ? param1(m.base, m.base_dt, c, 0.f) + v : v;
  };
  auto inval = [&](int64_t c) -> float {
    float xv = load1<T>(p.x, row * p.x_rs + c);
    if constexpr (MODE == ROW_RESID_LN) {
      float av = load1<T>(p.a, row * p.a_rs + c);
      const float ls = p.g_dt >= 0 ? mul_rn(av, param1(p.g, p.g_dt, c, 1.f)) : av;
      xv = Chunk<T>::round_trip(add_rn(ls, xv));
    } else if constexpr (MODE == ROW_GATE_MOD) {
      const float hv = load1<T>(p.a, row * p.a_rs + c);
      xv = Chunk<T>::round_trip(add_rn(xv, mul_rn(hv, piece(p.gate, c, 1.f))));
    }
    return xv;
  };
  if constexpr (MODE == ROW_GATE) {
    for (int64_t c = threadIdx.x; c < p.d; c += kBlock) {
      float hv = load1<T>(p.a, row * p.a_rs + c);
      store1<T>(p.y, row * p.y_rs + c, add_rn(load1<T>(p.x, row * p.x_rs + c), mul_rn(hv, piece(p.gate, c, 1.f))));
    }
    return;
  }
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < p.d; c += kBlock) s += inval(c);
  const float inv_d = 1.0f / (float)p.d;
  const float mean = row_total<kBlock>(s, red_a) * inv_d;
  float s2 = 0.f;
  for (int64_t c = threadIdx.x; c < p.d; c += kBlock) {
    const float dv = inval(c) - mean;
    s2 += dv * dv;
  }
  const float rstd = 1.0f / sqrtf(row_total<kBlock>(s2, red_b) * inv_d + p.eps);
  for (int64_t c = threadIdx.x; c < p.d; c += kBlock) {
    const float xv = inval(c);
    if constexpr (MODE == ROW_RESID_LN || MODE == ROW_GATE_MOD) store1<T>(p.h, row * p.h_rs + c, xv);
    float out;
    if constexpr (MODE == ROW_MODULATE || MODE == ROW_GATE_MOD) {
      out = (xv - mean) * rstd * (piece(p.scale, c, 0.f) + 1.0f) + piece(p.shift, c, 0.f);
      if (MODE == ROW_MODULATE && p.gate.dt >= 0) out = piece(p.gate, c, 1.f) * out + xv;
    } else {
      out = (xv - mean) * rstd * param1(p.w, p.w_dt, c, 1.f) + param1(p.b, p.b_dt, c, 0.f);
    }
    store1<T>(p.y, row * p.y_rs + c, out);
  }
}

template <typename T, int MODE>
hipError_t launch_typed(const RowParams &p0, bool vec, hipStream_t s) {
  if (p0.rows <= 0) return hipSuccess;
  RowParams p = p0;
  if (!p.seg_off && p.rows < (int64_t(1) << 31) && p.rows_per_seg > 0 && p.rows_per_seg < (int64_t(1) << 31))
    div_magic(p.rows_per_seg, p.rps_m, p.rps_s);
  const int64_t chunks = p.d / 8;
  // Layout: threads per row (TPR), chunks per lane (NC) and workgroup size.
  // Short jobs (DINOv2/DINOv3's ~1k tokens) split each row over 2-4
  // wavefronts, one row per workgroup, so the chip is still occupied. For
  // long jobs the layout is the one measured fastest on MI355X at the configs
  // shapes: the fused residual + LayerNorm and the gated residual run a row on
  // 2 wavefronts with one or two chunks per lane (configs[1] F1: 18.0 us vs
  // 20.4 us on one wavefront; the gate without a base vector on 4 wavefronts
  // when a row is 256 chunks), the single-stream LayerNorm / modulate on one
  // wavefront with NC chunks per lane (configs[2] modulate: 7.1 us vs 9.4 us),
  // and so does the gated residual + modulate (configs[2]: 13.1 us against
  // 19.2 us on 2 wavefronts and 18.9 us on 4).
  // Workgroups of several rows let modulate / gate share the staged segment
  // pieces (256 threads; 512 for the one-wavefront modulate rows).
  int tpr = 0, nc = 0;
  bool row_per_block = false;
  if (vec) {
    int ord[3] = {64, 128, 256};
    if (p.rows < 2048) {
      ord[0] = 256; ord[1] = 128; ord[2] = 64;
      row_per_block = true;
    } else if (MODE == ROW_RESID_LN) {
      if (chunks % 128 == 0 && chunks / 128 <= 2) { ord[0] = 128; ord[1] = 64; }
    } else if (MODE == ROW_GATE) {
      // one gate vector per row read straight from the cache is cheapest on
      // 4 wavefronts (configs[2]: 9.7 us vs 10.3 us staged); gate + base
      // is cheaper staged on 2-row workgroups (10.9 us vs 11.3 us)
      if (chunks == 256 && p.gate.base_dt < 0) { ord[0] = 256; ord[1] = 128; ord[2] = 64; }
      else if (chunks % 128 == 0 && chunks / 128 <= 2) { ord[0] = 128; ord[1] = 64; }
    }
    for (int i = 0; i < 3 && !tpr; ++i) {
      const int cand = ord[i];
      if (chunks % cand) continue;
      const int64_t n = chunks / cand;
      if (n == 1 || n == 2 || n == 3 || n == 4 || (n == 8 && cand == 64)) { tpr = cand; nc = (int)n; }
    }
    if (tpr == 64) row_per_block = false;
  }
  if (!tpr) {  // any width / alignment: one 256-thread block per row
    hipLaunchKernelGGL((row_kernel_any<T, MODE>), dim3((unsigned)p.rows), dim3(kBlock), 0, s, p);
    return hipGetLastError();
  }
  // the long residual + LayerNorm jobs on 2-byte rows of 1024: the persistent
  // kernel, two workgroups per CU
  // the long residual + LayerNorm jobs on 2-byte rows of 1024: the persistent
  // kernel, one 256-thread workgroup per CU
  if constexpr (MODE == ROW_RESID_LN && T::bytes == 2) {
    if (tpr == 128 && nc == 1 && !row_per_block && p.rows < INT32_MAX) {
      const int64_t need = (p.rows + 3) / 4, cap = cu_count(s);
      const int64_t grid = need < cap ? need : cap;
      hipLaunchKernelGGL((resid_ln_persist_kernel<T>), dim3((unsigned)grid), dim3(256), 0, s, p, (int)p.rows);
      return hipGetLastError();
    }
  }
  int block = row_per_block ? tpr : kBlock;
  // staged segment pieces: larger workgroups stage them for more rows
  if ((MODE == ROW_MODULATE || MODE == ROW_GATE_MOD) && !row_per_block && tpr == 64 && kStagedBlock > kBlock)
    block = kStagedBlock;
  const int64_t rpb = block / tpr;
  const dim3 grid((unsigned)((p.rows + rpb - 1) / rpb));
  // Stage the segment pieces in LDS when a workgroup holds several rows.
  const int npieces = (MODE == ROW_MODULATE || MODE == ROW_GATE_MOD) ? 2 + (p.gate.dt >= 0 ? 1 : 0)
                                                                      : (MODE == ROW_GATE ? 1 : 0);
  size_t lds = (size_t)npieces * (size_t)p.d * sizeof(float);
  const bool stage = npieces > 0 && rpb > 1 && lds <= 64 * 1024;
  // resident-workgroup caps (lds_for_occupancy), each measured in one
  // process with the cap on and off: the two-wavefront 2-byte residual rows
  // at 6 per CU (configs[1] F1: 17.67 against 18.04 us; the f32 rows are
  // not faster capped: 31.5 against 31.3), the 512-thread staged modulate
  // rows at 2 (configs[3] modulate 64.4 against 66.0 us, configs[2] even).
  // The ragged gated residual + modulate rows are slower capped (139.1
  // against 134.6 us at 2) and run uncapped.
  size_t lds_launch = stage ? lds : 0;
  if (MODE == ROW_RESID_LN && T::bytes == 2 && !row_per_block && block == 256 && tpr == 128)
    lds_launch = lds_for_occupancy(s, 6, lds_launch);
  if (MODE == ROW_MODULATE && stage && block == 512) lds_launch = lds_for_occupancy(s, 2, lds_launch);
#define LUX3D_ROW_CASE(TPR_, NC_, BLK_)                                                                 \
  if (tpr == TPR_ && nc == NC_ && block == BLK_) {                                                      \
    if constexpr (MODE == ROW_MODULATE || MODE == ROW_GATE || MODE == ROW_GATE_MOD) {                   \
      if (stage && BLK_ > TPR_) {                                                                       \
        hipLaunchKernelGGL((row_kernel<T, TPR_, NC_, MODE, BLK_, (BLK_ > TPR_)>), grid, dim3(BLK_), lds_launch, \
                           s, p);                                                                       \
        return hipGetLastError();                                                                       \
      }                                                                                                 \
    }                                                                                                   \
    hipLaunchKernelGGL((row_kernel<T, TPR_, NC_, MODE, BLK_>), grid, dim3(BLK_), lds_launch, s, p);     \
    return hipGetLastError();                                                                           \
  }
  LUX3D_ROW_CASE(64, 1, 256) LUX3D_ROW_CASE(64, 2, 256) LUX3D_ROW_CASE(64, 3, 256)
  LUX3D_ROW_CASE(64, 4, 256) LUX3D_ROW_CASE(64, 8, 256)
  LUX3D_ROW_CASE(128, 1, 256) LUX3D_ROW_CASE(128, 2, 256) LUX3D_ROW_CASE(128, 3, 256) LUX3D_ROW_CASE(128, 4, 256)
  LUX3D_ROW_CASE(128, 1, 128) LUX3D_ROW_CASE(128, 2, 128) LUX3D_ROW_CASE(128, 3, 128) LUX3D_ROW_CASE(128, 4, 128)
  LUX3D_ROW_CASE(256, 1, 256) LUX3D_ROW_CASE(256, 2, 256) LUX3D_ROW_CASE(256, 3, 256) LUX3D_ROW_CASE(256, 4, 256)
  if constexpr (MODE == ROW_MODULATE || MODE == ROW_GATE_MOD) {
    LUX3D_ROW_CASE(64, 1, kStagedBlock) LUX3D_ROW_CASE(64, 2, kStagedBlock) LUX3D_ROW_CASE(64, 3, kStagedBlock)
    LUX3D_ROW_CASE(64, 4, kStagedBlock) LUX3D_ROW_CASE(64, 8, kStagedBlock)
  }
#undef LUX3D_ROW_CASE
  return hipErrorInvalidValue;
}

template <typename T>
hipError_t launch_mode(int mode, const RowParams &p, bool vec, hipStream_t s) {
  switch (mode) {
    case ROW_LN: return launch_typed<T, ROW_LN>(p, vec, s);
    case ROW_RESID_LN: return launch_typed<T, ROW_RESID_LN>(p, vec, s);
    case ROW_MODULATE: return launch_typed<T, ROW_MODULATE>(p, vec, s);
    case ROW_GATE: return launch_typed<T, ROW_GATE>(p, vec, s);
    case ROW_GATE_MOD: return launch_typed<T, ROW_GATE_MOD>(p, vec, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_rows(int mode, int dt, const RowParams &p, bool vec, hipStream_t s) {
  switch (dt) {
    case LUX3D_F32: return launch_mode<F32>(mode, p, vec, s);
    case LUX3D_BF16: return launch_mode<BF16>(mode, p, vec, s);
    case LUX3D_F16: return launch_mode<F16>(mode, p, vec, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace lux3d
