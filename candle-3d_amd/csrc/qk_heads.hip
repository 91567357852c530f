// qk_heads.hip -- per-head normalisation + rotary kernels for gfx950 on
// [B, H, N, D] head views (D = 64 or 128): VGGT QK-LayerNorm + 2D RoPE,
// TripoSG per-head RMSNorm, TRELLIS.2 L2 norm + 3D RoPE, DINOv3 2D RoPE.
//
// Mapping. One workgroup per token (b, n) processes every head of q and k
// for that token: LPR = D/8 lanes own one head row, 8 elements each, so a
// wavefront covers 8 (D=64) or 4 (D=128) head rows. 2-byte types: lane l
// holds elements 8l..8l+7 (one 16-byte load); f32: elements 4l..4l+3 and
// D/2+4l..D/2+4l+3, so each 16-byte load instruction of the wavefront covers
// whole 64-byte runs of the row instead of every other 16 bytes. The token's rotation phases are computed (or read from the caller's
// tables) once into LDS and shared by all 2H head rows; head statistics are
// reduced in-register with DPP over the LPR lanes. Every rotation in the
// reference has the form out[j] = y[j]*C[j] + y[j ^ M]*S[j] for a fixed
// partner distance M (VGGT: D/4, TRELLIS interleaved pairs: 1, DINOv3
// rotate_half: D/2), with the rotate-half sign folded into S.
#include "common.hpp"
#include "kernels.hpp"

namespace lux3d {

namespace {

template <int ROT, int D> struct RotPartner;
template <int D> struct RotPartner<HR_NONE, D> { static constexpr int M = 0; };
template <int D> struct RotPartner<HR_R1_TAB, D> { static constexpr int M = D / 4; };
template <int D> struct RotPartner<HR_R1_POS, D> { static constexpr int M = D / 4; };
template <int D> struct RotPartner<HR_R2_TAB, D> { static constexpr int M = 1; };
template <int D> struct RotPartner<HR_R2_COORD, D> { static constexpr int M = 1; };
template <int D> struct RotPartner<HR_R3_TAB, D> { static constexpr int M = D / 2; };

// Element of the head row that a lane's x[k] holds (see Mapping above).
template <typename T, int D> __device__ __forceinline__ int head_elem(int lane, int k) {
  if constexpr (T::bytes == 4) return (k >> 2) * (D / 2) + lane * 4 + (k & 3);
  else return lane * 8 + k;
}
// A lane's 8 elements of the row at `row` (byte address of element 0).
template <typename T, int D> __device__ __forceinline__ void head_load(const char *row, int lane, float (&v)[8]) {
  if constexpr (T::bytes == 4) {
    const uint4 a = ld16<LUX3D_NT_STREAMS != 0>(row + lane * 16);
    const uint4 b = ld16<LUX3D_NT_STREAMS != 0>(row + D * 2 + lane * 16);
    v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
    v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y); v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
  } else {
    Chunk<T>::load(row + lane * 16, v);
  }
}
template <typename T, int D> __device__ __forceinline__ void head_store(char *row, int lane, const float (&v)[8]) {
  if constexpr (T::bytes == 4) {
    st16(row + lane * 16, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                     __float_as_uint(v[3])));
    st16(row + D * 2 + lane * 16, make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                                             __float_as_uint(v[7])));
  } else {
    Chunk<T>::store(row + lane * 16, v);
  }
}
// Per-channel parameters of the lane's 8 elements, channel 0 at element `off`.
template <typename T, int D>
__device__ __forceinline__ void head_param(const void *p, int dt, int64_t off, int lane, float dflt, float (&v)[8]) {
  if constexpr (T::bytes == 4) {
    param4(p, dt, off + lane * 4, dflt, v);
    param4(p, dt, off + D / 2 + lane * 4, dflt, v + 4);
  } else {
    param8(p, dt, off + lane * 8, dflt, v);
  }
}

// Element offset of (b, h, n) + c in a [B, H, N, D] view. O32: the launcher
// has checked that every byte offset of the views is below 2^31 and that
// every index and every stride of an axis longer than 1 is below 2^24, so
// the products are full-rate 24-bit multiplies (an axis of length 1 has
// index 0, whatever its stride).
template <bool O32> __device__ __forceinline__ uint32_t imul(uint32_t a, uint32_t b) {
  if constexpr (O32) return __umul24(a, b);
  else return a * b;
}
template <bool O32>
__device__ __forceinline__ auto view_off(uint32_t b, uint32_t h, uint32_t n, int64_t sB, int64_t sH, int64_t sN,
                                         uint32_t c) {
  if constexpr (O32) return imul<O32>(b, (uint32_t)sB) + imul<O32>(h, (uint32_t)sH) + imul<O32>(n, (uint32_t)sN) + c;
  else return (int64_t)b * sB + (int64_t)h * sH + (int64_t)n * sN + c;
}

__device__ __forceinline__ int64_t load_index(const void *p, int dt, int64_t i) {
  return dt == LUX3D_I64 ? reinterpret_cast<const int64_t *>(p)[i]
                         : (int64_t)reinterpret_cast<const int32_t *>(p)[i];
}

// Stage the rotation of the tile's tokens into LDS: Cs[t*D + j], Ss[t*D + j]
// for tile token t and element j, so that out[j] = y[j]*C[j] + y[j^M]*S[j].
// Angle-based sources compute each distinct angle once (D/2 per token) and
// write the two elements that share it.
template <int ROT, int D>
__device__ __forceinline__ void stage_phases(const HeadParams &p, uint32_t tok0, int tb, uint32_t ntok,
                                             uint32_t N, float *Cs, float *Ss) {
  constexpr int half = D / 2, quarter = D / 4;
  if constexpr (ROT == HR_R1_TAB || ROT == HR_R3_TAB) {
    for (int e = threadIdx.x; e < tb * D; e += blockDim.x) {
      const int t = e / D, j = e % D;
      uint32_t tok = tok0 + t;
      tok = tok < ntok ? tok : ntok - 1;
      const uint32_t b = fdiv(tok, p.div_n_m, p.div_n_s), n = tok - b * N;
      float C = 1.f, S = 0.f;
      if constexpr (ROT == HR_R1_TAB) {
        const int64_t off = (int64_t)b * p.tab_sB + (int64_t)n * p.tab_sN + j;
        C = param1(p.tab_c, p.tab_dt, off, 1.f);
        S = param1(p.tab_s, p.tab_dt, off, 0.f);
      } else if (n >= p.prefix) {
        const int64_t off = (int64_t)(n - p.prefix) * p.tab_sN + j;
        C = param1(p.tab_c, p.tab_dt, off, 1.f);
        const float sv = param1(p.tab_s, p.tab_dt, off, 0.f);
        S = j < half ? -sv : sv;  // rotate_half = cat(-x2, x1)
      }
      Cs[e] = C;
      Ss[e] = S;
    }
  } else {
    for (int e = threadIdx.x; e < tb * half; e += blockDim.x) {
      const int t = e / half, a = e % half;
      uint32_t tok = tok0 + t;
      tok = tok < ntok ? tok : ntok - 1;
      const uint32_t b = fdiv(tok, p.div_n_m, p.div_n_s), n = tok - b * N;
      float cv, sv;
      int j0, j1;
      if constexpr (ROT == HR_R1_POS) {
        // Rope2d: angle a = (axis, k); elements axis*half + k (sin negated:
        // the sin_alt quarter) and axis*half + quarter + k share it.
        const int axis = a / quarter, k = a % quarter;
        const uint32_t pv = (uint32_t)load_index(
            p.pos, p.pos_dt, (int64_t)b * p.pos_sB + (int64_t)n * p.pos_sN + axis * p.pos_sC);
        sincosf((float)pv * p.freq[k], &sv, &cv);
        j0 = axis * half + k;
        j1 = j0 + quarter;
      } else {
        // TRELLIS.2: pair a = (re, im) = elements (2a, 2a+1); angle axis-major,
        // the trailing pad pairs have angle 0.
        if constexpr (ROT == HR_R2_TAB) {
          const int64_t off = (int64_t)n * p.tab_sN + a;
          cv = param1(p.tab_c, p.tab_dt, off, 1.f);
          sv = param1(p.tab_s, p.tab_dt, off, 0.f);
        } else {
          float ang = 0.f;
          if (a < 3 * p.nfreq) {
            const int axis = a / p.nfreq;
            const int32_t cval = reinterpret_cast<const int32_t *>(p.pos)[(int64_t)n * p.pos_sN + axis * p.pos_sC];
            ang = (float)cval * p.freq[a % p.nfreq];
          }
          sincosf(ang, &sv, &cv);
        }
        j0 = 2 * a;
        j1 = 2 * a + 1;
      }
      Cs[t * D + j0] = cv;
      Ss[t * D + j0] = -sv;
      Cs[t * D + j1] = cv;
      Ss[t * D + j1] = sv;
    }
  }
}

// Phase sources of one angle item e < tb * D/2 (R1_POS: a position and a
// frequency; R2_COORD: a coordinate and a frequency), issued as plain loads
// with no branch on loaded data (an item past the tile reads item 0's
// sources), so that the head rows issued after them stay in flight while
// the phases are computed; phase_finish then writes the two LDS entries the
// angle feeds, exactly as stage_phases does.
struct PhaseSrc {
  uint32_t v;  // position / coordinate bits
  float f;     // frequency
};
template <int ROT, int D>
__device__ __forceinline__ PhaseSrc phase_issue(const HeadParams &p, uint32_t tok0, int tb, uint32_t ntok, uint32_t N,
                                                int e) {
  constexpr int half = D / 2, quarter = D / 4;
  if (e >= tb * half) e = 0;
  const int t = e / half, a = e % half;
  uint32_t tok = tok0 + t;
  tok = tok < ntok ? tok : ntok - 1;
  const uint32_t b = fdiv(tok, p.div_n_m, p.div_n_s), n = tok - b * N;
  PhaseSrc s;
  if constexpr (ROT == HR_R1_POS) {
    const int axis = a / quarter, k = a % quarter;
    const int64_t idx = (int64_t)b * p.pos_sB + (int64_t)n * p.pos_sN + axis * p.pos_sC;
    // the low 32 bits of an int64 position (little-endian), or the int32
    s.v = *reinterpret_cast<const uint32_t *>(reinterpret_cast<const char *>(p.pos) +
                                              (idx << (p.pos_dt == LUX3D_I64 ? 3 : 2)));
    s.f = p.freq[k];
  } else {
    const int axis = a < 3 * p.nfreq ? a / p.nfreq : 0;
    s.v = (uint32_t)reinterpret_cast<const int32_t *>(p.pos)[(int64_t)n * p.pos_sN + axis * p.pos_sC];
    s.f = p.freq[a < 3 * p.nfreq ? a % p.nfreq : 0];
  }
  return s;
}
// The angle is evaluated for every thread (an item past the tile evaluates
// item 0's) and only the LDS writes are conditional: a use of the loaded
// sources under a branch let the compiler sink their loads into it, behind
// the row loads.
template <int ROT, int D>
__device__ __forceinline__ void phase_finish(const HeadParams &p, int tb, int e, PhaseSrc s, float *Cs, float *Ss) {
  constexpr int half = D / 2, quarter = D / 4;
  const bool in_tile = e < tb * half;
  const int ec = in_tile ? e : 0;
  const int t = ec / half, a = ec % half;
  float cv, sv;
  int j0, j1;
  if constexpr (ROT == HR_R1_POS) {
    const int axis = a / quarter, k = a % quarter;
    sincosf((float)s.v * s.f, &sv, &cv);
    j0 = axis * half + k;
    j1 = j0 + quarter;
  } else {
    const float ang = a < 3 * p.nfreq ? (float)(int32_t)s.v * s.f : 0.f;
    sincosf(ang, &sv, &cv);
    j0 = 2 * a;
    j1 = 2 * a + 1;
  }
  if (in_tile) {
    Cs[t * D + j0] = cv;
    Ss[t * D + j0] = -sv;
    Cs[t * D + j1] = cv;
    Ss[t * D + j1] = sv;
  }
}

// Rotation tables (R1_TAB) issued before the head rows: the raw bits of the
// table elements a thread stages (up to two), decoded into LDS after the
// rows are in flight (as stage_phases would read them: C defaults to 1, S to
// 0 for an absent table). Loaded after the rows and converted at once, their
// wait had to wait for every row too.
__device__ __forceinline__ uint32_t tab_raw(const void *p, int dt, int64_t i) {
  if (dt == LUX3D_F32) return reinterpret_cast<const uint32_t *>(p)[i];
  if (dt == LUX3D_BF16 || dt == LUX3D_F16) return reinterpret_cast<const uint16_t *>(p)[i];
  return 0;
}
__device__ __forceinline__ float tab_decode(uint32_t v, int dt, float dflt) {
  if (dt == LUX3D_F32) return __uint_as_float(v);
  if (dt == LUX3D_BF16) return bf16_bits_to_f32(v);
  if (dt == LUX3D_F16) return f16_bits_to_f32(v);
  return dflt;
}

// Grid: x = tiles of `tb` consecutive tokens; y = tensor (q, k) when NTB = 1,
// or 1 when NTB = 2 (each workgroup then handles q and k of its tokens, whose
// rows lie side by side in a packed qkv buffer, and stages the phases once).
// Work items are (token, head) rows of LPR lanes; each thread owns R of the
// tile's rows per tensor. Order of work per workgroup: issue the phase
// sources, every row load and the per-channel parameters, then stage the
// tile's rotation phases in LDS while the rows are in flight, one LDS
// barrier, then normalise / rotate / store. Each workgroup therefore waits
// on one HBM round trip. Rows of one head are adjacent in the [B, H, N, D]
// output across the tile's tokens, so a head's stores form contiguous runs
// of tb*D elements.
template <typename T, int D, int NORM, int ROT, int R, int NTB, bool O32>
__global__ __launch_bounds__(256) void head_kernel(HeadParams p, int tb) {
  constexpr int LPR = D / 8;
  constexpr int M = RotPartner<ROT, D>::M;
  constexpr int EB = T::bytes;
  extern __shared__ float lds[];
  float *Cs = lds, *Ss = lds + tb * D;

  const uint32_t N = (uint32_t)p.N, H = (uint32_t)p.H;
  const uint32_t ntok = (uint32_t)(p.B * p.N);
  const uint32_t tok0 = blockIdx.x * (uint32_t)tb;
  const int lane = threadIdx.x % LPR;
  const int ipp = blockDim.x / LPR;
  const uint32_t items = (uint32_t)tb * H;

  uint32_t tt[R], hh[R], nn[R], bb[R];
  bool live[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t it = (uint32_t)(r * ipp) + threadIdx.x / LPR;
    uint32_t t = fdiv(it, p.div_h_m, p.div_h_s), h = it - imul<O32>(t, H);
    uint32_t tok = tok0 + t;
    live[r] = it < items && tok < ntok;
    if (!live[r]) { t = 0; h = 0; tok = tok0; }
    const uint32_t b = fdiv(tok, p.div_n_m, p.div_n_s);
    tt[r] = t; hh[r] = h; nn[r] = tok - imul<O32>(b, N); bb[r] = b;
  }
  // Order of the loads (vmcnt counts loads and stores in issue order, so a
  // wait for one load waits for all issued before it): (1) this thread's
  // phase sources, (2) the head rows, (3) the per-channel parameters as raw
  // bytes (pissue). The phases are then computed and staged while the rows
  // are in flight (their wait leaves (2) and (3) outstanding), and one
  // barrier and one wait later every row is normalised, rotated and stored.
  // Unrotated rows (HR_NONE) keep the plain order -- each tensor's rows, then
  // its parameters read where they are converted -- which measured faster
  // for them (configs[2] RMS heads 13.0 against 14.1 us, same-box A/B at
  // equal occupancy) than issuing every load first.
  constexpr bool SRC = ROT == HR_R1_POS || ROT == HR_R2_COORD;
  constexpr bool EARLY = ROT != HR_NONE;
  const int e0 = threadIdx.x;
  PhaseSrc ps{};
  if constexpr (SRC) ps = phase_issue<ROT, D>(p, tok0, tb, ntok, N, e0);
  // R1_TAB: this thread's (up to two) table elements, issued first when the
  // tile's tb * D elements fit two per thread (always, for the launcher's
  // tiles); otherwise stage_phases reads them after the rows
  constexpr bool TABE = ROT == HR_R1_TAB;
  const bool tab_early = TABE && tb * D <= 2 * (int)blockDim.x;
  uint32_t tcr[2] = {0u, 0u}, tsr[2] = {0u, 0u};
  if constexpr (TABE) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      int e = e0 + i * (int)blockDim.x;
      if (e >= tb * D) e = 0;
      const int t = e / D, j = e % D;
      uint32_t tok = tok0 + t;
      tok = tok < ntok ? tok : ntok - 1;
      const uint32_t b = fdiv(tok, p.div_n_m, p.div_n_s), n = tok - b * N;
      const int64_t off = (int64_t)b * p.tab_sB + (int64_t)n * p.tab_sN + j;
      tcr[i] = tab_raw(p.tab_c, p.tab_dt, off);
      tsr[i] = tab_raw(p.tab_s, p.tab_dt, off);
    }
  }
  issue_fence();

  float v[NTB][R][8];
  float w[NTB][8], bias[NTB][8];
  PRaw qw[NTB], qb[NTB], qg[NORM == HN_L2 && EARLY ? NTB : 1][NORM == HN_L2 && EARLY ? R : 1];
  // lane's elements of a head row: i..i+3 and j..j+3 (see head_elem)
  const int pi = EB == 4 ? lane * 4 : lane * 8, pj = EB == 4 ? D / 2 + lane * 4 : lane * 8 + 4;
#pragma unroll
  for (int q = 0; q < NTB; ++q) {
    const HeadIO &io = p.io[NTB == 1 ? blockIdx.y : q];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const char *xp = reinterpret_cast<const char *>(io.x) +
                       view_off<O32>(bb[r], hh[r], nn[r], io.sB, io.sH, io.sN, 0) * EB;
      head_load<T, D>(xp, lane, v[q][r]);
    }
    if constexpr (!EARLY) {
      if constexpr (NORM == HN_LN || NORM == HN_RMS) head_param<T, D>(io.p0, io.p0_dt, 0, lane, 1.f, w[q]);
      if constexpr (NORM == HN_LN) head_param<T, D>(io.p1, io.p1_dt, 0, lane, 0.f, bias[q]);
    }
  }
  if constexpr (EARLY) {
    issue_fence();
#pragma unroll
    for (int q = 0; q < NTB; ++q) {
      const HeadIO &io = p.io[NTB == 1 ? blockIdx.y : q];
      if constexpr (NORM == HN_LN || NORM == HN_RMS) qw[q] = pissue(param_rsrc(io.p0, io.p0_dt, D), io.p0_dt, pi, pj);
      if constexpr (NORM == HN_LN) qb[q] = pissue(param_rsrc(io.p1, io.p1_dt, D), io.p1_dt, pi, pj);
      if constexpr (NORM == HN_L2) {
        const rsrc_t rg = param_rsrc(io.p0, io.p0_dt, (int64_t)H * D);
#pragma unroll
        for (int r = 0; r < R; ++r) qg[q][r] = pissue(rg, io.p0_dt, (int64_t)hh[r] * D + pi, (int64_t)hh[r] * D + pj);
      }
    }
    issue_fence();
  }

  if constexpr (ROT != HR_NONE) {
    if constexpr (SRC) {
      phase_finish<ROT, D>(p, tb, e0, ps, Cs, Ss);
      // tiles with more angles than threads: the rest the plain way
      for (int e = e0 + (int)blockDim.x; e < tb * (D / 2); e += blockDim.x)
        phase_finish<ROT, D>(p, tb, e, phase_issue<ROT, D>(p, tok0, tb, ntok, N, e), Cs, Ss);
    } else if (tab_early) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = e0 + i * (int)blockDim.x;
        if (e < tb * D) {
          Cs[e] = tab_decode(tcr[i], p.tab_dt, 1.f);
          Ss[e] = tab_decode(tsr[i], p.tab_dt, 0.f);
        }
      }
    } else {
      stage_phases<ROT, D>(p, tok0, tb, ntok, N, Cs, Ss);
    }
    lds_barrier();
  }
  if constexpr (EARLY) {
#pragma unroll
    for (int q = 0; q < NTB; ++q) {
      const HeadIO &io = p.io[NTB == 1 ? blockIdx.y : q];
      if constexpr (NORM == HN_LN || NORM == HN_RMS) pdecode(qw[q], io.p0_dt, 1.f, w[q]);
      if constexpr (NORM == HN_LN) pdecode(qb[q], io.p1_dt, 0.f, bias[q]);
    }
  }

#pragma unroll
  for (int q = 0; q < NTB; ++q) {
    const HeadIO &io = p.io[NTB == 1 ? blockIdx.y : q];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float (&x)[8] = v[q][r];
      if constexpr (NORM == HN_LN) {
        const float mean = group_sum<LPR>(ln_chunk_sum(x)) * (1.0f / D);
        const float rstd = ln_rstd(group_sum<LPR>(ln_chunk_center_sq(x, mean)), 1.0f / D, p.eps);
        ln_chunk_affine(x, rstd, w[q], bias[q]);
      } else if constexpr (NORM == HN_RMS) {
        head_rms_chunk<LPR, D>(x, w[q], p.eps);
      } else if constexpr (NORM == HN_L2) {
        float g[8];
        if constexpr (EARLY) pdecode(qg[q][r], io.p0_dt, 1.f, g);
        else head_param<T, D>(io.p0, io.p0_dt, (int64_t)hh[r] * D, lane, 1.f, g);
        head_l2_chunk<LPR, D>(x, g);
      }
      if constexpr (ROT != HR_NONE) {
        bool rotate = true;
        if constexpr (ROT == HR_R3_TAB) rotate = nn[r] >= (uint32_t)p.prefix;  // prefix tokens pass through
        if (rotate) {
          // partner of element j = head_elem(lane, k): j ^ M
          float pv[8];
          if constexpr (EB == 4 && (M < 4 || M == D / 2)) {
            constexpr int KM = M == D / 2 ? 4 : M;  // in the lane: the other half, or the same 4
#pragma unroll
            for (int k = 0; k < 8; ++k) pv[k] = x[k ^ KM];
          } else if constexpr (EB == 4) {
#pragma unroll
            for (int k = 0; k < 8; ++k) pv[k] = lane_xor<M / 4>(x[k]);
          } else if constexpr (M < 8) {
#pragma unroll
            for (int k = 0; k < 8; ++k) pv[k] = x[k ^ M];
          } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) pv[k] = lane_xor<M / 8>(x[k]);
          }
          const float *C = Cs + tt[r] * D;
          const float *S = Ss + tt[r] * D;
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const int j = head_elem<T, D>(lane, k);
            x[k] = rotate1(x[k], C[j], pv[k], S[j]);
          }
        }
      }
      if (live[r]) {
        char *yp = reinterpret_cast<char *>(io.y) + view_off<O32>(bb[r], hh[r], nn[r], io.oB, io.oH, io.oN, 0) * EB;
        head_store<T, D>(yp, lane, v[q][r]);
      }
    }
  }
}

// Generic path for any head dim and any alignment (the reference's own
// tests use head dims 4, 6 and 12): one wavefront per (tensor, b, h, n) row,
// lanes striding over the D elements, element loads re-read from the cache
// instead of held in registers, and each element's phase evaluated where it
// is used. Same arithmetic as head_kernel, element for element.
template <int ROT>
__device__ __forceinline__ void phase_any(const HeadParams &p, int64_t b, int64_t n, int64_t j, float &C,
                                          float &S, int64_t &partner) {
  const int64_t D = p.D, half = D / 2, quarter = D / 4;
  C = 1.f;
  S = 0.f;
  partner = j;
  if constexpr (ROT == HR_R1_TAB || ROT == HR_R1_POS) {
    const int64_t jj = j % half;
    partner = j - jj + (jj < quarter ? jj + quarter : jj - quarter);
    if constexpr (ROT == HR_R1_TAB) {
      const int64_t off = b * p.tab_sB + n * p.tab_sN + j;
      C = param1(p.tab_c, p.tab_dt, off, 1.f);
      S = param1(p.tab_s, p.tab_dt, off, 0.f);
    } else {
      const int64_t axis = j / half;
      const uint32_t pv = (uint32_t)load_index(p.pos, p.pos_dt, b * p.pos_sB + n * p.pos_sN + axis * p.pos_sC);
      float sv, cv;
      sincosf((float)pv * p.freq[jj % quarter], &sv, &cv);
      C = cv;
      S = jj < quarter ? -sv : sv;
    }
  } else if constexpr (ROT == HR_R2_TAB || ROT == HR_R2_COORD) {
    const int64_t a = j / 2;
    partner = j ^ 1;
    float sv, cv;
    if constexpr (ROT == HR_R2_TAB) {
      cv = param1(p.tab_c, p.tab_dt, n * p.tab_sN + a, 1.f);
      sv = param1(p.tab_s, p.tab_dt, n * p.tab_sN + a, 0.f);
    } else {
      float ang = 0.f;
      if (a < 3 * p.nfreq) {
        const int32_t cval = reinterpret_cast<const int32_t *>(p.pos)[n * p.pos_sN + (a / p.nfreq) * p.pos_sC];
        ang = (float)cval * p.freq[a % p.nfreq];
      }
      sincosf(ang, &sv, &cv);
    }
    C = cv;
    S = (j & 1) ? sv : -sv;
  } else if constexpr (ROT == HR_R3_TAB) {
    partner = j < half ? j + half : j - half;
    if (n >= p.prefix) {
      const int64_t off = (n - p.prefix) * p.tab_sN + j;
      C = param1(p.tab_c, p.tab_dt, off, 1.f);
      const float sv = param1(p.tab_s, p.tab_dt, off, 0.f);
      S = j < half ? -sv : sv;
    } else {
      partner = j;  // prefix tokens pass through
    }
  }
}

template <typename T, int NORM, int ROT>
__global__ __launch_bounds__(256) void head_kernel_any(HeadParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t per = p.B * p.H * p.N;
  const int64_t row = uniform((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6));
  if (row >= per * p.ntens) return;  // wave-uniform
  const int q = (int)(row / per);
  int64_t r = row % per;
  const int64_t n = r % p.N;
  r /= p.N;
  const int64_t h = r % p.H, b = r / p.H;
  const HeadIO &io = p.io[q];
  const int64_t D = p.D;
  const int64_t xo = b * io.sB + h * io.sH + n * io.sN;
  const int64_t yo = b * io.oB + h * io.oH + n * io.oN;

  float mean = 0.f, rs = 1.f;
  if constexpr (NORM == HN_LN) {
    float s = 0.f;
    for (int64_t j = lane; j < D; j += 64) s += load1<T>(io.x, xo + j);
    mean = wave_sum(s) * (1.0f / (float)D);
    float s2 = 0.f;
    for (int64_t j = lane; j < D; j += 64) {
      const float c = load1<T>(io.x, xo + j) - mean;
      s2 += c * c;
    }
    rs = rsqrt_f32(wave_sum(s2) * (1.0f / (float)D) + p.eps);
  } else if constexpr (NORM == HN_RMS || NORM == HN_L2) {
    float s2 = 0.f;
    for (int64_t j = lane; j < D; j += 64) {
      const float v = load1<T>(io.x, xo + j);
      s2 += v * v;
    }
    if constexpr (NORM == HN_RMS) {
      rs = rsqrt_f32(wave_sum(s2) * (1.0f / (float)D) + p.eps);
    } else {
      rs = l2_rnorm(wave_sum(s2));
    }
  }
  auto normed = [&](int64_t j) -> float {
    const float v = load1<T>(io.x, xo + j);
    if constexpr (NORM == HN_LN) {
      return (v - mean) * rs * param1(io.p0, io.p0_dt, j, 1.f) + param1(io.p1, io.p1_dt, j, 0.f);
    } else if constexpr (NORM == HN_RMS) {
      return (v * rs) * param1(io.p0, io.p0_dt, j, 1.f);
    } else if constexpr (NORM == HN_L2) {
      return ((v * rs) * param1(io.p0, io.p0_dt, h * D + j, 1.f)) * sqrtf((float)D);
    } else {
      return v;
    }
  };
  for (int64_t j = lane; j < D; j += 64) {
    float out = normed(j);
    if constexpr (ROT != HR_NONE) {
      float C, S;
      int64_t pj;
      phase_any<ROT>(p, b, n, j, C, S, pj);
      if (pj != j) out = rotate1(out, C, normed(pj), S);
    }
    store1<T>(io.y, yo + j, out);
  }
}

template <typename T>
hipError_t launch_any(int norm, int rot, const HeadParams &p, hipStream_t s) {
  const int64_t rows = p.B * p.H * p.N * p.ntens;
  if (rows <= 0 || p.D <= 0) return hipSuccess;
  const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
#define LUX3D_ANY_CASE(NORM_, ROT_)                                                 \
  if (norm == NORM_ && rot == ROT_) {                                               \
    hipLaunchKernelGGL((head_kernel_any<T, NORM_, ROT_>), grid, block, 0, s, p);    \
    return hipGetLastError();                                                       \
  }
  LUX3D_ANY_CASE(HN_LN, HR_R1_TAB) LUX3D_ANY_CASE(HN_LN, HR_R1_POS)
  LUX3D_ANY_CASE(HN_NONE, HR_R1_TAB) LUX3D_ANY_CASE(HN_NONE, HR_R1_POS)
  LUX3D_ANY_CASE(HN_LN, HR_NONE)
  LUX3D_ANY_CASE(HN_RMS, HR_NONE)
  LUX3D_ANY_CASE(HN_L2, HR_NONE) LUX3D_ANY_CASE(HN_L2, HR_R2_TAB) LUX3D_ANY_CASE(HN_L2, HR_R2_COORD)
  LUX3D_ANY_CASE(HN_NONE, HR_R2_TAB) LUX3D_ANY_CASE(HN_NONE, HR_R2_COORD)
  LUX3D_ANY_CASE(HN_NONE, HR_R3_TAB)
  LUX3D_ANY_CASE(HN_NONE, HR_NONE)
#undef LUX3D_ANY_CASE
  return hipErrorInvalidValue;
}

// Every byte offset the vector kernel forms in the views of p is below 2^31
// (non-negative strides), and every index and every stride of an axis longer
// than 1 below 2^24: offsets may then be computed in 32 bits from 24-bit
// products.
bool offsets_fit_32(const HeadParams &p, int eb) {
  const int64_t lim = (int64_t(1) << 31) / eb, lim24 = int64_t(1) << 24;
  const int64_t ext[3] = {p.B - 1, p.H - 1, p.N - 1};
  for (int a = 0; a < 3; ++a)
    if (ext[a] >= lim24) return false;
  for (int i = 0; i < p.ntens; ++i) {
    const HeadIO &io = p.io[i];
    const int64_t in[3] = {io.sB, io.sH, io.sN}, out[3] = {io.oB, io.oH, io.oN};
    int64_t mi = p.D, mo = p.D;
    for (int a = 0; a < 3; ++a) {
      if (in[a] < 0 || out[a] < 0) return false;
      if (ext[a] > 0 && (in[a] >= lim24 || out[a] >= lim24)) return false;
      mi += ext[a] * in[a];
      mo += ext[a] * out[a];
    }
    if (mi >= lim || mo >= lim) return false;
  }
  return true;
}

template <typename T, int D, int NTB, int R, bool O32>
hipError_t launch_cases(int norm, int rot, const HeadParams &p, int tb, const dim3 &grid, const dim3 &block, size_t lds,
                        hipStream_t s) {
#define LUX3D_HEAD_CASE(NORM_, ROT_)                                                                          \
  if (norm == NORM_ && rot == ROT_) {                                                                         \
    hipLaunchKernelGGL((head_kernel<T, D, NORM_, ROT_, R, NTB, O32>), grid, block, lds, s, p, tb);            \
    return hipGetLastError();                                                                                 \
  }
  LUX3D_HEAD_CASE(HN_LN, HR_R1_TAB) LUX3D_HEAD_CASE(HN_LN, HR_R1_POS)
  LUX3D_HEAD_CASE(HN_NONE, HR_R1_TAB) LUX3D_HEAD_CASE(HN_NONE, HR_R1_POS)
  LUX3D_HEAD_CASE(HN_LN, HR_NONE)
  LUX3D_HEAD_CASE(HN_RMS, HR_NONE)
  LUX3D_HEAD_CASE(HN_L2, HR_NONE) LUX3D_HEAD_CASE(HN_L2, HR_R2_TAB) LUX3D_HEAD_CASE(HN_L2, HR_R2_COORD)
  LUX3D_HEAD_CASE(HN_NONE, HR_R2_TAB) LUX3D_HEAD_CASE(HN_NONE, HR_R2_COORD)
  LUX3D_HEAD_CASE(HN_NONE, HR_R3_TAB)
  LUX3D_HEAD_CASE(HN_NONE, HR_NONE)
#undef LUX3D_HEAD_CASE
  return hipErrorInvalidValue;
}

template <typename T, int D, int NTB, int R>
hipError_t launch_dn(int norm, int rot, const HeadParams &p0, hipStream_t s) {
  const int64_t tokens = p0.B * p0.N;
  constexpr int LPR = D / 8;
  // Whole heads per pass: threads = k*H*LPR rounded to wavefronts, <= 256.
  const int64_t hl = p0.H * LPR;
  int64_t k = hl >= 256 ? 1 : 256 / hl;
  int64_t threads = ((k * hl + 63) / 64) * 64;
  if (threads > 256) threads = 256;
  const int64_t ipp = threads / LPR;
  int64_t tb = (R * ipp) / p0.H;
  // more heads than R passes of a workgroup hold (H * D / 8 > 256 R): the
  // generic kernel, one wavefront per row
  if (tb < 1) {
    if (p0.B * p0.H * p0.N > INT32_MAX / 2) return hipErrorInvalidValue;
    return launch_any<T>(norm, rot, p0, s);
  }
  HeadParams p = p0;
  div_magic(p.H, p.div_h_m, p.div_h_s);
  div_magic(p.N, p.div_n_m, p.div_n_s);
  size_t lds = rot != HR_NONE ? (size_t)2 * tb * D * sizeof(float) : 0;
  // resident-workgroup cap (lds_for_occupancy), measured in one process with
  // the cap on and off: the VGGT D = 64 f32 rotation from positions at 6
  // per CU (configs[1] QK LayerNorm + RoPE in f32: 30.1 against 30.5 us);
  // the 2-byte form is faster uncapped (17.13 against 17.36 us), and the
  // unrotated D = 128 rows measure even.
  if (D == 64 && T::bytes == 4 && threads == 256 && rot == HR_R1_POS) lds = lds_for_occupancy(s, 6, lds);
  const dim3 grid((unsigned)((tokens + tb - 1) / tb), NTB == 2 ? 1u : (unsigned)p.ntens), block((unsigned)threads);
  if (offsets_fit_32(p, T::bytes)) return launch_cases<T, D, NTB, R, true>(norm, rot, p, (int)tb, grid, block, lds, s);
  return launch_cases<T, D, NTB, R, false>(norm, rot, p, (int)tb, grid, block, lds, s);
}

// q and k share a workgroup for D = 128 (measured: configs[2] RMS and
// configs[3] L2+RoPE gain 7-9%); for D = 64 one tensor per workgroup is
// faster. Rows per thread R: 1 for f32, 2 for 2-byte types,
// and 4 for 2-byte D = 128 rows without a rotation (configs[2] RMS heads:
// 13.0 against 14.0 us with R = 2; with a rotation the phase staging grows
// with R, and configs[3] L2 + 3D RoPE takes 140.7 against 133.3 us).
template <typename T, int D>
hipError_t launch_d(int norm, int rot, const HeadParams &p, hipStream_t s) {
  const int64_t tokens = p.B * p.N;
  if (tokens <= 0 || p.H <= 0) return hipSuccess;
  if (tokens > INT32_MAX || p.H > 4096) return hipErrorInvalidValue;
  constexpr int R = T::bytes == 4 ? 1 : 2;
  if constexpr (T::bytes == 2 && D == 128) {
    if (rot == HR_NONE) {
      if (p.ntens == 2) return launch_dn<T, D, 2, 4>(norm, rot, p, s);
      return launch_dn<T, D, 1, 4>(norm, rot, p, s);
    }
  }
  if (D == 128 && p.ntens == 2) return launch_dn<T, D, 2, R>(norm, rot, p, s);
  return launch_dn<T, D, 1, R>(norm, rot, p, s);
}

template <typename T>
hipError_t launch_t(int norm, int rot, const HeadParams &p, hipStream_t s) {
  if (p.vec && p.D == 64) return launch_d<T, 64>(norm, rot, p, s);
  if (p.vec && p.D == 128) return launch_d<T, 128>(norm, rot, p, s);
  if (p.B * p.H * p.N > INT32_MAX / 2) return hipErrorInvalidValue;
  return launch_any<T>(norm, rot, p, s);
}

// ---- table builders ---------------------------------------------------------

struct FreqArgs { float f[64]; };

__global__ __launch_bounds__(256) void rope2d_tables_kernel_args(const void *pos, int pos_dt,
                                                                 int64_t psB, int64_t psN,
                                                                 int64_t psC, int64_t N, int64_t D,
                                                                 int64_t total, FreqArgs fa,
                                                                 float *cos_full, float *sin_alt) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int64_t tok = e / D, j = e % D;
  const int64_t b = tok / N, n = tok % N;
  const int64_t half = D / 2, quarter = D / 4;
  const int64_t axis = j / half, jj = j % half;
  const uint32_t pv = (uint32_t)load_index(pos, pos_dt, b * psB + n * psN + axis * psC);
  const float ang = (float)pv * fa.f[jj % quarter];
  float sv, cv;
  sincosf(ang, &sv, &cv);
  cos_full[e] = cv;
  sin_alt[e] = jj < quarter ? -sv : sv;
}

__global__ __launch_bounds__(256) void rope3d_tables_kernel(const int32_t *coords, int64_t csN,
                                                            int64_t csC, int64_t half, int fd,
                                                            int64_t total, FreqArgs fa, float *cos,
                                                            float *sin) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int64_t n = e / half, i = e % half;
  float ang = 0.f;
  if (i < 3 * fd) ang = (float)coords[n * csN + (i / fd) * csC] * fa.f[i % fd];
  float sv, cv;
  sincosf(ang, &sv, &cv);
  cos[e] = cv;
  sin[e] = sv;
}

}  // namespace

hipError_t launch_heads(int norm, int rot, int dt, const HeadParams &p, hipStream_t s) {
  switch (dt) {
    case LUX3D_F32: return launch_t<F32>(norm, rot, p, s);
    case LUX3D_BF16: return launch_t<BF16>(norm, rot, p, s);
    case LUX3D_F16: return launch_t<F16>(norm, rot, p, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_rope2d_tables(const void *pos, int pos_dt, int64_t psB, int64_t psN, int64_t psC,
                                int64_t B, int64_t N, int64_t D, const float *inv_freq,
                                float *cos_full, float *sin_alt, hipStream_t s) {
  const int64_t total = B * N * D;
  if (total <= 0) return hipSuccess;
  FreqArgs fa{};
  for (int64_t k = 0; k < D / 4 && k < 64; ++k) fa.f[k] = inv_freq[k];
  hipLaunchKernelGGL(rope2d_tables_kernel_args, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     pos, pos_dt, psB, psN, psC, N, D, total, fa, cos_full, sin_alt);
  return hipGetLastError();
}

hipError_t launch_rope3d_tables(const int32_t *coords, int64_t csN, int64_t csC, int64_t N,
                                int64_t half, int64_t fd, const float *freq, float *cos, float *sin,
                                hipStream_t s) {
  const int64_t total = N * half;
  if (total <= 0) return hipSuccess;
  FreqArgs fa{};
  for (int64_t k = 0; k < fd && k < 64; ++k) fa.f[k] = freq[k];
  hipLaunchKernelGGL(rope3d_tables_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     coords, csN, csC, half, (int)fd, total, fa, cos, sin);
  return hipGetLastError();
}

}  // namespace lux3d
