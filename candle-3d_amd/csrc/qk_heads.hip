// qk_heads.hip -- per-head normalisation + rotary kernels for gfx950 on
// [B, H, N, D] head views (D = 64 or 128): VGGT QK-LayerNorm + 2D RoPE,
// TripoSG per-head RMSNorm, TRELLIS.2 L2 norm + 3D RoPE, DINOv3 2D RoPE.
//
// Mapping. One workgroup per token (b, n) processes every head of q and k
// for that token: LPR = D/8 lanes own one head row (8 elements each, one
// 16-byte load for bf16), so a wavefront covers 8 (D=64) or 4 (D=128) head
// rows. The token's rotation phases are computed (or read from the caller's
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

__device__ __forceinline__ int64_t load_index(const void *p, int dt, int64_t i) {
  return dt == LUX3D_I64 ? reinterpret_cast<const int64_t *>(p)[i]
                         : (int64_t)reinterpret_cast<const int32_t *>(p)[i];
}

// Phase (C[j], S[j]) of element j for token (b, n): out[j] = y[j]*C[j] +
// y[j ^ M]*S[j]. (DINOv3 prefix tokens never reach this: they are not rotated.)
template <int ROT, int D>
__device__ __forceinline__ void phase(const HeadParams &p, int64_t b, int64_t n, int j, float &C,
                                      float &S) {
  if constexpr (ROT == HR_R1_TAB) {
    const int64_t off = b * p.tab_sB + n * p.tab_sN + j;
    C = param1(p.tab_c, p.tab_dt, off, 1.f);
    S = param1(p.tab_s, p.tab_dt, off, 0.f);
  } else if constexpr (ROT == HR_R1_POS) {
    // Rope2d: half = D/2 per axis (y then x), table row [f, f] of D/4 freqs,
    // sin negated on the first quarter of each half (sin_alt).
    constexpr int half = D / 2, quarter = D / 4;
    const int axis = j / half, jj = j % half;
    const uint32_t pv = (uint32_t)load_index(p.pos, p.pos_dt, b * p.pos_sB + n * p.pos_sN + axis * p.pos_sC);
    const float ang = (float)pv * p.freq[jj % quarter];
    float sv, cv;
    sincosf(ang, &sv, &cv);
    C = cv;
    S = jj < quarter ? -sv : sv;
  } else if constexpr (ROT == HR_R2_TAB || ROT == HR_R2_COORD) {
    const int i = j >> 1;
    float cv, sv;
    if constexpr (ROT == HR_R2_TAB) {
      const int64_t off = n * p.tab_sN + i;
      cv = param1(p.tab_c, p.tab_dt, off, 1.f);
      sv = param1(p.tab_s, p.tab_dt, off, 0.f);
    } else {
      float ang = 0.f;
      if (i < 3 * p.nfreq) {
        const int axis = i / p.nfreq;
        const int32_t cval = reinterpret_cast<const int32_t *>(p.pos)[n * p.pos_sN + axis * p.pos_sC];
        ang = (float)cval * p.freq[i % p.nfreq];
      }
      sincosf(ang, &sv, &cv);
    }
    C = cv;
    S = (j & 1) ? sv : -sv;
  } else if constexpr (ROT == HR_R3_TAB) {
    const int64_t off = (n - p.prefix) * p.tab_sN + j;
    C = param1(p.tab_c, p.tab_dt, off, 1.f);
    const float sv = param1(p.tab_s, p.tab_dt, off, 0.f);
    S = j < D / 2 ? -sv : sv;
  } else {
    C = 1.f;
    S = 0.f;
  }
}

template <typename T, int D, int NORM, int ROT>
__global__ __launch_bounds__(512) void head_kernel(HeadParams p) {
  constexpr int LPR = D / 8;
  constexpr int M = RotPartner<ROT, D>::M;
  constexpr int EB = T::bytes;
  __shared__ float Cs[D], Ss[D];

  const int64_t tok = blockIdx.x;
  const int64_t b = tok / p.N, n = tok % p.N;
  bool rotate = ROT != HR_NONE;
  if constexpr (ROT == HR_R3_TAB) rotate = n >= p.prefix;
  if constexpr (ROT != HR_NONE) {
    if (rotate) {
      for (int j = threadIdx.x; j < D; j += blockDim.x) phase<ROT, D>(p, b, n, j, Cs[j], Ss[j]);
    }
    __syncthreads();
  }

  const int lane = threadIdx.x % LPR;
  const int rows_per_pass = blockDim.x / LPR;
  const int64_t nrows = (int64_t)p.ntens * p.H;
  for (int64_t slot = threadIdx.x / LPR; slot < nrows; slot += rows_per_pass) {
    const int ti = slot >= p.H ? 1 : 0;
    const int64_t h = slot - (int64_t)ti * p.H;
    const HeadIO &io = ti ? p.io[1] : p.io[0];
    float v[8];
    const char *xp = reinterpret_cast<const char *>(io.x) +
                     (b * io.sB + h * io.sH + n * io.sN + lane * 8) * EB;
    Chunk<T>::load(xp, v);

    if constexpr (NORM == HN_LN) {
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) s += v[k];
      const float mean = group_sum<LPR>(s) * (1.0f / D);
      float s2 = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        v[k] -= mean;
        s2 += v[k] * v[k];
      }
      const float rstd = 1.0f / sqrtf(group_sum<LPR>(s2) * (1.0f / D) + p.eps);
      float w[8], bb[8];
      param8(io.p0, io.p0_dt, lane * 8, 1.f, w);
      param8(io.p1, io.p1_dt, lane * 8, 0.f, bb);
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = v[k] * rstd * w[k] + bb[k];
    } else if constexpr (NORM == HN_RMS) {
      float s2 = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) s2 += v[k] * v[k];
      const float r = 1.0f / sqrtf(group_sum<LPR>(s2) * (1.0f / D) + p.eps);
      float w[8];
      param8(io.p0, io.p0_dt, lane * 8, 1.f, w);
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = (v[k] * r) * w[k];
    } else if constexpr (NORM == HN_L2) {
      float s2 = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) s2 += v[k] * v[k];
      const float nrm = fminf(fmaxf(sqrtf(group_sum<LPR>(s2)), 1e-12f), 1.0e30f);
      const float r = 1.0f / nrm;
      const float scale = sqrtf((float)D);
      float g[8];
      param8(io.p0, io.p0_dt, h * D + lane * 8, 1.f, g);
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = ((v[k] * r) * g[k]) * scale;
    }

    if constexpr (ROT != HR_NONE) {
      if (rotate) {
        float pv[8];
        if constexpr (M < 8) {
#pragma unroll
          for (int k = 0; k < 8; ++k) pv[k] = v[k ^ M];
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k) pv[k] = lane_xor<M / 8>(v[k]);
        }
        const int j0 = lane * 8;
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = __fadd_rn(__fmul_rn(v[k], Cs[j0 + k]), __fmul_rn(pv[k], Ss[j0 + k]));
      }
    }

    char *yp = reinterpret_cast<char *>(io.y) + (b * io.oB + h * io.oH + n * io.oN + lane * 8) * EB;
    Chunk<T>::store(yp, v);
  }
}

template <typename T, int D>
hipError_t launch_d(int norm, int rot, const HeadParams &p, hipStream_t s) {
  const int64_t tokens = p.B * p.N;
  if (tokens <= 0) return hipSuccess;
  constexpr int LPR = D / 8;
  int64_t threads = (int64_t)p.ntens * p.H * LPR;
  if (threads <= 0) return hipSuccess;  // no heads: nothing to do
  threads = ((threads + 63) / 64) * 64;
  if (threads > 512) threads = 512;
  const dim3 grid((unsigned)tokens), block((unsigned)threads);
#define LUX3D_HEAD_CASE(NORM_, ROT_)                                                  \
  if (norm == NORM_ && rot == ROT_) {                                                 \
    hipLaunchKernelGGL((head_kernel<T, D, NORM_, ROT_>), grid, block, 0, s, p);       \
    return hipGetLastError();                                                         \
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

template <typename T>
hipError_t launch_t(int norm, int rot, const HeadParams &p, hipStream_t s) {
  if (p.D == 64) return launch_d<T, 64>(norm, rot, p, s);
  if (p.D == 128) return launch_d<T, 128>(norm, rot, p, s);
  return hipErrorInvalidValue;
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
