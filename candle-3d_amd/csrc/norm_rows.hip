// norm_rows.hip -- row-reduction kernels for gfx950: LayerNorm (affine or
// not), LayerScale + residual + LayerNorm, AdaLN modulate (dense or ragged
// segments) and the gated residual.
//
// Mapping. A row of D elements is owned by TPR threads (one wavefront for
// TPR = 64, or 2 / 4 wavefronts reducing through LDS for short row counts).
// Thread t holds chunks c = 0..NC-1 of 8 elements at element
// (c*TPR + t)*8, so each load instruction of a wavefront reads 1 KiB (bf16)
// or 2 KiB (f32) of contiguous row data. The whole row stays in registers:
// HBM traffic is exactly one read of every input and one write of every
// output. Statistics are two-pass over the registers (mean, then centred sum
// of squares), reduced with DPP + permlane swaps (no LDS for TPR = 64).
#include "common.hpp"
#include "kernels.hpp"

namespace lux3d {

namespace {

constexpr int kBlock = 256;

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

template <typename T, int TPR, int NC, int MODE, int BLOCK = kBlock>
__global__ __launch_bounds__(BLOCK) void row_kernel(RowParams p) {
  static_assert(BLOCK % TPR == 0, "a block holds whole rows");
  constexpr int RPB = BLOCK / TPR;
  constexpr int EB = T::bytes;
  __shared__ float red_a[BLOCK / 64], red_b[BLOCK / 64];

  const int t = threadIdx.x % TPR;
  int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const bool live = row < p.rows;
  row = uniform(live ? row : p.rows - 1);

  float v[NC][8];
  const char *xr = reinterpret_cast<const char *>(p.x) + row * p.x_rs * EB;
#pragma unroll
  for (int c = 0; c < NC; ++c) Chunk<T>::load(xr + (int64_t)(c * TPR + t) * 8 * EB, v[c]);

  if constexpr (MODE == ROW_GATE) {
    const int64_t seg = segment_of(p.seg_off, p.nseg, p.rows_per_seg, row);
    const char *ar = reinterpret_cast<const char *>(p.a) + row * p.a_rs * EB;
    char *yr = reinterpret_cast<char *>(p.y) + row * p.y_rs * EB;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t idx = (int64_t)(c * TPR + t) * 8;
      float hv[8], g[8];
      Chunk<T>::load(ar + idx * EB, hv);
      mod8(p.gate, seg, idx, 1.f, g);
#pragma unroll
      for (int k = 0; k < 8; ++k) v[c][k] = __fadd_rn(v[c][k], __fmul_rn(hv[k], g[k]));
      if (live) Chunk<T>::store(yr + idx * EB, v[c]);
    }
    return;
  }

  if constexpr (MODE == ROW_RESID_LN) {
    const char *ar = reinterpret_cast<const char *>(p.a) + row * p.a_rs * EB;
    char *hr = reinterpret_cast<char *>(p.h) + row * p.h_rs * EB;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t idx = (int64_t)(c * TPR + t) * 8;
      float av[8], g[8];
      Chunk<T>::load(ar + idx * EB, av);
      param8(p.g, p.g_dt, idx, 1.f, g);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        // LayerScale product and residual add as two roundings (no FMA
        // contraction), exactly broadcast_mul then add.
        const float ls = p.g_dt >= 0 ? __fmul_rn(av[k], g[k]) : av[k];
        v[c][k] = Chunk<T>::round_trip(__fadd_rn(ls, v[c][k]));  // the norm reads the stored h
      }
      if (live) Chunk<T>::store(hr + idx * EB, v[c]);
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
  if constexpr (MODE == ROW_MODULATE) {
    const int64_t seg = segment_of(p.seg_off, p.nseg, p.rows_per_seg, row);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t idx = (int64_t)(c * TPR + t) * 8;
      float sh[8], sc[8], out[8];
      mod8(p.shift, seg, idx, 0.f, sh);
      mod8(p.scale, seg, idx, 0.f, sc);
#pragma unroll
      for (int k = 0; k < 8; ++k) out[k] = (v[c][k] - mean) * rstd * (sc[k] + 1.0f) + sh[k];
      if (p.gate.dt >= 0) {
        float g[8];
        mod8(p.gate, seg, idx, 1.f, g);
#pragma unroll
        for (int k = 0; k < 8; ++k) out[k] = g[k] * out[k] + v[c][k];
      }
      if (live) Chunk<T>::store(yr + idx * EB, out);
    }
  } else {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t idx = (int64_t)(c * TPR + t) * 8;
      float w[8], b[8], out[8];
      param8(p.w, p.w_dt, idx, 1.f, w);
      param8(p.b, p.b_dt, idx, 0.f, b);
#pragma unroll
      for (int k = 0; k < 8; ++k) out[k] = (v[c][k] - mean) * rstd * w[k] + b[k];
      if (live) Chunk<T>::store(yr + idx * EB, out);
    }
  }
}

// Fallback for any D and any alignment: one 256-thread block per row, three
// passes over the row (the second and third hit L2).
template <typename T, int MODE>
__global__ __launch_bounds__(kBlock) void row_kernel_any(RowParams p) {
  __shared__ float red_a[kBlock / 64], red_b[kBlock / 64];
  const int64_t row = blockIdx.x;
  const int64_t seg = segment_of(p.seg_off, p.nseg, p.rows_per_seg, row);
  auto inval = [&](int64_t c) -> float {
    float xv = load1<T>(p.x, row * p.x_rs + c);
    if constexpr (MODE == ROW_RESID_LN) {
      float av = load1<T>(p.a, row * p.a_rs + c);
      const float ls = p.g_dt >= 0 ? __fmul_rn(av, param1(p.g, p.g_dt, c, 1.f)) : av;
      xv = Chunk<T>::round_trip(__fadd_rn(ls, xv));
    }
    return xv;
  };
  auto piece = [&](const ModPiece &m, int64_t c, float dflt) -> float {
    float v = param1(m.p, m.dt, seg * m.ld + c, dflt);
    return m.base_dt >= 0 ? param1(m.base, m.base_dt, c, 0.f) + v : v;
  };
  if constexpr (MODE == ROW_GATE) {
    for (int64_t c = threadIdx.x; c < p.d; c += kBlock) {
      float hv = load1<T>(p.a, row * p.a_rs + c);
      store1<T>(p.y, row * p.y_rs + c, __fadd_rn(load1<T>(p.x, row * p.x_rs + c), __fmul_rn(hv, piece(p.gate, c, 1.f))));
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
    if constexpr (MODE == ROW_RESID_LN) store1<T>(p.h, row * p.h_rs + c, xv);
    float out;
    if constexpr (MODE == ROW_MODULATE) {
      out = (xv - mean) * rstd * (piece(p.scale, c, 0.f) + 1.0f) + piece(p.shift, c, 0.f);
      if (p.gate.dt >= 0) out = piece(p.gate, c, 1.f) * out + xv;
    } else {
      out = (xv - mean) * rstd * param1(p.w, p.w_dt, c, 1.f) + param1(p.b, p.b_dt, c, 0.f);
    }
    store1<T>(p.y, row * p.y_rs + c, out);
  }
}

template <typename T, int MODE>
hipError_t launch_typed(const RowParams &p, bool vec, hipStream_t s) {
  if (p.rows <= 0) return hipSuccess;
  const int64_t chunks = p.d / 8;
  // Layout: threads per row (TPR), chunks per lane (NC) and workgroup size.
  // Short jobs (DINOv2/DINOv3's ~1k tokens) split each row over 2-4
  // wavefronts, one row per workgroup, so the chip is still occupied. For
  // long jobs the layout is the one measured fastest on MI355X at the configs
  // shapes: the fused residual + LayerNorm runs a row on 2 wavefronts with one
  // chunk per lane (configs[1] F1: 18.0 us vs 20.4 us on one wavefront), the
  // gated residual on 4 wavefronts when a row is 256 chunks (configs[2]:
  // 9.9 us vs 10.8 us), the single-stream LayerNorm / modulate on one
  // wavefront with NC chunks per lane (configs[2] modulate: 7.1 us vs 9.4 us).
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
      if (chunks == 256) { ord[0] = 256; ord[1] = 128; ord[2] = 64; }
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
  const int block = row_per_block ? tpr : kBlock;
  const int64_t rpb = block / tpr;
  const dim3 grid((unsigned)((p.rows + rpb - 1) / rpb));
#define LUX3D_ROW_CASE(TPR_, NC_, BLK_)                                                      \
  if (tpr == TPR_ && nc == NC_ && block == BLK_) {                                           \
    hipLaunchKernelGGL((row_kernel<T, TPR_, NC_, MODE, BLK_>), grid, dim3(BLK_), 0, s, p);   \
    return hipGetLastError();                                                                \
  }
  LUX3D_ROW_CASE(64, 1, 256) LUX3D_ROW_CASE(64, 2, 256) LUX3D_ROW_CASE(64, 3, 256)
  LUX3D_ROW_CASE(64, 4, 256) LUX3D_ROW_CASE(64, 8, 256)
  LUX3D_ROW_CASE(128, 1, 256) LUX3D_ROW_CASE(128, 2, 256) LUX3D_ROW_CASE(128, 3, 256) LUX3D_ROW_CASE(128, 4, 256)
  LUX3D_ROW_CASE(128, 1, 128) LUX3D_ROW_CASE(128, 2, 128) LUX3D_ROW_CASE(128, 3, 128) LUX3D_ROW_CASE(128, 4, 128)
  LUX3D_ROW_CASE(256, 1, 256) LUX3D_ROW_CASE(256, 2, 256) LUX3D_ROW_CASE(256, 3, 256) LUX3D_ROW_CASE(256, 4, 256)
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
