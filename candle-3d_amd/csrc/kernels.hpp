// kernels.hpp -- host-side launch interface between the C ABI (abi.cpp) and
// the gfx950 kernels. Everything here is internal to liblux3d_fused.so: the
// ABI validates descriptors, resolves strides and dtypes, fills one of these
// parameter blocks and calls the launcher, which picks the kernel variant.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

namespace lux3d {

// ---- row family: LayerNorm / residual+LayerNorm / AdaLN modulate / gate ----
// ROW_GATE_MOD: the gated residual x + h*gate stored as the new residual
// stream, then AdaLN modulate of it (one pass: read x, h; write x', y).
enum RowMode : int { ROW_LN = 0, ROW_RESID_LN = 1, ROW_MODULATE = 2, ROW_GATE = 3, ROW_GATE_MOD = 4 };

// A modulation piece p[s, c] (+ base[c]); dt < 0 when absent.
struct ModPiece {
  const void *p = nullptr;
  int64_t ld = 0;
  int dt = -1;
  const void *base = nullptr;
  int base_dt = -1;
};

struct RowParams {
  const void *x = nullptr;  int64_t x_rs = 0;   // input rows
  const void *a = nullptr;  int64_t a_rs = 0;   // residual branch (RESID) or h (GATE, GATE_MOD)
  void *h = nullptr;        int64_t h_rs = 0;   // RESID, GATE_MOD: stored residual stream
  void *y = nullptr;        int64_t y_rs = 0;   // output rows
  int64_t rows = 0, d = 0;
  float eps = 0.f;
  const void *w = nullptr; int w_dt = -1;       // LN weight
  const void *b = nullptr; int b_dt = -1;       // LN bias
  const void *g = nullptr; int g_dt = -1;       // LayerScale gamma
  const int64_t *seg_off = nullptr;             // [nseg+1] or NULL
  int64_t nseg = 1, rows_per_seg = 1;
  uint32_t rps_m = 0; int rps_s = 0;            // set by the launcher: rows_per_seg's div_magic (dense, rows < 2^31)
  ModPiece shift, scale, gate;
};

// Returns hipSuccess or the launch error. `vec` selects the 16-byte vector
// kernels (the caller has checked alignment and d % 8 == 0).
hipError_t launch_rows(int mode, int dt, const RowParams &p, bool vec, hipStream_t s);

// ---- head family: per-head norm + rotary on [B, H, N, D] views ------------
enum HeadNorm : int { HN_NONE = 0, HN_LN = 1, HN_RMS = 2, HN_L2 = 3 };
enum HeadRot : int {
  HR_NONE = 0,
  HR_R1_TAB = 1,   // VGGT 2D RoPE, [B, N, D] cos / sin_alt tables
  HR_R1_POS = 2,   // VGGT 2D RoPE from integer positions [B, N, 2]
  HR_R2_TAB = 3,   // TRELLIS.2 3D RoPE, [N, D/2] cos / sin tables
  HR_R2_COORD = 4, // TRELLIS.2 3D RoPE from int32 coords [N, 3]
  HR_R3_TAB = 5    // DINOv3 2D RoPE, [N - prefix, D] tables, prefix untouched
};

struct HeadIO {
  const void *x = nullptr; int64_t sB = 0, sH = 0, sN = 0;  // input view
  void *y = nullptr;       int64_t oB = 0, oH = 0, oN = 0;  // output view
  const void *p0 = nullptr; int p0_dt = -1;                 // LN w / RMS w / L2 gamma
  const void *p1 = nullptr; int p1_dt = -1;                 // LN b
};

struct HeadParams {
  HeadIO io[2];
  int ntens = 1;
  int64_t B = 0, H = 0, N = 0, D = 0;
  float eps = 0.f;
  // rotation source
  const void *tab_c = nullptr, *tab_s = nullptr; int tab_dt = -1;
  int64_t tab_sB = 0, tab_sN = 0;               // element (b, n, j) at b*sB + n*sN + j
  const void *pos = nullptr; int pos_dt = -1;
  int64_t pos_sB = 0, pos_sN = 0, pos_sC = 0;   // positions/coords element strides
  float freq[64] = {};
  int nfreq = 0;
  int64_t prefix = 0;
  // Vector path allowed: D is 64 or 128 and every head row and per-channel
  // parameter vector is 16-byte aligned. Otherwise the generic kernel runs.
  bool vec = true;
  // Filled by the launcher: x / H and x / N for x < 2^31 as (x * m) >> s.
  uint32_t div_h_m = 0, div_n_m = 0;
  int div_h_s = 0, div_n_s = 0;
};

hipError_t launch_heads(int norm, int rot, int dt, const HeadParams &p, hipStream_t s);

// ---- table builders ---------------------------------------------------------
hipError_t launch_rope2d_tables(const void *pos, int pos_dt, int64_t psB, int64_t psN,
                                int64_t psC, int64_t B, int64_t N, int64_t D,
                                const float *inv_freq, float *cos_full, float *sin_alt,
                                hipStream_t s);
hipError_t launch_rope3d_tables(const int32_t *coords, int64_t csN, int64_t csC, int64_t N,
                                int64_t half, int64_t fd, const float *freq, float *cos,
                                float *sin, hipStream_t s);

// ---- elementwise -------------------------------------------------------------
enum Act : int { ACT_GELU_ERF = 0, ACT_GELU_TANH = 1, ACT_SILU = 2 };
hipError_t launch_act(int act, int dt, const void *x, void *y, int64_t n, bool vec, hipStream_t s);

hipError_t launch_timestep(const float *t, int64_t n, const float *freqs, int64_t dim,
                           int cos_first, float neg_log_period, float *out, hipStream_t s);

hipError_t launch_dequant_q8_0(const uint8_t *blocks, int64_t nblocks, int out_dt, void *y,
                               bool vec, hipStream_t s);

// ---- Q8_0 quantized linear ---------------------------------------------------
// y[m, n] = sum_k x[m, k] * bf16(q[n, k] * scale[n, k / 32]) (+ bias[n]).
struct Q8GemmParams {
  const void *x = nullptr; int64_t ldx = 0;   // bf16 (or f32 when x_f32) [M, K] rows, 16-byte aligned
  bool x_f32 = false;                         // f32 activations: exact f32 weights, f32 matrix cores
  const int8_t *qs = nullptr;                 // [N, K] contiguous, 16-byte aligned
  const float *scales = nullptr;              // [N, K / 32] contiguous
  const float *bias = nullptr;                // [N] or null
  void *y = nullptr; int64_t ldy = 0;         // [M, N] rows
  int64_t M = 0, N = 0, K = 0;
};
hipError_t launch_q8_0_repack(const uint8_t *blocks, int64_t nblocks, int8_t *qs, float *scales, hipStream_t s);
hipError_t launch_q8_0_gemm(int out_dt, const Q8GemmParams &p, hipStream_t s);

// candle's CPU QMatMul for a Q8_0 weight: x f32 rows quantized to Q8_0
// blocks (int8 values xq [M, K] + the f16 scale widened to f32, xd
// block-major [K/32, ldxd]), then y = sum over blocks of (f32)(isum) * wd * xd in block
// order (+ bias), f32 out. K % 32 == 0; every pointer 16-byte aligned.
struct Q8IntParams {
  const float *x = nullptr; int64_t ldx = 0;  // f32 rows
  int8_t *xq = nullptr;                       // [M, K] contiguous (workspace)
  float *xd = nullptr; int64_t ldxd = 0;      // block-major [K / 32, ldxd >= M rounded up to 64] (workspace)
  const int8_t *qs = nullptr;                 // [N, K] from the repack
  const float *scales = nullptr;              // [N, K / 32]
  const float *bias = nullptr;                // [N] or null
  float *y = nullptr; int64_t ldy = 0;        // [M, N] rows
  int64_t M = 0, N = 0, K = 0;
};
hipError_t launch_q8_0_quantize_rows(const Q8IntParams &p, hipStream_t s);
hipError_t launch_q8_0_int8_gemm(const Q8IntParams &p, hipStream_t s);

// Scaled dot-product attention over [B, H, L, D] views (element strides per
// batch, head and token; unit inner stride). out = softmax(q k^T * scale) v.
// `mfma` selects the matrix-core kernels (D 64 or 128, every row
// 16-byte aligned); otherwise the generic kernel (any float dtype, D <= 512).
struct AttnParams {
  const void *q = nullptr, *k = nullptr, *v = nullptr;
  void *o = nullptr;
  int64_t B = 0, H = 0, Lq = 0, Lk = 0, D = 0;
  int64_t q_sb = 0, q_sh = 0, q_st = 0;
  int64_t k_sb = 0, k_sh = 0, k_st = 0;
  int64_t v_sb = 0, v_sh = 0, v_st = 0;
  int64_t o_sb = 0, o_sh = 0, o_st = 0;
  float scale = 0.f;
  bool mfma = false;
  // exact_p: f32 probabilities and sums whatever the input type (the
  // reference's exact_sdpa_heads); out_f32: out is f32 (exact_p or f32 inputs)
  bool exact_p = false, out_f32 = false;
  // Head norm / rotation of q applied in the Q load (matrix-core paths): q is
  // the raw head view, qpro one of QP_*:
  //   QP_LN_R1 LayerNorm (qw, qb: [D]) + Rope2d tables cos_full / sin_alt_full,
  //            element (b, n, j) at b*tab_sB + n*tab_sN + j
  //   QP_RMS   RMSNorm, weight qw [D]
  //   QP_L2_R2 L2 norm with gamma qw [H, D] + TRELLIS.2 pair rotation, tables
  //            [L, D/2], pair a of token n at n*tab_sN + a
  //   QP_R3    DINOv3 rotate_half rotation, tables [L - prefix, D], row
  //            n - prefix at (n - prefix)*tab_sN; tokens n < prefix unchanged
  int qpro = 0;
  const void *qw = nullptr, *qb = nullptr;
  int qw_dt = -1, qb_dt = -1;
  float eps = 0.f;
  const void *tab_c = nullptr, *tab_s = nullptr;
  int tab_dt = -1;
  int64_t tab_sB = 0, tab_sN = 0;
  int64_t prefix = 0;
  // Key split (nsplit > 1): each (batch, head, query block) runs as nsplit
  // workgroups over consecutive ranges of split_blocks key blocks; each
  // writes its unnormalised partial O and (m, l) to ws_part and the last to
  // arrive (counter ws_cnt[tile], zero on entry and left zero) merges the
  // nsplit partials in split order and writes out.
  int nsplit = 1;
  int64_t split_blocks = 0;
  float *ws_part = nullptr;
  uint32_t *ws_cnt = nullptr;
};
enum { QP_NONE = 0, QP_LN_R1 = 1, QP_RMS = 2, QP_L2_R2 = 3, QP_R3 = 4 };
hipError_t launch_attention(int dt, const AttnParams &p, hipStream_t s);

// TRELLIS.2 sparse voxel ops.
// Coordinate hash (cap: a power of two >= 2n) and neighbour table nbr [n, 27].
hipError_t launch_sparse_map(const int32_t *coords, int64_t n, unsigned long long *keys, int32_t *vals, int64_t cap,
                             int32_t *nbr, int32_t *bad, hipStream_t s);
// The same with the hash table in a per-device static array (no allocation):
// n <= kNoAllocMaxVoxels; the table holds kNoAllocCap slots.
constexpr int64_t kNoAllocMaxVoxels = int64_t(1) << 20;
constexpr int64_t kNoAllocCap = 2 * kNoAllocMaxVoxels;
constexpr int64_t kNoAllocTableBytes = kNoAllocCap * (8 + 4);  // 24 MiB
hipError_t launch_sparse_map_noalloc(const int32_t *coords, int64_t n, int32_t *nbr, int32_t *bad, hipStream_t s);
struct SparseConvParams {
  const float *x = nullptr;       // [n, cin]
  const int32_t *nbr = nullptr;   // [n, 27]
  const float *w = nullptr;       // [27, cout, cin]
  const float *bias = nullptr;    // [cout] or null
  float *out = nullptr;           // [n, cout]
  int64_t n = 0, cin = 0, cout = 0;
  bool mfma = false;              // cin % 16 == 0, 16-byte aligned x and w
};
hipError_t launch_sparse_conv(const SparseConvParams &p, hipStream_t s);
// Rulebook: pairs [27, n, 2] (dst, src) per tap and counts [27] from nbr;
// the conv then runs one gather-GEMM-add pass per tap (p.mfma must hold).
hipError_t launch_sparse_rulebook(const int32_t *nbr, int64_t n, int32_t *pairs, int32_t *counts, hipStream_t s);
hipError_t launch_sparse_conv_rulebook(const SparseConvParams &p, const int32_t *pairs, const int32_t *counts,
                                       hipStream_t s);
// out[m] = src[ids[m]] for m < rows (and m < *count when count is given);
// rows of row_bytes bytes; ids out of range give zero rows.
hipError_t launch_gather_rows(const void *src, int64_t nsrc, const void *ids, bool ids64, int64_t rows,
                              const int32_t *count, void *out, int64_t row_bytes, int32_t *bad, hipStream_t s);
struct C2SParams {
  const int32_t *coords = nullptr;  // [n, 3]
  const void *feats = nullptr;      // [n, C], rows of 8 children x child_row_bytes
  const void *logits = nullptr;     // [n, 8]
  int logits_dt = 0;
  int64_t n = 0, child_row_bytes = 0;
  int32_t *offs = nullptr, *block_sums = nullptr;  // workspace [n], [ceil(n / 1024)]
  int32_t *out_coords = nullptr, *src_rows = nullptr, *count = nullptr;  // [8n, 3], [8n], [1]
  void *out_feats = nullptr;        // [8n, C / 8]
  float *sub = nullptr;             // [n, 8] or null
};
hipError_t launch_c2s(const C2SParams &p, hipStream_t s);

}  // namespace lux3d
