// ceiling.hip -- copy kernels that move exactly the bytes of a fused op, with
// no arithmetic, for bench.py's per-op bandwidth ceiling. Measurement code
// only (liblux3d_ceiling.so); it is not part of the C ABI in
// include/lux3d_fused.h and nothing in liblux3d_fused.so uses it.
//
// Three forms:
//  - streams: NIN contiguous inputs and NOUT contiguous outputs, one 16-byte
//    chunk per thread per stream (the activation kernels' layout); inputs and
//    outputs may differ in size (Q8_0 dequant reads 34-byte blocks and writes
//    twice as many bytes);
//  - rows: the row kernels' layout -- a row of `row_bytes` owned by TPR
//    threads, thread t holding 16-byte units c*TPR + t (c < NC), 256-thread
//    workgroups of whole rows (or one row per workgroup when TPR is 128 /
//    256 and the op runs a row per workgroup). The row kernels move 16-byte
//    units for every dtype (an f32 chunk is two 16-byte halves TPR units
//    apart), so f32 rows are copied as 16-byte units with twice the chunk
//    count;
//  - heads: the head kernels' layout -- [B, H, N, D] views with any outer
//    strides, D / 8 lanes per head row, R rows per thread as the kernel
//    runs them (f32: 1, its lane l holding 16 bytes at 16 l of each half
//    row; 2-byte types: 2, or 4 for unrotated D = 128 rows), workgroups of `tb` consecutive tokens x all heads, q and k in
//    grid.y (or both in one workgroup, as the D = 128 kernels do).
//  - best: the fastest plain copy this file can offer at a size, for the
//    question "how close to the HBM peak can anything get here": NIN
//    contiguous input streams and NOUT output streams in three launch forms
//    (one-shot grids of CPT chunks per thread; persistent grids that stride
//    over tiles; persistent grids that load the next tile before storing the
//    current one), at 256, 512 or 1024 threads per workgroup.
// Every output word is the XOR of the loaded words that map to it, so no
// load can be dropped by the compiler.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 ld(const char *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}
__device__ __forceinline__ void st(char *p, u32x4 v) { __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(p)); }

struct Streams {
  const char *in[4];
  char *out[4];
  int64_t in_chunks, out_chunks;  // 16-byte chunks per input / output stream
};

template <int NIN, int NOUT>
__global__ __launch_bounds__(256) void streams_kernel(Streams s) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  if (i < s.in_chunks) {
#pragma unroll
    for (int k = 0; k < NIN; ++k) acc ^= ld(s.in[k] + i * 16);
  }
  if (i < s.out_chunks) {
#pragma unroll
    for (int k = 0; k < NOUT; ++k) st(s.out[k] + i * 16, acc);
  }
}

struct Rows {
  const char *in[4];
  char *out[4];
  int64_t rows, row_bytes;
};

template <int TPR, int NC, int NIN, int NOUT, int BLOCK>
__global__ __launch_bounds__(BLOCK) void rows_kernel(Rows p) {
  constexpr int RPB = BLOCK / TPR;
  const int t = threadIdx.x % TPR;
  int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const bool live = row < p.rows;
  row = live ? row : p.rows - 1;
  u32x4 v[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) v[c] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < NIN; ++k) {
    const char *r = p.in[k] + row * p.row_bytes;
#pragma unroll
    for (int c = 0; c < NC; ++c) v[c] ^= ld(r + (int64_t)(c * TPR + t) * 16);
  }
  if (!live) return;
#pragma unroll
  for (int k = 0; k < NOUT; ++k) {
    char *r = p.out[k] + row * p.row_bytes;
#pragma unroll
    for (int c = 0; c < NC; ++c) st(r + (int64_t)(c * TPR + t) * 16, v[c]);
  }
}

struct Heads {
  const char *x[2];
  char *y[2];
  int64_t sB, sH, sN, oB, oH, oN;  // element strides (input, output)
  int64_t B, H, N;
  int ntens, tb;
};

// EB: element bytes; D: head dim; R: rows per thread; NTB: tensors per workgroup
template <int EB, int D, int R, int NTB>
__global__ __launch_bounds__(256) void heads_kernel(Heads p) {
  // CB: bytes per lane per row; f32 rows in two halves of D / 2 elements,
  // lane l holding the 16 bytes at 16 l of each (HS apart)
  constexpr int LPR = D / 8, CB = 8 * EB, HS = D * 2;
  const int lane = threadIdx.x % LPR, ipp = blockDim.x / LPR;
  // token and head counts below 2^31 (checked on the host): 32-bit indices
  const uint32_t H = (uint32_t)p.H, N = (uint32_t)p.N, ntok = (uint32_t)(p.B * p.N);
  const uint32_t tok0 = blockIdx.x * (uint32_t)p.tb, items = (uint32_t)p.tb * H;
  int64_t xo[R], yo[R];
  bool live[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t it = (uint32_t)(r * ipp) + threadIdx.x / LPR;
    uint32_t t = it / H, h = it - t * H, tok = tok0 + t;
    live[r] = it < items && tok < ntok;
    if (!live[r]) { h = 0; tok = tok0; }
    const uint32_t b = tok / N, n = tok - b * N;
    xo[r] = ((int64_t)b * p.sB + (int64_t)h * p.sH + (int64_t)n * p.sN) * EB + lane * 16;
    yo[r] = ((int64_t)b * p.oB + (int64_t)h * p.oH + (int64_t)n * p.oN) * EB + lane * 16;
  }
  u32x4 v[NTB][R][CB / 16];
#pragma unroll
  for (int q = 0; q < NTB; ++q) {
    const char *x = p.x[NTB == 1 ? blockIdx.y : q];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int h = 0; h < CB / 16; ++h) v[q][r][h] = ld(x + xo[r] + h * HS);
  }
#pragma unroll
  for (int q = 0; q < NTB; ++q) {
    char *y = p.y[NTB == 1 ? blockIdx.y : q];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (live[r])
#pragma unroll
        for (int h = 0; h < CB / 16; ++h) st(y + yo[r] + h * HS, v[q][r][h]);
  }
}

// ---- best: plain copies in three launch forms ------------------------------
// A tile is BLOCK * CPT consecutive 16-byte chunks of every stream; thread t
// of a workgroup moves chunks t, t + BLOCK, ... of its tile, so each load or
// store instruction of a wavefront covers 1 KiB of contiguous memory.
struct Best {
  const char *in[4];
  char *out[4];
  int64_t in_chunks, out_chunks;  // 16-byte chunks per input / output stream
  int64_t tiles;                  // ceil(max(in_chunks, out_chunks) / (BLOCK * CPT))
  int64_t full_tiles;             // tiles wholly inside every stream: min(in, out) / (BLOCK * CPT)
};

// Whole tiles (every chunk of the tile inside every stream) move
// unconditionally; only the last tiles check each chunk.
template <int NIN, int CPT, int BLOCK>
__device__ __forceinline__ void best_load(const Best &s, int64_t tile, u32x4 (&v)[CPT]) {
  const int64_t i0 = tile * CPT * BLOCK + threadIdx.x;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    v[c] = ld(s.in[0] + (i0 + c * BLOCK) * 16);
#pragma unroll
    for (int k = 1; k < NIN; ++k) v[c] ^= ld(s.in[k] + (i0 + c * BLOCK) * 16);
  }
}

// s_waitcnt immediates (gfx9 encoding: vmcnt in bits 3:0 and 15:14,
// expcnt 6:4, lgkmcnt 11:8; the counters not waited on at their maximum)
constexpr int kWaitVm0 = 0x0F70;  // vmcnt(0)
constexpr int kWaitVm1 = 0x0F71;  // vmcnt(1)

// THROTTLE 0: the stores issue back to back; 1: each store waits until
// the wavefront has no other memory operation outstanding (one store in
// flight per wavefront); 2: at most two stores in flight.
template <int NOUT, int CPT, int BLOCK, int THROTTLE = 0>
__device__ __forceinline__ void best_store(const Best &s, int64_t tile, const u32x4 (&v)[CPT]) {
  const int64_t i0 = tile * CPT * BLOCK + threadIdx.x;
#pragma unroll
  for (int c = 0; c < CPT; ++c)
#pragma unroll
    for (int k = 0; k < NOUT; ++k) {
      if (THROTTLE == 1) __builtin_amdgcn_s_waitcnt(kWaitVm0);
      if (THROTTLE == 2) __builtin_amdgcn_s_waitcnt(kWaitVm1);
      st(s.out[k] + (i0 + c * BLOCK) * 16, v[c]);
    }
}

// The last, partial tile: one chunk at a time (no register array, so the
// tail path does not raise the kernel's register count).
template <int NIN, int NOUT, int CPT, int BLOCK>
__device__ __forceinline__ void best_tile_checked(const Best &s, int64_t tile) {
  const int64_t i0 = tile * CPT * BLOCK + threadIdx.x;
#pragma unroll 1
  for (int c = 0; c < CPT; ++c) {
    const int64_t i = i0 + c * BLOCK;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (i < s.in_chunks)
      for (int k = 0; k < NIN; ++k) v ^= ld(s.in[k] + i * 16);
    if (i < s.out_chunks)
      for (int k = 0; k < NOUT; ++k) st(s.out[k] + i * 16, v);
  }
}

// FORM 0: one-shot (a workgroup per tile); 1: persistent, striding over the
// tiles; 2: persistent, the next tile's loads issued before this tile's
// stores (two register sets, the loop unrolled by two so neither is copied);
// 3 / 4: forms 1 / 0 with one store in flight per wavefront (THROTTLE 1);
// 5 / 6: forms 1 / 0 with two (THROTTLE 2).
// `full` tiles (below s.full_tiles) lie wholly inside every stream.
template <int NIN, int NOUT, int CPT, int BLOCK, int FORM>
__global__ __launch_bounds__(BLOCK) void best_kernel(Best s) {
  constexpr int TH = FORM >= 5 ? 2 : FORM >= 3 ? 1 : 0;
  if constexpr (FORM == 0 || FORM == 4 || FORM == 6) {
    if (blockIdx.x < s.full_tiles) {
      u32x4 v[CPT];
      best_load<NIN, CPT, BLOCK>(s, blockIdx.x, v);
      best_store<NOUT, CPT, BLOCK, TH>(s, blockIdx.x, v);
    } else {
      best_tile_checked<NIN, NOUT, CPT, BLOCK>(s, blockIdx.x);
    }
  } else if constexpr (FORM == 1 || FORM == 3 || FORM == 5) {
    int64_t t = blockIdx.x;
    for (; t < s.full_tiles; t += gridDim.x) {
      u32x4 v[CPT];
      best_load<NIN, CPT, BLOCK>(s, t, v);
      best_store<NOUT, CPT, BLOCK, TH>(s, t, v);
    }
    for (; t < s.tiles; t += gridDim.x) best_tile_checked<NIN, NOUT, CPT, BLOCK>(s, t);
  } else {
    const int64_t g = gridDim.x;
    int64_t t = blockIdx.x;
    if (t < s.full_tiles) {
      u32x4 a[CPT], b[CPT];
      best_load<NIN, CPT, BLOCK>(s, t, a);
      for (;;) {
        const bool more_b = t + g < s.full_tiles;
        if (more_b) best_load<NIN, CPT, BLOCK>(s, t + g, b);
        best_store<NOUT, CPT, BLOCK>(s, t, a);
        t += g;
        if (!more_b) break;
        const bool more_a = t + g < s.full_tiles;
        if (more_a) best_load<NIN, CPT, BLOCK>(s, t + g, a);
        best_store<NOUT, CPT, BLOCK>(s, t, b);
        t += g;
        if (!more_a) break;
      }
    }
    for (; t < s.tiles; t += g) best_tile_checked<NIN, NOUT, CPT, BLOCK>(s, t);
  }
}

int status(hipError_t e) { return e == hipSuccess ? 0 : -5; }

}  // namespace

extern "C" {

// nin / nout in 1..4; in_bytes / out_bytes per stream, multiples of 16.
int lux3d_ceiling_streams(const void *const *in, int nin, void *const *out, int nout, int64_t in_bytes,
                          int64_t out_bytes, void *stream) {
  if (nin < 1 || nin > 4 || nout < 1 || nout > 4 || in_bytes % 16 || out_bytes % 16) return -6;
  Streams s{};
  for (int k = 0; k < nin; ++k) s.in[k] = static_cast<const char *>(in[k]);
  for (int k = 0; k < nout; ++k) s.out[k] = static_cast<char *>(out[k]);
  s.in_chunks = in_bytes / 16;
  s.out_chunks = out_bytes / 16;
  const int64_t n = s.in_chunks > s.out_chunks ? s.in_chunks : s.out_chunks;
  if (n == 0) return 0;
  const dim3 grid((unsigned)((n + 255) / 256));
  hipStream_t st = static_cast<hipStream_t>(stream);
#define LUX3D_STREAMS(I, O)                                                    \
  if (nin == I && nout == O) {                                                 \
    hipLaunchKernelGGL((streams_kernel<I, O>), grid, dim3(256), 0, st, s);     \
    return status(hipGetLastError());                                          \
  }
  LUX3D_STREAMS(1, 1) LUX3D_STREAMS(2, 1) LUX3D_STREAMS(2, 2) LUX3D_STREAMS(1, 2)
#undef LUX3D_STREAMS
  return -6;
}

// Contiguous rows of row_bytes moved as 16-byte units (the row kernels'
// unit for every dtype); tpr 64 / 128 / 256; row_per_block: one row per
// workgroup of tpr threads (else 256-thread workgroups of 256 / tpr rows).
// row_bytes must be tpr * nc * 16 for nc in 1..8.
int lux3d_ceiling_rows(const void *const *in, int nin, void *const *out, int nout, int64_t rows, int64_t row_bytes,
                       int tpr, int row_per_block, void *stream) {
  if (rows <= 0) return 0;
  if (tpr != 64 && tpr != 128 && tpr != 256) return -6;
  if (row_bytes % ((int64_t)tpr * 16)) return -6;
  const int nc = (int)(row_bytes / ((int64_t)tpr * 16));
  if (nc < 1 || nc > 8) return -6;
  Rows p{};
  for (int k = 0; k < nin; ++k) p.in[k] = static_cast<const char *>(in[k]);
  for (int k = 0; k < nout; ++k) p.out[k] = static_cast<char *>(out[k]);
  p.rows = rows;
  p.row_bytes = row_bytes;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int block = row_per_block ? tpr : 256;
  const dim3 grid((unsigned)((rows + block / tpr - 1) / (block / tpr)));
#define LUX3D_ROWS(TPR_, NC_, I, O, BLK)                                                          \
  if (tpr == TPR_ && nc == NC_ && nin == I && nout == O && block == BLK) {                        \
    hipLaunchKernelGGL((rows_kernel<TPR_, NC_, I, O, BLK>), grid, dim3(BLK), 0, st, p);           \
    return status(hipGetLastError());                                                             \
  }
#define LUX3D_ROWS_IO(TPR_, NC_, BLK)                                                              \
  LUX3D_ROWS(TPR_, NC_, 1, 1, BLK) LUX3D_ROWS(TPR_, NC_, 2, 1, BLK) LUX3D_ROWS(TPR_, NC_, 2, 2, BLK)
#define LUX3D_ROWS_NC(TPR_, BLK)                                                                   \
  LUX3D_ROWS_IO(TPR_, 1, BLK) LUX3D_ROWS_IO(TPR_, 2, BLK) LUX3D_ROWS_IO(TPR_, 3, BLK)              \
  LUX3D_ROWS_IO(TPR_, 4, BLK) LUX3D_ROWS_IO(TPR_, 6, BLK) LUX3D_ROWS_IO(TPR_, 8, BLK)
  LUX3D_ROWS_NC(64, 256) LUX3D_ROWS_NC(128, 256) LUX3D_ROWS_NC(256, 256) LUX3D_ROWS_NC(128, 128)
#undef LUX3D_ROWS_NC
#undef LUX3D_ROWS_IO
#undef LUX3D_ROWS
  return -6;
}

// q, k: [B, H, N, D] views (element strides in_s = {sB, sH, sN}, unit inner
// stride) -> contiguous-or-strided outputs (out_s); k / ko may be NULL.
// D 64 / 128; elem_bytes 2 / 4; both_in_one: q and k in one workgroup;
// rows_per_thread: the head kernel's R (0: 1 for f32, 2 for 2-byte types;
// 4 for the 2-byte D = 128 rows without a rotation).
// Workgroup shape as the head kernels: whole heads per pass, tb tokens.
int lux3d_ceiling_heads(const void *q, const void *k, void *qo, void *ko, int64_t B, int64_t H, int64_t N, int64_t D,
                        int elem_bytes, const int64_t *in_s, const int64_t *out_s, int both_in_one,
                        int rows_per_thread, void *stream) {
  if (B * N <= 0 || H <= 0) return 0;
  if ((D != 64 && D != 128) || (elem_bytes != 2 && elem_bytes != 4)) return -6;
  if (B * N >= (int64_t(1) << 31) || H > 4096) return -6;
  const int ntens = k ? 2 : 1;
  const int lpr = (int)(D / 8), r = rows_per_thread > 0 ? rows_per_thread : (elem_bytes == 4 ? 1 : 2);
  if (r != 1 && r != 2 && r != 4) return -6;
  const int64_t hl = H * lpr;
  const int64_t kk = hl >= 256 ? 1 : 256 / hl;
  int64_t threads = ((kk * hl + 63) / 64) * 64;
  if (threads > 256) threads = 256;
  const int64_t ipp = threads / lpr, tb = (r * ipp) / H;
  if (tb < 1) return -6;
  Heads p{};
  p.x[0] = static_cast<const char *>(q);
  p.x[1] = static_cast<const char *>(k);
  p.y[0] = static_cast<char *>(qo);
  p.y[1] = static_cast<char *>(ko);
  p.sB = in_s[0]; p.sH = in_s[1]; p.sN = in_s[2];
  p.oB = out_s[0]; p.oH = out_s[1]; p.oN = out_s[2];
  p.B = B; p.H = H; p.N = N; p.ntens = ntens; p.tb = (int)tb;
  const bool two = both_in_one && ntens == 2;
  const dim3 grid((unsigned)((B * N + tb - 1) / tb), two ? 1u : (unsigned)ntens), block((unsigned)threads);
  hipStream_t st = static_cast<hipStream_t>(stream);
#define LUX3D_HEADS(EB, D_, R_, NTB)                                                         \
  if (elem_bytes == EB && D == D_ && r == R_ && (two ? 2 : 1) == NTB) {                    \
    hipLaunchKernelGGL((heads_kernel<EB, D_, R_, NTB>), grid, block, 0, st, p);            \
    return status(hipGetLastError());                                                      \
  }
  LUX3D_HEADS(2, 64, 2, 1) LUX3D_HEADS(2, 64, 2, 2) LUX3D_HEADS(2, 128, 2, 1) LUX3D_HEADS(2, 128, 2, 2)
  LUX3D_HEADS(4, 64, 1, 1) LUX3D_HEADS(4, 64, 1, 2) LUX3D_HEADS(4, 128, 1, 1) LUX3D_HEADS(4, 128, 1, 2)
  LUX3D_HEADS(2, 128, 4, 1) LUX3D_HEADS(2, 128, 4, 2)
#undef LUX3D_HEADS
  return -6;
}

// Plain copy of nin input streams of in_bytes each into nout output streams
// of out_bytes each (multiples of 16; nin / nout: 1/1, 2/1, 2/2, 1/2), in
// launch form `form` (0 one-shot, 1 persistent strided, 2 persistent with
// the next tile prefetched; 3 / 4 = 1 / 0 with one store in flight per
// wavefront, 5 / 6 = 1 / 0 with two), cpt 16-byte chunks per thread per tile (1, 2,
// 4, 8), block threads per workgroup (256, 512, 1024). Persistent forms run
// `grid` workgroups (at most the tile count); one-shot forms ignore it.
int lux3d_ceiling_best(const void *const *in, int nin, void *const *out, int nout, int64_t in_bytes,
                       int64_t out_bytes, int form, int cpt, int block, int grid, void *stream) {
  if (nin < 1 || nin > 2 || nout < 1 || nout > 2 || in_bytes % 16 || out_bytes % 16) return -6;
  if (form < 0 || form > 6 || (cpt != 1 && cpt != 2 && cpt != 4 && cpt != 8)) return -6;
  if (block != 256 && block != 512 && block != 1024) return -6;
  Best s{};
  for (int k = 0; k < nin; ++k) s.in[k] = static_cast<const char *>(in[k]);
  for (int k = 0; k < nout; ++k) s.out[k] = static_cast<char *>(out[k]);
  s.in_chunks = in_bytes / 16;
  s.out_chunks = out_bytes / 16;
  const int64_t n = s.in_chunks > s.out_chunks ? s.in_chunks : s.out_chunks;
  if (n == 0) return 0;
  s.tiles = (n + (int64_t)block * cpt - 1) / ((int64_t)block * cpt);
  s.full_tiles = (s.in_chunks < s.out_chunks ? s.in_chunks : s.out_chunks) / ((int64_t)block * cpt);
  if (s.tiles >= (int64_t(1) << 31)) return -6;
  int64_t g = s.tiles;
  if (form != 0 && form != 4 && form != 6) {
    if (grid < 1) return -6;
    g = grid < s.tiles ? grid : s.tiles;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
#define LUX3D_BEST(I, O, C, B, F)                                                                     \
  if (nin == I && nout == O && cpt == C && block == B && form == F) {                                 \
    hipLaunchKernelGGL((best_kernel<I, O, C, B, F>), dim3((unsigned)g), dim3(B), 0, st, s);           \
    return status(hipGetLastError());                                                                 \
  }
#define LUX3D_BEST_F(I, O, C, B)                                                                       \
  LUX3D_BEST(I, O, C, B, 0) LUX3D_BEST(I, O, C, B, 1) LUX3D_BEST(I, O, C, B, 2) LUX3D_BEST(I, O, C, B, 3)  \
  LUX3D_BEST(I, O, C, B, 4) LUX3D_BEST(I, O, C, B, 5) LUX3D_BEST(I, O, C, B, 6)
#define LUX3D_BEST_B(I, O, C) LUX3D_BEST_F(I, O, C, 256) LUX3D_BEST_F(I, O, C, 512) LUX3D_BEST_F(I, O, C, 1024)
#define LUX3D_BEST_C(I, O) LUX3D_BEST_B(I, O, 1) LUX3D_BEST_B(I, O, 2) LUX3D_BEST_B(I, O, 4) LUX3D_BEST_B(I, O, 8)
  LUX3D_BEST_C(1, 1) LUX3D_BEST_C(2, 1) LUX3D_BEST_C(2, 2) LUX3D_BEST_C(1, 2)
#undef LUX3D_BEST_C
#undef LUX3D_BEST_B
#undef LUX3D_BEST_F
#undef LUX3D_BEST
  return -6;
}

}  // extern "C"
