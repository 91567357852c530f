// abi.cpp -- the extern "C" entry points of liblux3d_fused.so (declared in
// include/lux3d_fused.h). Each entry validates its descriptors on the host
// (shapes, dtypes, strides, alignment), resolves the layout into a kernel
// parameter block and enqueues one kernel on the caller's stream. Nothing
// here synchronises, allocates device memory or touches the GPU before all
// checks have passed, so argument errors are reported without side effects.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <utility>

#include "kernels.hpp"
#include "lux3d_fused.h"

using namespace lux3d;

namespace {

thread_local std::string g_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int ok() {
  g_error.clear();
  return LUX3D_OK;
}

int hip_status(hipError_t e, const char *what) {
  if (e == hipSuccess) return ok();
  return fail(LUX3D_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
}

bool is_float(int dt) { return dt == LUX3D_F32 || dt == LUX3D_BF16 || dt == LUX3D_F16; }
int elem_bytes(int dt) {
  switch (dt) {
    case LUX3D_F32: case LUX3D_I32: return 4;
    case LUX3D_BF16: case LUX3D_F16: return 2;
    case LUX3D_I64: return 8;
    case LUX3D_U8: case LUX3D_I8: return 1;
  }
  return 0;
}
bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int64_t numel(const lux3d_tensor_t *t) {
  int64_t n = 1;
  for (int i = 0; i < t->rank; ++i) n *= t->shape[i];
  return n;
}

// Basic descriptor sanity shared by every tensor argument.
int check_desc(const lux3d_tensor_t *t, const char *fn, const char *name) {
  if (!t) return fail(LUX3D_ERR_NULL, "%s: `%s` is NULL", fn, name);
  if (t->rank < 1 || t->rank > LUX3D_MAX_RANK)
    return fail(LUX3D_ERR_SHAPE, "%s: `%s` has rank %d (1..%d supported)", fn, name, t->rank, LUX3D_MAX_RANK);
  if (elem_bytes(t->dtype) == 0) return fail(LUX3D_ERR_DTYPE, "%s: `%s` has unknown dtype %d", fn, name, t->dtype);
  for (int i = 0; i < t->rank; ++i)
    if (t->shape[i] < 0) return fail(LUX3D_ERR_SHAPE, "%s: `%s` has a negative dim", fn, name);
  if (!t->data && numel(t) > 0) return fail(LUX3D_ERR_NULL, "%s: `%s` has a NULL data pointer", fn, name);
  return LUX3D_OK;
}

bool is_contiguous(const lux3d_tensor_t *t) {
  if (numel(t) == 0) return true;  // no element to address: any strides will do
  int64_t expect = 1;
  for (int i = t->rank - 1; i >= 0; --i) {
    if (t->shape[i] != 1 && t->stride[i] != expect) return false;
    expect *= t->shape[i];
  }
  return true;
}

// View a tensor as [rows, d] rows with a uniform row stride and unit inner
// stride (every contiguous tensor qualifies; so does a row slice).
int rows_view(const lux3d_tensor_t *t, const char *fn, const char *name, int64_t &rows, int64_t &d,
              int64_t &rs) {
  d = t->shape[t->rank - 1];
  if (d > 1 && t->stride[t->rank - 1] != 1)
    return fail(LUX3D_ERR_LAYOUT, "%s: `%s` must have a unit innermost stride", fn, name);
  rows = 1;
  for (int i = 0; i < t->rank - 1; ++i) rows *= t->shape[i];
  if (t->rank == 1) {
    rs = d;
    return LUX3D_OK;
  }
  // innermost non-trivial leading dim gives the row stride; outer ones must nest
  rs = -1;
  int64_t expect = -1;
  for (int i = t->rank - 2; i >= 0; --i) {
    if (t->shape[i] == 1) continue;
    if (rs < 0) {
      rs = t->stride[i];
      expect = rs * t->shape[i];
    } else {
      if (t->stride[i] != expect)
        return fail(LUX3D_ERR_LAYOUT, "%s: `%s` leading dims do not form a uniform row stride", fn, name);
      expect *= t->shape[i];
    }
  }
  if (rs < 0) rs = d;  // a single row
  if (rs < d && rows > 1) return fail(LUX3D_ERR_LAYOUT, "%s: `%s` rows overlap (row stride %lld < %lld)", fn, name,
                                      (long long)rs, (long long)d);
  return LUX3D_OK;
}

// A per-channel parameter vector of length d (any float dtype, contiguous).
int param_vec(const lux3d_tensor_t *p, int64_t d, const char *fn, const char *name, const void *&ptr, int &dt) {
  ptr = nullptr;
  dt = -1;
  if (!p) return LUX3D_OK;
  int r = check_desc(p, fn, name);
  if (r) return r;
  if (!is_float(p->dtype)) return fail(LUX3D_ERR_DTYPE, "%s: `%s` must be f32/bf16/f16", fn, name);
  if (numel(p) != d) return fail(LUX3D_ERR_SHAPE, "%s: `%s` has %lld elements, expected %lld", fn, name,
                                 (long long)numel(p), (long long)d);
  if (!is_contiguous(p)) return fail(LUX3D_ERR_LAYOUT, "%s: `%s` must be contiguous", fn, name);
  ptr = p->data;
  dt = p->dtype;
  return LUX3D_OK;
}

hipStream_t stream_of(lux3d_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// --------------------------------------------------------------------------
// Row family helpers
// --------------------------------------------------------------------------

struct RowView {
  const void *p;
  int64_t rows, d, rs;
};

int row_tensor(const lux3d_tensor_t *t, const char *fn, const char *name, int dt_expect, RowView &v) {
  int r = check_desc(t, fn, name);
  if (r) return r;
  if (!is_float(t->dtype)) return fail(LUX3D_ERR_DTYPE, "%s: `%s` must be f32/bf16/f16", fn, name);
  if (dt_expect >= 0 && t->dtype != dt_expect)
    return fail(LUX3D_ERR_DTYPE, "%s: `%s` dtype %d differs from the input dtype %d", fn, name, t->dtype, dt_expect);
  r = rows_view(t, fn, name, v.rows, v.d, v.rs);
  if (r) return r;
  v.p = t->data;
  return LUX3D_OK;
}

int same_rows(const RowView &a, const RowView &b, const char *fn, const char *name) {
  if (a.rows != b.rows || a.d != b.d)
    return fail(LUX3D_ERR_SHAPE, "%s: `%s` is [%lld, %lld], expected [%lld, %lld]", fn, name, (long long)b.rows,
                (long long)b.d, (long long)a.rows, (long long)a.d);
  return LUX3D_OK;
}

bool vec_ok_rows(std::initializer_list<RowView> vs) {
  for (const RowView &v : vs) {
    if (v.d % 8) return false;
    if (!aligned16(v.p)) return false;
    if (v.rows > 1 && v.rs % 8) return false;
  }
  return true;
}

// Modulation piece [S, C] (or [S, 1, C] / [C]); base [C] optional.
int mod_piece(const lux3d_tensor_t *p, const lux3d_tensor_t *base, int64_t d, const char *fn, const char *name,
              ModPiece &m, int64_t &nseg) {
  m = ModPiece{};
  nseg = 0;
  if (!p) {
    if (base) return fail(LUX3D_ERR_NULL, "%s: `%s_base` given without `%s`", fn, name, name);
    return LUX3D_OK;
  }
  int r = check_desc(p, fn, name);
  if (r) return r;
  if (!is_float(p->dtype)) return fail(LUX3D_ERR_DTYPE, "%s: `%s` must be f32/bf16/f16", fn, name);
  if (p->shape[p->rank - 1] != d)
    return fail(LUX3D_ERR_SHAPE, "%s: `%s` last dim %lld != %lld", fn, name, (long long)p->shape[p->rank - 1],
                (long long)d);
  if (d > 1 && p->stride[p->rank - 1] != 1)
    return fail(LUX3D_ERR_LAYOUT, "%s: `%s` must have a unit innermost stride", fn, name);
  if (p->rank == 1) {
    nseg = 1;
    m.ld = 0;
  } else if (p->rank == 2 || (p->rank == 3 && p->shape[1] == 1)) {
    nseg = p->shape[0];
    m.ld = p->stride[0];
  } else {
    return fail(LUX3D_ERR_SHAPE, "%s: `%s` must be [S, C], [S, 1, C] or [C]", fn, name);
  }
  m.p = p->data;
  m.dt = p->dtype;
  const void *bp = nullptr;
  int bdt = -1;
  r = param_vec(base, d, fn, name, bp, bdt);
  if (r) return r;
  m.base = bp;
  m.base_dt = bdt;
  return LUX3D_OK;
}

bool vec_ok_piece(const ModPiece &m) {
  if (m.dt < 0) return true;
  if (!aligned16(m.p) || (m.ld % 8)) return false;
  if (m.base_dt >= 0 && !aligned16(m.base)) return false;
  return true;
}

// Resolve the segment structure shared by modulate and gate.
int segments(const lux3d_tensor_t *seg_offsets, int64_t rows, int64_t piece_segs, const char *fn, RowParams &p) {
  if (seg_offsets) {
    int r = check_desc(seg_offsets, fn, "seg_offsets");
    if (r) return r;
    if (seg_offsets->dtype != LUX3D_I64) return fail(LUX3D_ERR_DTYPE, "%s: `seg_offsets` must be int64", fn);
    if (seg_offsets->rank != 1 || seg_offsets->shape[0] < 2 || seg_offsets->stride[0] != 1)
      return fail(LUX3D_ERR_SHAPE, "%s: `seg_offsets` must be a contiguous [S+1] vector, S >= 1", fn);
    p.nseg = seg_offsets->shape[0] - 1;
    if (piece_segs != p.nseg && piece_segs != 1)
      return fail(LUX3D_ERR_SHAPE, "%s: modulation has %lld segments but seg_offsets describes %lld", fn,
                  (long long)piece_segs, (long long)p.nseg);
    if (piece_segs == 1) p.nseg = 1;  // one vector broadcast over every segment
    p.seg_off = piece_segs == 1 ? nullptr : reinterpret_cast<const int64_t *>(seg_offsets->data);
    p.rows_per_seg = rows > 0 ? rows : 1;
    return LUX3D_OK;
  }
  p.nseg = piece_segs;
  if (p.nseg < 1) p.nseg = 1;
  if (rows % p.nseg)
    return fail(LUX3D_ERR_SHAPE, "%s: %lld rows do not split into %lld equal segments (pass seg_offsets)", fn,
                (long long)rows, (long long)p.nseg);
  p.rows_per_seg = rows / p.nseg > 0 ? rows / p.nseg : 1;
  return LUX3D_OK;
}

// --------------------------------------------------------------------------
// Head family helpers
// --------------------------------------------------------------------------

// 4-D head view: (dim_b, dim_h, dim_n) name which descriptor dims play B, H, N.
struct HeadView {
  const void *p;
  int64_t B, H, N, D, sB, sH, sN;
  bool vec;  // D is 64 or 128 and the rows (and parameters) are 16-byte aligned
};

int head_tensor(const lux3d_tensor_t *t, const char *fn, const char *name, int ib, int ih, int in,
                HeadView &v) {
  int r = check_desc(t, fn, name);
  if (r) return r;
  if (!is_float(t->dtype)) return fail(LUX3D_ERR_DTYPE, "%s: `%s` must be f32/bf16/f16", fn, name);
  if (t->rank != 4) return fail(LUX3D_ERR_SHAPE, "%s: `%s` must be rank 4", fn, name);
  v.p = t->data;
  v.B = t->shape[ib];
  v.H = t->shape[ih];
  v.N = t->shape[in];
  v.D = t->shape[3];
  v.sB = t->stride[ib];
  v.sH = t->stride[ih];
  v.sN = t->stride[in];
  if (t->stride[3] != 1 && v.D > 1)
    return fail(LUX3D_ERR_LAYOUT, "%s: `%s` must have a unit innermost stride", fn, name);
  if (v.D < 1 || v.D > 8192) return fail(LUX3D_ERR_SHAPE, "%s: head dim %lld out of range [1, 8192]", fn, (long long)v.D);
  const int64_t e = elem_bytes(t->dtype);
  const bool al = aligned16(v.p) && ((v.sB * e) % 16 == 0 || v.B == 1) && ((v.sH * e) % 16 == 0 || v.H == 1) &&
                  ((v.sN * e) % 16 == 0 || v.N == 1);
  // other head dims and unaligned views take the generic kernel
  v.vec = (v.D == 64 || v.D == 128) && al;
  return LUX3D_OK;
}

int same_heads(const HeadView &a, const HeadView &b, const char *fn, const char *name) {
  if (a.B != b.B || a.H != b.H || a.N != b.N || a.D != b.D)
    return fail(LUX3D_ERR_SHAPE, "%s: `%s` shape differs from its input", fn, name);
  return LUX3D_OK;
}

bool param_aligned(const void *p, int dt) { return dt < 0 || aligned16(p); }

// One q/k side: input view, output view and up to two parameter vectors.
int head_side(const lux3d_tensor_t *x, const lux3d_tensor_t *y, const lux3d_tensor_t *p0, int64_t p0_len,
              const lux3d_tensor_t *p1, const char *fn, const char *xn, const char *yn, const char *p0n,
              const char *p1n, int ib, int ih, int in, HeadIO &io, HeadView &xv) {
  int r = head_tensor(x, fn, xn, ib, ih, in, xv);
  if (r) return r;
  HeadView yv;
  r = head_tensor(y, fn, yn, ib, ih, in, yv);
  if (r) return r;
  if ((r = same_heads(xv, yv, fn, yn))) return r;
  if (y->dtype != x->dtype) return fail(LUX3D_ERR_DTYPE, "%s: `%s` dtype differs from `%s`", fn, yn, xn);
  io.x = xv.p;
  io.sB = xv.sB; io.sH = xv.sH; io.sN = xv.sN;
  io.y = const_cast<void *>(yv.p);
  io.oB = yv.sB; io.oH = yv.sH; io.oN = yv.sN;
  if ((r = param_vec(p0, p0_len, fn, p0n, io.p0, io.p0_dt))) return r;
  if ((r = param_vec(p1, xv.D, fn, p1n, io.p1, io.p1_dt))) return r;
  xv.vec = xv.vec && yv.vec && param_aligned(io.p0, io.p0_dt) && param_aligned(io.p1, io.p1_dt);
  return LUX3D_OK;
}

int index_tensor(const lux3d_tensor_t *t, const char *fn, const char *name, int64_t lead, int64_t n, int64_t c,
                 bool allow_i64) {
  int r = check_desc(t, fn, name);
  if (r) return r;
  if (!(t->dtype == LUX3D_I32 || (allow_i64 && t->dtype == LUX3D_I64)))
    return fail(LUX3D_ERR_DTYPE, "%s: `%s` must be int32%s", fn, name, allow_i64 ? " or int64" : "");
  const bool shape_ok = lead > 0 ? (t->rank == 3 && t->shape[0] == lead && t->shape[1] == n && t->shape[2] == c)
                                 : (t->rank == 2 && t->shape[0] == n && t->shape[1] == c);
  if (!shape_ok) return fail(LUX3D_ERR_SHAPE, "%s: `%s` has the wrong shape", fn, name);
  return LUX3D_OK;
}

// Rope2d inverse frequencies, computed exactly as Rope2d::cos_sin does on the
// host (f32 powf), for token_dim d: inv[k] = 1 / base^((2k) / (d/2)).
void rope2d_inv_freq(float base, int64_t d, float *out) {
  const int64_t half = d / 2;
  for (int64_t k = 0; k < d / 4; ++k) out[k] = 1.0f / powf(base, (float)(2 * k) / (float)half);
}

// Trellis2Rope3d frequencies: f[i] = 1 / base^(i / freq_dim) (f32 powf).
int64_t rope3d_freq(float base, int64_t head_dim, float *out) {
  const int64_t fd = head_dim / 2 / 3;
  for (int64_t i = 0; i < fd; ++i) out[i] = 1.0f / powf(base, (float)i / (float)fd);
  return fd;
}

}  // namespace

extern "C" {

int lux3d_abi_version(void) { return LUX3D_ABI_VERSION; }

const char *lux3d_last_error(void) { return g_error.c_str(); }

// ---------------------------------------------------------------------------

int lux3d_layer_norm(const lux3d_tensor_t *x, const lux3d_tensor_t *w, const lux3d_tensor_t *b, float eps,
                     const lux3d_tensor_t *y, lux3d_stream_t stream) {
  const char *fn = "lux3d_layer_norm";
  RowView xv, yv;
  int r;
  if ((r = row_tensor(x, fn, "x", -1, xv))) return r;
  if ((r = row_tensor(y, fn, "y", x->dtype, yv))) return r;
  if ((r = same_rows(xv, yv, fn, "y"))) return r;
  if (!(eps >= 0.f)) return fail(LUX3D_ERR_VALUE, "%s: eps must be >= 0", fn);
  if (xv.d == 0) return fail(LUX3D_ERR_SHAPE, "%s: empty rows", fn);
  RowParams p;
  p.x = xv.p; p.x_rs = xv.rs;
  p.y = const_cast<void *>(yv.p); p.y_rs = yv.rs;
  p.rows = xv.rows; p.d = xv.d; p.eps = eps;
  if ((r = param_vec(w, xv.d, fn, "w", p.w, p.w_dt))) return r;
  if ((r = param_vec(b, xv.d, fn, "b", p.b, p.b_dt))) return r;
  const bool vec = vec_ok_rows({xv, yv}) && (p.w_dt < 0 || aligned16(p.w)) && (p.b_dt < 0 || aligned16(p.b));
  return hip_status(launch_rows(ROW_LN, x->dtype, p, vec, stream_of(stream)), fn);
}

int lux3d_residual_layer_norm(const lux3d_tensor_t *x, const lux3d_tensor_t *a, const lux3d_tensor_t *ls_gamma,
                              const lux3d_tensor_t *w, const lux3d_tensor_t *b, float eps,
                              const lux3d_tensor_t *h_out, const lux3d_tensor_t *y, lux3d_stream_t stream) {
  const char *fn = "lux3d_residual_layer_norm";
  RowView xv, av, hv, yv;
  int r;
  if ((r = row_tensor(x, fn, "x", -1, xv))) return r;
  if ((r = row_tensor(a, fn, "a", x->dtype, av))) return r;
  if ((r = row_tensor(h_out, fn, "h_out", x->dtype, hv))) return r;
  if ((r = row_tensor(y, fn, "y", x->dtype, yv))) return r;
  if ((r = same_rows(xv, av, fn, "a")) || (r = same_rows(xv, hv, fn, "h_out")) || (r = same_rows(xv, yv, fn, "y")))
    return r;
  if (!(eps >= 0.f)) return fail(LUX3D_ERR_VALUE, "%s: eps must be >= 0", fn);
  if (xv.d == 0) return fail(LUX3D_ERR_SHAPE, "%s: empty rows", fn);
  RowParams p;
  p.x = xv.p; p.x_rs = xv.rs;
  p.a = av.p; p.a_rs = av.rs;
  p.h = const_cast<void *>(hv.p); p.h_rs = hv.rs;
  p.y = const_cast<void *>(yv.p); p.y_rs = yv.rs;
  p.rows = xv.rows; p.d = xv.d; p.eps = eps;
  if ((r = param_vec(ls_gamma, xv.d, fn, "ls_gamma", p.g, p.g_dt))) return r;
  if ((r = param_vec(w, xv.d, fn, "w", p.w, p.w_dt))) return r;
  if ((r = param_vec(b, xv.d, fn, "b", p.b, p.b_dt))) return r;
  const bool vec = vec_ok_rows({xv, av, hv, yv}) && (p.g_dt < 0 || aligned16(p.g)) &&
                   (p.w_dt < 0 || aligned16(p.w)) && (p.b_dt < 0 || aligned16(p.b));
  return hip_status(launch_rows(ROW_RESID_LN, x->dtype, p, vec, stream_of(stream)), fn);
}

int lux3d_adaln_modulate(const lux3d_tensor_t *x, const lux3d_tensor_t *seg_offsets, const lux3d_tensor_t *shift,
                         const lux3d_tensor_t *shift_base, const lux3d_tensor_t *scale,
                         const lux3d_tensor_t *scale_base, const lux3d_tensor_t *gate,
                         const lux3d_tensor_t *gate_base, float eps, const lux3d_tensor_t *y,
                         lux3d_stream_t stream) {
  const char *fn = "lux3d_adaln_modulate";
  RowView xv, yv;
  int r;
  if ((r = row_tensor(x, fn, "x", -1, xv))) return r;
  if ((r = row_tensor(y, fn, "y", x->dtype, yv))) return r;
  if ((r = same_rows(xv, yv, fn, "y"))) return r;
  if (!(eps >= 0.f)) return fail(LUX3D_ERR_VALUE, "%s: eps must be >= 0", fn);
  if (xv.d == 0) return fail(LUX3D_ERR_SHAPE, "%s: empty rows", fn);
  if (!shift || !scale) return fail(LUX3D_ERR_NULL, "%s: `shift` and `scale` are required", fn);
  RowParams p;
  int64_t s_sh = 0, s_sc = 0, s_g = 0;
  if ((r = mod_piece(shift, shift_base, xv.d, fn, "shift", p.shift, s_sh))) return r;
  if ((r = mod_piece(scale, scale_base, xv.d, fn, "scale", p.scale, s_sc))) return r;
  if ((r = mod_piece(gate, gate_base, xv.d, fn, "gate", p.gate, s_g))) return r;
  if (s_sh != s_sc || (gate && s_g != s_sh))
    return fail(LUX3D_ERR_SHAPE, "%s: shift/scale/gate have different segment counts", fn);
  if ((r = segments(seg_offsets, xv.rows, s_sh, fn, p))) return r;
  p.x = xv.p; p.x_rs = xv.rs;
  p.y = const_cast<void *>(yv.p); p.y_rs = yv.rs;
  p.rows = xv.rows; p.d = xv.d; p.eps = eps;
  const bool vec = vec_ok_rows({xv, yv}) && vec_ok_piece(p.shift) && vec_ok_piece(p.scale) && vec_ok_piece(p.gate);
  return hip_status(launch_rows(ROW_MODULATE, x->dtype, p, vec, stream_of(stream)), fn);
}

int lux3d_gated_residual(const lux3d_tensor_t *x, const lux3d_tensor_t *h, const lux3d_tensor_t *seg_offsets,
                         const lux3d_tensor_t *gate, const lux3d_tensor_t *gate_base, const lux3d_tensor_t *out,
                         lux3d_stream_t stream) {
  const char *fn = "lux3d_gated_residual";
  RowView xv, hv, ov;
  int r;
  if ((r = row_tensor(x, fn, "x", -1, xv))) return r;
  if ((r = row_tensor(h, fn, "h", x->dtype, hv))) return r;
  if ((r = row_tensor(out, fn, "out", x->dtype, ov))) return r;
  if ((r = same_rows(xv, hv, fn, "h")) || (r = same_rows(xv, ov, fn, "out"))) return r;
  if (!gate) return fail(LUX3D_ERR_NULL, "%s: `gate` is required", fn);
  RowParams p;
  int64_t s_g = 0;
  if ((r = mod_piece(gate, gate_base, xv.d, fn, "gate", p.gate, s_g))) return r;
  if ((r = segments(seg_offsets, xv.rows, s_g, fn, p))) return r;
  p.x = xv.p; p.x_rs = xv.rs;
  p.a = hv.p; p.a_rs = hv.rs;
  p.y = const_cast<void *>(ov.p); p.y_rs = ov.rs;
  p.rows = xv.rows; p.d = xv.d;
  if (xv.d == 0 || xv.rows == 0) return ok();
  const bool vec = vec_ok_rows({xv, hv, ov}) && vec_ok_piece(p.gate);
  return hip_status(launch_rows(ROW_GATE, x->dtype, p, vec, stream_of(stream)), fn);
}

int lux3d_gated_residual_adaln_modulate(const lux3d_tensor_t *x, const lux3d_tensor_t *h,
                                        const lux3d_tensor_t *seg_offsets, const lux3d_tensor_t *gate,
                                        const lux3d_tensor_t *gate_base, const lux3d_tensor_t *shift,
                                        const lux3d_tensor_t *shift_base, const lux3d_tensor_t *scale,
                                        const lux3d_tensor_t *scale_base, float eps, const lux3d_tensor_t *x_out,
                                        const lux3d_tensor_t *y, lux3d_stream_t stream) {
  const char *fn = "lux3d_gated_residual_adaln_modulate";
  RowView xv, hv, xov, yv;
  int r;
  if ((r = row_tensor(x, fn, "x", -1, xv))) return r;
  if ((r = row_tensor(h, fn, "h", x->dtype, hv))) return r;
  if ((r = row_tensor(x_out, fn, "x_out", x->dtype, xov))) return r;
  if ((r = row_tensor(y, fn, "y", x->dtype, yv))) return r;
  if ((r = same_rows(xv, hv, fn, "h")) || (r = same_rows(xv, xov, fn, "x_out")) || (r = same_rows(xv, yv, fn, "y")))
    return r;
  if (!(eps >= 0.f)) return fail(LUX3D_ERR_VALUE, "%s: eps must be >= 0", fn);
  if (xv.d == 0) return fail(LUX3D_ERR_SHAPE, "%s: empty rows", fn);
  if (!shift || !scale) return fail(LUX3D_ERR_NULL, "%s: `shift` and `scale` are required", fn);
  if (xv.rows > 0 && (yv.p == xv.p || yv.p == xov.p))
    return fail(LUX3D_ERR_LAYOUT, "%s: `y` must not alias `x` or `x_out`", fn);
  RowParams p;
  int64_t s_sh = 0, s_sc = 0, s_g = 0;
  if ((r = mod_piece(shift, shift_base, xv.d, fn, "shift", p.shift, s_sh))) return r;
  if ((r = mod_piece(scale, scale_base, xv.d, fn, "scale", p.scale, s_sc))) return r;
  if ((r = mod_piece(gate, gate_base, xv.d, fn, "gate", p.gate, s_g))) return r;
  if (s_sh != s_sc || (gate && s_g != s_sh))
    return fail(LUX3D_ERR_SHAPE, "%s: shift/scale/gate have different segment counts", fn);
  if ((r = segments(seg_offsets, xv.rows, s_sh, fn, p))) return r;
  p.x = xv.p; p.x_rs = xv.rs;
  p.a = hv.p; p.a_rs = hv.rs;
  p.h = const_cast<void *>(xov.p); p.h_rs = xov.rs;
  p.y = const_cast<void *>(yv.p); p.y_rs = yv.rs;
  p.rows = xv.rows; p.d = xv.d; p.eps = eps;
  const bool vec = vec_ok_rows({xv, hv, xov, yv}) && vec_ok_piece(p.shift) && vec_ok_piece(p.scale) &&
                   vec_ok_piece(p.gate);
  return hip_status(launch_rows(ROW_GATE_MOD, x->dtype, p, vec, stream_of(stream)), fn);
}

// ---------------------------------------------------------------------------

namespace {

// Shared body of the two R1 entries.
int qk_rope2d_common(const char *fn, const lux3d_tensor_t *q, const lux3d_tensor_t *q_w, const lux3d_tensor_t *q_b,
                     const lux3d_tensor_t *k, const lux3d_tensor_t *k_w, const lux3d_tensor_t *k_b, float eps,
                     const lux3d_tensor_t *q_out, const lux3d_tensor_t *k_out, HeadParams &p, int &norm) {
  HeadView qv, kv;
  int r;
  if (!q_out) return fail(LUX3D_ERR_NULL, "%s: `q_out` is NULL", fn);
  if ((r = head_side(q, q_out, q_w, q ? q->shape[3] : 0, q_b, fn, "q", "q_out", "q_w", "q_b", 0, 1, 2, p.io[0], qv)))
    return r;
  p.ntens = 1;
  if (k) {
    if (!k_out) return fail(LUX3D_ERR_NULL, "%s: `k_out` is NULL while `k` is given", fn);
    if ((r = head_side(k, k_out, k_w, k->shape[3], k_b, fn, "k", "k_out", "k_w", "k_b", 0, 1, 2, p.io[1], kv)))
      return r;
    if ((r = same_heads(qv, kv, fn, "k"))) return r;
    if (k->dtype != q->dtype) return fail(LUX3D_ERR_DTYPE, "%s: `k` dtype differs from `q`", fn);
    p.ntens = 2;
  }
  // LayerNorm when the weight is given; its bias is optional (a candle
  // LayerNorm without bias); a bias without a weight is an error
  const bool qn = p.io[0].p0_dt >= 0;
  const bool kn = p.ntens == 2 && p.io[1].p0_dt >= 0;
  if (p.ntens == 2 && qn != kn) return fail(LUX3D_ERR_NULL, "%s: q and k must both be normalised or both not", fn);
  if (p.io[0].p1_dt >= 0 && !qn) return fail(LUX3D_ERR_NULL, "%s: LayerNorm bias given without a weight", fn);
  if (p.ntens == 2 && p.io[1].p1_dt >= 0 && !kn)
    return fail(LUX3D_ERR_NULL, "%s: LayerNorm bias given without a weight", fn);
  if (qn && !(eps >= 0.f)) return fail(LUX3D_ERR_VALUE, "%s: eps must be >= 0", fn);
  norm = qn ? HN_LN : HN_NONE;
  p.B = qv.B; p.H = qv.H; p.N = qv.N; p.D = qv.D; p.eps = eps;
  p.vec = qv.vec && (p.ntens == 1 || kv.vec);
  // Rope2d rotates the quarters of each half (attention_math.rs:28-30)
  if (p.D % 4) return fail(LUX3D_ERR_SHAPE, "%s: rope token_dim must be divisible by 4, got %lld", fn, (long long)p.D);
  return LUX3D_OK;
}

// [B, N, D] or [B, 1, N, D] f32/bf16/f16 table with unit inner stride.
int rope2d_table(const lux3d_tensor_t *t, const char *fn, const char *name, int64_t B, int64_t N, int64_t D,
                 int64_t &sB, int64_t &sN) {
  int r = check_desc(t, fn, name);
  if (r) return r;
  if (!is_float(t->dtype)) return fail(LUX3D_ERR_DTYPE, "%s: `%s` must be f32/bf16/f16", fn, name);
  if (t->rank == 3 && t->shape[0] == B && t->shape[1] == N && t->shape[2] == D) {
    sB = t->stride[0]; sN = t->stride[1];
  } else if (t->rank == 4 && t->shape[0] == B && t->shape[1] == 1 && t->shape[2] == N && t->shape[3] == D) {
    sB = t->stride[0]; sN = t->stride[2];
  } else {
    return fail(LUX3D_ERR_SHAPE, "%s: `%s` must be [B, N, D] or [B, 1, N, D] = [%lld, %lld, %lld]", fn, name,
                (long long)B, (long long)N, (long long)D);
  }
  if (t->stride[t->rank - 1] != 1) return fail(LUX3D_ERR_LAYOUT, "%s: `%s` must have a unit innermost stride", fn, name);
  if (B == 1) sB = 0;
  return LUX3D_OK;
}

}  // namespace

int lux3d_qk_layernorm_rope2d(const lux3d_tensor_t *q, const lux3d_tensor_t *q_w, const lux3d_tensor_t *q_b,
                              const lux3d_tensor_t *k, const lux3d_tensor_t *k_w, const lux3d_tensor_t *k_b, float eps,
                              const lux3d_tensor_t *cos_full, const lux3d_tensor_t *sin_alt_full,
                              const lux3d_tensor_t *q_out, const lux3d_tensor_t *k_out, lux3d_stream_t stream) {
  const char *fn = "lux3d_qk_layernorm_rope2d";
  HeadParams p;
  int norm = HN_NONE, r;
  if ((r = qk_rope2d_common(fn, q, q_w, q_b, k, k_w, k_b, eps, q_out, k_out, p, norm))) return r;
  int64_t cB, cN, sB, sN;
  if ((r = rope2d_table(cos_full, fn, "cos_full", p.B, p.N, p.D, cB, cN))) return r;
  if ((r = rope2d_table(sin_alt_full, fn, "sin_alt_full", p.B, p.N, p.D, sB, sN))) return r;
  if (cB != sB || cN != sN || cos_full->dtype != sin_alt_full->dtype)
    return fail(LUX3D_ERR_LAYOUT, "%s: cos_full and sin_alt_full must share layout and dtype", fn);
  p.tab_c = cos_full->data; p.tab_s = sin_alt_full->data; p.tab_dt = cos_full->dtype;
  p.tab_sB = cB; p.tab_sN = cN;
  return hip_status(launch_heads(norm, HR_R1_TAB, q->dtype, p, stream_of(stream)), fn);
}

int lux3d_qk_layernorm_rope2d_pos(const lux3d_tensor_t *q, const lux3d_tensor_t *q_w, const lux3d_tensor_t *q_b,
                                  const lux3d_tensor_t *k, const lux3d_tensor_t *k_w, const lux3d_tensor_t *k_b,
                                  float eps, const lux3d_tensor_t *positions, float base,
                                  const lux3d_tensor_t *q_out, const lux3d_tensor_t *k_out, lux3d_stream_t stream) {
  const char *fn = "lux3d_qk_layernorm_rope2d_pos";
  HeadParams p;
  int norm = HN_NONE, r;
  if ((r = qk_rope2d_common(fn, q, q_w, q_b, k, k_w, k_b, eps, q_out, k_out, p, norm))) return r;
  if ((r = index_tensor(positions, fn, "positions", p.B, p.N, 2, true))) return r;
  if (!(base > 0.f) || !std::isfinite(base)) return fail(LUX3D_ERR_VALUE, "%s: base must be a positive number", fn);
  if (p.D / 4 > 64) return fail(LUX3D_ERR_SHAPE, "%s: token_dim %lld above 256 (use the tables entry)", fn, (long long)p.D);
  p.pos = positions->data; p.pos_dt = positions->dtype;
  p.pos_sB = positions->stride[0]; p.pos_sN = positions->stride[1]; p.pos_sC = positions->stride[2];
  rope2d_inv_freq(base, p.D, p.freq);
  p.nfreq = (int)(p.D / 4);
  return hip_status(launch_heads(norm, HR_R1_POS, q->dtype, p, stream_of(stream)), fn);
}

int lux3d_rope2d_tables(const lux3d_tensor_t *positions, float base, const lux3d_tensor_t *cos_full,
                        const lux3d_tensor_t *sin_alt_full, lux3d_stream_t stream) {
  const char *fn = "lux3d_rope2d_tables";
  int r;
  if ((r = check_desc(positions, fn, "positions"))) return r;
  if ((r = check_desc(cos_full, fn, "cos_full")) || (r = check_desc(sin_alt_full, fn, "sin_alt_full"))) return r;
  if (positions->rank != 3) return fail(LUX3D_ERR_SHAPE, "%s: positions must be [B, N, 2]", fn);
  const int64_t B = positions->shape[0], N = positions->shape[1];
  if ((r = index_tensor(positions, fn, "positions", B, N, 2, true))) return r;
  const int64_t D = cos_full->shape[cos_full->rank - 1];
  if (D % 4 || D < 4 || D > 256) return fail(LUX3D_ERR_SHAPE, "%s: token_dim %lld must be a multiple of 4 in [4, 256]", fn, (long long)D);
  for (const lux3d_tensor_t *t : {cos_full, sin_alt_full}) {
    if (t->dtype != LUX3D_F32) return fail(LUX3D_ERR_DTYPE, "%s: tables must be f32", fn);
    if (!is_contiguous(t) || numel(t) != B * N * D) return fail(LUX3D_ERR_SHAPE, "%s: tables must be contiguous [B, N, D]", fn);
  }
  if (!(base > 0.f) || !std::isfinite(base)) return fail(LUX3D_ERR_VALUE, "%s: base must be a positive number", fn);
  float inv[64];
  rope2d_inv_freq(base, D, inv);
  return hip_status(launch_rope2d_tables(positions->data, positions->dtype, positions->stride[0], positions->stride[1],
                                         positions->stride[2], B, N, D, inv, reinterpret_cast<float *>(cos_full->data),
                                         reinterpret_cast<float *>(sin_alt_full->data), stream_of(stream)),
                    fn);
}

int lux3d_rms_norm_heads(const lux3d_tensor_t *q, const lux3d_tensor_t *q_w, const lux3d_tensor_t *k,
                         const lux3d_tensor_t *k_w, float eps, const lux3d_tensor_t *q_out,
                         const lux3d_tensor_t *k_out, lux3d_stream_t stream) {
  const char *fn = "lux3d_rms_norm_heads";
  HeadParams p;
  HeadView qv, kv;
  int r;
  if (!q_w) return fail(LUX3D_ERR_NULL, "%s: `q_w` is NULL", fn);
  if ((r = head_side(q, q_out, q_w, q ? q->shape[3] : 0, nullptr, fn, "q", "q_out", "q_w", "-", 0, 1, 2, p.io[0], qv)))
    return r;
  p.ntens = 1;
  if (k) {
    if (!k_w) return fail(LUX3D_ERR_NULL, "%s: `k_w` is NULL", fn);
    if ((r = head_side(k, k_out, k_w, k->shape[3], nullptr, fn, "k", "k_out", "k_w", "-", 0, 1, 2, p.io[1], kv)))
      return r;
    if ((r = same_heads(qv, kv, fn, "k"))) return r;
    if (k->dtype != q->dtype) return fail(LUX3D_ERR_DTYPE, "%s: `k` dtype differs from `q`", fn);
    p.ntens = 2;
  }
  if (!(eps >= 0.f)) return fail(LUX3D_ERR_VALUE, "%s: eps must be >= 0", fn);
  p.B = qv.B; p.H = qv.H; p.N = qv.N; p.D = qv.D; p.eps = eps;
  p.vec = qv.vec && (p.ntens == 1 || kv.vec);
  return hip_status(launch_heads(HN_RMS, HR_NONE, q->dtype, p, stream_of(stream)), fn);
}

int lux3d_qk_l2norm_rope3d(const lux3d_tensor_t *q, const lux3d_tensor_t *q_gamma, const lux3d_tensor_t *k,
                           const lux3d_tensor_t *k_gamma, const lux3d_tensor_t *cos, const lux3d_tensor_t *sin,
                           const lux3d_tensor_t *coords, float base, const lux3d_tensor_t *q_out,
                           const lux3d_tensor_t *k_out, lux3d_stream_t stream) {
  const char *fn = "lux3d_qk_l2norm_rope3d";
  HeadParams p;
  HeadView qv, kv;
  int r;
  // [B, L, H, D] views: B = dim 0, H = dim 2, N (tokens) = dim 1
  const int64_t H = q ? (q->rank == 4 ? q->shape[2] : 0) : 0;
  const int64_t D = (q && q->rank >= 1 && q->rank <= LUX3D_MAX_RANK) ? q->shape[q->rank - 1] : 0;
  if ((r = head_side(q, q_out, q_gamma, H * D, nullptr, fn, "q", "q_out", "q_gamma", "-", 0, 2, 1, p.io[0], qv)))
    return r;
  p.ntens = 1;
  if (k) {
    if ((r = head_side(k, k_out, k_gamma, H * D, nullptr, fn, "k", "k_out", "k_gamma", "-", 0, 2, 1, p.io[1], kv)))
      return r;
    if ((r = same_heads(qv, kv, fn, "k"))) return r;
    if (k->dtype != q->dtype) return fail(LUX3D_ERR_DTYPE, "%s: `k` dtype differs from `q`", fn);
    if ((q_gamma != nullptr) != (k_gamma != nullptr))
      return fail(LUX3D_ERR_NULL, "%s: q and k must both be normalised or both not", fn);
    p.ntens = 2;
  }
  p.B = qv.B; p.H = qv.H; p.N = qv.N; p.D = qv.D;
  p.vec = qv.vec && (p.ntens == 1 || kv.vec);
  const int norm = q_gamma ? HN_L2 : HN_NONE;
  int rot = HR_NONE;
  if ((cos || sin || coords) && p.D % 2)
    return fail(LUX3D_ERR_SHAPE, "%s: head dim %lld must be even to rotate (re, im) pairs", fn, (long long)p.D);
  if (cos || sin) {
    if (!cos || !sin) return fail(LUX3D_ERR_NULL, "%s: pass both cos and sin tables", fn);
    if (coords) return fail(LUX3D_ERR_VALUE, "%s: pass tables or coords, not both", fn);
    if ((r = check_desc(cos, fn, "cos")) || (r = check_desc(sin, fn, "sin"))) return r;
    for (const lux3d_tensor_t *t : {cos, sin}) {
      if (!is_float(t->dtype)) return fail(LUX3D_ERR_DTYPE, "%s: tables must be f32/bf16/f16", fn);
      if (t->rank != 2 || t->shape[0] != p.N || t->shape[1] != p.D / 2 || t->stride[1] != 1)
        return fail(LUX3D_ERR_SHAPE, "%s: tables must be [L, D/2] = [%lld, %lld] with unit inner stride", fn,
                    (long long)p.N, (long long)(p.D / 2));
    }
    if (cos->stride[0] != sin->stride[0] || cos->dtype != sin->dtype)
      return fail(LUX3D_ERR_LAYOUT, "%s: cos and sin must share layout and dtype", fn);
    p.tab_c = cos->data; p.tab_s = sin->data; p.tab_dt = cos->dtype; p.tab_sN = cos->stride[0];
    rot = HR_R2_TAB;
  } else if (coords) {
    if ((r = index_tensor(coords, fn, "coords", 0, p.N, 3, false))) return r;
    if (!(base > 0.f) || !std::isfinite(base)) return fail(LUX3D_ERR_VALUE, "%s: base must be a positive number", fn);
    if (p.D / 2 / 3 < 1 || p.D / 2 / 3 > 64)
      return fail(LUX3D_ERR_SHAPE, "%s: head dim %lld gives %lld frequencies per axis (1..64)", fn, (long long)p.D,
                  (long long)(p.D / 2 / 3));
    p.pos = coords->data; p.pos_dt = LUX3D_I32; p.pos_sN = coords->stride[0]; p.pos_sC = coords->stride[1];
    p.nfreq = (int)rope3d_freq(base, p.D, p.freq);
    rot = HR_R2_COORD;
  }
  return hip_status(launch_heads(norm, rot, q->dtype, p, stream_of(stream)), fn);
}

int lux3d_rope3d_tables(const lux3d_tensor_t *coords, int64_t head_dim, float base, const lux3d_tensor_t *cos,
                        const lux3d_tensor_t *sin, lux3d_stream_t stream) {
  const char *fn = "lux3d_rope3d_tables";
  int r;
  if ((r = check_desc(coords, fn, "coords"))) return r;
  if (coords->rank != 2) return fail(LUX3D_ERR_SHAPE, "%s: coords must be [L, 3]", fn);
  const int64_t L = coords->shape[0];
  if ((r = index_tensor(coords, fn, "coords", 0, L, 3, false))) return r;
  if (head_dim % 2 || head_dim / 2 / 3 < 1 || head_dim / 2 / 3 > 64)
    return fail(LUX3D_ERR_SHAPE, "%s: head_dim %lld unsupported", fn, (long long)head_dim);
  if ((r = check_desc(cos, fn, "cos")) || (r = check_desc(sin, fn, "sin"))) return r;
  for (const lux3d_tensor_t *t : {cos, sin}) {
    if (t->dtype != LUX3D_F32) return fail(LUX3D_ERR_DTYPE, "%s: tables must be f32", fn);
    if (!is_contiguous(t) || numel(t) != L * (head_dim / 2))
      return fail(LUX3D_ERR_SHAPE, "%s: tables must be contiguous [L, head_dim/2]", fn);
  }
  if (!(base > 0.f) || !std::isfinite(base)) return fail(LUX3D_ERR_VALUE, "%s: base must be a positive number", fn);
  float f[64];
  const int64_t fd = rope3d_freq(base, head_dim, f);
  return hip_status(launch_rope3d_tables(reinterpret_cast<const int32_t *>(coords->data), coords->stride[0],
                                         coords->stride[1], L, head_dim / 2, fd, f,
                                         reinterpret_cast<float *>(cos->data), reinterpret_cast<float *>(sin->data),
                                         stream_of(stream)),
                    fn);
}

int lux3d_dinov3_rope(const lux3d_tensor_t *q, const lux3d_tensor_t *k, const lux3d_tensor_t *cos,
                      const lux3d_tensor_t *sin, int64_t num_prefix, const lux3d_tensor_t *q_out,
                      const lux3d_tensor_t *k_out, lux3d_stream_t stream) {
  const char *fn = "lux3d_dinov3_rope";
  HeadParams p;
  HeadView qv, kv;
  int r;
  if ((r = head_side(q, q_out, nullptr, 0, nullptr, fn, "q", "q_out", "-", "-", 0, 1, 2, p.io[0], qv))) return r;
  p.ntens = 1;
  if (k) {
    if ((r = head_side(k, k_out, nullptr, 0, nullptr, fn, "k", "k_out", "-", "-", 0, 1, 2, p.io[1], kv))) return r;
    if ((r = same_heads(qv, kv, fn, "k"))) return r;
    if (k->dtype != q->dtype) return fail(LUX3D_ERR_DTYPE, "%s: `k` dtype differs from `q`", fn);
    p.ntens = 2;
  }
  p.B = qv.B; p.H = qv.H; p.N = qv.N; p.D = qv.D;
  p.vec = qv.vec && (p.ntens == 1 || kv.vec);
  if (p.D % 2) return fail(LUX3D_ERR_SHAPE, "%s: head dim %lld must be even (rotate_half)", fn, (long long)p.D);
  if (num_prefix < 0 || num_prefix > p.N) return fail(LUX3D_ERR_VALUE, "%s: num_prefix out of range", fn);
  if ((r = check_desc(cos, fn, "cos")) || (r = check_desc(sin, fn, "sin"))) return r;
  for (const lux3d_tensor_t *t : {cos, sin}) {
    if (!is_float(t->dtype)) return fail(LUX3D_ERR_DTYPE, "%s: tables must be f32/bf16/f16", fn);
    if (t->rank != 2 || t->shape[0] != p.N - num_prefix || t->shape[1] != p.D || t->stride[1] != 1)
      return fail(LUX3D_ERR_SHAPE, "%s: tables must be [S - num_prefix, D] = [%lld, %lld]", fn,
                  (long long)(p.N - num_prefix), (long long)p.D);
  }
  if (cos->stride[0] != sin->stride[0] || cos->dtype != sin->dtype)
    return fail(LUX3D_ERR_LAYOUT, "%s: cos and sin must share layout and dtype", fn);
  p.tab_c = cos->data; p.tab_s = sin->data; p.tab_dt = cos->dtype; p.tab_sN = cos->stride[0];
  p.prefix = num_prefix;
  return hip_status(launch_heads(HN_NONE, HR_R3_TAB, q->dtype, p, stream_of(stream)), fn);
}

// ---------------------------------------------------------------------------

namespace {
int act_common(int a, const char *fn, const lux3d_tensor_t *x, const lux3d_tensor_t *y, lux3d_stream_t stream) {
  int r;
  if ((r = check_desc(x, fn, "x")) || (r = check_desc(y, fn, "y"))) return r;
  if (!is_float(x->dtype)) return fail(LUX3D_ERR_DTYPE, "%s: `x` must be f32/bf16/f16", fn);
  if (y->dtype != x->dtype) return fail(LUX3D_ERR_DTYPE, "%s: `y` dtype differs from `x`", fn);
  if (numel(x) != numel(y)) return fail(LUX3D_ERR_SHAPE, "%s: `x` and `y` sizes differ", fn);
  if (!is_contiguous(x) || !is_contiguous(y)) return fail(LUX3D_ERR_LAYOUT, "%s: tensors must be contiguous", fn);
  const bool vec = aligned16(x->data) && aligned16(y->data);
  return hip_status(launch_act(a, x->dtype, x->data, y->data, numel(x), vec, stream_of(stream)), fn);
}
}  // namespace

int lux3d_gelu_erf(const lux3d_tensor_t *x, const lux3d_tensor_t *y, lux3d_stream_t stream) {
  return act_common(ACT_GELU_ERF, "lux3d_gelu_erf", x, y, stream);
}
int lux3d_gelu_tanh(const lux3d_tensor_t *x, const lux3d_tensor_t *y, lux3d_stream_t stream) {
  return act_common(ACT_GELU_TANH, "lux3d_gelu_tanh", x, y, stream);
}
int lux3d_silu(const lux3d_tensor_t *x, const lux3d_tensor_t *y, lux3d_stream_t stream) {
  return act_common(ACT_SILU, "lux3d_silu", x, y, stream);
}

int lux3d_timestep_embedding(const lux3d_tensor_t *t, const lux3d_tensor_t *freqs, int64_t dim, int32_t cos_first,
                             const lux3d_tensor_t *out, lux3d_stream_t stream) {
  const char *fn = "lux3d_timestep_embedding";
  int r;
  if ((r = check_desc(t, fn, "t")) || (r = check_desc(out, fn, "out"))) return r;
  if (t->dtype != LUX3D_F32 || out->dtype != LUX3D_F32) return fail(LUX3D_ERR_DTYPE, "%s: t and out must be f32", fn);
  if (!is_contiguous(t) || !is_contiguous(out)) return fail(LUX3D_ERR_LAYOUT, "%s: t and out must be contiguous", fn);
  if (dim < 1) return fail(LUX3D_ERR_VALUE, "%s: dim must be >= 1", fn);
  if (!cos_first && dim % 2) return fail(LUX3D_ERR_VALUE, "%s: the sin-first embedding needs an even dim", fn);
  const int64_t n = numel(t);
  if (numel(out) != n * dim) return fail(LUX3D_ERR_SHAPE, "%s: out must hold [n, dim] = [%lld, %lld]", fn,
                                         (long long)n, (long long)dim);
  const float *fp = nullptr;
  if (freqs) {
    if ((r = check_desc(freqs, fn, "freqs"))) return r;
    if (freqs->dtype != LUX3D_F32 || !is_contiguous(freqs) || numel(freqs) != dim / 2)
      return fail(LUX3D_ERR_SHAPE, "%s: freqs must be a contiguous f32 [dim/2] vector", fn);
    fp = reinterpret_cast<const float *>(freqs->data);
  }
  // -ln(10000) in f32: identical for `-(10000f32).ln()` (TripoSG) and
  // `-(10000f64.ln()) as f32` (TRELLIS.2).
  const float nlp = (float)(-std::log(10000.0));
  return hip_status(launch_timestep(reinterpret_cast<const float *>(t->data), n, fp, dim, cos_first ? 1 : 0, nlp,
                                    reinterpret_cast<float *>(out->data), stream_of(stream)),
                    fn);
}

int lux3d_dequant_q8_0(const lux3d_tensor_t *blocks, const lux3d_tensor_t *y, lux3d_stream_t stream) {
  const char *fn = "lux3d_dequant_q8_0";
  int r;
  if ((r = check_desc(blocks, fn, "blocks")) || (r = check_desc(y, fn, "y"))) return r;
  if (blocks->dtype != LUX3D_U8) return fail(LUX3D_ERR_DTYPE, "%s: blocks must be u8", fn);
  if (!is_float(y->dtype)) return fail(LUX3D_ERR_DTYPE, "%s: y must be f32/bf16/f16", fn);
  if (!is_contiguous(blocks) || !is_contiguous(y)) return fail(LUX3D_ERR_LAYOUT, "%s: tensors must be contiguous", fn);
  const int64_t nbytes = numel(blocks);
  if (nbytes % 34) return fail(LUX3D_ERR_SHAPE, "%s: %lld bytes is not a whole number of 34-byte Q8_0 blocks", fn,
                               (long long)nbytes);
  const int64_t nblocks = nbytes / 34;
  if (numel(y) != nblocks * 32)
    return fail(LUX3D_ERR_SHAPE, "%s: y has %lld elements, expected %lld", fn, (long long)numel(y),
                (long long)(nblocks * 32));
  if (reinterpret_cast<uintptr_t>(blocks->data) & 1u)
    return fail(LUX3D_ERR_LAYOUT, "%s: blocks must be 2-byte aligned", fn);
  const bool vec = aligned16(y->data);
  return hip_status(launch_dequant_q8_0(reinterpret_cast<const uint8_t *>(blocks->data), nblocks, y->dtype, y->data,
                                        vec, stream_of(stream)),
                    fn);
}

int lux3d_q8_0_repack(const lux3d_tensor_t *blocks, int64_t n, int64_t k, const lux3d_tensor_t *qs,
                      const lux3d_tensor_t *scales, lux3d_stream_t stream) {
  const char *fn = "lux3d_q8_0_repack";
  int r;
  if ((r = check_desc(blocks, fn, "blocks")) || (r = check_desc(qs, fn, "qs")) ||
      (r = check_desc(scales, fn, "scales")))
    return r;
  if (n < 0 || k < 0 || k % 32) return fail(LUX3D_ERR_SHAPE, "%s: weight [%lld, %lld] needs k %% 32 == 0", fn,
                                           (long long)n, (long long)k);
  if (blocks->dtype != LUX3D_U8) return fail(LUX3D_ERR_DTYPE, "%s: blocks must be u8", fn);
  if (qs->dtype != LUX3D_I8) return fail(LUX3D_ERR_DTYPE, "%s: qs must be int8", fn);
  if (scales->dtype != LUX3D_F32) return fail(LUX3D_ERR_DTYPE, "%s: scales must be f32", fn);
  if (!is_contiguous(blocks) || !is_contiguous(qs) || !is_contiguous(scales))
    return fail(LUX3D_ERR_LAYOUT, "%s: tensors must be contiguous", fn);
  const int64_t nblocks = n * (k / 32);
  if (numel(blocks) != nblocks * 34)
    return fail(LUX3D_ERR_SHAPE, "%s: %lld bytes of blocks for a [%lld, %lld] weight (expected %lld)", fn,
                (long long)numel(blocks), (long long)n, (long long)k, (long long)(nblocks * 34));
  if (numel(qs) != n * k || numel(scales) != nblocks)
    return fail(LUX3D_ERR_SHAPE, "%s: qs must hold n*k values and scales n*k/32", fn);
  if (reinterpret_cast<uintptr_t>(blocks->data) & 1u)
    return fail(LUX3D_ERR_LAYOUT, "%s: blocks must be 2-byte aligned", fn);
  if (!aligned16(qs->data) || !aligned16(scales->data))
    return fail(LUX3D_ERR_LAYOUT, "%s: qs and scales must be 16-byte aligned", fn);
  return hip_status(launch_q8_0_repack(reinterpret_cast<const uint8_t *>(blocks->data), nblocks,
                                       reinterpret_cast<int8_t *>(qs->data), reinterpret_cast<float *>(scales->data),
                                       stream_of(stream)),
                    fn);
}

int lux3d_q8_0_linear(const lux3d_tensor_t *x, const lux3d_tensor_t *qs, const lux3d_tensor_t *scales,
                      const lux3d_tensor_t *bias, const lux3d_tensor_t *y, lux3d_stream_t stream) {
  const char *fn = "lux3d_q8_0_linear";
  int r;
  RowView xv, yv;
  if ((r = row_tensor(x, fn, "x", -1, xv))) return r;
  if (x->dtype != LUX3D_BF16 && x->dtype != LUX3D_F32)
    return fail(LUX3D_ERR_DTYPE, "%s: x must be bf16 or f32", fn);
  const bool xf32 = x->dtype == LUX3D_F32;
  if ((r = row_tensor(y, fn, "y", -1, yv))) return r;
  if ((r = check_desc(qs, fn, "qs")) || (r = check_desc(scales, fn, "scales"))) return r;
  if (qs->dtype != LUX3D_I8 || qs->rank != 2 || !is_contiguous(qs))
    return fail(LUX3D_ERR_SHAPE, "%s: qs must be a contiguous int8 [n, k] (from lux3d_q8_0_repack)", fn);
  const int64_t n = qs->shape[0], k = qs->shape[1];
  if (k != xv.d) return fail(LUX3D_ERR_SHAPE, "%s: x has %lld features, the weight %lld", fn, (long long)xv.d,
                             (long long)k);
  if (k % 32 || k == 0) return fail(LUX3D_ERR_SHAPE, "%s: k must be a positive multiple of 32", fn);
  if (xf32 && k % 64) return fail(LUX3D_ERR_SHAPE, "%s: f32 x needs k to be a multiple of 64", fn);
  if (scales->dtype != LUX3D_F32 || !is_contiguous(scales) || numel(scales) != n * (k / 32))
    return fail(LUX3D_ERR_SHAPE, "%s: scales must be a contiguous f32 [n, k/32]", fn);
  if (yv.d != n || yv.rows != xv.rows)
    return fail(LUX3D_ERR_SHAPE, "%s: y must be [%lld, %lld]", fn, (long long)xv.rows, (long long)n);
  const float *bp = nullptr;
  if (bias) {
    if ((r = check_desc(bias, fn, "bias"))) return r;
    if (bias->dtype != LUX3D_F32 || !is_contiguous(bias) || numel(bias) != n)
      return fail(LUX3D_ERR_SHAPE, "%s: bias must be a contiguous f32 [n]", fn);
    bp = reinterpret_cast<const float *>(bias->data);
  }
  if (!aligned16(x->data) || (xv.rows > 1 && (xv.rs * (xf32 ? 4 : 2)) % 16) || !aligned16(qs->data))
    return fail(LUX3D_ERR_LAYOUT, "%s: x rows and qs must be 16-byte aligned", fn);
  if (xf32 && (xv.rs > (int64_t(1) << 20) || k > (int64_t(1) << 22)))
    return fail(LUX3D_ERR_SHAPE, "%s: f32 x rows of more than 2^20 elements are not supported", fn);
  Q8GemmParams p;
  p.x = xv.p; p.ldx = xv.rs; p.x_f32 = xf32;
  p.qs = reinterpret_cast<const int8_t *>(qs->data);
  p.scales = reinterpret_cast<const float *>(scales->data);
  p.bias = bp;
  p.y = const_cast<void *>(yv.p); p.ldy = yv.rs;
  p.M = xv.rows; p.N = n; p.K = k;
  return hip_status(launch_q8_0_gemm(y->dtype, p, stream_of(stream)), fn);
}

namespace {
// x f32 rows (16-byte aligned) and the Q8_0 quantization workspace for them:
// xq int8 [rows, k] and xd f32 block-major [k/32, rows rounded up to 64],
// both contiguous and 16-byte aligned.
int q8_act(const char *fn, const lux3d_tensor_t *x, const lux3d_tensor_t *xq, const lux3d_tensor_t *xd,
           Q8IntParams &p) {
  int r;
  RowView xv;
  if ((r = row_tensor(x, fn, "x", LUX3D_F32, xv))) return r;
  if ((r = check_desc(xq, fn, "xq")) || (r = check_desc(xd, fn, "xd"))) return r;
  const int64_t k = xv.d;
  if (k % 32 || k == 0) return fail(LUX3D_ERR_SHAPE, "%s: x rows must hold a positive multiple of 32 values", fn);
  if (xq->dtype != LUX3D_I8 || !is_contiguous(xq) || numel(xq) != xv.rows * k)
    return fail(LUX3D_ERR_SHAPE, "%s: xq must be a contiguous int8 [%lld, %lld]", fn, (long long)xv.rows,
                (long long)k);
  const int64_t mpad = (xv.rows + 63) / 64 * 64;
  if (xd->dtype != LUX3D_F32 || !is_contiguous(xd) || numel(xd) != mpad * (k / 32))
    return fail(LUX3D_ERR_SHAPE, "%s: xd must be a contiguous f32 [%lld, %lld] (block-major, rows rounded up to 64)",
                fn, (long long)(k / 32), (long long)mpad);
  if (!aligned16(x->data) || (xv.rows > 1 && (xv.rs * 4) % 16) || !aligned16(xq->data) || !aligned16(xd->data))
    return fail(LUX3D_ERR_LAYOUT, "%s: x rows, xq and xd must be 16-byte aligned", fn);
  p.x = reinterpret_cast<const float *>(xv.p);
  p.ldx = xv.rs;
  p.xq = reinterpret_cast<int8_t *>(xq->data);
  p.xd = reinterpret_cast<float *>(xd->data);
  p.ldxd = mpad;
  p.M = xv.rows;
  p.K = k;
  return LUX3D_OK;
}
}  // namespace

int lux3d_q8_0_quantize(const lux3d_tensor_t *x, const lux3d_tensor_t *xq, const lux3d_tensor_t *xd,
                        lux3d_stream_t stream) {
  const char *fn = "lux3d_q8_0_quantize";
  Q8IntParams p;
  int r;
  if ((r = q8_act(fn, x, xq, xd, p))) return r;
  return hip_status(launch_q8_0_quantize_rows(p, stream_of(stream)), fn);
}

int lux3d_q8_0_linear_int8(const lux3d_tensor_t *x, const lux3d_tensor_t *qs, const lux3d_tensor_t *scales,
                           const lux3d_tensor_t *bias, const lux3d_tensor_t *xq, const lux3d_tensor_t *xd,
                           const lux3d_tensor_t *y, lux3d_stream_t stream) {
  const char *fn = "lux3d_q8_0_linear_int8";
  Q8IntParams p;
  int r;
  if ((r = q8_act(fn, x, xq, xd, p))) return r;
  if ((r = check_desc(qs, fn, "qs")) || (r = check_desc(scales, fn, "scales"))) return r;
  if (qs->dtype != LUX3D_I8 || qs->rank != 2 || !is_contiguous(qs))
    return fail(LUX3D_ERR_SHAPE, "%s: qs must be a contiguous int8 [n, k] (from lux3d_q8_0_repack)", fn);
  const int64_t n = qs->shape[0];
  if (qs->shape[1] != p.K)
    return fail(LUX3D_ERR_SHAPE, "%s: x has %lld features, the weight %lld", fn, (long long)p.K,
                (long long)qs->shape[1]);
  if (scales->dtype != LUX3D_F32 || !is_contiguous(scales) || numel(scales) != n * (p.K / 32))
    return fail(LUX3D_ERR_SHAPE, "%s: scales must be a contiguous f32 [n, k/32]", fn);
  if (!aligned16(qs->data)) return fail(LUX3D_ERR_LAYOUT, "%s: qs must be 16-byte aligned", fn);
  RowView yv;
  if ((r = row_tensor(y, fn, "y", LUX3D_F32, yv))) return r;
  if (yv.d != n || yv.rows != p.M)
    return fail(LUX3D_ERR_SHAPE, "%s: y must be f32 [%lld, %lld]", fn, (long long)p.M, (long long)n);
  if (bias) {
    if ((r = check_desc(bias, fn, "bias"))) return r;
    if (bias->dtype != LUX3D_F32 || !is_contiguous(bias) || numel(bias) != n)
      return fail(LUX3D_ERR_SHAPE, "%s: bias must be a contiguous f32 [n]", fn);
    p.bias = reinterpret_cast<const float *>(bias->data);
  }
  p.qs = reinterpret_cast<const int8_t *>(qs->data);
  p.scales = reinterpret_cast<const float *>(scales->data);
  p.y = reinterpret_cast<float *>(const_cast<void *>(yv.p));
  p.ldy = yv.rs;
  p.N = n;
  hipStream_t s = stream_of(stream);
  hipError_t e = launch_q8_0_quantize_rows(p, s);
  if (e == hipSuccess) e = launch_q8_0_int8_gemm(p, s);
  return hip_status(e, fn);
}

namespace {
// Validates q, k, v, out for attention and fills the strides; `mfma` tells
// whether every row is 16-byte aligned with D 64 / 128. `f32_out_ok`: out
// may also be f32 when q, k, v are 2-byte.
int attn_params(const char *fn, const lux3d_tensor_t *q, const lux3d_tensor_t *k, const lux3d_tensor_t *v,
                float scale, const lux3d_tensor_t *out, AttnParams &p, bool f32_out_ok = false);
}  // namespace

int lux3d_sdpa(const lux3d_tensor_t *q, const lux3d_tensor_t *k, const lux3d_tensor_t *v, float scale,
               const lux3d_tensor_t *out, lux3d_stream_t stream) {
  const char *fn = "lux3d_sdpa";
  AttnParams p;
  int r;
  if ((r = attn_params(fn, q, k, v, scale, out, p))) return r;
  return hip_status(launch_attention(q->dtype, p, stream_of(stream)), fn);
}

int lux3d_sdpa_heads_f32(const lux3d_tensor_t *q, const lux3d_tensor_t *k, const lux3d_tensor_t *v, float scale,
                         const lux3d_tensor_t *out, lux3d_stream_t stream) {
  const char *fn = "lux3d_sdpa_heads_f32";
  AttnParams p;
  int r;
  if ((r = attn_params(fn, q, k, v, scale, out, p, true))) return r;
  p.exact_p = true;
  p.out_f32 = out->dtype == LUX3D_F32;
  return hip_status(launch_attention(q->dtype, p, stream_of(stream)), fn);
}

int lux3d_sdpa_layernorm_rope2d(const lux3d_tensor_t *q, const lux3d_tensor_t *q_w, const lux3d_tensor_t *q_b,
                                float eps, const lux3d_tensor_t *cos_full, const lux3d_tensor_t *sin_alt_full,
                                const lux3d_tensor_t *k, const lux3d_tensor_t *v, float scale, const lux3d_tensor_t *out,
                                lux3d_stream_t stream) {
  const char *fn = "lux3d_sdpa_layernorm_rope2d";
  AttnParams p;
  int r;
  if ((r = attn_params(fn, q, k, v, scale, out, p))) return r;
  if (!q_w) return fail(LUX3D_ERR_NULL, "%s: LayerNorm needs a weight (the bias may be NULL)", fn);
  const void *wp, *bp;
  int wdt, bdt;
  if ((r = param_vec(q_w, p.D, fn, "q_w", wp, wdt)) || (r = param_vec(q_b, p.D, fn, "q_b", bp, bdt))) return r;
  if (!(eps >= 0.f)) return fail(LUX3D_ERR_VALUE, "%s: eps must be >= 0", fn);
  if (p.D % 4) return fail(LUX3D_ERR_SHAPE, "%s: rope token_dim must be divisible by 4, got %lld", fn, (long long)p.D);
  int64_t cB, cN, sB, sN;
  if ((r = rope2d_table(cos_full, fn, "cos_full", p.B, p.Lq, p.D, cB, cN))) return r;
  if ((r = rope2d_table(sin_alt_full, fn, "sin_alt_full", p.B, p.Lq, p.D, sB, sN))) return r;
  if (cB != sB || cN != sN || cos_full->dtype != sin_alt_full->dtype)
    return fail(LUX3D_ERR_LAYOUT, "%s: cos_full and sin_alt_full must share layout and dtype", fn);
  // fused: the matrix-core path, and 16-byte aligned parameters and table rows
  const int tb = elem_bytes(cos_full->dtype);
  const bool fused = p.mfma && q->dtype != LUX3D_F32 && (p.D == 64 || p.D == 128) && aligned16(wp) &&
                     (bdt < 0 || aligned16(bp)) &&
                     aligned16(cos_full->data) && aligned16(sin_alt_full->data) && (cN * tb) % 16 == 0 &&
                     (cB * tb) % 16 == 0;
  if (!fused) {
    // the two launches, out holding the normalised q (each attention
    // workgroup reads its query rows before it writes the same rows)
    if ((r = lux3d_qk_layernorm_rope2d(q, q_w, q_b, nullptr, nullptr, nullptr, eps, cos_full, sin_alt_full, out,
                                       nullptr, stream)))
      return r;
    return lux3d_sdpa(out, k, v, scale, out, stream);
  }
  p.qpro = QP_LN_R1;
  p.qw = wp; p.qw_dt = wdt; p.qb = bp; p.qb_dt = bdt; p.eps = eps;
  p.tab_c = cos_full->data; p.tab_s = sin_alt_full->data; p.tab_dt = cos_full->dtype;
  p.tab_sB = cB; p.tab_sN = cN;
  return hip_status(launch_attention(q->dtype, p, stream_of(stream)), fn);
}

int lux3d_sdpa_rms_norm_heads(const lux3d_tensor_t *q, const lux3d_tensor_t *q_w, float eps, const lux3d_tensor_t *k,
                              const lux3d_tensor_t *v, float scale, const lux3d_tensor_t *out,
                              lux3d_stream_t stream) {
  const char *fn = "lux3d_sdpa_rms_norm_heads";
  AttnParams p;
  int r;
  if ((r = attn_params(fn, q, k, v, scale, out, p))) return r;
  if (!q_w) return fail(LUX3D_ERR_NULL, "%s: `q_w` is NULL", fn);
  const void *wp;
  int wdt;
  if ((r = param_vec(q_w, p.D, fn, "q_w", wp, wdt))) return r;
  if (!(eps >= 0.f)) return fail(LUX3D_ERR_VALUE, "%s: eps must be >= 0", fn);
  const bool fused = p.mfma && q->dtype != LUX3D_F32 && aligned16(wp);
  if (!fused) {
    // the two launches, out holding the normalised q
    if ((r = lux3d_rms_norm_heads(q, q_w, nullptr, nullptr, eps, out, nullptr, stream))) return r;
    return lux3d_sdpa(out, k, v, scale, out, stream);
  }
  p.qpro = QP_RMS;
  p.qw = wp; p.qw_dt = wdt; p.eps = eps;
  return hip_status(launch_attention(q->dtype, p, stream_of(stream)), fn);
}

namespace {
// The [B, L, H, D] view of a [B, H, L, D] descriptor (dims 1 and 2 swapped).
lux3d_tensor_t swap_heads_tokens(const lux3d_tensor_t *t) {
  lux3d_tensor_t u = *t;
  std::swap(u.shape[1], u.shape[2]);
  std::swap(u.stride[1], u.stride[2]);
  return u;
}
// A rotation table [rows, cols] with a unit inner stride in f32 / bf16 / f16
// (cos and sin alike); its row stride in sN.
int rot_tables(const lux3d_tensor_t *cos, const lux3d_tensor_t *sin, int64_t rows, int64_t cols, const char *fn,
               const char *what, int64_t &sN) {
  int r;
  if (!cos || !sin) return fail(LUX3D_ERR_NULL, "%s: pass both cos and sin tables", fn);
  if ((r = check_desc(cos, fn, "cos")) || (r = check_desc(sin, fn, "sin"))) return r;
  for (const lux3d_tensor_t *t : {cos, sin}) {
    if (!is_float(t->dtype)) return fail(LUX3D_ERR_DTYPE, "%s: tables must be f32/bf16/f16", fn);
    if (t->rank != 2 || t->shape[0] != rows || t->shape[1] != cols || (cols > 1 && t->stride[1] != 1))
      return fail(LUX3D_ERR_SHAPE, "%s: tables must be %s = [%lld, %lld] with unit inner stride", fn, what,
                  (long long)rows, (long long)cols);
  }
  if (cos->stride[0] != sin->stride[0] || cos->dtype != sin->dtype)
    return fail(LUX3D_ERR_LAYOUT, "%s: cos and sin must share layout and dtype", fn);
  sN = cos->stride[0];
  return LUX3D_OK;
}
// Both tables 16-byte aligned with 16-byte aligned rows.
bool tables_aligned(const lux3d_tensor_t *cos, const lux3d_tensor_t *sin, int64_t sN) {
  return aligned16(cos->data) && aligned16(sin->data) && (sN * elem_bytes(cos->dtype)) % 16 == 0;
}
}  // namespace

int lux3d_sdpa_l2norm_rope3d(const lux3d_tensor_t *q, const lux3d_tensor_t *q_gamma, const lux3d_tensor_t *cos,
                             const lux3d_tensor_t *sin, const lux3d_tensor_t *k, const lux3d_tensor_t *v, float scale,
                             const lux3d_tensor_t *out, lux3d_stream_t stream) {
  const char *fn = "lux3d_sdpa_l2norm_rope3d";
  AttnParams p;
  int r;
  if ((r = attn_params(fn, q, k, v, scale, out, p))) return r;
  if (!q_gamma) return fail(LUX3D_ERR_NULL, "%s: `q_gamma` is NULL", fn);
  const void *gp;
  int gdt;
  if ((r = param_vec(q_gamma, p.H * p.D, fn, "q_gamma", gp, gdt))) return r;
  if (p.D % 2) return fail(LUX3D_ERR_SHAPE, "%s: head dim %lld must be even to rotate (re, im) pairs", fn, (long long)p.D);
  int64_t sN;
  if ((r = rot_tables(cos, sin, p.Lq, p.D / 2, fn, "[L, D/2]", sN))) return r;
  const bool fused = p.mfma && q->dtype != LUX3D_F32 && aligned16(gp) && tables_aligned(cos, sin, sN);
  if (!fused) {
    // the two launches on the [B, L, H, D] views, out holding the rotated q
    const lux3d_tensor_t qt = swap_heads_tokens(q), ot = swap_heads_tokens(out);
    if ((r = lux3d_qk_l2norm_rope3d(&qt, q_gamma, nullptr, nullptr, cos, sin, nullptr, 0.f, &ot, nullptr, stream)))
      return r;
    return lux3d_sdpa(out, k, v, scale, out, stream);
  }
  p.qpro = QP_L2_R2;
  p.qw = gp; p.qw_dt = gdt;
  p.tab_c = cos->data; p.tab_s = sin->data; p.tab_dt = cos->dtype; p.tab_sN = sN;
  return hip_status(launch_attention(q->dtype, p, stream_of(stream)), fn);
}

int lux3d_sdpa_dinov3_rope(const lux3d_tensor_t *q, const lux3d_tensor_t *cos, const lux3d_tensor_t *sin,
                           int64_t num_prefix, const lux3d_tensor_t *k, const lux3d_tensor_t *v, float scale,
                           const lux3d_tensor_t *out, lux3d_stream_t stream) {
  const char *fn = "lux3d_sdpa_dinov3_rope";
  AttnParams p;
  int r;
  if ((r = attn_params(fn, q, k, v, scale, out, p))) return r;
  if (p.D % 2) return fail(LUX3D_ERR_SHAPE, "%s: head dim %lld must be even (rotate_half)", fn, (long long)p.D);
  if (num_prefix < 0 || num_prefix > p.Lq) return fail(LUX3D_ERR_VALUE, "%s: num_prefix out of range", fn);
  int64_t sN;
  if ((r = rot_tables(cos, sin, p.Lq - num_prefix, p.D, fn, "[S - num_prefix, D]", sN))) return r;
  const bool fused = p.mfma && (q->dtype == LUX3D_F32 || q->dtype == LUX3D_BF16) && tables_aligned(cos, sin, sN);
  if (!fused) {
    // the two launches, out holding the rotated q
    if ((r = lux3d_dinov3_rope(q, nullptr, cos, sin, num_prefix, out, nullptr, stream))) return r;
    return lux3d_sdpa_heads_f32(out, k, v, scale, out, stream);
  }
  p.exact_p = true;
  p.qpro = QP_R3;
  p.tab_c = cos->data; p.tab_s = sin->data; p.tab_dt = cos->dtype; p.tab_sN = sN;
  p.prefix = num_prefix;
  return hip_status(launch_attention(q->dtype, p, stream_of(stream)), fn);
}

namespace {
int attn_params(const char *fn, const lux3d_tensor_t *q, const lux3d_tensor_t *k, const lux3d_tensor_t *v,
                float scale, const lux3d_tensor_t *out, AttnParams &p, bool f32_out_ok) {
  int r;
  const lux3d_tensor_t *ts[4] = {q, k, v, out};
  const char *names[4] = {"q", "k", "v", "out"};
  for (int i = 0; i < 4; ++i) {
    if ((r = check_desc(ts[i], fn, names[i]))) return r;
    if (ts[i]->rank != 4)
      return fail(LUX3D_ERR_SHAPE, "%s: `%s` must be [B, H, L, D] (rank %d given)", fn, names[i], ts[i]->rank);
    if (ts[i]->dtype != q->dtype && !(i == 3 && f32_out_ok && ts[i]->dtype == LUX3D_F32))
      return fail(LUX3D_ERR_DTYPE, f32_out_ok ? "%s: q, k and v must share one dtype; out has it or is f32"
                                              : "%s: q, k, v and out must share one dtype", fn);
    if (ts[i]->shape[3] > 1 && ts[i]->stride[3] != 1)
      return fail(LUX3D_ERR_LAYOUT, "%s: `%s` must have a unit innermost stride", fn, names[i]);
  }
  if (!is_float(q->dtype)) return fail(LUX3D_ERR_DTYPE, "%s: dtype must be f32, bf16 or f16", fn);
  const int64_t B = q->shape[0], H = q->shape[1], Lq = q->shape[2], D = q->shape[3], Lk = k->shape[2];
  if (k->shape[0] != B || k->shape[1] != H || k->shape[3] != D)
    return fail(LUX3D_ERR_SHAPE, "%s: k must be [%lld, %lld, Lk, %lld]", fn, (long long)B, (long long)H, (long long)D);
  for (int i = 0; i < 4; ++i)
    if (ts[i]->shape[3] != D) return fail(LUX3D_ERR_SHAPE, "%s: head dims differ", fn);
  if (v->shape[0] != B || v->shape[1] != H || v->shape[2] != Lk)
    return fail(LUX3D_ERR_SHAPE, "%s: v must have the shape of k", fn);
  if (out->shape[0] != B || out->shape[1] != H || out->shape[2] != Lq)
    return fail(LUX3D_ERR_SHAPE, "%s: out must have the shape of q", fn);
  if (B * H * Lq > 0 && Lk == 0) return fail(LUX3D_ERR_SHAPE, "%s: k and v have no tokens", fn);
  if (D > 512 || D < 1) return fail(LUX3D_ERR_SHAPE, "%s: head dim %lld outside 1..512", fn, (long long)D);
  if (!(scale > 0.f) || !std::isfinite(scale)) return fail(LUX3D_ERR_VALUE, "%s: scale must be finite and > 0", fn);
  p = AttnParams();
  p.q = q->data; p.k = k->data; p.v = v->data; p.o = out->data;
  p.B = B; p.H = H; p.Lq = Lq; p.Lk = Lk; p.D = D;
  p.q_sb = q->stride[0]; p.q_sh = q->stride[1]; p.q_st = q->stride[2];
  p.k_sb = k->stride[0]; p.k_sh = k->stride[1]; p.k_st = k->stride[2];
  p.v_sb = v->stride[0]; p.v_sh = v->stride[1]; p.v_st = v->stride[2];
  p.o_sb = out->stride[0]; p.o_sh = out->stride[1]; p.o_st = out->stride[2];
  p.scale = scale;
  // matrix cores: D 64 / 128, every row start 16-byte aligned
  bool mfma = D == 64 || D == 128;
  for (int i = 0; i < 4 && mfma; ++i) {
    const lux3d_tensor_t *t = ts[i];
    const int64_t align_el = 16 / elem_bytes(t->dtype);
    mfma = aligned16(t->data);
    for (int a = 0; a < 3 && mfma; ++a)
      if (t->shape[a] > 1 && t->stride[a] % align_el) mfma = false;
  }
  p.mfma = mfma;
  return LUX3D_OK;
}
}  // namespace

// ---- sparse ops --------------------------------------------------------------

namespace {
int contiguous_of(const lux3d_tensor_t *t, const char *fn, const char *name, int dtype, int rank) {
  int r = check_desc(t, fn, name);
  if (r) return r;
  if (dtype >= 0 && t->dtype != dtype) return fail(LUX3D_ERR_DTYPE, "%s: `%s` has the wrong dtype", fn, name);
  if (rank > 0 && t->rank != rank) return fail(LUX3D_ERR_SHAPE, "%s: `%s` must have rank %d", fn, name, rank);
  if (!is_contiguous(t)) return fail(LUX3D_ERR_LAYOUT, "%s: `%s` must be contiguous", fn, name);
  return LUX3D_OK;
}
}  // namespace

int lux3d_sparse_neighbors(const lux3d_tensor_t *coords, const lux3d_tensor_t *keys, const lux3d_tensor_t *vals,
                           const lux3d_tensor_t *nbr, const lux3d_tensor_t *bad_coords, lux3d_stream_t stream) {
  const char *fn = "lux3d_sparse_neighbors";
  int r;
  if ((r = contiguous_of(coords, fn, "coords", LUX3D_I32, 2)) || (r = contiguous_of(keys, fn, "keys", LUX3D_I64, -1)) ||
      (r = contiguous_of(vals, fn, "vals", LUX3D_I32, -1)) || (r = contiguous_of(nbr, fn, "nbr", LUX3D_I32, 2)))
    return r;
  if (bad_coords && ((r = contiguous_of(bad_coords, fn, "bad_coords", LUX3D_I32, -1)) || numel(bad_coords) < 1))
    return r ? r : fail(LUX3D_ERR_SHAPE, "%s: bad_coords must hold one int32", fn);
  const int64_t n = coords->shape[0], cap = numel(keys);
  if (coords->shape[1] != 3) return fail(LUX3D_ERR_SHAPE, "%s: coords must be [N, 3]", fn);
  if (nbr->shape[0] != n || nbr->shape[1] != 27) return fail(LUX3D_ERR_SHAPE, "%s: nbr must be [%lld, 27]", fn,
                                                              (long long)n);
  if (numel(vals) != cap) return fail(LUX3D_ERR_SHAPE, "%s: keys and vals must have the same length", fn);
  if (cap < 2 * n || cap <= 0 || (cap & (cap - 1)))
    return fail(LUX3D_ERR_SHAPE, "%s: the table needs a power-of-two capacity >= 2 N = %lld (got %lld)", fn,
                (long long)(2 * n), (long long)cap);
  if (n > INT32_MAX / 27) return fail(LUX3D_ERR_SHAPE, "%s: too many voxels", fn);
  return hip_status(launch_sparse_map(static_cast<const int32_t *>(coords->data), n,
                                      static_cast<unsigned long long *>(keys->data), static_cast<int32_t *>(vals->data),
                                      cap, static_cast<int32_t *>(nbr->data),
                                      bad_coords ? static_cast<int32_t *>(bad_coords->data) : nullptr,
                                      stream_of(stream)),
                    fn);
}

int lux3d_sparse_neighbors_noalloc(const lux3d_tensor_t *coords, const lux3d_tensor_t *nbr,
                                   const lux3d_tensor_t *bad_coords, lux3d_stream_t stream) {
  const char *fn = "lux3d_sparse_neighbors_noalloc";
  int r;
  if ((r = contiguous_of(coords, fn, "coords", LUX3D_I32, 2)) || (r = contiguous_of(nbr, fn, "nbr", LUX3D_I32, 2)))
    return r;
  if (bad_coords && ((r = contiguous_of(bad_coords, fn, "bad_coords", LUX3D_I32, -1)) || numel(bad_coords) < 1))
    return r ? r : fail(LUX3D_ERR_SHAPE, "%s: bad_coords must hold one int32", fn);
  const int64_t n = coords->shape[0];
  if (coords->shape[1] != 3) return fail(LUX3D_ERR_SHAPE, "%s: coords must be [N, 3]", fn);
  if (nbr->shape[0] != n || nbr->shape[1] != 27) return fail(LUX3D_ERR_SHAPE, "%s: nbr must be [%lld, 27]", fn,
                                                              (long long)n);
  if (n > kNoAllocMaxVoxels)
    return fail(LUX3D_ERR_SHAPE, "%s: %lld voxels exceed the allocation-free table's limit of %lld (use "
                "lux3d_sparse_neighbors with a caller-provided table)", fn, (long long)n, (long long)kNoAllocMaxVoxels);
  return hip_status(launch_sparse_map_noalloc(static_cast<const int32_t *>(coords->data), n,
                                              static_cast<int32_t *>(nbr->data),
                                              bad_coords ? static_cast<int32_t *>(bad_coords->data) : nullptr,
                                              stream_of(stream)),
                    fn);
}

int lux3d_sparse_conv3d(const lux3d_tensor_t *x, const lux3d_tensor_t *nbr, const lux3d_tensor_t *weight,
                        const lux3d_tensor_t *bias, const lux3d_tensor_t *out, lux3d_stream_t stream) {
  const char *fn = "lux3d_sparse_conv3d";
  int r;
  if ((r = contiguous_of(x, fn, "x", LUX3D_F32, 2)) || (r = contiguous_of(nbr, fn, "nbr", LUX3D_I32, 2)) ||
      (r = contiguous_of(weight, fn, "weight", LUX3D_F32, 3)) || (r = contiguous_of(out, fn, "out", LUX3D_F32, 2)))
    return r;
  const int64_t n = x->shape[0], cin = x->shape[1], cout = weight->shape[1];
  if (nbr->shape[0] != n || nbr->shape[1] != 27) return fail(LUX3D_ERR_SHAPE, "%s: nbr must be [%lld, 27]", fn,
                                                              (long long)n);
  if (weight->shape[0] != 27 || weight->shape[2] != cin)
    return fail(LUX3D_ERR_SHAPE, "SparseConv3d expects [N, %lld] with weight [27, Cout, %lld]", (long long)cin,
                (long long)weight->shape[2]);
  if (out->shape[0] != n || out->shape[1] != cout) return fail(LUX3D_ERR_SHAPE, "%s: out must be [%lld, %lld]", fn,
                                                                (long long)n, (long long)cout);
  const float *bp = nullptr;
  if (bias) {
    if ((r = contiguous_of(bias, fn, "bias", LUX3D_F32, -1))) return r;
    if (numel(bias) != cout) return fail(LUX3D_ERR_SHAPE, "%s: bias must have %lld elements", fn, (long long)cout);
    bp = static_cast<const float *>(bias->data);
  }
  SparseConvParams p;
  p.x = static_cast<const float *>(x->data);
  p.nbr = static_cast<const int32_t *>(nbr->data);
  p.w = static_cast<const float *>(weight->data);
  p.bias = bp;
  p.out = static_cast<float *>(out->data);
  p.n = n; p.cin = cin; p.cout = cout;
  p.mfma = cin % 16 == 0 && cin > 0 && aligned16(x->data) && aligned16(weight->data);
  return hip_status(launch_sparse_conv(p, stream_of(stream)), fn);
}

int lux3d_sparse_rulebook(const lux3d_tensor_t *nbr, const lux3d_tensor_t *pairs, const lux3d_tensor_t *counts,
                          lux3d_stream_t stream) {
  const char *fn = "lux3d_sparse_rulebook";
  int r;
  if ((r = contiguous_of(nbr, fn, "nbr", LUX3D_I32, 2)) || (r = contiguous_of(pairs, fn, "pairs", LUX3D_I32, 3)) ||
      (r = contiguous_of(counts, fn, "counts", LUX3D_I32, -1)))
    return r;
  const int64_t n = nbr->shape[0];
  if (nbr->shape[1] != 27) return fail(LUX3D_ERR_SHAPE, "%s: nbr must be [N, 27]", fn);
  if (pairs->shape[0] != 27 || pairs->shape[1] != n || pairs->shape[2] != 2 || numel(counts) != 27)
    return fail(LUX3D_ERR_SHAPE, "%s: pairs must be [27, %lld, 2] and counts [27]", fn, (long long)n);
  if (n > INT32_MAX / 27) return fail(LUX3D_ERR_SHAPE, "%s: too many voxels", fn);
  return hip_status(launch_sparse_rulebook(static_cast<const int32_t *>(nbr->data), n,
                                           static_cast<int32_t *>(pairs->data), static_cast<int32_t *>(counts->data),
                                           stream_of(stream)),
                    fn);
}

int lux3d_sparse_conv3d_rulebook(const lux3d_tensor_t *x, const lux3d_tensor_t *pairs, const lux3d_tensor_t *counts,
                                 const lux3d_tensor_t *weight, const lux3d_tensor_t *bias, const lux3d_tensor_t *out,
                                 lux3d_stream_t stream) {
  const char *fn = "lux3d_sparse_conv3d_rulebook";
  int r;
  if ((r = contiguous_of(x, fn, "x", LUX3D_F32, 2)) || (r = contiguous_of(pairs, fn, "pairs", LUX3D_I32, 3)) ||
      (r = contiguous_of(counts, fn, "counts", LUX3D_I32, -1)) ||
      (r = contiguous_of(weight, fn, "weight", LUX3D_F32, 3)) || (r = contiguous_of(out, fn, "out", LUX3D_F32, 2)))
    return r;
  const int64_t n = x->shape[0], cin = x->shape[1], cout = weight->shape[1];
  if (pairs->shape[0] != 27 || pairs->shape[1] != n || pairs->shape[2] != 2 || numel(counts) != 27)
    return fail(LUX3D_ERR_SHAPE, "%s: pairs must be [27, %lld, 2] and counts [27]", fn, (long long)n);
  if (weight->shape[0] != 27 || weight->shape[2] != cin)
    return fail(LUX3D_ERR_SHAPE, "SparseConv3d expects [N, %lld] with weight [27, Cout, %lld]", (long long)cin,
                (long long)weight->shape[2]);
  if (out->shape[0] != n || out->shape[1] != cout) return fail(LUX3D_ERR_SHAPE, "%s: out must be [%lld, %lld]", fn,
                                                                (long long)n, (long long)cout);
  if (cin % 16 || cin == 0)
    return fail(LUX3D_ERR_SHAPE, "%s: Cin must be a positive multiple of 16 (use lux3d_sparse_conv3d)", fn);
  if (!aligned16(x->data) || !aligned16(weight->data))
    return fail(LUX3D_ERR_LAYOUT, "%s: x and weight must be 16-byte aligned", fn);
  const float *bp = nullptr;
  if (bias) {
    if ((r = contiguous_of(bias, fn, "bias", LUX3D_F32, -1))) return r;
    if (numel(bias) != cout) return fail(LUX3D_ERR_SHAPE, "%s: bias must have %lld elements", fn, (long long)cout);
    bp = static_cast<const float *>(bias->data);
  }
  SparseConvParams p;
  p.x = static_cast<const float *>(x->data);
  p.w = static_cast<const float *>(weight->data);
  p.bias = bp;
  p.out = static_cast<float *>(out->data);
  p.n = n; p.cin = cin; p.cout = cout;
  p.mfma = true;
  return hip_status(launch_sparse_conv_rulebook(p, static_cast<const int32_t *>(pairs->data),
                                                static_cast<const int32_t *>(counts->data), stream_of(stream)),
                    fn);
}

int lux3d_index_select_rows(const lux3d_tensor_t *src, const lux3d_tensor_t *ids, const lux3d_tensor_t *out,
                            const lux3d_tensor_t *bad_ids, lux3d_stream_t stream) {
  const char *fn = "lux3d_index_select_rows";
  int r;
  if ((r = contiguous_of(src, fn, "src", -1, -1)) || (r = contiguous_of(ids, fn, "ids", -1, 1)) ||
      (r = contiguous_of(out, fn, "out", src->dtype, src->rank)))
    return r;
  if (bad_ids && ((r = contiguous_of(bad_ids, fn, "bad_ids", LUX3D_I32, -1)) || numel(bad_ids) < 1))
    return r ? r : fail(LUX3D_ERR_SHAPE, "%s: bad_ids must hold one int32", fn);
  if (ids->dtype != LUX3D_I32 && ids->dtype != LUX3D_I64)
    return fail(LUX3D_ERR_DTYPE, "%s: ids must be int32 or int64", fn);
  if (out->shape[0] != ids->shape[0]) return fail(LUX3D_ERR_SHAPE, "%s: out must have one row per id", fn);
  int64_t row = 1;
  for (int i = 1; i < src->rank; ++i) {
    if (out->shape[i] != src->shape[i]) return fail(LUX3D_ERR_SHAPE, "%s: out rows must match src rows", fn);
    row *= src->shape[i];
  }
  return hip_status(launch_gather_rows(src->data, src->shape[0], ids->data, ids->dtype == LUX3D_I64, ids->shape[0],
                                       nullptr, out->data, row * elem_bytes(src->dtype),
                                       bad_ids ? static_cast<int32_t *>(bad_ids->data) : nullptr, stream_of(stream)),
                    fn);
}

int lux3d_channel_to_spatial(const lux3d_tensor_t *coords, const lux3d_tensor_t *feats, const lux3d_tensor_t *logits,
                             const lux3d_tensor_t *workspace, const lux3d_tensor_t *out_coords,
                             const lux3d_tensor_t *src_rows, const lux3d_tensor_t *out_feats,
                             const lux3d_tensor_t *sub, const lux3d_tensor_t *count, lux3d_stream_t stream) {
  const char *fn = "lux3d_channel_to_spatial";
  int r;
  if ((r = contiguous_of(coords, fn, "coords", LUX3D_I32, 2)) || (r = contiguous_of(feats, fn, "feats", -1, 2)) ||
      (r = contiguous_of(logits, fn, "logits", -1, 2)) || (r = contiguous_of(workspace, fn, "workspace", LUX3D_I32, -1)) ||
      (r = contiguous_of(out_coords, fn, "out_coords", LUX3D_I32, 2)) ||
      (r = contiguous_of(src_rows, fn, "src_rows", LUX3D_I32, -1)) ||
      (r = contiguous_of(out_feats, fn, "out_feats", feats->dtype, 2)) ||
      (r = contiguous_of(count, fn, "count", LUX3D_I32, -1)))
    return r;
  const int64_t n = coords->shape[0], c = feats->shape[1];
  if (coords->shape[1] != 3) return fail(LUX3D_ERR_SHAPE, "%s: coords must be [N, 3]", fn);
  if (feats->shape[0] != n)
    return fail(LUX3D_ERR_SHAPE, "channel_to_spatial coords/features mismatch: %lld coords vs %lld rows",
                (long long)n, (long long)feats->shape[0]);
  if (c % 8) return fail(LUX3D_ERR_SHAPE,
                         "channel_to_spatial expects channels divisible by 8 (layout [child, channel]), got %lld",
                         (long long)c);
  if (!is_float(logits->dtype)) return fail(LUX3D_ERR_DTYPE, "%s: logits must be f32, bf16 or f16", fn);
  if (logits->shape[0] != n || logits->shape[1] != 8)
    return fail(LUX3D_ERR_SHAPE, "subdivision logits must be [%lld, 8], got [%lld, %lld]", (long long)n,
                (long long)logits->shape[0], (long long)logits->shape[1]);
  const int64_t nb = (n + 1023) / 1024;
  if (numel(workspace) < n + nb)
    return fail(LUX3D_ERR_SHAPE, "%s: workspace needs N + ceil(N / 1024) = %lld int32", fn, (long long)(n + nb));
  if (out_coords->shape[0] != 8 * n || out_coords->shape[1] != 3 || numel(src_rows) != 8 * n ||
      out_feats->shape[0] != 8 * n || out_feats->shape[1] != c / 8 || numel(count) != 1)
    return fail(LUX3D_ERR_SHAPE, "%s: outputs must hold 8 N = %lld rows (out_feats [8 N, C / 8]) and count 1", fn,
                (long long)(8 * n));
  float *sp = nullptr;
  if (sub) {
    if ((r = contiguous_of(sub, fn, "sub", LUX3D_F32, -1))) return r;
    if (numel(sub) != 8 * n) return fail(LUX3D_ERR_SHAPE, "%s: sub must be [N, 8]", fn);
    sp = static_cast<float *>(sub->data);
  }
  if (n > INT32_MAX / 8) return fail(LUX3D_ERR_SHAPE, "%s: too many parents", fn);
  C2SParams p;
  p.coords = static_cast<const int32_t *>(coords->data);
  p.feats = feats->data;
  p.logits = logits->data;
  p.logits_dt = logits->dtype;
  p.n = n;
  p.child_row_bytes = (c / 8) * elem_bytes(feats->dtype);
  p.offs = static_cast<int32_t *>(workspace->data);
  p.block_sums = p.offs + n;
  p.out_coords = static_cast<int32_t *>(out_coords->data);
  p.src_rows = static_cast<int32_t *>(src_rows->data);
  p.count = static_cast<int32_t *>(count->data);
  p.out_feats = out_feats->data;
  p.sub = sp;
  return hip_status(launch_c2s(p, stream_of(stream)), fn);
}

}  // extern "C"
