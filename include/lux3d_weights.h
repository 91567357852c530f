/*
 * lux3d_weights.h -- C ABI of the weight-file readers in liblux3d_candle.so:
 * GGUF (the container candle-3d's quantizer writes, weights/quantize.rs:
 * 102-317, and VarBuilder::from_gguf reads, weights/mod.rs:121-140) and
 * safetensors (VarBuilder::from_mmaped_safetensors, weights/mod.rs:134-140).
 *
 * Host only: files are memory-mapped read-only; tensor data pointers point
 * into the mapping and stay valid until the handle is closed. No GPU call is
 * made here; the C++ interface (lux3d_candle.hpp: GgufFile,
 * SafetensorsFile) uploads tensors, repacks Q8_0 weights for the quantized
 * linear and converts dtypes on the device.
 *
 * Every function that can fail returns a negative lux3d_status (or NULL)
 * and leaves a message for lux3d_weights_last_error() (thread-local).
 */
#ifndef LUX3D_WEIGHTS_H
#define LUX3D_WEIGHTS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML tensor types this reader knows the size of (ggml_type ids). */
enum {
  LUX3D_GGML_F32 = 0,
  LUX3D_GGML_F16 = 1,
  LUX3D_GGML_Q8_0 = 8,
  LUX3D_GGML_BF16 = 30
};

/* GGUF metadata value types (gguf_type ids). */
enum {
  LUX3D_GGUF_U8 = 0, LUX3D_GGUF_I8 = 1, LUX3D_GGUF_U16 = 2, LUX3D_GGUF_I16 = 3,
  LUX3D_GGUF_U32 = 4, LUX3D_GGUF_I32 = 5, LUX3D_GGUF_F32 = 6, LUX3D_GGUF_BOOL = 7,
  LUX3D_GGUF_STRING = 8, LUX3D_GGUF_ARRAY = 9, LUX3D_GGUF_U64 = 10,
  LUX3D_GGUF_I64 = 11, LUX3D_GGUF_F64 = 12
};

#define LUX3D_WEIGHTS_MAX_RANK 8

typedef struct lux3d_weights_tensor {
  const char *name;
  int32_t dtype;        /* GGUF: a LUX3D_GGML_* id; safetensors: a lux3d_dtype (LUX3D_F32 ...) */
  int32_t rank;
  int64_t shape[LUX3D_WEIGHTS_MAX_RANK]; /* candle order: the outermost dim first */
  const void *data;     /* into the mapping */
  uint64_t nbytes;
} lux3d_weights_tensor_t;

const char *lux3d_weights_last_error(void);

/* ---- GGUF ------------------------------------------------------------------
 * Versions 1-3; little-endian; `general.alignment` (default 32) aligns the
 * data section and every tensor. GGUF stores dims innermost first; the shape
 * reported here is reversed to candle order, as candle's reader does. A
 * tensor of an unknown ggml type is reported with its type id and
 * nbytes = 0 (it cannot be sized); opening fails only if the file itself is
 * malformed (bad magic, truncation, data past the end of the file). */
typedef struct lux3d_gguf lux3d_gguf_t;
lux3d_gguf_t *lux3d_gguf_open(const char *path);
void lux3d_gguf_close(lux3d_gguf_t *g);
uint32_t lux3d_gguf_version(const lux3d_gguf_t *g);
int64_t lux3d_gguf_tensor_count(const lux3d_gguf_t *g);
/* index of `name`, or -1 */
int64_t lux3d_gguf_find(const lux3d_gguf_t *g, const char *name);
int lux3d_gguf_tensor(const lux3d_gguf_t *g, int64_t index, lux3d_weights_tensor_t *out);
int64_t lux3d_gguf_metadata_count(const lux3d_gguf_t *g);
/* Metadata entry `index`: key, value type and value. Scalars: `value`
 * points at the little-endian bytes, count = 1. Strings: `value` points at
 * the (not NUL-terminated) bytes, count = length. Arrays: `elem_type` is the
 * element type, count the element count, and `value` the packed elements for
 * scalar elements (NULL for arrays of strings or arrays). */
int lux3d_gguf_metadata(const lux3d_gguf_t *g, int64_t index, const char **key, int32_t *type,
                        int32_t *elem_type, const void **value, uint64_t *count);
/* index of metadata `key`, or -1 */
int64_t lux3d_gguf_metadata_find(const lux3d_gguf_t *g, const char *key);

/* ---- safetensors -----------------------------------------------------------
 * u64 header length, a JSON header {name: {dtype, shape, data_offsets}, ...,
 * "__metadata__": {string: string}}, then the data. Dtypes F32, BF16, F16,
 * I32, I64, U8, I8 map to lux3d_dtype codes; other dtypes are reported as -1
 * with their bytes. */
typedef struct lux3d_safetensors lux3d_safetensors_t;
lux3d_safetensors_t *lux3d_safetensors_open(const char *path);
void lux3d_safetensors_close(lux3d_safetensors_t *s);
int64_t lux3d_safetensors_tensor_count(const lux3d_safetensors_t *s);
int64_t lux3d_safetensors_find(const lux3d_safetensors_t *s, const char *name);
int lux3d_safetensors_tensor(const lux3d_safetensors_t *s, int64_t index, lux3d_weights_tensor_t *out);
/* "__metadata__" value for `key` (NUL-terminated), or NULL */
const char *lux3d_safetensors_metadata(const lux3d_safetensors_t *s, const char *key);

#ifdef __cplusplus
}
#endif
#endif /* LUX3D_WEIGHTS_H */
