/*
 * sqx.h — C ABI of libsqx_hip.so, the MI355X (gfx950) kernels behind scratch_llm's quantized-linear
 * path. Every pointer is a device pointer owned by the caller; the library never allocates device
 * memory. Every call is asynchronous on `stream` (a hipStream_t passed as void*) and returns 0 on
 * success or a negative SQX_E_* code, with a message in sqx_last_error() (per host thread).
 *
 * Reference interface each entry point replaces is cited as file:line in andreidhoang/scratch_llm.
 * All tensors are dense row-major with the shapes given.
 */
#ifndef SQX_H_
#define SQX_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* sqx_stream_t; /* hipStream_t */

/* element type tags */
enum {
  SQX_DTYPE_F32 = 0,
  SQX_DTYPE_BF16 = 1,
  SQX_DTYPE_F16 = 2,
};

/* status codes */
enum {
  SQX_OK = 0,
  SQX_E_ARG = -1,   /* bad shape / pointer / dtype: the call was rejected before any launch */
  SQX_E_HIP = -2,   /* a HIP runtime call failed */
  SQX_E_SPACE = -3, /* the workspace passed in is too small */
};

/* Message describing the last failure on this host thread ("" if none). */
const char* sqx_last_error(void);

/* ABI version; bumped on any incompatible change of the entry points below. */
int sqx_abi_version(void);

/* ============================================================================================
 * INT4, group-wise (src/scratch_llm/quant/int4_group.py)
 * ============================================================================================ */

/* quantize_groupwise_int4 (int4_group.py:108-129), symmetric codes in [-8, 7]:
 *   s[r,g] = max(absmax(w[r, g*group:(g+1)*group]) / 7, FLT_MIN)   (IEEE fp32 division)
 *   q[r,c] = clamp(rint(w[r,c] / s[r, c/group]), -8, 7)             (round half to even)
 * w: [rows, cols] of w_dtype (F32 / BF16 / F16, converted exactly to fp32). cols % group == 0.
 * q: int8 [rows, cols]; scales: fp32 [rows, cols/group]. Bit-exact with the reference. */
int sqx_int4_quantize_sym(const void* w, int w_dtype, int64_t rows, int64_t cols, int64_t group,
                          int8_t* q, float* scales, sqx_stream_t stream);

/* pack_int4 (int4_group.py:62-82): packed[i] = (q[2i] & 0xF) << 4 | (q[2i+1] & 0xF); an odd n
 * packs a zero low nibble into the last byte. q: int8 [n]; packed: uint8 [(n+1)/2]. */
int sqx_int4_pack(const int8_t* q, int64_t n, uint8_t* packed, sqx_stream_t stream);

/* unpack_int4 (int4_group.py:85-102): high nibble first, each nibble sign-extended from 4 bits.
 * packed: uint8 [(n+1)/2]; q: int8 [n]. */
int sqx_int4_unpack(const uint8_t* packed, int64_t n, int8_t* q, sqx_stream_t stream);

/* dequantize_groupwise_int4 (int4_group.py:132-142): out[r,c] = fp32(q[r,c]) * scales[r, c/group].
 * q: int8 [rows, cols]; scales: fp32 [rows, cols/group]; out: fp32 [rows, cols]. */
int sqx_int4_dequantize(const int8_t* q, const float* scales, int64_t rows, int64_t cols,
                        int64_t group, float* out, sqx_stream_t stream);

/* Size in bytes of the tiled weight / per-group parameter buffers sqx_int4_tile writes for a
 * [rows, cols] weight (no reference counterpart: this is the kernel's HBM layout). */
int64_t sqx_int4_tiled_weight_bytes(int64_t rows, int64_t cols);
int64_t sqx_int4_tiled_param_count(int64_t rows, int64_t cols, int64_t group);

/* Re-lay int4 codes into the GEMV/GEMM tile layout (no reference counterpart).
 * codes: int8 [rows, cols]; code_kind 0 = signed symmetric codes in [-8, 7] (the reference's
 * format), 1 = unsigned asymmetric codes in [0, 15]. scales (and zeros when code_kind == 1): [rows,
 * cols/group] of param_dtype (F32 or BF16). group must be 32, 64 or 128, and cols % group == 0.
 * Outputs: wt (sqx_int4_tiled_weight_bytes bytes), st (and zt when code_kind == 1):
 * sqx_int4_tiled_param_count elements of param_dtype. Padding rows/columns hold a zero weight. */
int sqx_int4_tile(const int8_t* codes, int code_kind, const void* scales, const void* zeros,
                  int param_dtype, int64_t rows, int64_t cols, int64_t group, uint8_t* wt,
                  void* st, void* zt, sqx_stream_t stream);

/* The same re-lay from the reference's packed byte stream (pack_int4 of the row-major codes,
 * int4_group.py:62-82): packed: uint8 [rows*cols/2], symmetric codes. */
int sqx_int4_tile_packed(const uint8_t* packed, const void* scales, int param_dtype, int64_t rows,
                         int64_t cols, int64_t group, uint8_t* wt, void* st, sqx_stream_t stream);

/* Number of k-slices (waves per 16-row tile) the library picks for a shape when the caller passes
 * k_slices <= 0. */
int sqx_int4_linear_default_kslices(int64_t m, int64_t rows, int64_t cols);

/* W4A16 linear (w4a16_linear, int4_group.py:148-164; awq_linear, awq.py:184-192 once the AWQ
 * channel scale is folded): y[m, r] = sum_c x[m, c] * w[r, c] (+ bias[r]), with
 * w[r, c] = (u - z) * s for the tiled codes u, zero z (8 for symmetric codes) and scale s of the
 * group. x: [m, cols] of act_dtype (BF16 or F16); y: [m, rows] of act_dtype; bias: [rows] of
 * act_dtype or NULL. wt/st/zt from sqx_int4_tile (zt NULL for symmetric codes). fp32 accumulation.
 * Any m >= 1 (processed 64 rows of x per pass). One workgroup per 16-row tile; k_slices (1..16, or
 * <= 0 for the default) waves split its columns and sum their partials in a fixed order, so results
 * are deterministic for a given k_slices. Needs no workspace. */
int sqx_int4_linear(const uint8_t* wt, const void* st, const void* zt, int param_dtype,
                    const void* x, int act_dtype, void* y, const void* bias, int64_t m, int64_t rows,
                    int64_t cols, int64_t group, int k_slices, sqx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SQX_H_ */
