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
  SQX_DTYPE_F64 = 3, /* accepted by sqx_nvfp4_ceil_quantize only */
};

/* FP4 weight formats and the source of their scales for sqx_fp4_tile */
enum {
  SQX_FP4_MX = 0, /* MXFP4: E2M1 codes, E8M0 scale per 32 columns */
  SQX_FP4_NV = 1, /* NVFP4: E2M1 codes, E4M3 scale per 16 columns, fp32 global scale */
};
enum {
  SQX_FP4_SCALE_MX_F32 = 0,  /* MXFP4 s_block as fp32 powers of two [rows, cols/32] */
  SQX_FP4_SCALE_MX_E8M0 = 1, /* MXFP4 scales as E8M0 bytes [rows, cols/32] (the on-disk form) */
  SQX_FP4_SCALE_NV_F32 = 2,  /* NVFP4 s_block as fp32 E4M3 values [rows, cols/16] */
  SQX_FP4_SCALE_NV_E4M3 = 3, /* NVFP4 scales as E4M3 bytes [rows, cols/16] (sqx_nvfp4_ceil_quantize's) */
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
 * sqx_int4_tiled_param_count elements of param_dtype. Asymmetric codes with BF16 parameters instead
 * keep each (scale, zero) pair in one dword of st (scale bits | zero bits << 16: 2 x
 * sqx_int4_tiled_param_count BF16 elements), so the kernels fetch both with one load; zt is then
 * neither written nor read, but must be non-NULL wherever it marks the codes asymmetric (pass st).
 * Padding rows/columns hold a zero weight. */
int sqx_int4_tile(const int8_t* codes, int code_kind, const void* scales, const void* zeros,
                  int param_dtype, int64_t rows, int64_t cols, int64_t group, uint8_t* wt,
                  void* st, void* zt, sqx_stream_t stream);

/* The same re-lay from the reference's packed byte stream (pack_int4 of the row-major codes,
 * int4_group.py:62-82): packed: uint8 [rows*cols/2], symmetric codes. */
int sqx_int4_tile_packed(const uint8_t* packed, const void* scales, int param_dtype, int64_t rows,
                         int64_t cols, int64_t group, uint8_t* wt, void* st, sqx_stream_t stream);

/* The inverse of sqx_int4_tile (no reference counterpart: it gives back the reference's tensors from
 * the kernel layout, so a module can hold the tiled copy only). codes: int8 [rows, cols] (code_kind 0:
 * signed symmetric codes, 1: unsigned asymmetric codes); scales (and zeros for code_kind 1):
 * [rows, cols/group] of param_dtype. Bit-exact round trip. */
int sqx_int4_untile(const uint8_t* wt, const void* st, const void* zt, int param_dtype, int code_kind,
                    int64_t rows, int64_t cols, int64_t group, int8_t* codes, void* scales, void* zeros,
                    sqx_stream_t stream);

/* Number of k-slices (waves per 16-row tile) the decode GEMV takes when sqx_int4_linear runs it
 * with k_slices <= 0; passing this value explicitly always selects the GEMV. */
int sqx_int4_linear_default_kslices(int64_t m, int64_t rows, int64_t cols);

/* W4A16 linear (w4a16_linear, int4_group.py:148-164; awq_linear, awq.py:184-192 once the AWQ
 * channel scale is folded): y[m, r] = sum_c x[m, c] * w[r, c] (+ bias[r]), with
 * w[r, c] = (u - z) * s for the tiled codes u, zero z (8 for symmetric codes) and scale s of the
 * group. x: [m, cols] of act_dtype (BF16 or F16); y: [m, rows] of act_dtype; bias: [rows] of
 * act_dtype or NULL. wt/st/zt from sqx_int4_tile (zt NULL for symmetric codes). fp32 accumulation.
 * Any m >= 1. k_slices 1..16 runs the decode GEMV (one workgroup per 16-row tile, k_slices waves
 * splitting its columns, 64 rows of x per pass). k_slices <= 0 lets the library pick by shape: for
 * 2..64 rows the decode-regime kernels of sqx_int4_skinny (without K splits) where they are faster,
 * otherwise the GEMV with sqx_int4_linear_default_kslices. Sums run in a fixed order, so a call is
 * deterministic for a given shape and k_slices. Needs no workspace. */
int sqx_int4_linear(const uint8_t* wt, const void* st, const void* zt, int param_dtype,
                    const void* x, int act_dtype, void* y, const void* bias, int64_t m, int64_t rows,
                    int64_t cols, int64_t group, int k_slices, sqx_stream_t stream);

/* The same W4A16 linear for 1 <= m <= 64 activation rows (the decode regime of batched serving) with
 * an explicit launch shape. Each wave owns `tiles` 16-row weight tiles and applies each k-block's
 * activation fragments to all of them; the codes' offset is removed through per-group activation
 * sums. variant 0: `waves` (1..8) split each workgroup's k-blocks, tiles 2 or 4. variant 1: the
 * activations are staged through LDS and shared by `waves` compute waves (4, or 8 as two k-groups)
 * that own disjoint tiles (tiles 1, 2 or 4). variant 2: the multi-row GEMV (2 <= m <= 8; one
 * workgroup per tile whose `waves` (0: default, at most 16) take k-slices of at most 8 blocks for
 * m <= 4 or 4 blocks for 5..8 rows in one workgroup, each wave copying its slice of the rows into LDS;
 * tiles = the row groups: 1 = one workgroup per tile, 2 = (5..8 rows) two workgroups of four rows per
 * tile on one XCD, 0 = the library's choice; splits 1). splits >= 1 workgroups split K further and
 * write fp32
 * partials to ws, added in split order by a second kernel. variant < 0 is the library's choice for
 * the shape, the decode GEMV included when tiles, waves and splits are all <= 0; tiles, waves or
 * splits <= 0 pick the default of the variant (splits > 1 only when ws is given). The library may
 * lower `tiles` where the registers would not hold it. Deterministic for a given shape. ws: 16-byte
 * aligned, sqx_int4_skinny_workspace_bytes(m, rows, cols, splits) bytes (0 when splits resolves to
 * 1; splits <= 0 asks for the library choice's). Other arguments and results as sqx_int4_linear. No
 * counterpart in the reference (a launch shape of w4a16_linear, int4_group.py:148-164). */
int64_t sqx_int4_skinny_workspace_bytes(int64_t m, int64_t rows, int64_t cols, int splits);
int sqx_int4_skinny(const uint8_t* wt, const void* st, const void* zt, int param_dtype, const void* x,
                    int act_dtype, void* y, const void* bias, int64_t m, int64_t rows, int64_t cols,
                    int64_t group, int variant, int tiles, int waves, int splits, void* ws,
                    int64_t ws_bytes, sqx_stream_t stream);

/* The K-split count of the library's launch shape for sqx_int4_skinny with a workspace (1 when that
 * shape does not split, the GEMV included). No counterpart in the reference (launch planning). */
int sqx_int4_skinny_default_splits(int64_t m, int64_t rows, int64_t cols);

/* sqx_int4_skinny with the library's shape (which must split K: sqx_int4_skinny_default_splits >= 2),
 * stopping before its reduce: the fp32 partials [S][m][rows] stay in ws, to be added in split order
 * by the consumer (sqx_rmsnorm_partials). No bias. No counterpart in the reference (it fuses the
 * linear's last kernel into the decode step's residual add + RMSNorm, model.py:365-372). */
int sqx_int4_skinny_partials(const uint8_t* wt, const void* st, const void* zt, int param_dtype, const void* x,
                             int act_dtype, int64_t m, int64_t rows, int64_t cols, int64_t group, void* ws,
                             int64_t ws_bytes, sqx_stream_t stream);

/* 1 when sqx_int4_linear_rmsnorm / sqx_int4_linear_silu take m activation rows of cols columns
 * (m <= 8, cols % 8 == 0, m * (cols rounded up to 128, + 8) * 2 <= 64 KiB), else 0. */
int sqx_int4_prologue_fits(int64_t m, int64_t cols);

/* A decode-step linear with the residual add and RMSNorm in front of it (TransformerBlock.forward,
 * model.py:394-403, then RMSNorm, model.py:158-162, then w4a16_linear): h = bf16(x + delta) (written
 * to h_out; delta NULL means h = x and h_out unused), x' = bf16(h * (1 / sqrt(mean(h^2) + eps)) * gain),
 * y = x' @ W^T. Symmetric codes with fp32 scales (sqx_int4_tile code_kind 0), bf16 x/delta/gain/h_out/y
 * ([m, cols], [cols] for gain). Runs the decode GEMV: bit-identical to sqx_rmsnorm followed by
 * sqx_int4_linear with the same k_slices (k_slices <= 0: sqx_int4_linear_default_kslices). */
int sqx_int4_linear_rmsnorm(const uint8_t* wt, const float* st, const void* x, const void* delta,
                            const void* gain, float eps, void* h_out, void* y, int64_t m, int64_t rows,
                            int64_t cols, int64_t group, int k_slices, sqx_stream_t stream);

/* SwiGLU's down projection with its gate in front (model.py:227-237): y = bf16(silu(g) * u) @ W^T with
 * gate_up = bf16 [m, 2 cols] laid out [g | u]. Bit-identical to sqx_silu_mul followed by the linear
 * the library picks for those rows: where that is the multi-row GEMV (2 <= m <= 8, k_slices <= 0;
 * sqx_int4_skinny's variant 2), each wave applies the gate to its own slice of the rows; otherwise the
 * GEMV form of sqx_int4_linear, as for sqx_int4_linear_rmsnorm, whose weight format it takes. */
int sqx_int4_linear_silu(const uint8_t* wt, const float* st, const void* gate_up, void* y, int64_t m,
                         int64_t rows, int64_t cols, int64_t group, int k_slices, sqx_stream_t stream);

/* 1 when sqx_int4_linear_silu takes m rows of a [rows, cols] weight with k_slices <= 0 (the
 * multi-row GEMV's slices, or sqx_int4_prologue_fits), else 0. No reference counterpart. */
int sqx_int4_linear_silu_fits(int64_t m, int64_t rows, int64_t cols);

/* The one-row decode step with the RMSNorm between the linears folded away (model.py:365-372, the
 * block's h = x + attn(attn_norm(x)) and h + ffn(ffn_norm(h))). A linear that feeds the residual
 * stream ends in the residual add and leaves the sums of squares the next norm needs; the linear
 * after the norm forms the norm from those sums while it loads its activations. m is 1, or 2..8 rows
 * through the multi-row form (sqx_int4_rows_fits; sqx_int4_linear_attn_residual takes one row only).
 *
 * sqx_int4_linear_residual: res_out = bf16(res + bf16(x @ W^T)) [rows] (res_out may be res), and
 * ss_out[t] = sum of res_out[16t .. 16t+15]^2 (fp32, ceil(rows/16) entries). With gain_next (bf16
 * [rows], the next RMSNorm's gain) it also writes hg_out = bf16(res_out * gain_next) [rows], the input
 * sqx_int4_linear_rowscale_sumsq takes (both NULL otherwise). The linear is the GEMV form of
 * sqx_int4_linear with the same k_slices, bit for bit, and the add rounds as the reference's bf16
 * tensor add. Weight format as sqx_int4_linear_rmsnorm. */
int sqx_int4_linear_residual(const uint8_t* wt, const float* st, const void* x, const void* res, void* res_out,
                             float* ss_out, const void* gain_next, void* hg_out, int64_t m, int64_t rows, int64_t cols,
                             int64_t group, int k_slices, sqx_stream_t stream);

/* sqx_int4_linear_silu with the residual epilogue of sqx_int4_linear_residual (the MLP's down
 * projection). */
int sqx_int4_linear_silu_residual(const uint8_t* wt, const float* st, const void* gate_up, const void* res,
                                  void* res_out, float* ss_out, const void* gain_next, void* hg_out, int64_t m,
                                  int64_t rows, int64_t cols, int64_t group, int k_slices, sqx_stream_t stream);

/* y = rmsnorm(h) @ W^T for one row h [cols] whose sums of squares per 16 columns are ss [nss],
 * nss = ceil(cols/16) <= 512 (as sqx_int4_linear_residual leaves them): the norm is the reference's
 * RMSNorm (model.py:160-172), bf16(h * (1 / sqrt(sum(ss) / cols + eps)) * gain), with the fp32 sum of
 * squares added in the tiles' order rather than sqx_rmsnorm's, so the normalised row can differ from
 * sqx_rmsnorm's by rounding. gain bf16 [cols], 16-byte aligned. At most 16 k-blocks of 128 columns
 * per wave (the k_slices default satisfies it up to cols = 8192). */
int sqx_int4_linear_rmsnorm_sumsq(const uint8_t* wt, const float* st, const void* h, const float* ss, int64_t nss,
                                  const void* gain, float eps, void* y, int64_t m, int64_t rows, int64_t cols,
                                  int64_t group, int k_slices, sqx_stream_t stream);

/* The same linear after RMSNorm with the norm's row factor moved past the product (one row):
 * y = bf16(r * (hg @ W^T)), r = 1 / sqrt(sum(ss) / cols + eps), where hg = bf16(h * gain) as
 * sqx_int4_linear_residual leaves it and ss the sums of squares of h per 16 columns (nss =
 * ceil(cols/16) <= 512, 16-byte aligned). The reference rounds the normalised row bf16(h * r * gain)
 * once before the product; here bf16(h * gain) is rounded and r scales the fp32 sum, the same bound
 * with another rounding. The GEMV runs its plain one-row form, without a per-wave prologue. */
int sqx_int4_linear_rowscale_sumsq(const uint8_t* wt, const float* st, const void* hg, const float* ss, int64_t nss,
                                   float eps, void* y, int64_t m, int64_t rows, int64_t cols, int64_t group,
                                   int k_slices, sqx_stream_t stream);

/* The SwiGLU linear of a fused gate|up weight in the layout of sqx_int4_linear_rowscale_swiglu (rows
 * alternating in groups of 8, rows a multiple of 16), without the norm's row factor: y [m, rows / 2] =
 * bf16(silu(g) * u) with g, u the bf16 outputs of sqx_int4_linear / sqx_int4_skinny on x [m, cols]
 * (model.py:223-237). 1..64 rows: the one-row GEMV, the multi-row GEMV or a row-tiled kernel by the
 * library's shape choice without K splits; bit for bit that linear (same kernel and shape) followed by
 * sqx_silu_mul_pairs8. Symmetric int4 tiles, fp32 group scales, bf16 x. */
int sqx_int4_linear_swiglu(const uint8_t* wt, const float* st, const void* x, void* y, int64_t m, int64_t rows,
                           int64_t cols, int64_t group, sqx_stream_t stream);

/* sqx_int4_linear_rowscale_sumsq for the decode step's fused gate|up weight with SwiGLU's product in
 * the epilogue (model.py:223-237, SwiGLU.forward's silu(w1 x) * w3 x): the weight's rows alternate in
 * groups of 8 (rows 16t..16t+7 are gate rows 8t..8t+7, rows 16t+8..16t+15 the matching up rows, so
 * rows = 2 d_ff, a multiple of 16), each output is rounded to bf16 as sqx_int4_linear_rowscale_sumsq
 * writes it, and y [m, rows / 2] = bf16(silu(g) * u) per pair, bit for bit sqx_int4_linear_rowscale_sumsq
 * followed by sqx_silu_mul_pairs8. m is 1 (rows the one-row form takes) or 2..8 (sqx_int4_rows_fits). */
int sqx_int4_linear_rowscale_swiglu(const uint8_t* wt, const float* st, const void* hg, const float* ss, int64_t nss,
                                    float eps, void* y, int64_t m, int64_t rows, int64_t cols, int64_t group,
                                    int k_slices, sqx_stream_t stream);

/* The decode step's fused q|k|v projection at one row with RoPE and the slot-cache write in its epilogue
 * (model.py:205-224, 281-305; kv_cache.py:194-205): the one-row GEMV of x [cols] (with ss given, the
 * row factor of sqx_int4_linear_rowscale_sumsq: x is bf16(h * gain) and ss the sums of squares of h),
 * rows = (n_heads + 2 n_kv_heads) * 128 laid out [q | k | v]. With p = lengths[0]: q and k are rotated
 * at position min(p, rope_rows - 1) as sqx_rope_kv rotates them (bf16 outputs, separate fp32
 * products and sums), q into q_out [n_heads * 128], k and v stored at row min(p, tmax - 1) of
 * k_cache / v_cache [n_kv_heads, tmax, 128] (one layer, one slot; bf16). The rotated bf16 values
 * equal sqx_rope_kv's on this linear's output. One row: fewer than 1024 row tiles. 2..8 rows (m): the
 * multi-row form below, row r at position lengths[r], x, q_out and the sums row after row, k_cache /
 * v_cache [m, n_kv_heads, tmax, 128] (one layer, m slots). */
int sqx_int4_linear_rope_kv(const uint8_t* wt, const float* st, const void* x, const float* ss, int64_t nss,
                            float eps, const int* lengths, const float* cos_t, const float* sin_t, int64_t rope_rows,
                            int64_t n_heads, int64_t n_kv_heads, int64_t tmax, void* q_out, void* k_cache,
                            void* v_cache, int64_t m, int64_t rows, int64_t cols, int64_t group, int k_slices,
                            sqx_stream_t stream);

/* 2..8 rows of the decode step's fused linears (sqx_int4_linear_residual, _silu_residual,
 * _rowscale_sumsq, _rope_kv with m >= 2) run on the multi-row GEMV (sqx_int4_skinny's variant 2):
 * every array is row after row ([m, cols] inputs, [m, rows] outputs, sums of squares [m, ceil(n/16)]
 * with n the columns they cover, a multiple of 4 for the row factor), each row computed as the one-row
 * form computes it, k_slices <= 0 the form's default waves. 1 when that form takes m rows of a [rows,
 * cols] weight (scale_sum: with the row factor's sums in LDS), else 0. No reference counterpart. */
int sqx_int4_rows_fits(int64_t m, int64_t rows, int64_t cols, int scale_sum);

/* Build-defined asymmetric uint4, group-wise (BASELINE config 2's "asymmetric, bf16 scale/zero";
 * no reference symbol: the 4-bit form of quantize_affine, int8.py:142-172, per group):
 * lo = min(min(w_g), 0), hi = max(max(w_g), 0), s = max((hi - lo) / 15, 1e-12) (rounded to bf16 first
 * when param_dtype is BF16), z = clamp(rint(-lo / s), 0, 15), q = clamp(rint(w / s + z), 0, 15).
 * q: uint8 [rows, cols]; scales, zeros: [rows, cols/group] of param_dtype (F32 or BF16). */
int sqx_int4_quantize_asym(const void* w, int w_dtype, int64_t rows, int64_t cols, int64_t group,
                           int param_dtype, uint8_t* q, void* scales, void* zeros, sqx_stream_t stream);

/* ============================================================================================
 * AWQ (src/scratch_llm/quant/awq.py)
 * ============================================================================================ */

/* quantize_awq_int4 with a channel scale (awq.py:154-175): the group-int4 codes and scales of the fp32
 * product w * chan_scale[col] (quantize_groupwise_int4 of W * s). Bit-exact. */
int sqx_awq_quantize(const void* w, int w_dtype, const float* chan_scale, int64_t rows, int64_t cols,
                     int64_t group, int8_t* q, float* scales, sqx_stream_t stream);

/* _awq_dequant_weight (awq.py:115-119): w_eff = dequant(quantize(W * s)) / s, fp32 [rows, cols]. */
int sqx_awq_fake_quant(const void* w, int w_dtype, const float* chan_scale, int64_t rows, int64_t cols,
                       int64_t group, float* w_eff, sqx_stream_t stream);

/* awq_dequantize (awq.py:178-181): out = q * group_scale / chan_scale[col], fp32 [rows, cols]. */
int sqx_awq_dequantize(const int8_t* q, const float* group_scales, const float* chan_scale, int64_t rows,
                       int64_t cols, int64_t group, float* out, sqx_stream_t stream);

/* act_scale (awq.py:94-101): out[c] = mean_r |x[r, c]| (fp64 accumulation, one rounding to fp32). */
int sqx_col_absmean(const void* x, int dtype, int64_t rows, int64_t cols, float* out, sqx_stream_t stream);

/* The channel scale of one AWQ grid point (awq.py:104-112, 141-142):
 * s = max(act ** ratio, 1e-4); out = s / sqrt(max(s) * min(s)). act, out: fp32 [n]. */
int sqx_awq_scale(const float* act, int64_t n, float ratio, float* out, sqx_stream_t stream);

/* out[r, c] = x[r, c] / s[c] rounded to act_dtype (BF16 or F16): the activations of the AWQ linear,
 * which folds 1/s into x (awq.py:15-16). */
int sqx_scale_columns(const void* x, int act_dtype, const float* s, int64_t rows, int64_t cols, void* out,
                      sqx_stream_t stream);

/* AWQ linear (awq_linear, awq.py:184-192): the W4A16 linear of the codes of W*s with the per-input
 * channel AWQ scale s folded into the activations, y = (x / s) @ (q*gs)^T; x / s is computed in fp32
 * per element and rounded to act_dtype while the workgroup copies x into LDS. col_scale: fp32 [cols].
 * Needs m <= 16 and m * (cols rounded up to 128, + 8) * 2 <= 66 KiB (larger inputs: divide x first,
 * then sqx_int4_linear).
 * Other arguments as sqx_int4_linear. */
int sqx_int4_linear_colscaled(const uint8_t* wt, const void* st, const void* zt, int param_dtype,
                              const void* x, int act_dtype, const float* col_scale, void* y,
                              const void* bias, int64_t m, int64_t rows, int64_t cols, int64_t group,
                              int k_slices, sqx_stream_t stream);

/* ============================================================================================
 * FP4: E2M1 codes with E4M3 (NVFP4) or E8M0 (MXFP4) block scales
 * (src/scratch_llm/quant/nvfp4_mxfp4.py). Bit-exact with the reference's fp32 arithmetic.
 * ============================================================================================ */

/* e2m1_round_to_code (nvfp4_mxfp4.py:85-98): codes[i] = sign(x<0) << 3 | index of the nearest
 * E2M1 magnitude by fp32 distance (first index on ties, NaN -> 0). x: n elements of dtype. */
int sqx_e2m1_round(const void* x, int dtype, int64_t n, uint8_t* codes, sqx_stream_t stream);

/* e2m1_decode (nvfp4_mxfp4.py:101-106): out[i] = +-FP4_MAGNITUDES[codes[i] & 7] (fp32). */
int sqx_e2m1_decode(const uint8_t* codes, int64_t n, float* out, sqx_stream_t stream);

/* pack_fp4 / unpack_fp4 (nvfp4_mxfp4.py:109-129): packed[i] = codes[2i] | codes[2i+1] << 4 (low nibble
 * = even element); an odd n pads a zero code. packed: (n+1)/2 bytes. */
int sqx_fp4_pack(const uint8_t* codes, int64_t n, uint8_t* packed, sqx_stream_t stream);
int sqx_fp4_unpack(const uint8_t* packed, int64_t n, uint8_t* codes, sqx_stream_t stream);

/* quantize_e4m3 (nvfp4_mxfp4.py:135-147) and quantize_e8m0 (:150-159), fp32 in and out. */
int sqx_quantize_e4m3(const float* v, int64_t n, float* out, sqx_stream_t stream);
int sqx_quantize_e8m0(const float* v, int64_t n, float* out, sqx_stream_t stream);

/* mxfp4_quantize (nvfp4_mxfp4.py:257-265) of the flattened x (n elements, zero-padded to whole
 * blocks): codes uint8 [n_blocks*block] (one code per byte, unpacked), s_block fp32 [n_blocks]
 * (2**ceil(log2(max(amax/6, 1e-30))), exponent clamped to +-127), and optionally e8m0 uint8
 * [n_blocks] (exponent + 127; NULL to skip). n_blocks = ceil(n / block). */
int sqx_mxfp4_quantize(const void* x, int dtype, int64_t n, int64_t block, uint8_t* codes,
                       float* s_block, uint8_t* e8m0, sqx_stream_t stream);

/* mxfp4_dequantize(mxfp4_quantize(x)) (nvfp4_mxfp4.py:257-272) of each row of x [m, k] (dtype F32 /
 * BF16 / F16, k a multiple of 32, 16-byte aligned), written as bf16 rows out [m, k]: every value is
 * exact in bf16 where it is finite in fp32. Config 4's activation-quantized linear at a few rows runs
 * these rows through the MXFP4 weight GEMV (the products of the two dequantized operands). */
int sqx_mxfp4_fake_quant_rows(const void* x, int dtype, int64_t m, int64_t k, uint16_t* out, sqx_stream_t stream);

/* mxfp4_dequantize (nvfp4_mxfp4.py:268-272): out[i] = decode(codes[i]) * s_block[i / block], i < n. */
int sqx_mxfp4_dequantize(const uint8_t* codes, const float* s_block, int64_t n, int64_t block,
                         float* out, sqx_stream_t stream);

/* Workspace bytes sqx_nvfp4_quantize needs (partial maxima of |x|). */
int64_t sqx_nvfp4_workspace_bytes(void);

/* nvfp4_quantize (nvfp4_mxfp4.py:212-223): s_global = max(amax(|x|) / 2688, 1e-30) (written to the
 * device fp32 *s_global), s_block[b] = quantize_e4m3(block_amax / 6 / s_global), codes =
 * e2m1(x / max(s_global * s_block, 1e-30)). Layout as sqx_mxfp4_quantize. */
int sqx_nvfp4_quantize(const void* x, int dtype, int64_t n, int64_t block, uint8_t* codes,
                       float* s_block, float* s_global, void* workspace, int64_t workspace_bytes,
                       sqx_stream_t stream);

/* nvfp4_dequantize (nvfp4_mxfp4.py:226-231): out[i] = decode(codes[i]) * (s_global * s_block[i/block]). */
int sqx_nvfp4_dequantize(const uint8_t* codes, const float* s_block, const float* s_global, int64_t n,
                         int64_t block, float* out, sqx_stream_t stream);

/* Bytes of the tiled FP4 weight and scale buffers sqx_fp4_tile writes for a [rows, cols] weight
 * (no reference counterpart: the kernels' HBM layout). fmt: SQX_FP4_MX or SQX_FP4_NV. */
int64_t sqx_fp4_tiled_weight_bytes(int64_t rows, int64_t cols);
int64_t sqx_fp4_tiled_scale_bytes(int64_t rows, int64_t cols, int fmt);

/* Re-lay an FP4 weight [rows, cols] for the linear kernels (no reference counterpart). codes: the
 * E2M1 codes, unpacked (codes_packed = 0, one per byte) or in the reference's packed row-major
 * stream (codes_packed = 1, pack_fp4 order, also the on-disk weight_packed of k3/checkpoint.py:92-144).
 * scales by scale_kind, one per `block` columns of a row: SQX_FP4_SCALE_MX_F32 (s_block fp32
 * [rows, cols/block], block a multiple of 32), SQX_FP4_SCALE_MX_E8M0 (bytes, same shape),
 * SQX_FP4_SCALE_NV_F32 (s_block fp32 E4M3 values [rows, cols/block], block a multiple of 16) or
 * SQX_FP4_SCALE_NV_E4M3 (the same scales as E4M3 bytes). */
int sqx_fp4_tile(const uint8_t* codes, int codes_packed, const void* scales, int scale_kind, int64_t block,
                 int64_t rows, int64_t cols, uint8_t* wt, uint8_t* st, sqx_stream_t stream);

/* The inverse of sqx_fp4_tile (no reference counterpart): packed uint8 [rows, cols/2] in the
 * reference's pack_fp4 order (the on-disk weight_packed), scales uint8 row-major: E8M0 [rows, cols/32]
 * (fmt SQX_FP4_MX) or E4M3 [rows, cols/16] (SQX_FP4_NV, one byte per 16-column block). */
int sqx_fp4_untile(const uint8_t* wt, const uint8_t* st, int fmt, int64_t rows, int64_t cols, uint8_t* packed,
                   uint8_t* scales, sqx_stream_t stream);

/* dequantize_mxfp4 into float64 (k3/checkpoint.py:92-144): out[r, c] = E2M1(code) * 2**(s - 127) for
 * the on-disk pair, packed uint8 [rows, cols/2] (low nibble = even column) and E8M0 bytes uint8
 * [rows, cols/32]; every value is exact in float64. out: float64 [rows, cols], 16-byte aligned. The
 * caller refuses scale byte 0xFF (NaN) beforehand, as the reference does. */
int sqx_mxfp4_pair_dequantize_f64(const uint8_t* packed, const uint8_t* scales, int64_t rows, int64_t cols,
                                  double* out, sqx_stream_t stream);

/* The second NVFP4 convention, the b_r6 GEMM rung's operands (kernels/gemm/cuda/b_r6.py:155-244 with
 * kernels/gemm/nvfp4_layout.py:341-416). Per block of 16 along k, in float64: scale = the smallest
 * unsigned-E4M3 value >= amax / 6 (ceil onto the grid; no global scale; an all-zero block gets 0),
 * code = the nearest E2M1 magnitude of x / scale with ties to the even magnitude index (saturating
 * at 6), the sign bit only on a non-zero magnitude. x: [rows, k] of dtype (F32 / BF16 / F16 / F64; the
 * block amax and every quotient are float64, as the reference's x.to(float64)), k a
 * multiple of 16; packed: uint8 [rows, k/2], the lower k in the low nibble (the reference's bytes);
 * scales: uint8 [rows, k/16] row-major E4M3 codes (the reference swizzles them for CUTLASS; this
 * layout is the library's). *status (device int, zeroed by the caller) gets bit 0 for a NaN or Inf
 * input and bit 1 for a block whose amax / 6 exceeds 448; the reference raises on both. */
int sqx_nvfp4_ceil_quantize(const void* x, int dtype, int64_t rows, int64_t k, uint8_t* packed,
                            uint8_t* scales, int* status, sqx_stream_t stream);

/* dequantize_nvfp4 (b_r6.py:228-244): out = e2m1 value * scale, exact in F32 and in BF16 (out_dtype). */
int sqx_nvfp4_ceil_dequantize(const uint8_t* packed, const uint8_t* scales, int64_t rows, int64_t k, void* out,
                              int out_dtype, sqx_stream_t stream);

/* Elementwise forms of the scalar rules (nvfp4_layout.py:341-416) over float64 device arrays:
 * sqx_ue4m3_ceil: codes[i] = ue4m3_ceil_code(v[i] / divisor) and values[i] its value (values may be
 * NULL); divisor 6 gives scale_for_amax (amax 0 -> code 0). Status bit 0: a negative or non-finite
 * v; bit 1: v / divisor > 448 (the code is then 0). sqx_e2m1_round_rne: e2m1_round_code (status bit
 * 0 for NaN or Inf), with the scalar rule's sign bit: set for every v < 0, so a negative v that
 * rounds to magnitude 0 gives 0x8 (nvfp4_layout.py:402), unlike the quantizer's canonical +0. */
int sqx_ue4m3_ceil(const double* v, int64_t n, double divisor, uint8_t* codes, double* values, int* status,
                   sqx_stream_t stream);
int sqx_e2m1_round_rne(const double* v, int64_t n, uint8_t* codes, int* status, sqx_stream_t stream);

/* FP4 weight linear: y[m, r] = sum_c x[m, c] * W[r, c] (* *s_global for NVFP4) (+ bias[r]) with W the
 * dequantized tiled weight: the config-4 MXFP4 linear F.linear(x, mxfp4_dequantize(W).to(x.dtype))
 * (nvfp4_mxfp4.py:268-272 composed with F.linear) and the NVFP4 block-scaled linear
 * (quant_linear_nvfp4, nvfp4_mxfp4.py:296-328). x: [m, cols] BF16 or F16; y: [m, rows] of act_dtype
 * or F32 (y_dtype); bias: [rows] of act_dtype or NULL (needs y_dtype == act_dtype); s_global: the
 * NVFP4 global scale, a device fp32 (NULL for MXFP4). fp32 accumulation; k_slices as
 * sqx_int4_linear. */
int sqx_fp4_linear(const uint8_t* wt, const uint8_t* st, int fmt, const float* s_global, const void* x,
                   int act_dtype, void* y, int y_dtype, const void* bias, int64_t m, int64_t rows,
                   int64_t cols, int k_slices, sqx_stream_t stream);

/* mxfp4_quantize (nvfp4_mxfp4.py:257-265, block 32) of each row of x [m, k] (k a multiple of 32, so
 * every block lies in one row), written in the tiled FP4 layout sqx_fp4_tile produces: xt
 * (sqx_fp4_tiled_weight_bytes(m, k) bytes) and E8M0 scale bytes xst (sqx_fp4_tiled_scale_bytes(m, k,
 * SQX_FP4_MX)). Codes and scales are bit-exact with the reference's; this is the activation side
 * of the config-4 MXFP4 x MXFP4 linear. x: F32, BF16 or F16, 16-byte aligned. */
int sqx_mxfp4_quantize_tiled(const void* x, int dtype, int64_t m, int64_t k, uint8_t* xt, uint8_t* xst,
                             sqx_stream_t stream);

/* MXFP4 x MXFP4 GEMM on the block-scaled fp4 MFMA: y[i, r] = sum_c X[i, c] W[r, c] (+ bias[r]) with
 * X = mxfp4_dequantize of the tiled activations (xt, xst from sqx_mxfp4_quantize_tiled) and W of the
 * tiled weight (wt, st from sqx_fp4_tile with MXFP4 scales). Replaces the config-4 composition
 * F.linear(mxfp4_dequantize(mxfp4_quantize(x)), mxfp4_dequantize(W)) (nvfp4_mxfp4.py:257-272 with
 * F.linear); this is the mxfp4 GEMM export with act_fmt = MXFP4. fp32 accumulation;
 * y [m, rows] of y_dtype (BF16, F16 or F32); bias (NULL or [rows] of y_dtype, not with F32).
 * One pass per 256 x 256 output tile: for few output tiles (small m) use sqx_mxfp4_gemm_ws. */
int sqx_mxfp4_gemm(const uint8_t* xt, const uint8_t* xst, const uint8_t* wt, const uint8_t* wst, void* y,
                   int y_dtype, const void* bias, int64_t m, int64_t rows, int64_t cols, sqx_stream_t stream);

/* Workspace bytes sqx_mxfp4_gemm_ws needs for a shape and a number of K splits (splits <= 0: the
 * automatic choice; 0 bytes when that is one split). */
int64_t sqx_mxfp4_gemm_workspace_bytes(int64_t m, int64_t rows, int64_t cols, int splits);

/* sqx_mxfp4_gemm with the k range split over `splits` workgroups per output tile (1..16; <= 0: the
 * automatic choice, which splits when the output tiles leave CUs idle and falls back to one pass when
 * ws is NULL or too small). Each split writes fp32 partial sums to ws ([splits][m][rows], 16-byte
 * aligned); a second kernel adds them in split order, adds the bias and rounds to y_dtype, so the
 * result is deterministic for a given shape and split count and differs from the one-pass result
 * only by the order of the fp32 additions. An explicit split count that leaves a split empty is
 * refused (SQX_E_ARG); a workspace smaller than it needs returns SQX_E_SPACE. */
int sqx_mxfp4_gemm_ws(const uint8_t* xt, const uint8_t* xst, const uint8_t* wt, const uint8_t* wst, void* y,
                      int y_dtype, const void* bias, int64_t m, int64_t rows, int64_t cols, int splits, void* ws,
                      int64_t ws_bytes, sqx_stream_t stream);

/* Prefill / large-batch W4A16 GEMM (the int4 GEMM export): the same operation and tiled weight as
 * sqx_int4_linear (w4a16_linear, int4_group.py:148-164, and the AWQ linear awq.py:184-192 on x / s),
 * for any m, on the bf16 / fp16 MFMA with the weight tile decoded in registers to the reference's
 * bf16(fp32((q - z) * s)). group: 32, 64 or 128; cols a multiple of 32 and of group. y [m, rows] in
 * act_dtype; bias NULL or [rows] in act_dtype. ws: see sqx_gemm_workspace_bytes. */
int sqx_int4_gemm(const uint8_t* wt, const void* st, const void* zt, int param_dtype, const void* x,
                  int act_dtype, void* y, const void* bias, int64_t m, int64_t rows, int64_t cols, int64_t group,
                  void* ws, int64_t ws_bytes, sqx_stream_t stream);

/* Workspace bytes the prefill GEMMs (sqx_int4_gemm, sqx_fp4_gemm) use for a shape: when few output
 * tiles would leave CUs idle, the k range is split over workgroups that write fp32 partial sums to
 * the workspace, added in a fixed order by a second kernel (deterministic). 0 = no split. A NULL or
 * smaller workspace runs without the split (same result, slower for small m). */
int64_t sqx_gemm_workspace_bytes(int64_t m, int64_t rows, int64_t cols);

/* W4A16 linear with fp32 activations (w4a16_linear, int4_group.py:157-164, and awq_linear,
 * awq.py:184-192, which accept any x.dtype and then run F.linear in fp32): x [m, cols] fp32,
 * optionally divided by col_scale [cols] (the AWQ channel scale; NULL for none), splits into the
 * bf16 rows a = bf16(v), b = bf16(v - a), c = bf16(v - a - b), whose sum is v exactly for normal v;
 * the 3m rows run through the int4 decode GEMV with fp32 outputs (exact code products, fp32 group
 * scales, 64 rows per pass over the weight; the prefill GEMM's bf16 weight decode is not
 * fp32-faithful), and y [m, rows] fp32 = (y_a + y_b) + y_c (+ bias [rows] fp32, or NULL). Weight
 * arguments as sqx_int4_linear. ws: device workspace of at least
 * sqx_int4_linear_f32_workspace_bytes(m, rows, cols), 256-byte aligned. */
int64_t sqx_int4_linear_f32_workspace_bytes(int64_t m, int64_t rows, int64_t cols);
int sqx_int4_linear_f32(const uint8_t* wt, const void* st, const void* zt, int param_dtype, const float* x,
                        const float* col_scale, float* y, const float* bias, int64_t m, int64_t rows, int64_t cols,
                        int64_t group, void* ws, int64_t ws_bytes, sqx_stream_t stream);

/* Prefill / large-batch FP4-weight GEMM with BF16 / F16 activations (the mxfp4 GEMM export with
 * act_fmt = bf16, and the nvfp4 GEMM): the same operation and tiled weight as sqx_fp4_linear (the
 * config-4 F.linear(x, mxfp4_dequantize(W).to(x.dtype)) and the NVFP4 linear) on the 16-bit MFMA,
 * each weight decoded in registers (MXFP4 exactly; NVFP4 as e2m1 * s_block with *s_global applied to
 * the fp32 result). cols a multiple of 32; y_dtype act_dtype or F32; bias as sqx_fp4_linear. */
int sqx_fp4_gemm(const uint8_t* wt, const uint8_t* st, int fmt, const float* s_global, const void* x,
                 int act_dtype, void* y, int y_dtype, const void* bias, int64_t m, int64_t rows, int64_t cols,
                 void* ws, int64_t ws_bytes, sqx_stream_t stream);

/* fp32 activations as two bf16 rows (quant_linear_nvfp4 keeps x in fp32): hi = bf16(x),
 * lo = bf16(x - hi); sqx_sum_halves: y[i] = y2[i] + y2[n + i] (the two rows' products). */
int sqx_split_bf16(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, sqx_stream_t stream);
int sqx_sum_halves(const float* y2, int64_t n, float* y, sqx_stream_t stream);

/* ============================================================================================
 * INT8 (src/scratch_llm/quant/int8.py). The input is viewed as [A, B, C] with B the kept axis of the
 * reference's `axis` argument (A = product of the dims before it, C = product of those after it);
 * axis=None is A = C = 1, B = 1 over all elements. Scales (and zero-points) have B elements in the
 * input's dtype, and every intermediate is rounded to that dtype where torch rounds it, so codes and
 * scales are bit-exact with the reference for fp32, bf16 and fp16 inputs.
 * ============================================================================================ */

/* Workspace bytes a per-tensor (B == 1) quantize needs. */
int64_t sqx_int8_workspace_bytes(void);

/* quantize_symmetric (int8.py:102-125): s = max(amax(|x|) / 127, eps), q = clamp(rint(x / s), +-127).
 * x: A*B*C elements of dtype; q: int8, same count; s: B elements of dtype. */
int sqx_int8_quantize_sym(const void* x, int dtype, int64_t A, int64_t B, int64_t C, float eps,
                          int8_t* q, void* s, void* workspace, int64_t workspace_bytes,
                          sqx_stream_t stream);

/* quantize_affine (int8.py:142-172): lo = min(min(x), 0), hi = max(max(x), 0),
 * s = max((hi - lo) / 255, eps), z = clamp(rint(-lo / s), 0, 255), q = clamp(rint(x / s + z), 0, 255).
 * q: uint8; s, z: B elements of dtype. */
int sqx_int8_quantize_affine(const void* x, int dtype, int64_t A, int64_t B, int64_t C, float eps,
                             uint8_t* q, void* s, void* z, void* workspace, int64_t workspace_bytes,
                             sqx_stream_t stream);

/* dequantize_symmetric (int8.py:128-130): out = q * s; dequantize_affine (int8.py:175-177):
 * out = (q - z) * s; in the scale dtype, with the [A, B, C] view of sqx_int8_quantize_*. */
int sqx_int8_dequantize_sym(const int8_t* q, int64_t A, int64_t B, int64_t C, const void* s, int dtype,
                            void* out, sqx_stream_t stream);
int sqx_int8_dequantize_affine(const uint8_t* q, int64_t A, int64_t B, int64_t C, const void* s,
                               const void* z, int dtype, void* out, sqx_stream_t stream);

/* w8a8_linear's integer GEMM and epilogue (int8.py:189-213): y[m, n] = fp32(sum_k qx[m,k] * qw[n,k])
 * * (sx[m] * sw[n]) with int32 accumulation (k <= 131072) and the scale product in the promoted
 * dtype of the two scales. qx: int8 [m, k]; qw: int8 [n, k]; sx: [m], sw: [n]; y: fp32 [m, n]. */
int sqx_w8a8_gemm(const int8_t* qx, const void* sx, int sx_dtype, const int8_t* qw, const void* sw,
                  int sw_dtype, float* y, int64_t m, int64_t n, int64_t k, sqx_stream_t stream);

/* Bytes of the tiled int8 weight (16-row x 64-column blocks of 1 KiB; no reference counterpart). */
int64_t sqx_int8_tiled_weight_bytes(int64_t rows, int64_t cols);

/* Re-lay symmetric int8 codes q [rows, cols] for sqx_int8_linear (no reference counterpart). */
int sqx_int8_tile(const int8_t* q, int64_t rows, int64_t cols, uint8_t* wt, sqx_stream_t stream);

/* The inverse of sqx_int8_tile (no reference counterpart): q int8 [rows, cols]. */
int sqx_int8_untile(const uint8_t* wt, int64_t rows, int64_t cols, int8_t* q, sqx_stream_t stream);

/* Int8 weight-only linear, BASELINE config 1 (quantize_symmetric(W, axis=0) + dequantize_symmetric,
 * int8.py:102-130, composed with F.linear): y[m, r] = scale[r] * sum_c x[m, c] * q[r, c] (+ bias[r]).
 * x: [m, cols] BF16 or F16 (cols % 8 == 0); y: [m, rows] of act_dtype; scale: fp32 [rows]; bias:
 * [rows] of act_dtype or NULL. fp32 accumulation; k_slices as sqx_int4_linear. */
int sqx_int8_linear(const uint8_t* wt, const float* scale, const void* x, int act_dtype, void* y,
                    const void* bias, int64_t m, int64_t rows, int64_t cols, int k_slices,
                    sqx_stream_t stream);

/* ============================================================================================
 * FP8 E4M3 (src/scratch_llm/quant/fp8_weights.py, fp8_kv_per_head.py). Codes are OCP e4m3fn bytes
 * (torch.float8_e4m3fn); every quantizer is saturating_cast_e4m3 (clamp to +-448, round to nearest
 * even; fp8_weights.py:117-124) of fp32(x) / scale, bit-exact with the reference.
 * ============================================================================================ */

/* quantize_per_channel (fp8_weights.py:133-143) of a weight [rows, cols], or quantize_per_token
 * (:146-155) of activations [rows, cols]: scale[r] = max(amax_c |x[r, c]| / 448, 1 / (448 * 512)) in
 * fp32, codes[r, c] = saturating_cast(fp32(x[r, c]) / scale[r]). x: F32 / BF16 / F16. */
int sqx_fp8_quantize_rows(const void* x, int dtype, int64_t rows, int64_t cols, uint8_t* codes, float* scale,
                          sqx_stream_t stream);

/* dequantize (fp8_weights.py:158-160): out[r, c] = fp32(codes[r, c]) * scale[r]; out fp32. */
int sqx_fp8_dequantize_rows(const uint8_t* codes, const float* scale, int64_t rows, int64_t cols, float* out,
                            sqx_stream_t stream);

/* per_head_amax / per_head_scale (fp8_kv_per_head.py:77-91) of a KV block x [B, H, inner]
 * (inner = T * D): amax[h] = max over (b, t, d) of |x| and scale[h] = max(amax[h] / 448,
 * 1 / (448 * 512)), fp32 [H] each (either pointer may be NULL). */
int sqx_fp8_head_scale(const void* x, int dtype, int64_t B, int64_t H, int64_t inner, float* amax, float* scale,
                       sqx_stream_t stream);

/* quantize_per_head (fp8_kv_per_head.py:93-96): codes = saturating_cast(fp32(x) / scale[h]) over
 * [B, H, inner]. saturated (NULL or one uint64 in device memory): incremented by the number of
 * elements with |x| > 448 * scale[h] (saturated_count, :104-107). */
int sqx_fp8_quantize_heads(const void* x, int dtype, int64_t B, int64_t H, int64_t inner, const float* scale,
                           uint8_t* codes, unsigned long long* saturated, sqx_stream_t stream);

/* dequantize_per_head (fp8_kv_per_head.py:99-101): out = fp32(codes) * scale[h], fp32 [B, H, inner]. */
int sqx_fp8_dequantize_heads(const uint8_t* codes, const float* scale, int64_t B, int64_t H, int64_t inner,
                             float* out, sqx_stream_t stream);

/* Bytes of the tiled FP8 weight and its re-lay from codes [rows, cols] (no reference counterpart:
 * 1 KiB blocks of 16 rows x 64 columns). */
int64_t sqx_fp8_tiled_weight_bytes(int64_t rows, int64_t cols);
int sqx_fp8_tile(const uint8_t* codes, int64_t rows, int64_t cols, uint8_t* wt, sqx_stream_t stream);

/* fp8_linear (fp8_weights.py:211-262): x [m, cols] (F32 / BF16 / F16) is quantized per token,
 * y[i, r] = (sum_c qx[i, c] * qw[r, c]) * s_x[i] * w_scale[r] (+ bias[r]) with exact products and fp32
 * accumulation; y [m, rows] of y_dtype (BF16, or F32 without bias); bias BF16 or NULL. wt from
 * sqx_fp8_tile; w_scale fp32 [rows]. cols % 8 == 0. ws: sqx_fp8_linear_workspace_bytes(m, rows, cols)
 * bytes (the quantized activations and, where the library's launch splits K, fp32 partial sums),
 * 16-byte aligned. k_slices <= 0 lets the library pick the launch: for 2..64 rows and a BF16 output
 * the kernel of sqx_fp8_skinny where it is faster, otherwise the GEMV (k_slices > 0: the GEMV with
 * that many waves per tile). */
int64_t sqx_fp8_linear_workspace_bytes(int64_t m, int64_t rows, int64_t cols);
int sqx_fp8_linear(const uint8_t* wt, const float* w_scale, const void* x, int act_dtype, void* y, int y_dtype,
                   const void* bias, int64_t m, int64_t rows, int64_t cols, int k_slices, void* ws,
                   int64_t ws_bytes, sqx_stream_t stream);

/* sqx_fp8_linear (BF16 output, m <= 64) on the decode-regime kernel with an explicit launch shape:
 * a workgroup owns `tiles` (2 or 4) tiles of 16 weight rows and applies each activation fragment to
 * all of them, `waves` (1..8) waves split its k-blocks, `splits` workgroups split K (partials added
 * in split order by a second kernel, which applies the scales). Same results as sqx_fp8_linear to
 * its bound; fp32 sums in a different order. ws: sqx_fp8_skinny_workspace_bytes(m, rows, cols,
 * splits) bytes. No counterpart in the reference (launch planning). */
int64_t sqx_fp8_skinny_workspace_bytes(int64_t m, int64_t rows, int64_t cols, int splits);
int sqx_fp8_skinny(const uint8_t* wt, const float* w_scale, const void* x, int act_dtype, void* y, const void* bias,
                   int64_t m, int64_t rows, int64_t cols, int tiles, int waves, int splits, void* ws,
                   int64_t ws_bytes, sqx_stream_t stream);

/* ============================================================================================
 * Decode step around the quantized linears: the ops that src/scratch_llm/
 * model.py runs between the Linear calls of one token, against the dense slot KV cache of
 * kv_cache.py:234-262 (BatchedKVCache). Activations are bf16 rows; lengths[b] (int32) is the slot's
 * valid length before this step's write (SlotKVCache.lengths, kv_cache.py:126). All arithmetic is
 * fp32 with one round-to-nearest-even to bf16 per written tensor.
 * ============================================================================================ */

/* RMSNorm (model.py:148-162) with the residual add before it (TransformerBlock.forward,
 * model.py:394-403): with delta, h = bf16(x + delta) is written to h_out; without, h = x.
 * y = bf16(h * (1 / sqrt(mean(h^2) + eps)) * w). x, delta, h_out, y: bf16 [rows, d]; w: bf16 [d];
 * d % 8 == 0, d <= 16384; 16-byte aligned. h_out must not alias x or delta. */
int sqx_rmsnorm(const void* x, const void* delta, const void* w, float eps, int64_t rows, int64_t d,
                void* h_out, void* y, sqx_stream_t stream);

/* sqx_rmsnorm with delta given as the S fp32 partials [S][rows][d] of a K-split linear
 * (sqx_int4_skinny_partials): delta = bf16(sum of the partials in split order), the bits that
 * linear's own reduce writes, so the result is bit-identical to sqx_int4_skinny followed by
 * sqx_rmsnorm. h_out receives x + delta. */
int sqx_rmsnorm_partials(const void* x, const float* part, int splits, const void* w, float eps, int64_t rows,
                         int64_t d, void* h_out, void* y, sqx_stream_t stream);

/* The attention block's o projection of one decode row with the attention combine folded into its
 * activation load (MultiHeadSelfAttention.forward's output projection, model.py:349-366, after the
 * flash-decoding merge of the key-chunk partials): x is not an input but the merge of the partials that
 * sqx_decode_attention_partials left in `part` for this row (B = 1) at the row's length lengths[0]
 * (tmax the cache length given to that call), computed per wave for its own columns with the
 * arithmetic of sqx_attn_partials_combine, so the result equals sqx_attn_partials_combine followed by
 * sqx_int4_linear_residual (same k_slices) bit for bit. Residual epilogue, outputs and weight format as
 * sqx_int4_linear_residual; m = 1, cols = H * 128, two k-blocks per wave (k_slices = cols / 256,
 * the default for cols = 4096), at most 8 key chunks (sqx_attn_partials_chunk). */
int sqx_int4_linear_attn_residual(const uint8_t* wt, const float* st, const float* part, const int* lengths,
                                  int64_t tmax, const void* res, void* res_out, float* ss_out, const void* gain_next,
                                  void* hg_out, int64_t m, int64_t rows, int64_t cols, int64_t group, int k_slices,
                                  sqx_stream_t stream);

/* RoPE of q and k (RotaryPositionalEmbedding.forward, model.py:205-224: interleaved pairs, position
 * lengths[b], fp32 cos/sin tables [rope_rows, hd/2]) and the cache write of SlotKVCache.write_decode
 * (kv_cache.py:194-205, at min(lengths[b], tmax - 1)). qkv: bf16 [B, (H + 2 Hkv) hd] laid out
 * [q | k | v]; q_out: bf16 [B, H, hd]; k_cache, v_cache: bf16 [B, Hkv, tmax, hd]. */
int sqx_rope_kv(const void* qkv, const int* lengths, const float* cos_t, const float* sin_t,
                int64_t rope_rows, int64_t B, int64_t H, int64_t Hkv, int64_t hd, int64_t tmax,
                void* q_out, void* k_cache, void* v_cache, sqx_stream_t stream);

/* Keys per workgroup of sqx_decode_attention, and the bytes of fp32 workspace it needs. */
int sqx_attn_chunk(int64_t B, int64_t Hkv, int64_t tmax);
int64_t sqx_attn_workspace_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t tmax);

/* One-token GQA attention over the slot cache (MultiHeadSelfAttention.forward's SlotKVCache branch,
 * model.py:281-305 and :313-349): out[b, h] = softmax(q[b,h] k[b,h/G]^T / sqrt(hd)) v[b,h/G] over the
 * keys j <= lengths[b] (G = H / Hkv in {1, 2, 4, 8}; hd == 128). out: bf16 [B, H * hd]. Split over
 * the keys into fp32 partials in ws (sqx_attn_workspace_bytes) and combined in a second launch; with
 * one chunk per row (sqx_attn_chunk >= tmax, as when B * Hkv >= 256) one launch writes out, with the
 * bits the combine of that single chunk would give. */
int sqx_decode_attention(const void* q, const void* k_cache, const void* v_cache, const int* lengths,
                         int64_t B, int64_t H, int64_t Hkv, int64_t hd, int64_t tmax, void* out, void* ws,
                         int64_t ws_bytes, sqx_stream_t stream);

/* sqx_rope_kv and sqx_decode_attention in one pass: qkv is the fused projection row of
 * sqx_rope_kv; q and the new key are rotated in registers, the new key/value take the place of cache
 * row min(lengths[b], tmax - 1) and are written there. Same results, bit for bit, as the two calls. */
int sqx_decode_attention_rope(const void* qkv, const int* lengths, const float* cos_t, const float* sin_t,
                              int64_t rope_rows, void* k_cache, void* v_cache, int64_t B, int64_t H,
                              int64_t Hkv, int64_t hd, int64_t tmax, void* out, void* ws, int64_t ws_bytes,
                              sqx_stream_t stream);

/* The first half of sqx_decode_attention[_rope][_fp8kv] on its own: the key-chunk partials (m, l, o)
 * of every row and query head, written to ws, without the combine, for the o projection that merges
 * them in its prologue (sqx_int4_linear_attn_residual). cos_t == NULL: q is [B, H, hd] as
 * sqx_decode_attention takes it; otherwise qkv as sqx_decode_attention_rope (RoPE and the cache write
 * included). k_scale == v_scale == NULL: bf16 cache; both given: E4M3 cache as
 * sqx_decode_attention_fp8kv. Chunks of sqx_attn_partials_chunk(tmax) keys (at most 8 per head for
 * the merge), workspace of sqx_attn_partials_workspace_bytes(B, H, tmax) bytes: o as fp32
 * [B][H][nchunk][hd], then (m, l) as fp32 [B][H][nchunk][2]. */
int sqx_attn_partials_chunk(int64_t tmax);
int64_t sqx_attn_partials_workspace_bytes(int64_t B, int64_t H, int64_t tmax);
int sqx_decode_attention_partials(const void* q, const int* lengths, const float* cos_t, const float* sin_t,
                                  int64_t rope_rows, void* k_cache, void* v_cache, const float* k_scale,
                                  const float* v_scale, int64_t B, int64_t H, int64_t Hkv, int64_t hd, int64_t tmax,
                                  void* ws, int64_t ws_bytes, sqx_stream_t stream);
/* The second half: out[b, h*hd + d] (bf16 [B, H * hd]) from the partials of
 * sqx_decode_attention_partials (same B, H, tmax and lengths), merged in ascending chunk order. */
int sqx_attn_partials_combine(const void* ws, const int* lengths, int64_t B, int64_t H, int64_t tmax, void* out,
                              sqx_stream_t stream);

/* sqx_decode_attention_rope without a workspace argument and without any allocation. No counterpart in
 * the reference: it is for callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). The key-split partials go to a fixed 8 MiB device array
 * inside the library (one per GPU, held until the process ends), so the shape must satisfy
 * sqx_attn_workspace_bytes(B, H, Hkv, tmax) <= 8 MiB (e.g. B = 16, H = 32, Hkv = 8, tmax = 2048
 * needs 0.5 MB, B = 64 with one key chunk per row 1.1 MB); larger shapes return SQX_E_SPACE without launching. The stream's device must be the
 * current device. Calls that overlap on one GPU share that array and race; calls in one stream are
 * ordered. Other arguments and results as sqx_decode_attention_rope, bit for bit. */
int sqx_decode_attention_rope_noalloc(const void* qkv, const int* lengths, const float* cos_t, const float* sin_t,
                                      int64_t rope_rows, void* k_cache, void* v_cache, int64_t B, int64_t H,
                                      int64_t Hkv, int64_t hd, int64_t tmax, void* out, sqx_stream_t stream);

/* The two attention calls above on an FP8 cache (the per-head E4M3 cache of fp8_kv_per_head.py:120-223
 * as the slot cache): k/v hold E4M3 codes [B, Hkv, tmax, hd] (one byte each) with fp32 scales
 * k_scale, v_scale [Hkv]; attention runs on code * scale. The _rope variant quantizes the new key and
 * value with those scales (quantize_per_head: saturating_cast(fp32(x) / scale)) and uses and stores the
 * codes. */
int sqx_decode_attention_fp8kv(const void* q, const void* k_codes, const void* v_codes, const float* k_scale,
                               const float* v_scale, const int* lengths, int64_t B, int64_t H, int64_t Hkv,
                               int64_t hd, int64_t tmax, void* out, void* ws, int64_t ws_bytes,
                               sqx_stream_t stream);
int sqx_decode_attention_rope_fp8kv(const void* qkv, const int* lengths, const float* cos_t, const float* sin_t,
                                    int64_t rope_rows, void* k_codes, void* v_codes, const float* k_scale,
                                    const float* v_scale, int64_t B, int64_t H, int64_t Hkv, int64_t hd,
                                    int64_t tmax, void* out, void* ws, int64_t ws_bytes, sqx_stream_t stream);

/* sqx_decode_attention_rope (k_scale == v_scale == NULL) or sqx_decode_attention_rope_fp8kv (both
 * given) with the q|k|v rows given as the fp32 partials of a K-split projection (MultiHeadSelfAttention's
 * fused qkv projection, model.py:313-320, run by sqx_int4_skinny_partials): qkv_parts fp32
 * [splits][B][(H + 2 Hkv) hd], 16-byte aligned, 1 <= splits <= 64. Each row value is the partials
 * added in split order and rounded to bf16, the bits sqx_int4_skinny's reduce writes, so the result
 * (output and cache) equals that reduce followed by the bf16-row call, bit for bit, in one launch
 * fewer. */
int sqx_decode_attention_rope_parts(const float* qkv_parts, int64_t splits, const int* lengths, const float* cos_t,
                                    const float* sin_t, int64_t rope_rows, void* k_cache, void* v_cache,
                                    const float* k_scale, const float* v_scale, int64_t B, int64_t H, int64_t Hkv,
                                    int64_t hd, int64_t tmax, void* out, void* ws, int64_t ws_bytes,
                                    sqx_stream_t stream);

/* SwiGLU's gate (model.py:227-237): out = bf16(silu(g) * u) from gate_up = bf16 [B, 2F] laid out
 * [g | u] (the w1 and w3 outputs side by side); out: bf16 [B, F]. */
int sqx_silu_mul(const void* gate_up, int64_t B, int64_t F, void* out, sqx_stream_t stream);

/* sqx_silu_mul for a gate_up row laid out in 8-element groups [g 8j..8j+7 | u 8j..8j+7] (what a fused
 * gate|up weight with alternating 8-row groups writes); the same arithmetic per element. F a multiple
 * of 8; 16-byte aligned buffers. */
int sqx_silu_mul_pairs8(const void* gate_up, int64_t B, int64_t F, void* out, sqx_stream_t stream);

/* Embedding.forward (model.py:136-145): out[b] = table[tokens[b]]; table bf16 [V, d]. An id outside
 * [0, V) gives a zero row (the reference raises; callers validate host-side ids). */
int sqx_embed(const void* table, int64_t V, const int* tokens, int64_t B, int64_t d, void* out,
              sqx_stream_t stream);

/* Greedy pick (sampling.py:80-83, temperature 0): next_tok[b] = first index of the maximum of the bf16
 * logits [B, V], NaN counting as the maximum (torch.argmax). Rows are split over up to 64 workgroups
 * whose partial picks go through ws (sqx_argmax_workspace_bytes) to a second, one-wave-per-row pass. */
int64_t sqx_argmax_workspace_bytes(int64_t B, int64_t V);
int sqx_argmax(const void* logits, int64_t B, int64_t V, int* next_tok, void* ws, int64_t ws_bytes,
               sqx_stream_t stream);

/* SlotKVCache.advance(1) (kv_cache.py:207-213): lengths[b] += 1 where active[b] != 0 (every row when
 * active is NULL). */
int sqx_advance(int* lengths, const uint8_t* active, int64_t B, sqx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SQX_H_ */
