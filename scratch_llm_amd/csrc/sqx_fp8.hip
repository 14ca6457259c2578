// FP8 E4M3 (OCP e4m3fn: bias 7, no infinities, NaN = S.1111.111) on gfx950: the quantizers of
// src/scratch_llm/quant/fp8_weights.py (per output channel, per token) and fp8_kv_per_head.py (per
// head), bit-exact with the reference's torch casts, and the W8A8 linear (fp8_linear).
//
// The linear. fp8_linear multiplies per-token E4M3 activations by per-channel E4M3 weights with fp32
// accumulation and applies s_x[m] * s_w[n] (fp8_weights.py:14-31, 211-262). Every E4M3 value is exact
// in bf16 and every product of two is exact in fp32, so this build decodes both operands to bf16
// (v_cvt_pk_f32_fp8, exact for all 256 codes) and runs the bf16 MFMA: the only rounding left is the
// fp32 accumulation and the output cast, which keeps the result inside the reference's derived bound
// (|ref| eps_out/2 + sqrt(K) eps_f32 sum|x w|). The block-scaled fp8 MFMA aligns a step's 128
// products to the largest with a limited-width adder (measured error up to 1.4e-4 of sum|x w| per
// step) and does not meet that bound, nor does the library GEMM built on it.
//
// Tiled FP8 weights: block (t, kb) = 1 KiB covering 16 rows x 64 columns; lane L owns the 16 codes of
// row 16t + (L & 15), columns kb*64 + 16(L >> 4) + e, code e in byte e. Padding holds code 0.
#include "sqx_skinny.h"

namespace sqx {

// NaN-propagating maximum (torch's amax): once a NaN is seen it stays.
__device__ inline float nan_max(float acc, float a) { return (a > acc || a != a) ? a : acc; }

template <int DT>
__device__ inline float load_f(const void* p, int64_t i) {
  if (DT == SQX_DTYPE_F32) return static_cast<const float*>(p)[i];
  const uint16_t b = static_cast<const uint16_t*>(p)[i];
  return DT == SQX_DTYPE_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

__device__ inline float block_max_256(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = nan_max(v, __shfl_xor(v, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) r = nan_max(r, red[w]);
  return r;
}

// quantize_per_channel / quantize_per_token (fp8_weights.py:127-155): per row of x [rows, cols],
// s = max(amax(|x|) / 448, MIN_SCALE) in fp32, codes = saturating_cast(fp32(x) / s). One workgroup
// of 256 threads per row. Codes go to codes[r * cpitch + c] (cols <= cpitch, padding zero-filled),
// and, when vals is given, the codes' exact values as bf16 to vals[r * cpitch + c] (the activation
// operand of the linear).
template <int DT>
__global__ __launch_bounds__(256) void fp8_quantize_rows_kernel(const void* __restrict__ x, int64_t cols, int64_t cpitch,
                                                                uint8_t* __restrict__ codes, float* __restrict__ scale,
                                                                uint16_t* __restrict__ vals) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int64_t base = r * cols;
  float am = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) am = nan_max(am, fabsf(load_f<DT>(x, base + c)));
  am = block_max_256(am, red);
  const float q = __fdiv_rn(am, kE4M3Max);
  const float s = q != q ? q : fmaxf(q, kFp8MinScale);
  if (threadIdx.x == 0) scale[r] = s;
  for (int64_t c = threadIdx.x; c < cpitch; c += 256) {
    uint32_t code = 0;
    if (c < cols) code = e4m3_encode_sat(__fdiv_rn(load_f<DT>(x, base + c), s));
    if (codes != nullptr) codes[r * cpitch + c] = static_cast<uint8_t>(code);
    if (vals != nullptr) {
      const float d = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(code), false)[0];
      vals[r * cpitch + c] = static_cast<uint16_t>(__builtin_bit_cast(uint32_t, d) >> 16);  // exact
    }
  }
}

// The same quantizer for 16-bit rows with cols % 8 == 0: 1024 threads per row, 16-byte loads, the row
// held in registers between the amax and the encode (thread t owns 8-column chunks t + 1024 i, i < NCH).
template <int DT, int NCH>
__global__ __launch_bounds__(1024) void fp8_quantize_rows16_kernel(const uint16_t* __restrict__ x, int64_t cols,
                                                                   uint8_t* __restrict__ codes, float* __restrict__ scale,
                                                                   uint16_t* __restrict__ vals) {
  __shared__ float red[16];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t nch = cols / 8;
  u32x4_t v[NCH];
  float am = 0.0f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int64_t c = tid + 1024 * i;
    if (c < nch) {
      v[i] = *reinterpret_cast<const u32x4_t*>(x + r * cols + 8 * c);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = DT == SQX_DTYPE_BF16 ? bf16_lo(v[i][j]) : f16_bits_to_f32(static_cast<uint16_t>(v[i][j]));
        const float hi = DT == SQX_DTYPE_BF16 ? bf16_hi(v[i][j]) : f16_bits_to_f32(static_cast<uint16_t>(v[i][j] >> 16));
        am = nan_max(nan_max(am, fabsf(lo)), fabsf(hi));
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) am = nan_max(am, __shfl_xor(am, o, 64));
  if ((tid & 63) == 0) red[tid >> 6] = am;
  __syncthreads();
  float tot = red[0];
#pragma unroll
  for (int w = 1; w < 16; ++w) tot = nan_max(tot, red[w]);
  const float q = __fdiv_rn(tot, kE4M3Max);
  const float s = q != q ? q : fmaxf(q, kFp8MinScale);
  if (tid == 0) scale[r] = s;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int64_t c = tid + 1024 * i;
    if (c < nch) {
      uint32_t cw[2] = {0u, 0u};
      u32x4_t vw;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = DT == SQX_DTYPE_BF16 ? bf16_lo(v[i][j]) : f16_bits_to_f32(static_cast<uint16_t>(v[i][j]));
        const float hi = DT == SQX_DTYPE_BF16 ? bf16_hi(v[i][j]) : f16_bits_to_f32(static_cast<uint16_t>(v[i][j] >> 16));
        const uint32_t c0 = e4m3_encode_sat(__fdiv_rn(lo, s));
        const uint32_t c1 = e4m3_encode_sat(__fdiv_rn(hi, s));
        cw[j >> 1] |= (c0 | (c1 << 8)) << (16 * (j & 1));
        const uint32_t pair = c0 | (c1 << 8);
        const f32x2_t d = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(pair), false);
        vw[j] = ActBF16::pack_exact(d[0], d[1]);
      }
      if (codes != nullptr) *reinterpret_cast<u32x2v_t*>(codes + r * cols + 8 * c) = u32x2v_t{cw[0], cw[1]};
      if (vals != nullptr) *reinterpret_cast<u32x4_t*>(vals + r * cols + 8 * c) = vw;
    }
  }
}

// dequantize (fp8_weights.py:158-160) and dequantize_per_head (fp8_kv_per_head.py:99-101):
// out[i] = fp32(code[i]) * scale[(i / inner) % nscale] (per-row scales: inner = cols, nscale = rows;
// per-head scales of [B, H, inner]: nscale = H).
__global__ __launch_bounds__(256) void fp8_dequantize_kernel(const uint8_t* __restrict__ codes, const float* __restrict__ scale,
                                                             int64_t n, int64_t inner, int64_t nscale,
                                                             float* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const float d = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(codes[i]), false)[0];
  out[i] = d * scale[(i / inner) % nscale];
}

// Per-head amax over (batch, tokens, head_dim) of x [B, H, inner] (fp8_kv_per_head.py:77-91), then
// scale = max(amax / 448, MIN_SCALE). One workgroup per head.
template <int DT>
__global__ __launch_bounds__(256) void fp8_head_scale_kernel(const void* __restrict__ x, int64_t B, int64_t H, int64_t inner,
                                                             float* __restrict__ amax, float* __restrict__ scale) {
  __shared__ float red[4];
  const int64_t h = blockIdx.x;
  float am = 0.0f;
  for (int64_t b = 0; b < B; ++b) {
    const int64_t base = (b * H + h) * inner;
    for (int64_t c = threadIdx.x; c < inner; c += 256) am = nan_max(am, fabsf(load_f<DT>(x, base + c)));
  }
  am = block_max_256(am, red);
  const float q = __fdiv_rn(am, kE4M3Max);
  if (threadIdx.x == 0) {
    if (amax != nullptr) amax[h] = am;
    if (scale != nullptr) scale[h] = q != q ? q : fmaxf(q, kFp8MinScale);
  }
}

// quantize_per_head (fp8_kv_per_head.py:93-96): codes = saturating_cast(fp32(x) / scale[h]) for
// x [B, H, inner]; sat (optional) counts the elements the clamp moved (|x| > 448 * scale, :104-107).
template <int DT>
__global__ __launch_bounds__(256) void fp8_quantize_heads_kernel(const void* __restrict__ x, int64_t n, int64_t H,
                                                                 int64_t inner, const float* __restrict__ scale,
                                                                 uint8_t* __restrict__ codes, unsigned long long* __restrict__ sat) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  bool over = false;
  if (i < n) {
    const float v = load_f<DT>(x, i);
    const float s = scale[(i / inner) % H];
    codes[i] = static_cast<uint8_t>(e4m3_encode_sat(__fdiv_rn(v, s)));
    over = fabsf(v) > kE4M3Max * s;
  }
  if (sat != nullptr) {
    const unsigned long long cnt = __popcll(__ballot(over));
    if ((threadIdx.x & 63) == 0 && cnt != 0) atomicAdd(sat, cnt);
  }
}

// One thread per dword of the tiled weight (layout in the file comment).
__global__ __launch_bounds__(256) void fp8_tile_kernel(const uint8_t* __restrict__ q, int64_t rows, int64_t cols, int64_t KB,
                                                       int64_t n_dwords, uint32_t* __restrict__ wt) {
  const int64_t d = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (d >= n_dwords) return;
  const int i = static_cast<int>(d & 3);
  const int L = static_cast<int>((d >> 2) & 63);
  const int64_t blk = d >> 8;
  const int64_t t = blk / KB;
  const int64_t kb = blk - t * KB;
  const int64_t r = 16 * t + (L & 15);
  const int64_t c0 = kb * 64 + 16 * (L >> 4) + 4 * i;
  uint32_t word = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t c = c0 + e;
    const uint32_t u = (r < rows && c < cols) ? static_cast<uint32_t>(q[r * cols + c]) : 0u;
    word |= u << (8 * e);
  }
  wt[d] = word;
}

// GEMV weight policy: E4M3 codes decoded exactly to bf16 (two per v_cvt_pk_f32_fp8), bf16 MFMA
// against the activations' E4M3 values (as bf16), and s_x[m] * s_w[n] on the fp32 result.
struct WFp8 {
  static constexpr int KBLK = 64, STEPS = 2;
  static constexpr bool kRowScale = true;
  struct Args {
    const uint8_t* wt;
    const float* wscale;  // [rows]
    const float* xscale;  // [m]
  };
  struct Ctx {
    rsrc_t wr;
    uint32_t wvo;
  };
  struct P {};
  __device__ static Ctx ctx(const Args& a, int t, int KB, int lane) {
    return Ctx{make_rsrc(a.wt + (int64_t)t * KB * 1024, (uint32_t)KB * 1024u), (uint32_t)lane * 16u};
  }
  __device__ static void load(const Ctx& c, int kb, u32x4_t& w, P&) { w = bload128<2>(c.wr, c.wvo, (uint32_t)kb * 1024u); }
  __device__ static int xk(int i, int jg) { return 16 * jg + 8 * i; }
  template <bool HI>
  __device__ static uint32_t pair(uint32_t d) {  // bytes 0,1 (HI false) or 2,3 of d as a bf16 pair
    const f32x2_t f = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(d), HI);
    return ActBF16::pack_exact(f[0], f[1]);
  }
  template <class A, int MCH>
  __device__ static void mma(const u32x4_t& w, const P&, const u32x4_t (&xv)[MCH][STEPS], f32x4_t (&yacc)[MCH]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t d0 = w[2 * i], d1 = w[2 * i + 1];
      const u32x4_t b = {pair<false>(d0), pair<true>(d0), pair<false>(d1), pair<true>(d1)};
#pragma unroll
      for (int c = 0; c < MCH; ++c) yacc[c] = A::mfma(xv[c][i], b, yacc[c]);
    }
  }
  __device__ static float out_scale(const Args& a, int n) { return a.wscale[n]; }
  __device__ static float row_scale(const Args& a, int m) { return a.xscale[m]; }
  static Args rows_from(const Args& a, int64_t m0) { return Args{a.wt, a.wscale, a.xscale + m0}; }
  static const float* row_scales(const Args& a) { return a.xscale; }
  static const float* out_scales(const Args& a) { return a.wscale; }

  // The skinny linear's hooks: the decoded values are the weights themselves (no offset, no group
  // scale), so each block's MFMAs chain straight into the output sums.
  static constexpr int NG = 1, MPG = STEPS;
  static constexpr bool kPlainBlocks = true, kConstOffset = true;
  __device__ static Ctx ctx_tiles(const Args& a, int t, int nt, int KB, int lane) {
    return Ctx{make_rsrc(a.wt + (int64_t)t * KB * 1024, (uint32_t)nt * (uint32_t)KB * 1024u), (uint32_t)lane * 16u};
  }
  template <class A>
  __device__ static u32x4_t bfrag(const u32x4_t& w, int i) {
    return u32x4_t{pair<false>(w[2 * i]), pair<true>(w[2 * i]), pair<false>(w[2 * i + 1]), pair<true>(w[2 * i + 1])};
  }
  template <class A>
  __device__ static float const_offset() { return 0.0f; }
  template <class A>
  __device__ static float offset(const P&, int) { return 0.0f; }
  __device__ static float scale(const P&, int) { return 1.0f; }
};

}  // namespace sqx

using namespace sqx;

// ==============================================================================================
// extern "C" entry points
// ==============================================================================================
static bool fp8_float_dtype(int d) { return d == SQX_DTYPE_F32 || d == SQX_DTYPE_BF16 || d == SQX_DTYPE_F16; }

#define SQX_FP8_DT(DT_, KERNEL, GRID, ...)                                                                  \
  switch (DT_) {                                                                                            \
    case SQX_DTYPE_F32: hipLaunchKernelGGL((KERNEL<SQX_DTYPE_F32>), GRID, dim3(256), 0, __VA_ARGS__); break;  \
    case SQX_DTYPE_BF16: hipLaunchKernelGGL((KERNEL<SQX_DTYPE_BF16>), GRID, dim3(256), 0, __VA_ARGS__); break; \
    default: hipLaunchKernelGGL((KERNEL<SQX_DTYPE_F16>), GRID, dim3(256), 0, __VA_ARGS__); break;           \
  }

// Per-row quantize into codes (optional) and bf16 values (optional): the 1024-thread register kernel
// for 16-bit rows with cols % 8 == 0 and cols <= 32768, else the generic one.
static void fp8_quantize_rows_launch(const void* x, int dtype, int64_t rows, int64_t cols, uint8_t* codes, float* scale,
                                     uint16_t* vals, hipStream_t s) {
  const bool vec = dtype != SQX_DTYPE_F32 && cols % 8 == 0 && cols <= 32768 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                   (codes == nullptr || reinterpret_cast<uintptr_t>(codes) % 8 == 0) &&
                   (vals == nullptr || reinterpret_cast<uintptr_t>(vals) % 16 == 0);
  if (vec) {
    const int nch = static_cast<int>(ceil_div(cols / 8, 1024));
    const auto* xp = static_cast<const uint16_t*>(x);
    const dim3 grid(static_cast<unsigned>(rows));
#define SQX_Q16(DT_, N_) hipLaunchKernelGGL((fp8_quantize_rows16_kernel<DT_, N_>), grid, dim3(1024), 0, s, xp, cols, codes, scale, vals)
#define SQX_Q16N(DT_)                   \
  if (nch <= 1) SQX_Q16(DT_, 1);        \
  else if (nch <= 2) SQX_Q16(DT_, 2);   \
  else SQX_Q16(DT_, 4);
    if (dtype == SQX_DTYPE_BF16) { SQX_Q16N(SQX_DTYPE_BF16) } else { SQX_Q16N(SQX_DTYPE_F16) }
#undef SQX_Q16N
#undef SQX_Q16
    return;
  }
  SQX_FP8_DT(dtype, fp8_quantize_rows_kernel, dim3(static_cast<unsigned>(rows)), s, x, cols, cols, codes, scale, vals);
}

extern "C" int sqx_fp8_quantize_rows(const void* x, int dtype, int64_t rows, int64_t cols, uint8_t* codes, float* scale,
                                     sqx_stream_t stream) {
  SQX_REQUIRE(fp8_float_dtype(dtype), SQX_E_ARG, "sqx_fp8_quantize_rows: unsupported dtype %d", dtype);
  SQX_REQUIRE(rows >= 0 && cols >= 0 && rows < (int64_t(1) << 31), SQX_E_ARG, "sqx_fp8_quantize_rows: bad shape");
  if (rows == 0) return SQX_OK;
  SQX_REQUIRE(x && codes && scale, SQX_E_ARG, "sqx_fp8_quantize_rows: null pointer");
  fp8_quantize_rows_launch(x, dtype, rows, cols, codes, scale, nullptr, as_stream(stream));
  SQX_LAUNCH_CHECK("sqx_fp8_quantize_rows");
  return SQX_OK;
}

extern "C" int sqx_fp8_dequantize_rows(const uint8_t* codes, const float* scale, int64_t rows, int64_t cols, float* out,
                                       sqx_stream_t stream) {
  SQX_REQUIRE(rows >= 0 && cols >= 0, SQX_E_ARG, "sqx_fp8_dequantize_rows: bad shape");
  const int64_t n = rows * cols;
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(codes && scale && out, SQX_E_ARG, "sqx_fp8_dequantize_rows: null pointer");
  hipLaunchKernelGGL(fp8_dequantize_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, as_stream(stream),
                     codes, scale, n, cols, rows, out);
  SQX_LAUNCH_CHECK("sqx_fp8_dequantize_rows");
  return SQX_OK;
}

extern "C" int sqx_fp8_head_scale(const void* x, int dtype, int64_t B, int64_t H, int64_t inner, float* amax, float* scale,
                                  sqx_stream_t stream) {
  SQX_REQUIRE(fp8_float_dtype(dtype), SQX_E_ARG, "sqx_fp8_head_scale: unsupported dtype %d", dtype);
  SQX_REQUIRE(B >= 0 && H >= 0 && inner >= 0 && H < (int64_t(1) << 31), SQX_E_ARG, "sqx_fp8_head_scale: bad shape");
  if (H == 0) return SQX_OK;
  SQX_REQUIRE((amax || scale) && (x || B * inner == 0), SQX_E_ARG, "sqx_fp8_head_scale: null pointer");
  SQX_FP8_DT(dtype, fp8_head_scale_kernel, dim3(static_cast<unsigned>(H)), as_stream(stream), x, B, H, inner, amax, scale);
  SQX_LAUNCH_CHECK("sqx_fp8_head_scale");
  return SQX_OK;
}

extern "C" int sqx_fp8_quantize_heads(const void* x, int dtype, int64_t B, int64_t H, int64_t inner, const float* scale,
                                      uint8_t* codes, unsigned long long* saturated, sqx_stream_t stream) {
  SQX_REQUIRE(fp8_float_dtype(dtype), SQX_E_ARG, "sqx_fp8_quantize_heads: unsupported dtype %d", dtype);
  SQX_REQUIRE(B >= 0 && H > 0 && inner >= 0, SQX_E_ARG, "sqx_fp8_quantize_heads: bad shape");
  const int64_t n = B * H * inner;
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(x && scale && codes, SQX_E_ARG, "sqx_fp8_quantize_heads: null pointer");
  SQX_FP8_DT(dtype, fp8_quantize_heads_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), as_stream(stream), x, n, H,
             inner, scale, codes, saturated);
  SQX_LAUNCH_CHECK("sqx_fp8_quantize_heads");
  return SQX_OK;
}

extern "C" int sqx_fp8_dequantize_heads(const uint8_t* codes, const float* scale, int64_t B, int64_t H, int64_t inner,
                                        float* out, sqx_stream_t stream) {
  SQX_REQUIRE(B >= 0 && H > 0 && inner > 0, SQX_E_ARG, "sqx_fp8_dequantize_heads: bad shape");
  const int64_t n = B * H * inner;
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(codes && scale && out, SQX_E_ARG, "sqx_fp8_dequantize_heads: null pointer");
  hipLaunchKernelGGL(fp8_dequantize_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256), 0, as_stream(stream),
                     codes, scale, n, inner, H, out);
  SQX_LAUNCH_CHECK("sqx_fp8_dequantize_heads");
  return SQX_OK;
}

extern "C" int64_t sqx_fp8_tiled_weight_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return ceil_div(rows, 16) * ceil_div(cols, 64) * 1024;
}

extern "C" int sqx_fp8_tile(const uint8_t* codes, int64_t rows, int64_t cols, uint8_t* wt, sqx_stream_t stream) {
  SQX_REQUIRE(rows > 0 && cols > 0, SQX_E_ARG, "sqx_fp8_tile: bad shape");
  SQX_REQUIRE(codes && wt, SQX_E_ARG, "sqx_fp8_tile: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 4 == 0, SQX_E_ARG, "sqx_fp8_tile: wt must be 4-byte aligned");
  const int64_t KB = ceil_div(cols, 64);
  const int64_t nd = sqx_fp8_tiled_weight_bytes(rows, cols) / 4;
  hipLaunchKernelGGL(fp8_tile_kernel, dim3(static_cast<unsigned>(ceil_div(nd, 256))), dim3(256), 0, as_stream(stream),
                     codes, rows, cols, KB, nd, reinterpret_cast<uint32_t*>(wt));
  SQX_LAUNCH_CHECK("sqx_fp8_tile");
  return SQX_OK;
}

// Workspace of the FP8 linear: the activations' E4M3 values as bf16 [m, cols], their per-token
// scales [m], then (when the launch splits K) the fp32 partials [S][m][rows]; each part starts on a
// 256-byte boundary.
static int64_t fp8_round256(int64_t b) { return (b + 255) / 256 * 256; }
static int64_t fp8_vals_bytes(int64_t m, int64_t cols) { return fp8_round256(m * cols * 2); }
static int64_t fp8_part_offset(int64_t m, int64_t cols) { return fp8_vals_bytes(m, cols) + fp8_round256(m * 4); }

// The launch the library picks for m rows (bf16 output), from a measured sweep of the Llama-3-8B
// shapes (4096 -> 1024 / 4096 / 6144 / 28672, 14336 -> 4096) at m = 2..64. R tiles of 16 weight rows
// per workgroup share each activation fragment, `waves` waves split its k-blocks, S workgroups split
// K; `gemv` marks shapes where the GEMV (one workgroup per tile) is faster:
//   >= 1024 tiles          R = 2 (m <= 8) or 4, 4 waves, no split;
//   384 .. 1023 tiles      the GEMV for m <= 4, else R = 2 with 8 waves;
//   fewer, K >= 8192       the GEMV for m <= 4, else 8 waves and 4 splits, R = 2 (m <= 8) or 4;
//   fewer, shorter K       the GEMV for m <= 16, else R = 2, 8 waves, 2 splits (4 below 256 tiles).
static SkinnyShape fp8_default_shape(int64_t m, int64_t rows, int64_t cols) {
  const int64_t T = ceil_div(rows, 16);
  const int64_t KB = ceil_div(cols, WFp8::KBLK);
  SkinnyShape sh{0, 2, 8, 1, true};
  if (m < 2 || m > 64) return sh;
  if (T >= 1024) return SkinnyShape{0, m <= 8 ? 2 : 4, 4, 1, false};
  if (T >= 384) return SkinnyShape{0, 2, 8, 1, m <= 4};
  if (KB >= 128) return SkinnyShape{0, m <= 8 ? 2 : 4, 8, 4, m <= 4};
  return SkinnyShape{0, 2, 8, T >= 256 ? 2 : 4, m <= 16};
}

static int64_t fp8_ws_bytes(int64_t m, int64_t rows, int64_t cols, const SkinnyShape& sh) {
  if (m <= 0 || rows <= 0 || cols <= 0) return 0;
  const int S = sh.gemv ? 1 : skinny_splits(ceil_div(cols, WFp8::KBLK), sh.S);
  return fp8_part_offset(m, cols) + skinny_workspace_bytes(m, rows, S);
}

extern "C" int64_t sqx_fp8_linear_workspace_bytes(int64_t m, int64_t rows, int64_t cols) {
  return fp8_ws_bytes(m, rows, cols, fp8_default_shape(m, rows, cols));
}

extern "C" int64_t sqx_fp8_skinny_workspace_bytes(int64_t m, int64_t rows, int64_t cols, int splits) {
  return fp8_ws_bytes(m, rows, cols, SkinnyShape{0, 2, 8, splits > 0 ? splits : 1, false});
}

// Shared by sqx_fp8_linear (sh from fp8_default_shape unless k_slices > 0) and sqx_fp8_skinny.
static int fp8_linear_impl(const uint8_t* wt, const float* w_scale, const void* x, int act_dtype, void* y, int y_dtype,
                           const void* bias, int64_t m, int64_t rows, int64_t cols, int k_slices, SkinnyShape sh,
                           void* ws, int64_t ws_bytes, sqx_stream_t stream, const char* fn) {
  SQX_REQUIRE(fp8_float_dtype(act_dtype), SQX_E_ARG, "%s: unsupported activation dtype %d", fn, act_dtype);
  SQX_REQUIRE(y_dtype == SQX_DTYPE_BF16 || y_dtype == SQX_DTYPE_F32, SQX_E_ARG, "%s: output must be BF16 or F32", fn);
  SQX_REQUIRE(m >= 0 && rows > 0 && cols > 0 && cols % 8 == 0 && rows < (int64_t(1) << 31) && m < (int64_t(1) << 31),
              SQX_E_ARG, "%s: bad shape m=%lld rows=%lld cols=%lld (cols %% 8 == 0)", fn, (long long)m, (long long)rows,
              (long long)cols);
  SQX_REQUIRE(ceil_div(cols, 64) * 1024 < (int64_t(1) << 31) && 64 * cols * 2 < (int64_t(1) << 31) &&
                  ceil_div(rows, 16) * ceil_div(cols, 64) * 1024 < (int64_t(1) << 31),
              SQX_E_ARG, "%s: shape too large for 32-bit buffer offsets", fn);
  SQX_REQUIRE(k_slices <= 16, SQX_E_ARG, "%s: k_slices %d > 16", fn, k_slices);
  if (!sh.gemv) {
    SQX_REQUIRE(m <= 64 && y_dtype == SQX_DTYPE_BF16, SQX_E_ARG, "%s: the skinny kernel takes m <= 64 and a BF16 output",
                fn);
    SQX_REQUIRE(sh.variant == 0 && (sh.R == 2 || sh.R == 4) && sh.waves >= 1 && sh.waves <= kSkinnyMaxWaves && sh.S >= 1,
                SQX_E_ARG, "%s: bad launch shape (tiles %d, waves %d, splits %d)", fn, sh.R, sh.waves, sh.S);
  }
  if (m == 0) return SQX_OK;
  SQX_REQUIRE(wt && w_scale && x && y && ws, SQX_E_ARG, "%s: null pointer", fn);
  const int64_t need = fp8_ws_bytes(m, rows, cols, sh);
  SQX_REQUIRE(ws_bytes >= need, SQX_E_SPACE, "%s: workspace of %lld bytes, %lld needed", fn, (long long)ws_bytes,
              (long long)need);
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0 && reinterpret_cast<uintptr_t>(ws) % 16 == 0, SQX_E_ARG,
              "%s: wt and the workspace must be 16-byte aligned", fn);
  SQX_REQUIRE(bias == nullptr || y_dtype == SQX_DTYPE_BF16, SQX_E_ARG, "%s: bias needs a BF16 output", fn);
  hipStream_t s = as_stream(stream);
  uint16_t* vals = static_cast<uint16_t*>(ws);
  float* xs = reinterpret_cast<float*>(static_cast<char*>(ws) + fp8_vals_bytes(m, cols));
  fp8_quantize_rows_launch(x, act_dtype, m, cols, nullptr, xs, vals, s);
  SQX_LAUNCH_CHECK(fn);
  const WFp8::Args a{wt, w_scale, xs};
  const uint16_t* b16 = static_cast<const uint16_t*>(bias);
  hipError_t e;
  if (!sh.gemv) {
    float* part = reinterpret_cast<float*>(static_cast<char*>(ws) + fp8_part_offset(m, cols));
    e = skinny_launch<ActBF16, WFp8>(a, vals, static_cast<uint16_t*>(y), b16, m, rows, cols, sh, part,
                                     ws_bytes - fp8_part_offset(m, cols), s);
  } else {
    e = y_dtype == SQX_DTYPE_F32
            ? gemv_launch<ActBF16, WFp8, 4, 2, true>(a, vals, y, b16, nullptr, m, rows, cols, k_slices, s)
            : gemv_launch<ActBF16, WFp8, 4, 2, false>(a, vals, y, b16, nullptr, m, rows, cols, k_slices, s);
  }
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}

extern "C" int sqx_fp8_linear(const uint8_t* wt, const float* w_scale, const void* x, int act_dtype, void* y, int y_dtype,
                              const void* bias, int64_t m, int64_t rows, int64_t cols, int k_slices, void* ws,
                              int64_t ws_bytes, sqx_stream_t stream) {
  SkinnyShape sh = fp8_default_shape(m, rows, cols);
  if (k_slices > 0 || y_dtype != SQX_DTYPE_BF16) sh.gemv = true;
  return fp8_linear_impl(wt, w_scale, x, act_dtype, y, y_dtype, bias, m, rows, cols, k_slices, sh, ws, ws_bytes, stream,
                         "sqx_fp8_linear");
}

extern "C" int sqx_fp8_skinny(const uint8_t* wt, const float* w_scale, const void* x, int act_dtype, void* y,
                              const void* bias, int64_t m, int64_t rows, int64_t cols, int tiles, int waves, int splits,
                              void* ws, int64_t ws_bytes, sqx_stream_t stream) {
  const SkinnyShape sh{0, tiles, waves, splits, false};
  return fp8_linear_impl(wt, w_scale, x, act_dtype, y, SQX_DTYPE_BF16, bias, m, rows, cols, 0, sh, ws, ws_bytes, stream,
                         "sqx_fp8_skinny");
}
