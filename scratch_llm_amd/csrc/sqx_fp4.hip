// FP4 (E2M1) weights on gfx950: the codecs of src/scratch_llm/quant/nvfp4_mxfp4.py (E2M1, E4M3,
// E8M0), MXFP4 / NVFP4 quantize and dequantize bit-exact with the reference, the tile re-layout and
// the decode linear (policies of the shared GEMV, sqx_gemv.h).
//
// Tiled FP4 layout: block (t, kb) = 1 KiB at (t*KB + kb)*1024; lane L owns the 16 bytes at 16L:
// the 32 codes of row 16t + (L & 15), columns kb*128 + 32(L >> 4) + e, two per byte with the even
// element in the low nibble (the reference's pack_fp4 order, and the fp4 operand order of CDNA4's
// MFMA and conversion instructions). A lane's 16 bytes are therefore 16 consecutive bytes of the
// reference's row-major packed weight. Scales per block (t, kb): MXFP4 64 bytes, byte L the E8M0
// scale of lane L's 32 columns; NVFP4 128 bytes, bytes 2L and 2L+1 the E4M3 scales of lane L's two
// 16-column halves. Padding rows / columns hold code 0 and scale byte 0.
#include "sqx_gemv.h"
#include "sqx_mx.h"

#include <float.h>

namespace sqx {

// ----------------------------------------------------------------------------------------------
// Codecs (nvfp4_mxfp4.py:85-174)
// ----------------------------------------------------------------------------------------------
__device__ __constant__ float kFp4Mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

__device__ inline float e2m1_value(uint32_t c) {
  const float m = kFp4Mag[c & 7u];
  return (c & 8u) ? -m : m;
}

// quantize_e4m3 (:135-147): nearest E4M3 value, half to even, binade exponent clamped to [-6, 8]
// (subnormal step 2**-9), saturating at 448, non-positive and NaN -> 0. floor(log2 v) is taken from
// the fp32 exponent field: where torch's fp32 log2 would round v just below 2**k up to k, both
// binades round v to 2**k, so the result is the same.
__device__ inline float quantize_e4m3(float v) {
  const float vf = fminf(fmaxf(v, 0.0f), 448.0f);
  if (!(vf > 0.0f)) return 0.0f;
  const uint32_t u = __builtin_bit_cast(uint32_t, vf);
  int e = static_cast<int>((u >> 23) & 0xffu) - 127;  // vf >= 2**-149; fp32 subnormals clamp below
  e = min(max(e, -6), 8);
  const float step = ldexpf(1.0f, e - 3);
  const float q = __builtin_rintf(__fdiv_rn(vf, step)) * step;
  return fminf(q, 448.0f);
}

// E4M3 value (one quantize_e4m3 returns) <-> OCP e4m3fn byte.
__device__ inline uint32_t e4m3_byte(float v) {
  if (!(v > 0.0f)) return 0u;
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const int e = static_cast<int>((u >> 23) & 0xffu) - 127;
  if (e < -6) return static_cast<uint32_t>(__builtin_rintf(v * 512.0f));  // subnormal: m * 2**-9
  const uint32_t mant = (u >> 20) & 7u;
  return (static_cast<uint32_t>(e + 7) << 3) | mant;
}


// quantize_e8m0 (:150-159): 2**clamp(rint(log2 v), +-127), 0 for v <= 0 (and NaN).
__device__ inline float quantize_e8m0(float v) {
  const float c = v < kTiny ? kTiny : v;  // clamp_min keeps NaN
  float e = __builtin_rintf(log2_f32(c));
  e = fminf(fmaxf(e, -127.0f), 127.0f);
  return v > 0.0f ? ldexpf(1.0f, static_cast<int>(e)) : 0.0f;
}

// ----------------------------------------------------------------------------------------------
// Elementwise codec kernels
// ----------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void e2m1_round_kernel(const void* __restrict__ x, int dtype, int64_t n,
                                                         uint8_t* __restrict__ codes) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) codes[i] = static_cast<uint8_t>(e2m1_code(load_as_f32(x, dtype, i)));
}

__global__ __launch_bounds__(256) void e2m1_decode_kernel(const uint8_t* __restrict__ codes, int64_t n,
                                                          float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = e2m1_value(codes[i]);
}

__global__ __launch_bounds__(256) void fp4_pack_kernel(const uint8_t* __restrict__ codes, int64_t n,
                                                       uint8_t* __restrict__ packed) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (2 * i >= n) return;
  const uint32_t lo = codes[2 * i] & 0xFu;
  const uint32_t hi = (2 * i + 1 < n) ? (codes[2 * i + 1] & 0xFu) : 0u;
  packed[i] = static_cast<uint8_t>(lo | (hi << 4));
}

__global__ __launch_bounds__(256) void fp4_unpack_kernel(const uint8_t* __restrict__ packed, int64_t n,
                                                         uint8_t* __restrict__ codes) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (2 * i >= n) return;
  const uint32_t b = packed[i];
  codes[2 * i] = static_cast<uint8_t>(b & 0xFu);
  if (2 * i + 1 < n) codes[2 * i + 1] = static_cast<uint8_t>(b >> 4);
}

template <int KIND>  // 0 = quantize_e4m3, 1 = quantize_e8m0
__global__ __launch_bounds__(256) void scale_codec_kernel(const float* __restrict__ v, int64_t n,
                                                          float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = KIND == 0 ? quantize_e4m3(v[i]) : quantize_e8m0(v[i]);
}

// ----------------------------------------------------------------------------------------------
// MXFP4 / NVFP4 quantize and dequantize (nvfp4_mxfp4.py:180-272)
// ----------------------------------------------------------------------------------------------
// One thread per block of the flattened, zero-padded input (_blockify, :180-187). Elements at or
// beyond n read as zero, exactly like the padding.
template <bool NV>
__global__ __launch_bounds__(256) void fp4_quantize_kernel(const void* __restrict__ x, int dtype, int64_t n,
                                                           int64_t n_blocks, int block, uint8_t* __restrict__ codes,
                                                           float* __restrict__ s_block, uint8_t* __restrict__ e8m0,
                                                           const float* __restrict__ s_global) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n_blocks) return;
  const int64_t base = b * block;
  float amax = 0.0f;
  for (int e = 0; e < block; ++e) amax = amax_step(amax, base + e < n ? load_as_f32(x, dtype, base + e) : 0.0f);
  float scale;
  if (NV) {
    // nvfp4_quantize (:212-223): s_b = E4M3(block_amax / 6 / s_global); scale = max(s_g * s_b, 1e-30)
    const float sg = *s_global;
    const float sb = quantize_e4m3(__fdiv_rn(__fdiv_rn(amax, 6.0f), sg));
    s_block[b] = sb;
    scale = sg * sb;
    if (scale < kTiny) scale = kTiny;
  } else {
    // mxfp4_quantize (:257-265): s_b = 2**ceil(log2(max(amax/6, 1e-30))), clamped to +-127
    const int e = mx_exponent(amax);
    scale = e == 128 ? __builtin_nanf("") : ldexpf(1.0f, e);
    s_block[b] = scale;
    if (e8m0) e8m0[b] = static_cast<uint8_t>(e == 128 ? 255 : e + 127);
  }
  for (int e = 0; e < block; ++e) {
    const float v = base + e < n ? load_as_f32(x, dtype, base + e) : 0.0f;
    codes[base + e] = static_cast<uint8_t>(e2m1_code(__fdiv_rn(v, scale)));
  }
}

// mxfp4_quantize of the rows of x [m, k] (k % 32 == 0, so each of the reference's flattened
// 32-blocks lies in one row) written straight into the tiled layout: one thread per 16-byte lane
// chunk q of the padded [16 * ceil(m/16), 128 * KB] grid, i.e. row 16t + (L & 15), columns
// 128kb + 32(L >> 4) .. +31, with its E8M0 scale at byte q of the scale buffer. Padding chunks get
// code 0 and scale byte 0. x / 2**e is formed as x * 2**-e: the same single rounding of the same
// real number (2**-e is exact for every e in [-99, 127], and NaN stays NaN).
template <int DT>
__global__ __launch_bounds__(256) void mxfp4_quantize_tiled_kernel(const void* __restrict__ x, int64_t m, int64_t k,
                                                                   int64_t KB, int64_t n_chunks,
                                                                   u32x4_t* __restrict__ xt,
                                                                   uint8_t* __restrict__ xst) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= n_chunks) return;
  const int L = static_cast<int>(q & 63);
  const int64_t blk = q >> 6;
  const int64_t t = blk / KB;
  const int64_t kb = blk - t * KB;
  const int64_t r = 16 * t + (L & 15);
  const int64_t c0 = kb * 128 + 32 * (L >> 4);
  uint32_t d[4] = {0u, 0u, 0u, 0u};
  uint32_t sbyte = 0;
  if (r < m && c0 < k) {
    float v[32];
    const int64_t base = r * k + c0;
    if (DT == SQX_DTYPE_F32) {
      const u32x4_t* p = reinterpret_cast<const u32x4_t*>(static_cast<const float*>(x) + base);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const u32x4_t w = p[j];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // copy the lane out first: __builtin_bit_cast of a vector subscript reads element 0
          const uint32_t u = w[e];
          v[4 * j + e] = __builtin_bit_cast(float, u);
        }
      }
    } else {
      const u32x4_t* p = reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + base);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4_t w = p[j];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint16_t h = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
          v[8 * j + e] = DT == SQX_DTYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
        }
      }
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e) amax = amax_step(amax, v[e]);
    const int ex = mx_exponent(amax);
    const float inv = ex == 128 ? __builtin_nanf("") : ldexpf(1.0f, -ex);
#pragma unroll
    for (int e = 0; e < 32; ++e) d[e >> 3] |= e2m1_code(v[e] * inv) << (4 * (e & 7));
    sbyte = ex == 128 ? 255u : static_cast<uint32_t>(ex + 127);
  }
  xt[q] = u32x4_t{d[0], d[1], d[2], d[3]};
  xst[q] = static_cast<uint8_t>(sbyte);
}

// bf16(mxfp4_dequantize(mxfp4_quantize(row))) for each row of x [m, k] (k % 32 == 0): eight lanes per
// 32-element block, four elements each, the same code and scale as mxfp4_quantize_tiled_kernel, then
// code value * 2**e. The block maximum joins the lanes' maxima (amax_step of two maxima is their joint
// maximum, NaN included). Every such value is exact in bf16 wherever it is finite in fp32 (the two
// share the exponent range, and an E2M1 value has 2 significant bits), so these rows times a weight
// are the products of the two dequantized operands. A single row of 8192 columns spreads over eight
// workgroups instead of one (one thread per block took 7.5 us at M = 1).
template <int DT>
__global__ __launch_bounds__(256) void mxfp4_fake_quant_rows_kernel(const void* __restrict__ x, int64_t n_blocks,
                                                                    uint16_t* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = (t >> 3) < n_blocks;  // the eight lanes of a block are live or not together
  const int64_t base = t * 4;
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (live) {
    if (DT == SQX_DTYPE_F32) {
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(static_cast<const float*>(x) + base);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t u = w[e];  // an element copy first: bit-casting the subscript reads element 0
        v[e] = __builtin_bit_cast(float, u);
      }
    } else {
      const u32x2v_t w = *reinterpret_cast<const u32x2v_t*>(static_cast<const uint16_t*>(x) + base);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint16_t h = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
        v[e] = DT == SQX_DTYPE_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
      }
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) amax = amax_step(amax, v[e]);
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) amax = amax_step(amax, __shfl_xor(amax, o, 64));
  if (!live) return;
  const int ex = mx_exponent(amax);
  *reinterpret_cast<u32x2v_t*>(out + base) = u32x2v_t{mx_fake_pair(v[0], v[1], ex), mx_fake_pair(v[2], v[3], ex)};
}

// NVFP4 global amax: P partial maxima, then s_global = max(amax / (448 * 6), 1e-30) from them.
static constexpr int kAmaxParts = 512;

__global__ __launch_bounds__(256) void amax_partial_kernel(const void* __restrict__ x, int dtype, int64_t n,
                                                           float* __restrict__ part) {
  __shared__ float red[256];
  float m = 0.0f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    m = amax_step(m, load_as_f32(x, dtype, i));
  red[threadIdx.x] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] = amax_step(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

__global__ __launch_bounds__(256) void nv_global_scale_kernel(const float* __restrict__ part, int parts,
                                                              float* __restrict__ s_global) {
  __shared__ float red[256];
  float m = 0.0f;
  for (int i = threadIdx.x; i < parts; i += blockDim.x) m = amax_step(m, part[i]);
  red[threadIdx.x] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] = amax_step(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float sg = __fdiv_rn(red[0], 2688.0f);  // E4M3_MAX * _FP4_MAX
    if (sg < kTiny) sg = kTiny;
    *s_global = sg;
  }
}

template <bool NV>
__global__ __launch_bounds__(256) void fp4_dequantize_kernel(const uint8_t* __restrict__ codes,
                                                             const float* __restrict__ s_block,
                                                             const float* __restrict__ s_global, int64_t n, int block,
                                                             float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float sb = s_block[i / block];
  // nvfp4_dequantize (:226-231): decode * (s_global * s_block); mxfp4_dequantize (:268-272): decode * s_block
  const float scale = NV ? (*s_global) * sb : sb;
  out[i] = e2m1_value(codes[i]) * scale;
}

// ----------------------------------------------------------------------------------------------
// Tile re-layout
// ----------------------------------------------------------------------------------------------
// One thread per lane chunk (16 bytes). PACKED: source is the reference's packed row-major stream
// (rows*cols/2 bytes); else unpacked codes (one per byte).
template <bool PACKED>
__global__ __launch_bounds__(256) void fp4_tile_weights_kernel(const uint8_t* __restrict__ src, int64_t rows,
                                                               int64_t cols, int64_t KB, int64_t n_chunks,
                                                               u32x4_t* __restrict__ wt) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= n_chunks) return;
  const int L = static_cast<int>(q & 63);
  const int64_t blk = q >> 6;
  const int64_t t = blk / KB;
  const int64_t kb = blk - t * KB;
  const int64_t r = 16 * t + (L & 15);
  const int64_t c0 = kb * 128 + 32 * (L >> 4);
  uint32_t d[4] = {0u, 0u, 0u, 0u};
  if (r < rows) {
#pragma unroll 4
    for (int e = 0; e < 32; ++e) {
      const int64_t c = c0 + e;
      if (c >= cols) break;
      const int64_t f = r * cols + c;
      const uint32_t code = PACKED ? ((src[f >> 1] >> (4 * (f & 1))) & 0xFu) : (src[f] & 0xFu);
      d[e >> 3] |= code << (4 * (e & 7));
    }
  }
  wt[q] = u32x4_t{d[0], d[1], d[2], d[3]};
}

// KIND: 0 = MXFP4 scales from fp32 powers of two (s_block), 1 = MXFP4 scales as E8M0 bytes,
// 2 = NVFP4 scales from fp32 E4M3 values, 3 = NVFP4 scales as E4M3 bytes; the source holds one
// scale per `block` columns (a
// multiple of the 32 / 16 columns a scale byte covers). One thread per output scale byte.
template <int KIND>
__global__ __launch_bounds__(256) void fp4_tile_scales_kernel(const void* __restrict__ src, int64_t rows,
                                                              int64_t cols, int64_t block, int64_t KB,
                                                              int64_t n_out, uint8_t* __restrict__ st) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= n_out) return;
  constexpr bool NVK = KIND >= 2;  // NVFP4: two 16-column scales per lane
  constexpr int PER_BLOCK = NVK ? 128 : 64;
  const int64_t blk = o / PER_BLOCK;
  const int j = static_cast<int>(o - blk * PER_BLOCK);
  const int L = NVK ? (j >> 1) : j;
  const int64_t t = blk / KB;
  const int64_t kb = blk - t * KB;
  const int64_t r = 16 * t + (L & 15);
  const int64_t c0 = kb * 128 + 32 * (L >> 4) + (NVK ? 16 * (j & 1) : 0);
  uint32_t byte = 0;
  if (r < rows && c0 < cols) {
    const int64_t si = r * (cols / block) + c0 / block;  // the source block holding column c0
    if (KIND == 2) {
      byte = e4m3_byte(static_cast<const float*>(src)[si]);
    } else if (KIND == 1 || KIND == 3) {
      byte = static_cast<const uint8_t*>(src)[si];
    } else {
      const float s = static_cast<const float*>(src)[si];
      byte = (__builtin_bit_cast(uint32_t, s) >> 23) & 0xffu;  // exponent of a normal power of two
    }
  }
  st[o] = static_cast<uint8_t>(byte);
}

// The inverse re-layout. A lane's 16 tiled bytes are the reference's packed bytes of columns
// c0 .. c0+31 of its row (even element in the low nibble), so each thread copies its chunk back to
// packed [rows, cols/2] (byte by byte at a ragged end); each tiled scale byte goes back to the
// row-major [rows, cols/32] (MXFP4 E8M0) or [rows, cols/16] (NVFP4 E4M3) array.
__global__ __launch_bounds__(256) void fp4_untile_weights_kernel(const u32x4_t* __restrict__ wt, int64_t rows,
                                                                 int64_t cols, int64_t KB, int64_t n_chunks,
                                                                 uint8_t* __restrict__ packed) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= n_chunks) return;
  const int L = static_cast<int>(q & 63);
  const int64_t blk = q >> 6;
  const int64_t t = blk / KB;
  const int64_t kb = blk - t * KB;
  const int64_t r = 16 * t + (L & 15);
  const int64_t c0 = kb * 128 + 32 * (L >> 4);
  if (r >= rows || c0 >= cols) return;
  const u32x4_t v = wt[q];
  uint8_t* dst = packed + r * (cols / 2) + c0 / 2;
  if (c0 + 32 <= cols && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
    *reinterpret_cast<u32x4_t*>(dst) = v;
  } else {
    for (int b = 0; b < 16 && c0 + 2 * b < cols; ++b) {
      const uint32_t w = v[b >> 2];  // through a scalar: hipcc's element access of a vector value
      dst[b] = static_cast<uint8_t>(w >> (8 * (b & 3)));
    }
  }
}

template <bool NVK>
__global__ __launch_bounds__(256) void fp4_untile_scales_kernel(const uint8_t* __restrict__ st, int64_t rows,
                                                                int64_t cols, int64_t KB, int64_t n_in,
                                                                uint8_t* __restrict__ scales) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= n_in) return;
  constexpr int PER_BLOCK = NVK ? 128 : 64;
  constexpr int BS = NVK ? 16 : 32;
  const int64_t blk = o / PER_BLOCK;
  const int j = static_cast<int>(o - blk * PER_BLOCK);
  const int L = NVK ? (j >> 1) : j;
  const int64_t t = blk / KB;
  const int64_t kb = blk - t * KB;
  const int64_t r = 16 * t + (L & 15);
  const int64_t c0 = kb * 128 + 32 * (L >> 4) + (NVK ? 16 * (j & 1) : 0);
  if (r < rows && c0 < cols) scales[r * (cols / BS) + c0 / BS] = st[o];
}

// ----------------------------------------------------------------------------------------------
// GEMV policies
// ----------------------------------------------------------------------------------------------
// Lane group jg feeds MFMA step i the 8 columns 32*jg + 8i .. +7 of the block: dword i of its chunk.
template <bool NV>
struct WFp4 {
  static constexpr int KBLK = 128, STEPS = 4;
  struct Args {
    const uint8_t* wt;
    const uint8_t* st;
    const float* s_global;  // NVFP4: device scalar
  };
  struct Ctx {
    rsrc_t wr, sr;
    uint32_t wvo, svo;
  };
  struct P {
    float s0, s1;
  };
  __device__ static Ctx ctx(const Args& a, int t, int KB, int lane) {
    Ctx c;
    c.wr = make_rsrc(a.wt + (int64_t)t * KB * 1024, (uint32_t)KB * 1024u);
    const uint32_t sbytes = (uint32_t)KB * (NV ? 128u : 64u);
    c.sr = make_rsrc(a.st + (int64_t)t * sbytes, sbytes);
    c.wvo = (uint32_t)lane * 16u;
    c.svo = (uint32_t)lane * (NV ? 2u : 1u);
    return c;
  }
  __device__ static void load(const Ctx& c, int kb, u32x4_t& w, P& p) {
    w = bload128<2>(c.wr, c.wvo, (uint32_t)kb * 1024u);
    if (NV) {
      const uint32_t b = bload16(c.sr, c.svo, (uint32_t)kb * 128u);
      p.s0 = e4m3_value(b & 0xffu);
      p.s1 = e4m3_value(b >> 8);
    } else {
      // E8M0 byte e -> the fp32 2**(e-127) (the conversion uses only the scale's exponent field)
      p.s0 = __builtin_bit_cast(float, bload8(c.sr, c.svo, (uint32_t)kb * 64u) << 23);
      p.s1 = p.s0;
    }
  }
  __device__ static int xk(int i, int jg) { return 32 * jg + 8 * i; }
  template <class A, int MCH>
  __device__ static void mma(const u32x4_t& w, const P& p, const u32x4_t (&xv)[MCH][4], f32x4_t (&yacc)[MCH]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t d = w[i];
      u32x4_t b;
      if (NV) {
        // E4M3 scales carry mantissa bits: decode to fp32, scale, pack (e2m1 * s_b has <= 6
        // significant bits, exact in bf16 / fp16, so taking the upper half is exact for bf16)
        const float s = i < 2 ? p.s0 : p.s1;
#pragma unroll
        for (int sel = 0; sel < 4; ++sel) {
          const f32x2_t f = A::fp4_pair_f32(d, sel);
          b[sel] = A::pack_exact(f[0] * s, f[1] * s);
        }
      } else {
#pragma unroll
        for (int sel = 0; sel < 4; ++sel) b[sel] = A::fp4_pair_scaled(d, p.s0, sel);
      }
#pragma unroll
      for (int c = 0; c < MCH; ++c) yacc[c] = A::mfma(xv[c][i], b, yacc[c]);
    }
  }
  __device__ static float out_scale(const Args& a, int) { return NV ? *a.s_global : 1.0f; }
};

template <class A, bool NV, bool YF32>
static hipError_t launch_fp4(const uint8_t* wt, const uint8_t* st, const float* s_global, const uint16_t* x, void* y,
                             const uint16_t* bias, int64_t m, int64_t rows, int64_t cols, int k_slices,
                             hipStream_t s) {
  using W = WFp4<NV>;
  const typename W::Args a{wt, st, s_global};
  return gemv_launch<A, W, 4, 2, YF32>(a, x, y, bias, nullptr, m, rows, cols, k_slices, s);
}

// ----------------------------------------------------------------------------------------------
// The second NVFP4 convention (the b_r6 rung's operands, kernels/gemm/cuda/b_r6.py:155-244 with the
// scalar rules of kernels/gemm/nvfp4_layout.py:341-416): per block of 16 along k, in float64,
// scale = the smallest unsigned-E4M3 value >= amax / 6 (no global scale), code = the nearest E2M1
// magnitude of x / scale with ties to the even magnitude index, sign only on a non-zero magnitude,
// two codes per byte with the lower k in the low nibble. Scales are stored as E4M3 codes in a
// row-major [rows, k/16] byte array (this library's layout; the E4M3 byte of a positive value is its
// unsigned-E4M3 code). Problems are reported through a status word: bit 0 = a NaN or Inf input,
// bit 1 = a block whose amax / 6 exceeds 448.
// ----------------------------------------------------------------------------------------------
constexpr int kCeilNonFinite = 1, kCeilRange = 2;

__device__ inline double ue4m3_value_d(uint32_t c) {
  const uint32_t e = (c >> 3) & 15u, m = c & 7u;
  return e == 0 ? static_cast<double>(m) * 0x1p-9 : ldexp(1.0 + static_cast<double>(m) * 0.125, static_cast<int>(e) - 7);
}

// Smallest unsigned-E4M3 code whose value is >= v, for finite v >= 0; 0x7F when v > 448. Every step
// is exact in float64: the subnormal grid is m * 2^-9 (and code 8 is 2^-6), a normal value is
// (1 + m/8) * 2^e, so the mantissa step of v's binade is one ceil of an exact scaled value.
__device__ inline uint32_t ue4m3_ceil_d(double v) {
  if (v <= 0.0) return 0u;
  if (v <= 0x1p-6) return static_cast<uint32_t>(ceil(v * 512.0));
  int e2;
  const double f = frexp(v, &e2);  // v = f * 2^e2, f in [0.5, 1)
  int ex = e2 - 1;
  int m = static_cast<int>(ceil((2.0 * f - 1.0) * 8.0));
  if (m == 8) {
    m = 0;
    ++ex;
  }
  const int eb = ex + 7;
  if (eb > 15 || (eb == 15 && m == 7)) return 0x7Fu;
  return static_cast<uint32_t>((eb << 3) | m);
}

// E2M1 magnitude index of a >= 0: round to nearest, ties to the even index, 7 (6.0) past 5.
__device__ inline uint32_t e2m1_rne_index(double a) {
  const uint32_t lo = (a > 0.25) + (a > 0.75) + (a > 1.25) + (a > 1.75) + (a > 2.5) + (a > 3.5) + (a > 5.0);
  const uint32_t hi = (a >= 0.25) + (a >= 0.75) + (a >= 1.25) + (a >= 1.75) + (a >= 2.5) + (a >= 3.5) + (a >= 5.0);
  return (hi > lo && (lo & 1u)) ? hi : lo;
}

// The quantizer's code (b_r6.py:205-223): a value that rounds to magnitude 0 is stored as +0.
__device__ inline uint32_t e2m1_rne_code(double y) {
  const uint32_t i = e2m1_rne_index(fabs(y));
  return i | ((y < 0.0 && i != 0u) ? 8u : 0u);
}

// The scalar helper's code (nvfp4_layout.py:390-416): the sign bit is set for every y < 0, so a
// negative value that rounds to magnitude 0 gives 0x8; -0.0 is not below zero and gives 0x0.
__device__ inline uint32_t e2m1_rne_code_signed(double y) {
  return e2m1_rne_index(fabs(y)) | (y < 0.0 ? 8u : 0u);
}

// One thread per block of 16: packed [rows, k/2] (8 bytes per block), scale codes [rows, k/16].
__global__ __launch_bounds__(256) void nvfp4_ceil_quantize_kernel(const void* __restrict__ x, int dtype, int64_t nblk,
                                                                  uint8_t* __restrict__ packed,
                                                                  uint8_t* __restrict__ scales, int* __restrict__ status) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (b >= nblk) return;
  // float64 throughout, as the reference's x.to(float64): every fp32 / bf16 / fp16 value is exact in it.
  double v[16];
#pragma unroll
  for (int j = 0; j < 16; ++j)
    v[j] = dtype == SQX_DTYPE_F64 ? static_cast<const double*>(x)[b * 16 + j]
                                  : static_cast<double>(load_as_f32(x, dtype, b * 16 + j));
  double amax = 0.0;
  bool finite = true;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    finite = finite && isfinite(v[j]);
    amax = fmax(amax, fabs(v[j]));
  }
  int bad = finite ? 0 : kCeilNonFinite;
  uint32_t code = 0u;
  double scale = 0.0;
  if (finite) {
    code = ue4m3_ceil_d(amax / 6.0);
    if (code == 0x7Fu) {
      bad |= kCeilRange;
      code = 0u;
    }
    scale = ue4m3_value_d(code);
  }
  if (bad) atomicOr(status, bad);
  const double div = scale > 0.0 ? scale : 1.0;
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t c = finite ? e2m1_rne_code(v[j] / div) : 0u;
    w[j >> 3] |= c << (4 * (j & 7));
  }
  *reinterpret_cast<u32x2v_t*>(packed + b * 8) = u32x2v_t{w[0], w[1]};
  scales[b] = static_cast<uint8_t>(code);
}

// One thread per block of 16: fp32 (YB16 = false) or bf16 code value * scale (exact in both).
template <bool YB16>
__global__ __launch_bounds__(256) void nvfp4_ceil_dequantize_kernel(const uint8_t* __restrict__ packed,
                                                                    const uint8_t* __restrict__ scales, int64_t nblk,
                                                                    void* __restrict__ out) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (b >= nblk) return;
  const u32x2v_t w = *reinterpret_cast<const u32x2v_t*>(packed + b * 8);
  const float sc = static_cast<float>(ue4m3_value_d(scales[b]));
  constexpr float kMag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t c = (w[j >> 3] >> (4 * (j & 7))) & 0xFu;
    const float val = (c & 8u ? -kMag[c & 7u] : kMag[c & 7u]) * sc;
    if (YB16)
      static_cast<uint16_t*>(out)[b * 16 + j] = f32_to_bf16_bits(val);
    else
      static_cast<float*>(out)[b * 16 + j] = val;
  }
}

// Elementwise: codes of the smallest unsigned-E4M3 value >= v / divisor (and that value), or the
// E2M1 round-to-nearest-even codes of v (MODE 1).
template <int MODE>
__global__ __launch_bounds__(256) void nvfp4_ceil_elem_kernel(const double* __restrict__ v, int64_t n, double divisor,
                                                              uint8_t* __restrict__ codes, double* __restrict__ values,
                                                              int* __restrict__ status) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const double a = v[i];
  uint32_t c = 0u;
  int bad = 0;
  if (!isfinite(a) || (MODE == 0 && a < 0.0)) {
    bad = kCeilNonFinite;
  } else if (MODE == 0) {
    c = ue4m3_ceil_d(a / divisor);
    if (c == 0x7Fu) {
      bad = kCeilRange;
      c = 0u;
    }
    if (values) values[i] = ue4m3_value_d(c);
  } else {
    c = e2m1_rne_code_signed(a);
  }
  if (bad) atomicOr(status, bad);
  codes[i] = static_cast<uint8_t>(c);
}

// ----------------------------------------------------------------------------------------------
// fp32 activations as two bf16 rows: x = hi + lo with hi = bf16(x), lo = bf16(x - hi)
// ----------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void split_bf16_kernel(const float* __restrict__ x, int64_t n,
                                                         uint16_t* __restrict__ hi, uint16_t* __restrict__ lo) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  const uint16_t h = f32_to_bf16_bits(v);
  hi[i] = h;
  lo[i] = f32_to_bf16_bits(v - bf16_bits_to_f32(h));
}

__global__ __launch_bounds__(256) void sum_halves_kernel(const float* __restrict__ y2, int64_t n,
                                                         float* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = y2[i] + y2[n + i];
}

}  // namespace sqx

using namespace sqx;

// ==============================================================================================
// extern "C" entry points
// ==============================================================================================
static bool is_float_dtype(int d) { return d == SQX_DTYPE_F32 || d == SQX_DTYPE_BF16 || d == SQX_DTYPE_F16; }
static dim3 grid_for(int64_t n) { return dim3(static_cast<unsigned>(ceil_div(n, 256))); }

extern "C" int sqx_e2m1_round(const void* x, int dtype, int64_t n, uint8_t* codes, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0 && is_float_dtype(dtype), SQX_E_ARG, "sqx_e2m1_round: bad n or dtype");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(x && codes, SQX_E_ARG, "sqx_e2m1_round: null pointer");
  hipLaunchKernelGGL(e2m1_round_kernel, grid_for(n), dim3(256), 0, as_stream(stream), x, dtype, n, codes);
  SQX_LAUNCH_CHECK("sqx_e2m1_round");
  return SQX_OK;
}

extern "C" int sqx_e2m1_decode(const uint8_t* codes, int64_t n, float* out, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0, SQX_E_ARG, "sqx_e2m1_decode: negative n");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(codes && out, SQX_E_ARG, "sqx_e2m1_decode: null pointer");
  hipLaunchKernelGGL(e2m1_decode_kernel, grid_for(n), dim3(256), 0, as_stream(stream), codes, n, out);
  SQX_LAUNCH_CHECK("sqx_e2m1_decode");
  return SQX_OK;
}

extern "C" int sqx_fp4_pack(const uint8_t* codes, int64_t n, uint8_t* packed, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0, SQX_E_ARG, "sqx_fp4_pack: negative n");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(codes && packed, SQX_E_ARG, "sqx_fp4_pack: null pointer");
  hipLaunchKernelGGL(fp4_pack_kernel, grid_for(ceil_div(n, 2)), dim3(256), 0, as_stream(stream), codes, n, packed);
  SQX_LAUNCH_CHECK("sqx_fp4_pack");
  return SQX_OK;
}

extern "C" int sqx_fp4_unpack(const uint8_t* packed, int64_t n, uint8_t* codes, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0, SQX_E_ARG, "sqx_fp4_unpack: negative n");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(codes && packed, SQX_E_ARG, "sqx_fp4_unpack: null pointer");
  hipLaunchKernelGGL(fp4_unpack_kernel, grid_for(ceil_div(n, 2)), dim3(256), 0, as_stream(stream), packed, n, codes);
  SQX_LAUNCH_CHECK("sqx_fp4_unpack");
  return SQX_OK;
}

extern "C" int sqx_quantize_e4m3(const float* v, int64_t n, float* out, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0, SQX_E_ARG, "sqx_quantize_e4m3: negative n");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(v && out, SQX_E_ARG, "sqx_quantize_e4m3: null pointer");
  hipLaunchKernelGGL(scale_codec_kernel<0>, grid_for(n), dim3(256), 0, as_stream(stream), v, n, out);
  SQX_LAUNCH_CHECK("sqx_quantize_e4m3");
  return SQX_OK;
}

extern "C" int sqx_quantize_e8m0(const float* v, int64_t n, float* out, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0, SQX_E_ARG, "sqx_quantize_e8m0: negative n");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(v && out, SQX_E_ARG, "sqx_quantize_e8m0: null pointer");
  hipLaunchKernelGGL(scale_codec_kernel<1>, grid_for(n), dim3(256), 0, as_stream(stream), v, n, out);
  SQX_LAUNCH_CHECK("sqx_quantize_e8m0");
  return SQX_OK;
}

extern "C" int sqx_mxfp4_quantize(const void* x, int dtype, int64_t n, int64_t block, uint8_t* codes,
                                  float* s_block, uint8_t* e8m0, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0 && block >= 1 && block <= 4096 && is_float_dtype(dtype), SQX_E_ARG,
              "sqx_mxfp4_quantize: bad n, block or dtype");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(x && codes && s_block, SQX_E_ARG, "sqx_mxfp4_quantize: null pointer");
  const int64_t nb = ceil_div(n, block);
  hipLaunchKernelGGL(fp4_quantize_kernel<false>, grid_for(nb), dim3(256), 0, as_stream(stream), x, dtype, n, nb,
                     static_cast<int>(block), codes, s_block, e8m0, nullptr);
  SQX_LAUNCH_CHECK("sqx_mxfp4_quantize");
  return SQX_OK;
}

extern "C" int sqx_mxfp4_dequantize(const uint8_t* codes, const float* s_block, int64_t n, int64_t block, float* out,
                                    sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0 && block >= 1, SQX_E_ARG, "sqx_mxfp4_dequantize: bad n or block");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(codes && s_block && out, SQX_E_ARG, "sqx_mxfp4_dequantize: null pointer");
  hipLaunchKernelGGL(fp4_dequantize_kernel<false>, grid_for(n), dim3(256), 0, as_stream(stream), codes, s_block,
                     nullptr, n, static_cast<int>(block), out);
  SQX_LAUNCH_CHECK("sqx_mxfp4_dequantize");
  return SQX_OK;
}

extern "C" int64_t sqx_nvfp4_workspace_bytes(void) { return (int64_t)kAmaxParts * 4; }

extern "C" int sqx_nvfp4_quantize(const void* x, int dtype, int64_t n, int64_t block, uint8_t* codes, float* s_block,
                                  float* s_global, void* workspace, int64_t workspace_bytes, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0 && block >= 1 && block <= 4096 && is_float_dtype(dtype), SQX_E_ARG,
              "sqx_nvfp4_quantize: bad n, block or dtype");
  SQX_REQUIRE(s_global && workspace && workspace_bytes >= sqx_nvfp4_workspace_bytes(), SQX_E_SPACE,
              "sqx_nvfp4_quantize: needs s_global and a workspace of %lld bytes", (long long)sqx_nvfp4_workspace_bytes());
  hipStream_t s = as_stream(stream);
  float* part = static_cast<float*>(workspace);
  const int parts = n == 0 ? 1 : static_cast<int>(std::min<int64_t>(kAmaxParts, ceil_div(n, 256)));
  if (n > 0) {
    SQX_REQUIRE(x && codes && s_block, SQX_E_ARG, "sqx_nvfp4_quantize: null pointer");
    hipLaunchKernelGGL(amax_partial_kernel, dim3(parts), dim3(256), 0, s, x, dtype, n, part);
  }
  hipLaunchKernelGGL(nv_global_scale_kernel, dim3(1), dim3(256), 0, s, part, n > 0 ? parts : 0, s_global);
  if (n > 0) {
    const int64_t nb = ceil_div(n, block);
    hipLaunchKernelGGL(fp4_quantize_kernel<true>, grid_for(nb), dim3(256), 0, s, x, dtype, n, nb,
                       static_cast<int>(block), codes, s_block, nullptr, s_global);
  }
  SQX_LAUNCH_CHECK("sqx_nvfp4_quantize");
  return SQX_OK;
}

extern "C" int sqx_nvfp4_dequantize(const uint8_t* codes, const float* s_block, const float* s_global, int64_t n,
                                    int64_t block, float* out, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0 && block >= 1, SQX_E_ARG, "sqx_nvfp4_dequantize: bad n or block");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(codes && s_block && s_global && out, SQX_E_ARG, "sqx_nvfp4_dequantize: null pointer");
  hipLaunchKernelGGL(fp4_dequantize_kernel<true>, grid_for(n), dim3(256), 0, as_stream(stream), codes, s_block,
                     s_global, n, static_cast<int>(block), out);
  SQX_LAUNCH_CHECK("sqx_nvfp4_dequantize");
  return SQX_OK;
}

extern "C" int64_t sqx_fp4_tiled_weight_bytes(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) return -1;
  return ceil_div(rows, 16) * ceil_div(cols, 128) * 1024;
}

extern "C" int64_t sqx_fp4_tiled_scale_bytes(int64_t rows, int64_t cols, int fmt) {
  if (rows < 0 || cols < 0 || (fmt != SQX_FP4_MX && fmt != SQX_FP4_NV)) return -1;
  return ceil_div(rows, 16) * ceil_div(cols, 128) * (fmt == SQX_FP4_NV ? 128 : 64);
}

extern "C" int sqx_fp4_tile(const uint8_t* codes, int codes_packed, const void* scales, int scale_kind, int64_t block,
                            int64_t rows, int64_t cols, uint8_t* wt, uint8_t* st, sqx_stream_t stream) {
  SQX_REQUIRE(rows > 0 && cols > 0 && rows <= ((int64_t)1 << 30) && cols <= ((int64_t)1 << 30), SQX_E_ARG,
              "sqx_fp4_tile: bad shape [%lld, %lld]", (long long)rows, (long long)cols);
  SQX_REQUIRE(scale_kind >= SQX_FP4_SCALE_MX_F32 && scale_kind <= SQX_FP4_SCALE_NV_E4M3, SQX_E_ARG,
              "sqx_fp4_tile: bad scale_kind %d", scale_kind);
  const bool nv = scale_kind == SQX_FP4_SCALE_NV_F32 || scale_kind == SQX_FP4_SCALE_NV_E4M3;
  SQX_REQUIRE(block > 0 && block % (nv ? 16 : 32) == 0 && cols % block == 0, SQX_E_ARG,
              "sqx_fp4_tile: block %lld must be a multiple of %d that divides cols=%lld", (long long)block,
              nv ? 16 : 32, (long long)cols);
  SQX_REQUIRE(!codes_packed || cols % 2 == 0, SQX_E_ARG, "sqx_fp4_tile: packed rows need an even cols");
  SQX_REQUIRE(codes && scales && wt && st, SQX_E_ARG, "sqx_fp4_tile: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0, SQX_E_ARG, "sqx_fp4_tile: wt must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const int64_t KB = ceil_div(cols, 128);
  const int64_t chunks = ceil_div(rows, 16) * KB * 64;
  u32x4_t* w4 = reinterpret_cast<u32x4_t*>(wt);
  if (codes_packed)
    hipLaunchKernelGGL(fp4_tile_weights_kernel<true>, grid_for(chunks), dim3(256), 0, s, codes, rows, cols, KB, chunks, w4);
  else
    hipLaunchKernelGGL(fp4_tile_weights_kernel<false>, grid_for(chunks), dim3(256), 0, s, codes, rows, cols, KB, chunks, w4);
  const int64_t ns = sqx_fp4_tiled_scale_bytes(rows, cols, nv ? SQX_FP4_NV : SQX_FP4_MX);
  if (scale_kind == SQX_FP4_SCALE_MX_F32)
    hipLaunchKernelGGL(fp4_tile_scales_kernel<0>, grid_for(ns), dim3(256), 0, s, scales, rows, cols, block, KB, ns, st);
  else if (scale_kind == SQX_FP4_SCALE_MX_E8M0)
    hipLaunchKernelGGL(fp4_tile_scales_kernel<1>, grid_for(ns), dim3(256), 0, s, scales, rows, cols, block, KB, ns, st);
  else if (scale_kind == SQX_FP4_SCALE_NV_F32)
    hipLaunchKernelGGL(fp4_tile_scales_kernel<2>, grid_for(ns), dim3(256), 0, s, scales, rows, cols, block, KB, ns, st);
  else
    hipLaunchKernelGGL(fp4_tile_scales_kernel<3>, grid_for(ns), dim3(256), 0, s, scales, rows, cols, block, KB, ns, st);
  SQX_LAUNCH_CHECK("sqx_fp4_tile");
  return SQX_OK;
}

extern "C" int sqx_fp4_untile(const uint8_t* wt, const uint8_t* st, int fmt, int64_t rows, int64_t cols,
                              uint8_t* packed, uint8_t* scales, sqx_stream_t stream) {
  SQX_REQUIRE(fmt == SQX_FP4_MX || fmt == SQX_FP4_NV, SQX_E_ARG, "sqx_fp4_untile: bad fmt %d", fmt);
  const int bs = fmt == SQX_FP4_NV ? 16 : 32;
  SQX_REQUIRE(rows > 0 && cols > 0 && cols % bs == 0 && rows <= ((int64_t)1 << 30) && cols <= ((int64_t)1 << 30),
              SQX_E_ARG, "sqx_fp4_untile: bad shape [%lld, %lld] (cols a multiple of %d)", (long long)rows,
              (long long)cols, bs);
  SQX_REQUIRE(wt && st && packed && scales, SQX_E_ARG, "sqx_fp4_untile: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0, SQX_E_ARG, "sqx_fp4_untile: wt must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const int64_t KB = ceil_div(cols, 128);
  const int64_t chunks = ceil_div(rows, 16) * KB * 64;
  hipLaunchKernelGGL(fp4_untile_weights_kernel, grid_for(chunks), dim3(256), 0, s,
                     reinterpret_cast<const u32x4_t*>(wt), rows, cols, KB, chunks, packed);
  const int64_t ns = sqx_fp4_tiled_scale_bytes(rows, cols, fmt);
  if (fmt == SQX_FP4_NV)
    hipLaunchKernelGGL(fp4_untile_scales_kernel<true>, grid_for(ns), dim3(256), 0, s, st, rows, cols, KB, ns, scales);
  else
    hipLaunchKernelGGL(fp4_untile_scales_kernel<false>, grid_for(ns), dim3(256), 0, s, st, rows, cols, KB, ns, scales);
  SQX_LAUNCH_CHECK("sqx_fp4_untile");
  return SQX_OK;
}

// The on-disk MXFP4 pair in float64 (k3/checkpoint.py:136-144): one thread per packed byte (columns
// 2j and 2j + 1 of its row, the low nibble first); the E8M0 byte s becomes 2**(s - 127) by writing
// s - 127 + 1023 into float64's exponent field, so every value and product is exact.
__global__ __launch_bounds__(256) void mxfp4_pair_f64_kernel(const uint8_t* __restrict__ packed,
                                                             const uint8_t* __restrict__ scales, int64_t half,
                                                             int64_t groups, int64_t nbytes, double* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= nbytes) return;
  const int64_t r = i / half;
  const int64_t j = i - r * half;
  const uint32_t b = packed[i];
  const uint64_t sb = scales[r * groups + (2 * j) / 32];
  const double sc = __longlong_as_double(static_cast<long long>((sb + (1023 - 127)) << 52));
  constexpr double kMag[8] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0};
  const uint32_t lo = b & 0xFu, hi = b >> 4;
  double2 v;
  v.x = (lo & 8u ? -kMag[lo & 7u] : kMag[lo & 7u]) * sc;
  v.y = (hi & 8u ? -kMag[hi & 7u] : kMag[hi & 7u]) * sc;
  reinterpret_cast<double2*>(out)[i] = v;
}

extern "C" int sqx_mxfp4_pair_dequantize_f64(const uint8_t* packed, const uint8_t* scales, int64_t rows, int64_t cols,
                                             double* out, sqx_stream_t stream) {
  SQX_REQUIRE(rows >= 0 && cols > 0 && cols % 32 == 0, SQX_E_ARG,
              "sqx_mxfp4_pair_dequantize_f64: bad shape [%lld, %lld] (cols a multiple of 32)", (long long)rows,
              (long long)cols);
  const int64_t nbytes = rows * (cols / 2);
  if (nbytes == 0) return SQX_OK;
  SQX_REQUIRE(packed && scales && out, SQX_E_ARG, "sqx_mxfp4_pair_dequantize_f64: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(out) % 16 == 0, SQX_E_ARG,
              "sqx_mxfp4_pair_dequantize_f64: out must be 16-byte aligned");
  hipLaunchKernelGGL(mxfp4_pair_f64_kernel, grid_for(nbytes), dim3(256), 0, as_stream(stream), packed, scales,
                     cols / 2, cols / 32, nbytes, out);
  SQX_LAUNCH_CHECK("sqx_mxfp4_pair_dequantize_f64");
  return SQX_OK;
}

extern "C" int sqx_mxfp4_fake_quant_rows(const void* x, int dtype, int64_t m, int64_t k, uint16_t* out,
                                         sqx_stream_t stream) {
  SQX_REQUIRE(is_float_dtype(dtype), SQX_E_ARG, "sqx_mxfp4_fake_quant_rows: bad dtype %d", dtype);
  SQX_REQUIRE(m >= 0 && k > 0 && k % 32 == 0 && m <= ((int64_t)1 << 31) && k <= ((int64_t)1 << 30), SQX_E_ARG,
              "sqx_mxfp4_fake_quant_rows: bad shape [%lld, %lld] (k must be a multiple of 32)", (long long)m,
              (long long)k);
  if (m == 0) return SQX_OK;
  SQX_REQUIRE(x && out, SQX_E_ARG, "sqx_mxfp4_fake_quant_rows: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0, SQX_E_ARG,
              "sqx_mxfp4_fake_quant_rows: x and out must be 16-byte aligned");
  const int64_t nb = m * (k / 32);
  SQX_REQUIRE(nb < (int64_t(1) << 36), SQX_E_ARG, "sqx_mxfp4_fake_quant_rows: %lld blocks (fewer than 2^36)",
              (long long)nb);
  hipStream_t s = as_stream(stream);
  const dim3 grid = grid_for(nb * 8);  // eight lanes per block
  if (dtype == SQX_DTYPE_BF16)
    hipLaunchKernelGGL(mxfp4_fake_quant_rows_kernel<SQX_DTYPE_BF16>, grid, dim3(256), 0, s, x, nb, out);
  else if (dtype == SQX_DTYPE_F16)
    hipLaunchKernelGGL(mxfp4_fake_quant_rows_kernel<SQX_DTYPE_F16>, grid, dim3(256), 0, s, x, nb, out);
  else
    hipLaunchKernelGGL(mxfp4_fake_quant_rows_kernel<SQX_DTYPE_F32>, grid, dim3(256), 0, s, x, nb, out);
  SQX_LAUNCH_CHECK("sqx_mxfp4_fake_quant_rows");
  return SQX_OK;
}

extern "C" int sqx_mxfp4_quantize_tiled(const void* x, int dtype, int64_t m, int64_t k, uint8_t* xt, uint8_t* xst,
                                        sqx_stream_t stream) {
  SQX_REQUIRE(is_float_dtype(dtype), SQX_E_ARG, "sqx_mxfp4_quantize_tiled: bad dtype %d", dtype);
  SQX_REQUIRE(m >= 0 && k > 0 && k % 32 == 0 && m <= ((int64_t)1 << 31) && k <= ((int64_t)1 << 30), SQX_E_ARG,
              "sqx_mxfp4_quantize_tiled: bad shape [%lld, %lld] (k must be a multiple of 32)", (long long)m,
              (long long)k);
  if (m == 0) return SQX_OK;
  SQX_REQUIRE(x && xt && xst, SQX_E_ARG, "sqx_mxfp4_quantize_tiled: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(xt) % 16 == 0, SQX_E_ARG,
              "sqx_mxfp4_quantize_tiled: x and xt must be 16-byte aligned");
  const int64_t KB = ceil_div(k, 128);
  const int64_t chunks = ceil_div(m, 16) * KB * 64;
  hipStream_t s = as_stream(stream);
  u32x4_t* x4 = reinterpret_cast<u32x4_t*>(xt);
  if (dtype == SQX_DTYPE_BF16)
    hipLaunchKernelGGL(mxfp4_quantize_tiled_kernel<SQX_DTYPE_BF16>, grid_for(chunks), dim3(256), 0, s, x, m, k, KB,
                       chunks, x4, xst);
  else if (dtype == SQX_DTYPE_F16)
    hipLaunchKernelGGL(mxfp4_quantize_tiled_kernel<SQX_DTYPE_F16>, grid_for(chunks), dim3(256), 0, s, x, m, k, KB,
                       chunks, x4, xst);
  else
    hipLaunchKernelGGL(mxfp4_quantize_tiled_kernel<SQX_DTYPE_F32>, grid_for(chunks), dim3(256), 0, s, x, m, k, KB,
                       chunks, x4, xst);
  SQX_LAUNCH_CHECK("sqx_mxfp4_quantize_tiled");
  return SQX_OK;
}

extern "C" int sqx_fp4_linear(const uint8_t* wt, const uint8_t* st, int fmt, const float* s_global, const void* x,
                              int act_dtype, void* y, int y_dtype, const void* bias, int64_t m, int64_t rows,
                              int64_t cols, int k_slices, sqx_stream_t stream) {
  SQX_REQUIRE(fmt == SQX_FP4_MX || fmt == SQX_FP4_NV, SQX_E_ARG, "sqx_fp4_linear: bad fmt %d", fmt);
  SQX_REQUIRE(m >= 0 && rows > 0 && cols > 0 && cols % (fmt == SQX_FP4_NV ? 16 : 32) == 0, SQX_E_ARG,
              "sqx_fp4_linear: bad shape m=%lld rows=%lld cols=%lld", (long long)m, (long long)rows, (long long)cols);
  SQX_REQUIRE(act_dtype == SQX_DTYPE_BF16 || act_dtype == SQX_DTYPE_F16, SQX_E_ARG,
              "sqx_fp4_linear: activations must be BF16 or F16");
  SQX_REQUIRE(y_dtype == act_dtype || y_dtype == SQX_DTYPE_F32, SQX_E_ARG,
              "sqx_fp4_linear: y_dtype must be the activation dtype or F32");
  SQX_REQUIRE(bias == nullptr || y_dtype == act_dtype, SQX_E_ARG, "sqx_fp4_linear: bias needs y in act_dtype");
  SQX_REQUIRE(rows < ((int64_t)1 << 31) && m < ((int64_t)1 << 31) && ceil_div(cols, 128) * 1024 < ((int64_t)1 << 31) &&
                  64 * cols * 2 < ((int64_t)1 << 31),
              SQX_E_ARG, "sqx_fp4_linear: shape too large for 32-bit buffer offsets");
  SQX_REQUIRE(k_slices <= 16, SQX_E_ARG, "sqx_fp4_linear: k_slices %d > 16", k_slices);
  if (m == 0) return SQX_OK;
  SQX_REQUIRE(wt && st && x && y && (fmt == SQX_FP4_MX || s_global), SQX_E_ARG, "sqx_fp4_linear: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0, SQX_E_ARG,
              "sqx_fp4_linear: wt and x must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* b16 = static_cast<const uint16_t*>(bias);
  const bool nv = fmt == SQX_FP4_NV;
  const bool yf = y_dtype == SQX_DTYPE_F32;
  hipError_t e;
#define SQX_F4(ACT, NV, YF) e = launch_fp4<ACT, NV, YF>(wt, st, s_global, xp, y, b16, m, rows, cols, k_slices, s)
  if (act_dtype == SQX_DTYPE_BF16) {
    if (nv) { if (yf) SQX_F4(ActBF16, true, true); else SQX_F4(ActBF16, true, false); }
    else { if (yf) SQX_F4(ActBF16, false, true); else SQX_F4(ActBF16, false, false); }
  } else {
    if (nv) { if (yf) SQX_F4(ActF16, true, true); else SQX_F4(ActF16, true, false); }
    else { if (yf) SQX_F4(ActF16, false, true); else SQX_F4(ActF16, false, false); }
  }
#undef SQX_F4
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "sqx_fp4_linear: launch failed: %s", hipGetErrorString(e));
  return SQX_OK;
}

extern "C" int sqx_split_bf16(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0, SQX_E_ARG, "sqx_split_bf16: negative n");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(x && hi && lo, SQX_E_ARG, "sqx_split_bf16: null pointer");
  hipLaunchKernelGGL(split_bf16_kernel, grid_for(n), dim3(256), 0, as_stream(stream), x, n, hi, lo);
  SQX_LAUNCH_CHECK("sqx_split_bf16");
  return SQX_OK;
}

extern "C" int sqx_sum_halves(const float* y2, int64_t n, float* y, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0, SQX_E_ARG, "sqx_sum_halves: negative n");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(y2 && y, SQX_E_ARG, "sqx_sum_halves: null pointer");
  hipLaunchKernelGGL(sum_halves_kernel, grid_for(n), dim3(256), 0, as_stream(stream), y2, n, y);
  SQX_LAUNCH_CHECK("sqx_sum_halves");
  return SQX_OK;
}

extern "C" int sqx_nvfp4_ceil_quantize(const void* x, int dtype, int64_t rows, int64_t k, uint8_t* packed,
                                       uint8_t* scales, int* status, sqx_stream_t stream) {
  SQX_REQUIRE(is_float_dtype(dtype) || dtype == SQX_DTYPE_F64, SQX_E_ARG, "sqx_nvfp4_ceil_quantize: bad dtype %d",
              dtype);
  SQX_REQUIRE(rows >= 0 && k > 0 && k % 16 == 0, SQX_E_ARG,
              "quantize_nvfp4: K=%lld is not a multiple of SF_VEC_SIZE=16", (long long)k);
  const int64_t nblk = rows * (k / 16);
  if (nblk == 0) return SQX_OK;
  SQX_REQUIRE(x && packed && scales && status, SQX_E_ARG, "sqx_nvfp4_ceil_quantize: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(packed) % 8 == 0, SQX_E_ARG,
              "sqx_nvfp4_ceil_quantize: packed must be 8-byte aligned");
  hipLaunchKernelGGL(nvfp4_ceil_quantize_kernel, grid_for(nblk), dim3(256), 0, as_stream(stream), x, dtype, nblk, packed,
                     scales, status);
  SQX_LAUNCH_CHECK("sqx_nvfp4_ceil_quantize");
  return SQX_OK;
}

extern "C" int sqx_nvfp4_ceil_dequantize(const uint8_t* packed, const uint8_t* scales, int64_t rows, int64_t k,
                                         void* out, int out_dtype, sqx_stream_t stream) {
  SQX_REQUIRE(rows >= 0 && k > 0 && k % 16 == 0, SQX_E_ARG, "sqx_nvfp4_ceil_dequantize: bad shape");
  SQX_REQUIRE(out_dtype == SQX_DTYPE_F32 || out_dtype == SQX_DTYPE_BF16, SQX_E_ARG,
              "sqx_nvfp4_ceil_dequantize: out_dtype must be F32 or BF16");
  const int64_t nblk = rows * (k / 16);
  if (nblk == 0) return SQX_OK;
  SQX_REQUIRE(packed && scales && out, SQX_E_ARG, "sqx_nvfp4_ceil_dequantize: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(packed) % 8 == 0, SQX_E_ARG,
              "sqx_nvfp4_ceil_dequantize: packed must be 8-byte aligned");
  if (out_dtype == SQX_DTYPE_BF16)
    hipLaunchKernelGGL(nvfp4_ceil_dequantize_kernel<true>, grid_for(nblk), dim3(256), 0, as_stream(stream), packed,
                       scales, nblk, out);
  else
    hipLaunchKernelGGL(nvfp4_ceil_dequantize_kernel<false>, grid_for(nblk), dim3(256), 0, as_stream(stream), packed,
                       scales, nblk, out);
  SQX_LAUNCH_CHECK("sqx_nvfp4_ceil_dequantize");
  return SQX_OK;
}

extern "C" int sqx_ue4m3_ceil(const double* v, int64_t n, double divisor, uint8_t* codes, double* values, int* status,
                              sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0 && divisor > 0.0, SQX_E_ARG, "sqx_ue4m3_ceil: bad n or divisor");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(v && codes && status, SQX_E_ARG, "sqx_ue4m3_ceil: null pointer");
  hipLaunchKernelGGL(nvfp4_ceil_elem_kernel<0>, grid_for(n), dim3(256), 0, as_stream(stream), v, n, divisor, codes, values,
                     status);
  SQX_LAUNCH_CHECK("sqx_ue4m3_ceil");
  return SQX_OK;
}

extern "C" int sqx_e2m1_round_rne(const double* v, int64_t n, uint8_t* codes, int* status, sqx_stream_t stream) {
  SQX_REQUIRE(n >= 0, SQX_E_ARG, "sqx_e2m1_round_rne: negative n");
  if (n == 0) return SQX_OK;
  SQX_REQUIRE(v && codes && status, SQX_E_ARG, "sqx_e2m1_round_rne: null pointer");
  hipLaunchKernelGGL(nvfp4_ceil_elem_kernel<1>, grid_for(n), dim3(256), 0, as_stream(stream), v, n, 1.0, codes, nullptr,
                     status);
  SQX_LAUNCH_CHECK("sqx_e2m1_round_rne");
  return SQX_OK;
}
