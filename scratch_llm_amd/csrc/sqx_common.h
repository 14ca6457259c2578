// Shared helpers for the sqx HIP kernels (gfx950 / CDNA4 only).
//
// Every extern "C" entry point returns 0 on success or a negative SQX_E* code and records a
// message retrievable with sqx_last_error() (thread-local). Kernels never allocate; callers pass
// device pointers and a hipStream_t.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include <algorithm>

#include "../../include/sqx.h"

namespace sqx {

// ---------------------------------------------------------------- error reporting (host) ----
void set_error(const char* fmt, ...);

#define SQX_REQUIRE(cond, code, ...)        \
  do {                                      \
    if (!(cond)) {                          \
      ::sqx::set_error(__VA_ARGS__);        \
      return (code);                        \
    }                                       \
  } while (0)

#define SQX_LAUNCH_CHECK(what)                                                        \
  do {                                                                                \
    hipError_t e_ = hipGetLastError();                                                \
    if (e_ != hipSuccess) {                                                           \
      ::sqx::set_error("%s: launch failed: %s", (what), hipGetErrorString(e_));       \
      return SQX_E_HIP;                                                               \
    }                                                                                 \
  } while (0)

inline hipStream_t as_stream(sqx_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// The int4 decode GEMV with fp32 outputs and no bias, for bf16 activation rows (sqx_int4.hip); the
// fp32-activation linear (sqx_gemm.hip) runs its hi/lo rows through it.
hipError_t int4_gemv_f32out(const uint8_t* wt, const void* st, const void* zt, bool pbf16, const uint16_t* x,
                            float* y, int64_t m, int64_t rows, int64_t cols, int group, hipStream_t s);

// ---------------------------------------------------------------- vector types (device) -----
typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef _Float16 f16x8_t __attribute__((__vector_size__(8 * sizeof(_Float16))));
typedef float f32x4_t __attribute__((__vector_size__(4 * sizeof(float))));
typedef unsigned u32x4_t __attribute__((__vector_size__(4 * sizeof(unsigned))));
typedef uint32_t u32x2v_t __attribute__((__vector_size__(8)));
typedef float f32x2_t __attribute__((__vector_size__(2 * sizeof(float))));
typedef __bf16 bf16x2_t __attribute__((__vector_size__(2 * sizeof(__bf16))));
typedef _Float16 f16x2_t __attribute__((__vector_size__(2 * sizeof(_Float16))));

// ---------------------------------------------------------------- scalar conversions --------
// bf16 <-> fp32 by bit manipulation. fp32 -> bf16 is round-to-nearest-even with NaN kept quiet,
// the same rounding torch's `.to(torch.bfloat16)` performs.
__host__ __device__ inline float bf16_bits_to_f32(uint16_t b) {
  uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

__host__ __device__ inline uint16_t f32_to_bf16_bits(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ inline float f16_bits_to_f32(uint16_t b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return static_cast<float>(h);
}

__device__ inline uint16_t f32_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);  // round-to-nearest-even
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// Load element i of an array whose element type is given at run time (fp32 / bf16 / fp16) as fp32.
// Every conversion here is exact.
__device__ inline float load_as_f32(const void* p, int dtype, int64_t i) {
  if (dtype == SQX_DTYPE_F32) return static_cast<const float*>(p)[i];
  uint16_t b = static_cast<const uint16_t*>(p)[i];
  return dtype == SQX_DTYPE_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// Activation element traits for the MFMA paths: the 16-bit storage type, the "magic" exponent that
// turns a 4-bit unsigned code u into the exactly representable value MAGIC + u by OR-ing it into
// the mantissa, and the conversions of the fp32 accumulator back to storage.
struct ActBF16 {
  static constexpr uint32_t kMagicPair = 0x43004300u;  // bf16 128.0 in both halves
  static constexpr float kMagic = 128.0f;
  __device__ static inline float to_f32(uint16_t b) { return bf16_bits_to_f32(b); }
  __device__ static inline uint16_t from_f32(float f) { return f32_to_bf16_bits(f); }
  __device__ static inline uint32_t pair_from_f32(float v) {  // v exactly representable
    uint32_t h = f32_to_bf16_bits(v);
    return h | (h << 16);
  }
  __device__ static inline f32x4_t mfma(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  // byte `sel` of d (two e2m1 codes, even element in the low nibble) times 2**exponent(scale)
  __device__ static inline uint32_t fp4_pair_scaled(uint32_t d, float scale, int sel) {
    switch (sel) {
      case 0: return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 0));
      case 1: return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 1));
      case 2: return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 2));
      default: return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(d, scale, 3));
    }
  }
  // two floats -> one bf16 pair, each rounded to nearest even (torch's .to(torch.bfloat16))
  __device__ static inline uint32_t pack_rne(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
  }
  // two floats exactly representable in bf16 -> one bf16 pair (upper halves of the fp32 bits)
  __device__ static inline uint32_t pack_exact(float lo, float hi) {
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hi), __builtin_bit_cast(uint32_t, lo), 0x07060302u);
  }
  __device__ static inline f32x2_t fp4_pair_f32(uint32_t d, int sel) { return fp4_pair_f32_any(d, sel); }


  __device__ static inline f32x2_t fp4_pair_f32_any(uint32_t d, int sel) {
    switch (sel) {
      case 0: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 0);
      case 1: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 1);
      case 2: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 2);
      default: return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(d, 1.0f, 3);
    }
  }
};

struct ActF16 {
  static constexpr uint32_t kMagicPair = 0x64006400u;  // fp16 1024.0 in both halves
  static constexpr float kMagic = 1024.0f;
  __device__ static inline float to_f32(uint16_t b) { return f16_bits_to_f32(b); }
  __device__ static inline uint16_t from_f32(float f) { return f32_to_f16_bits(f); }
  __device__ static inline uint32_t pair_from_f32(float v) {
    uint32_t h = f32_to_f16_bits(v);
    return h | (h << 16);
  }
  __device__ static inline f32x4_t mfma(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t fp4_pair_scaled(uint32_t d, float scale, int sel) {
    switch (sel) {
      case 0: return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, scale, 0));
      case 1: return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, scale, 1));
      case 2: return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, scale, 2));
      default: return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(d, scale, 3));
    }
  }
  // two floats -> one fp16 pair, each rounded to nearest even (torch's .to(torch.float16))
  __device__ static inline uint32_t pack_rne(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, f16x2_t));
  }
  // two floats exactly representable in fp16 -> one fp16 pair (round-toward-zero is exact here)
  __device__ static inline uint32_t pack_exact(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
  }
  __device__ static inline f32x2_t fp4_pair_f32(uint32_t d, int sel) { return ActBF16::fp4_pair_f32(d, sel); }
};

// ---------------------------------------------------------------- buffer loads (device) -----
// Raw buffer resources: SGPR base + 32-bit byte count. A load whose byte offset (voffset + soffset)
// is at or beyond `bytes` returns zero without touching memory, which the kernels use for rows of
// an MFMA operand beyond the last activation row. Word 3 is the gfx9 raw-buffer format.
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ inline rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// aux bit 1 = nt (streaming: the line is not kept in the caches once used).
template <int AUX = 0>
__device__ inline u32x4_t bload128(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, AUX));
}

__device__ inline uint32_t bload32(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}

template <int AUX = 0>
__device__ inline u32x2v_t bload64(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x2v_t, __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, AUX));
}

__device__ inline uint32_t bload16(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0);
}

__device__ inline uint32_t bload8(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, (int)voff, (int)soff, 0);
}

// (a & mask) | bits in one VALU op. gfx9 VOP3 encodings take no literal constants, so the compiler
// splits this into v_and + v_or; here the mask sits in an SGPR and `bits` in a VGPR.
__device__ inline uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(bits));
  return r;
}

// v_cvt_f32_ubyteN: byte SEL of d as fp32 in one instruction (the compiler forms a shift, a mask
// and a conversion from the plain expression).
template <int SEL>
__device__ inline float ubyte_f32(uint32_t d) {
  float f;
  if (SEL == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(d));
  if (SEL == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(d));
  if (SEL == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(d));
  if (SEL == 3) asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(d));
  return f;
}

// OCP e4m3fn byte (as quantize_e4m3 values are stored in the tiled NVFP4 scales) -> fp32.
__device__ inline float e4m3_value(uint32_t b) {
  const uint32_t e = (b >> 3) & 15u;
  const uint32_t m = b & 7u;
  return e ? ldexpf(static_cast<float>(8u + m), static_cast<int>(e) - 10) : ldexpf(static_cast<float>(m), -9);
}

// LDS pointers for the buffer loads that write LDS directly.
typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt[3:0] in bits
// 3:0 and vmcnt[5:4] in bits 15:14; expcnt and lgkmcnt at their maxima).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that also orders LDS accesses for the compiler (the memory clobber), without
// waiting for outstanding global loads: loads into registers stay in flight across it.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// All-lane sums over 16 lanes (one DPP row) and over the wave, in a fixed order.
__device__ inline float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));  // row_ror:8
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));  // row_ror:4
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false));   // quad_perm 2301
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));   // quad_perm 1032
  return v;
}

__device__ inline float wave_sum(float v) {
  v = row16_sum(v);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// The merge of a head's key-chunk attention partials (m, l, o) (flash decoding): with M the maximum
// of the merged chunks' m, a chunk's weight is a = 2^(m - M) (0 for a chunk whose keys were all
// masked), then l_sum = fmaf(l, a, l_sum) and o_sum = fmaf(o, a, o_sum) in ascending chunk order, and
// out = bf16(o_sum / l_sum). Every merge of chunk partials (the combine kernel, the o projection's
// prologue) runs exactly these operations, so they agree bit for bit.
__device__ inline float attn_chunk_weight(float m, float M) { return m == -INFINITY ? 0.0f : exp2f(m - M); }

// The two bf16 values of a 32-bit word as fp32 (low half first).
__device__ inline float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }

// SiLU in fp32, g * sigmoid(g) = g / (1 + e^-g), with the hardware reciprocal (1 ulp) in place of an
// IEEE division: a division costs about ten instructions, and the decode step's fused SiLU prologue
// sits in front of the first MFMA of every wave. e^-g overflowing to inf gives a signed zero, as the
// division does. Every SiLU of the library goes through this one function, so the fused prologues
// and the standalone kernel stay bit-identical.
__device__ inline float silu_f32(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }
__device__ inline float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

constexpr float kE4M3Max = 448.0f;
// MIN_SCALE = 1 / (448 * 512) (fp8_weights.py:100), as the fp32 value torch compares against.
constexpr float kFp8MinScale = static_cast<float>(1.0 / (448.0 * 512.0));

// saturating_cast_e4m3 (fp8_weights.py:117-124): clamp to +-448, then round to nearest even. NaN
// stays NaN (0x7f with the input's sign, as torch's cast encodes it).
__device__ inline uint32_t e4m3_encode_sat(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const uint32_t sign = (u >> 24) & 0x80u;
  if (v != v) return sign | 0x7fu;
  const float a = fminf(fabsf(v), kE4M3Max);
  uint32_t code;
  if (a < 0.015625f) {  // below the smallest normal 2**-6: multiples of 2**-9 (code 8 is 2**-6 itself)
    code = static_cast<uint32_t>(rintf(a * 512.0f));
  } else {
    const uint32_t b = __builtin_bit_cast(uint32_t, a);
    const int e = static_cast<int>(b >> 23) - 127;  // -6 .. 8
    const uint32_t mant = b & 0x7fffffu;
    const uint32_t r = mant + 0x7ffffu + ((mant >> 20) & 1u);  // 23 -> 3 bits, ties to even
    code = (static_cast<uint32_t>(e + 7) << 3) + (r >> 20);    // a mantissa carry bumps the exponent
  }
  return sign | code;
}

}  // namespace sqx
