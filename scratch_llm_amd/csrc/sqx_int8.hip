// INT8 on gfx950: the quantizers of src/scratch_llm/quant/int8.py bit-exact with the reference (which
// computes in the input's dtype: every fp32 intermediate is rounded back to bf16 / fp16 exactly where
// torch rounds it), w8a8_linear on int8 MFMA with exact int32 accumulation, and the int8 weight-only
// linear as a policy of the shared GEMV.
//
// Reductions see the input as [A, B, C] with B the kept axis (A = product of the dims before it,
// C = product of the dims after it); per-tensor is A = C = 1, B = 1 over all n elements.
//
// Tiled int8 layout (the weight-only linear): block (t, kb) = 1 KiB covering 16 rows x 64 columns;
// lane L owns the 16 codes of row 16t + (L & 15), columns kb*64 + 16(L >> 4) + e, stored as
// u = q + 128 in byte e. Per-row fp32 scales are read in the epilogue.
#include "sqx_gemv.h"

namespace sqx {

template <int DT>
__device__ inline float rd(float v) {  // round an fp32 result to the working dtype
  if (DT == SQX_DTYPE_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  if (DT == SQX_DTYPE_F16) return f16_bits_to_f32(f32_to_f16_bits(v));
  return v;
}

template <int DT>
__device__ inline void store_dt(void* p, int64_t i, float v) {  // v already representable in DT
  if (DT == SQX_DTYPE_F32)
    static_cast<float*>(p)[i] = v;
  else if (DT == SQX_DTYPE_BF16)
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  else
    static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
}

// NaN-propagating reductions (torch amax / amin propagate NaN)
__device__ inline float nmax(float m, float v) { return (v > m || v != v) ? v : m; }
__device__ inline float nmin(float m, float v) { return (v < m || v != v) ? v : m; }

// ----------------------------------------------------------------------------------------------
// Per-slice statistics. OP 0: amax of |x| -> symmetric scale; OP 1: min and max -> affine scale and
// zero-point. The scale math (int8.py:119-124, 163-170), in the working dtype DT:
//   symmetric: s = max(rd(amax / 127), rd(eps))
//   affine:    lo = min(xmin, 0), hi = max(xmax, 0); s = max(rd(rd(hi - lo) / 255), rd(eps));
//              z = clamp(rint(rd(-lo / s)), 0, 255)
// ----------------------------------------------------------------------------------------------
template <int DT, int OP>
__device__ inline void finish_stats(float a, float b, float eps, void* s_out, void* z_out, int64_t i) {
  const float e = rd<DT>(eps);
  if (OP == 0) {
    float s = rd<DT>(__fdiv_rn(a, 127.0f));
    if (s < e) s = e;
    store_dt<DT>(s_out, i, s);
  } else {
    const float lo = a < 0.0f || a != a ? a : 0.0f;  // torch.minimum(x, 0) propagates NaN
    const float hi = b > 0.0f || b != b ? b : 0.0f;
    float s = rd<DT>(__fdiv_rn(rd<DT>(hi - lo), 255.0f));
    if (s < e) s = e;
    float z = __builtin_rintf(rd<DT>(__fdiv_rn(-lo, s)));
    z = fminf(fmaxf(z, 0.0f), 255.0f);
    store_dt<DT>(s_out, i, s);
    store_dt<DT>(z_out, i, z);
  }
}

// One workgroup per kept index b (C >= 32 or A*C large): reduces x[a, b, c] over a and c.
template <int DT, int OP>
__global__ __launch_bounds__(256) void stats_wg_kernel(const void* __restrict__ x, int64_t A, int64_t B, int64_t C,
                                                       float eps, void* __restrict__ s_out,
                                                       void* __restrict__ z_out) {
  __shared__ float ra[256], rb[256];
  const int64_t b = blockIdx.x;
  float m0 = OP == 0 ? 0.0f : INFINITY, m1 = -INFINITY;
  const int64_t per = A * C;
  for (int64_t j = threadIdx.x; j < per; j += blockDim.x) {
    const int64_t a = j / C, c = j - a * C;
    const float v = load_as_f32(x, DT, (a * B + b) * C + c);
    if (OP == 0) m0 = nmax(m0, fabsf(v));
    else { m0 = nmin(m0, v); m1 = nmax(m1, v); }
  }
  ra[threadIdx.x] = m0;
  rb[threadIdx.x] = m1;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      if (OP == 0) ra[threadIdx.x] = nmax(ra[threadIdx.x], ra[threadIdx.x + s]);
      else {
        ra[threadIdx.x] = nmin(ra[threadIdx.x], ra[threadIdx.x + s]);
        rb[threadIdx.x] = nmax(rb[threadIdx.x], rb[threadIdx.x + s]);
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) finish_stats<DT, OP>(ra[0], rb[0], eps, s_out, z_out, b);
}

// One thread per kept index b (small C): coalesced across b.
template <int DT, int OP>
__global__ __launch_bounds__(256) void stats_thread_kernel(const void* __restrict__ x, int64_t A, int64_t B,
                                                           int64_t C, float eps, void* __restrict__ s_out,
                                                           void* __restrict__ z_out) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  float m0 = OP == 0 ? 0.0f : INFINITY, m1 = -INFINITY;
  for (int64_t a = 0; a < A; ++a)
    for (int64_t c = 0; c < C; ++c) {
      const float v = load_as_f32(x, DT, (a * B + b) * C + c);
      if (OP == 0) m0 = nmax(m0, fabsf(v));
      else { m0 = nmin(m0, v); m1 = nmax(m1, v); }
    }
  finish_stats<DT, OP>(m0, m1, eps, s_out, z_out, b);
}

// Per-tensor: grid-stride partials, then one workgroup finishes.
static constexpr int kStatParts = 512;

template <int DT, int OP>
__global__ __launch_bounds__(256) void stats_partial_kernel(const void* __restrict__ x, int64_t n,
                                                            float* __restrict__ part) {
  __shared__ float ra[256], rb[256];
  float m0 = OP == 0 ? 0.0f : INFINITY, m1 = -INFINITY;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float v = load_as_f32(x, DT, i);
    if (OP == 0) m0 = nmax(m0, fabsf(v));
    else { m0 = nmin(m0, v); m1 = nmax(m1, v); }
  }
  ra[threadIdx.x] = m0;
  rb[threadIdx.x] = m1;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      if (OP == 0) ra[threadIdx.x] = nmax(ra[threadIdx.x], ra[threadIdx.x + s]);
      else {
        ra[threadIdx.x] = nmin(ra[threadIdx.x], ra[threadIdx.x + s]);
        rb[threadIdx.x] = nmax(rb[threadIdx.x], rb[threadIdx.x + s]);
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    part[2 * blockIdx.x] = ra[0];
    part[2 * blockIdx.x + 1] = rb[0];
  }
}

template <int DT, int OP>
__global__ __launch_bounds__(256) void stats_final_kernel(const float* __restrict__ part, int parts, float eps,
                                                          void* __restrict__ s_out, void* __restrict__ z_out) {
  __shared__ float ra[256], rb[256];
  float m0 = OP == 0 ? 0.0f : INFINITY, m1 = -INFINITY;
  for (int i = threadIdx.x; i < parts; i += blockDim.x) {
    if (OP == 0) m0 = nmax(m0, part[2 * i]);
    else { m0 = nmin(m0, part[2 * i]); m1 = nmax(m1, part[2 * i + 1]); }
  }
  ra[threadIdx.x] = m0;
  rb[threadIdx.x] = m1;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      if (OP == 0) ra[threadIdx.x] = nmax(ra[threadIdx.x], ra[threadIdx.x + s]);
      else {
        ra[threadIdx.x] = nmin(ra[threadIdx.x], ra[threadIdx.x + s]);
        rb[threadIdx.x] = nmax(rb[threadIdx.x], rb[threadIdx.x + s]);
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) finish_stats<DT, OP>(ra[0], rb[0], eps, s_out, z_out, 0);
}

// ----------------------------------------------------------------------------------------------
// Elementwise quantize / dequantize with the scale of slice b = (i / C) % B
// ----------------------------------------------------------------------------------------------
// symmetric: q = clamp(rint(rd(x / s)), -127, 127); affine: q = clamp(rint(rd(rd(x / s) + z)), 0, 255)
template <int DT, int OP>
__global__ __launch_bounds__(256) void quantize_kernel(const void* __restrict__ x, int64_t n, int64_t B, int64_t C,
                                                       const void* __restrict__ s, const void* __restrict__ z,
                                                       uint8_t* __restrict__ q) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t b = (i / C) % B;
  const float v = load_as_f32(x, DT, i);
  const float sv = load_as_f32(s, DT, b);
  if (OP == 0) {
    const float r = fminf(fmaxf(__builtin_rintf(rd<DT>(__fdiv_rn(v, sv))), -127.0f), 127.0f);
    q[i] = static_cast<uint8_t>(static_cast<int8_t>(r == r ? r : 0.0f));
  } else {
    const float r = fminf(fmaxf(__builtin_rintf(rd<DT>(rd<DT>(__fdiv_rn(v, sv)) + load_as_f32(z, DT, b))), 0.0f), 255.0f);
    q[i] = static_cast<uint8_t>(r == r ? r : 0.0f);
  }
}

// symmetric: rd(q * s); affine: rd(rd(q - z) * s) (int8.py:127-129, 174-176), in the scale dtype.
template <int DT, int OP>
__global__ __launch_bounds__(256) void dequantize_kernel(const uint8_t* __restrict__ q, int64_t n, int64_t B,
                                                         int64_t C, const void* __restrict__ s,
                                                         const void* __restrict__ z, void* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t b = (i / C) % B;
  const float sv = load_as_f32(s, DT, b);
  float v;
  if (OP == 0) v = rd<DT>(static_cast<float>(static_cast<int8_t>(q[i])) * sv);
  else v = rd<DT>(rd<DT>(static_cast<float>(q[i]) - load_as_f32(z, DT, b)) * sv);
  store_dt<DT>(out, i, v);
}

// ----------------------------------------------------------------------------------------------
// w8a8_linear (int8.py:189-213): acc = q_x @ q_w^T in int32 (exact), y = fp32(acc) * (s_x[m] * s_w[n])
// with the scale product in the promoted scale dtype PD. One wave per 16x16 output tile, 4 waves per
// workgroup (32x32), v_mfma_i32_16x16x64_i8: lanes of group g = lane >> 4 carry the same 16 columns
// of A (row lane & 15) and B (column lane & 15), so each product pairs matching k.
// ----------------------------------------------------------------------------------------------
typedef int i32x4_t __attribute__((__vector_size__(4 * sizeof(int))));

template <int PD>
__global__ __launch_bounds__(256) void w8a8_kernel(const int8_t* __restrict__ qx, const int8_t* __restrict__ qw,
                                                   const void* __restrict__ sx, int sx_dt, const void* __restrict__ sw,
                                                   int sw_dt, float* __restrict__ y, int M, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m0 = blockIdx.y * 32 + (wave >> 1) * 16;
  const int n0 = blockIdx.x * 32 + (wave & 1) * 16;
  const int r = lane & 15, g = lane >> 4;
  const int am = m0 + r, bn = n0 + r;
  const rsrc_t ar = make_rsrc(qx, (uint32_t)M * (uint32_t)K);
  const rsrc_t br = make_rsrc(qw, (uint32_t)N * (uint32_t)K);
  i32x4_t acc = {0, 0, 0, 0};
  const bool kfull = K % 16 == 0;
  for (int k0 = 0; k0 < K; k0 += 64) {
    const int kk = k0 + 16 * g;
    u32x4_t a, b;
    if (kfull) {
      // rows at or beyond M / N read zero (past the end of the buffer); columns at or beyond K are
      // the next row's: masked below
      a = kk < K && am < M ? bload128(ar, (uint32_t)(am * K + kk), 0u) : u32x4_t{0u, 0u, 0u, 0u};
      b = kk < K && bn < N ? bload128(br, (uint32_t)(bn * K + kk), 0u) : u32x4_t{0u, 0u, 0u, 0u};
    } else {
      uint32_t av[4] = {0u, 0u, 0u, 0u}, bv[4] = {0u, 0u, 0u, 0u};
      for (int e = 0; e < 16; ++e) {
        if (kk + e < K) {
          if (am < M) av[e >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(qx[(int64_t)am * K + kk + e])) << (8 * (e & 3));
          if (bn < N) bv[e >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(qw[(int64_t)bn * K + kk + e])) << (8 * (e & 3));
        }
      }
      a = u32x4_t{av[0], av[1], av[2], av[3]};
      b = u32x4_t{bv[0], bv[1], bv[2], bv[3]};
    }
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4_t, a), __builtin_bit_cast(i32x4_t, b), acc,
                                                0, 0, 0);
  }
  const int n = n0 + r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + 4 * g + i;
    if (m < M && n < N) {
      const float p = rd<PD>(load_as_f32(sx, sx_dt, m) * load_as_f32(sw, sw_dt, n));
      y[(int64_t)m * N + n] = static_cast<float>(acc[i]) * p;
    }
  }
}

// ----------------------------------------------------------------------------------------------
// Int8 weight-only linear: the GEMV policy
// ----------------------------------------------------------------------------------------------
struct WInt8 {
  static constexpr int KBLK = 64, STEPS = 2;
  struct Args {
    const uint8_t* wt;
    const float* scale;  // [rows] fp32
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
  template <class A, int MCH>
  __device__ static void mma(const u32x4_t& w, const P&, const u32x4_t (&xv)[MCH][STEPS], f32x4_t (&yacc)[MCH]) {
    const uint32_t off = A::pair_from_f32(-128.0f);
    const u32x4_t boff = u32x4_t{off, off, off, off};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t d0 = w[2 * i], d1 = w[2 * i + 1];
      const u32x4_t b = {A::pack_exact(ubyte_f32<0>(d0), ubyte_f32<1>(d0)), A::pack_exact(ubyte_f32<2>(d0), ubyte_f32<3>(d0)),
                         A::pack_exact(ubyte_f32<0>(d1), ubyte_f32<1>(d1)), A::pack_exact(ubyte_f32<2>(d1), ubyte_f32<3>(d1))};
#pragma unroll
      for (int c = 0; c < MCH; ++c) {
        yacc[c] = A::mfma(xv[c][i], b, yacc[c]);
        yacc[c] = A::mfma(xv[c][i], boff, yacc[c]);
      }
    }
  }
  // One activation row (the GEMV's ONE form): the code chains only, with the offset -128 charged
  // through the block's activation sum sig[0].
  static constexpr bool kSumOffset = true;
  static constexpr int NG = 1;
  template <class A>
  __device__ static void mma_one(const u32x4_t& w, const P&, const u32x4_t (&xv)[STEPS], const float (&sig)[NG],
                                 float& y0) {
    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t d0 = w[2 * i], d1 = w[2 * i + 1];
      const u32x4_t b = {A::pack_exact(ubyte_f32<0>(d0), ubyte_f32<1>(d0)), A::pack_exact(ubyte_f32<2>(d0), ubyte_f32<3>(d0)),
                         A::pack_exact(ubyte_f32<0>(d1), ubyte_f32<1>(d1)), A::pack_exact(ubyte_f32<2>(d1), ubyte_f32<3>(d1))};
      acc = A::mfma(xv[i], b, acc);
    }
    y0 += fmaf(-128.0f, sig[0], acc[0]);
  }
  __device__ static float out_scale(const Args& a, int n) { return a.scale[n]; }
};

// One thread per output dword of the tiled int8 weight.
__global__ __launch_bounds__(256) void int8_tile_kernel(const int8_t* __restrict__ q, int64_t rows, int64_t cols,
                                                        int64_t KB, int64_t n_dwords, uint32_t* __restrict__ wt) {
  const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
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
    const uint32_t u = (r < rows && c < cols) ? static_cast<uint32_t>(q[r * cols + c] + 128) : 128u;
    word |= (u & 0xffu) << (8 * e);
  }
  wt[d] = word;
}

// The inverse re-layout: one thread per tiled dword writes its 4 codes back to q [rows, cols].
__global__ __launch_bounds__(256) void int8_untile_kernel(const uint32_t* __restrict__ wt, int64_t rows, int64_t cols,
                                                          int64_t KB, int64_t n_dwords, int8_t* __restrict__ q) {
  const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= n_dwords) return;
  const int i = static_cast<int>(d & 3);
  const int L = static_cast<int>((d >> 2) & 63);
  const int64_t blk = d >> 8;
  const int64_t t = blk / KB;
  const int64_t kb = blk - t * KB;
  const int64_t r = 16 * t + (L & 15);
  if (r >= rows) return;
  const int64_t c0 = kb * 64 + 16 * (L >> 4) + 4 * i;
  const uint32_t word = wt[d];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t c = c0 + e;
    if (c < cols) q[r * cols + c] = static_cast<int8_t>(static_cast<int>((word >> (8 * e)) & 0xffu) - 128);
  }
}

}  // namespace sqx

using namespace sqx;

// ==============================================================================================
// extern "C" entry points
// ==============================================================================================
static bool is_float_dtype(int d) { return d == SQX_DTYPE_F32 || d == SQX_DTYPE_BF16 || d == SQX_DTYPE_F16; }
static dim3 grid_for(int64_t n) { return dim3(static_cast<unsigned>(ceil_div(n, 256))); }

template <int OP>
static int int8_stats(const void* x, int dtype, int64_t A, int64_t B, int64_t C, float eps, void* s, void* z,
                      void* workspace, int64_t workspace_bytes, hipStream_t st, const char* fn) {
  const int64_t n = A * B * C;
  const bool per_tensor = B == 1;
  if (per_tensor) {
    SQX_REQUIRE(workspace && workspace_bytes >= (int64_t)kStatParts * 8, SQX_E_SPACE,
                "%s: a per-tensor scale needs a workspace of %d bytes", fn, kStatParts * 8);
    const int parts = n == 0 ? 1 : static_cast<int>(std::min<int64_t>(kStatParts, ceil_div(n, 256)));
    float* part = static_cast<float*>(workspace);
#define SQX_PT(DT)                                                                                                   \
  do {                                                                                                               \
    if (n > 0) hipLaunchKernelGGL((stats_partial_kernel<DT, OP>), dim3(parts), dim3(256), 0, st, x, n, part);        \
    hipLaunchKernelGGL((stats_final_kernel<DT, OP>), dim3(1), dim3(256), 0, st, part, n > 0 ? parts : 0, eps, s, z); \
  } while (0)
    if (dtype == SQX_DTYPE_F32) SQX_PT(SQX_DTYPE_F32);
    else if (dtype == SQX_DTYPE_BF16) SQX_PT(SQX_DTYPE_BF16);
    else SQX_PT(SQX_DTYPE_F16);
#undef SQX_PT
    return SQX_OK;
  }
  const bool wg = C >= 32 || A * C >= 4096;
#define SQX_AX(DT)                                                                                                   \
  do {                                                                                                               \
    if (wg) hipLaunchKernelGGL((stats_wg_kernel<DT, OP>), dim3(static_cast<unsigned>(B)), dim3(256), 0, st, x, A, B, \
                               C, eps, s, z);                                                                        \
    else hipLaunchKernelGGL((stats_thread_kernel<DT, OP>), grid_for(B), dim3(256), 0, st, x, A, B, C, eps, s, z);   \
  } while (0)
  if (dtype == SQX_DTYPE_F32) SQX_AX(SQX_DTYPE_F32);
  else if (dtype == SQX_DTYPE_BF16) SQX_AX(SQX_DTYPE_BF16);
  else SQX_AX(SQX_DTYPE_F16);
#undef SQX_AX
  return SQX_OK;
}

extern "C" int64_t sqx_int8_workspace_bytes(void) { return (int64_t)kStatParts * 8; }

template <int OP>
static int int8_quantize(const void* x, int dtype, int64_t A, int64_t B, int64_t C, float eps, uint8_t* q, void* s,
                         void* z, void* workspace, int64_t workspace_bytes, sqx_stream_t stream, const char* fn) {
  SQX_REQUIRE(is_float_dtype(dtype), SQX_E_ARG, "%s: unsupported dtype %d", fn, dtype);
  SQX_REQUIRE(A >= 1 && B >= 1 && C >= 1 && A * B * C < ((int64_t)1 << 40), SQX_E_ARG, "%s: bad view [%lld, %lld, %lld]",
              fn, (long long)A, (long long)B, (long long)C);
  SQX_REQUIRE(x && q && s && (OP == 0 || z), SQX_E_ARG, "%s: null pointer", fn);
  SQX_REQUIRE(B == 1 || B < ((int64_t)1 << 31), SQX_E_ARG, "%s: kept axis too long", fn);
  hipStream_t st = as_stream(stream);
  int rc = int8_stats<OP>(x, dtype, A, B, C, eps, s, z, workspace, workspace_bytes, st, fn);
  if (rc) return rc;
  const int64_t n = A * B * C;
  if (n > 0) {
    if (dtype == SQX_DTYPE_F32)
      hipLaunchKernelGGL((quantize_kernel<SQX_DTYPE_F32, OP>), grid_for(n), dim3(256), 0, st, x, n, B, C, s, z, q);
    else if (dtype == SQX_DTYPE_BF16)
      hipLaunchKernelGGL((quantize_kernel<SQX_DTYPE_BF16, OP>), grid_for(n), dim3(256), 0, st, x, n, B, C, s, z, q);
    else
      hipLaunchKernelGGL((quantize_kernel<SQX_DTYPE_F16, OP>), grid_for(n), dim3(256), 0, st, x, n, B, C, s, z, q);
  }
  SQX_LAUNCH_CHECK(fn);
  return SQX_OK;
}

extern "C" int sqx_int8_quantize_sym(const void* x, int dtype, int64_t A, int64_t B, int64_t C, float eps,
                                     int8_t* q, void* s, void* workspace, int64_t workspace_bytes,
                                     sqx_stream_t stream) {
  return int8_quantize<0>(x, dtype, A, B, C, eps, reinterpret_cast<uint8_t*>(q), s, nullptr, workspace,
                          workspace_bytes, stream, "sqx_int8_quantize_sym");
}

extern "C" int sqx_int8_quantize_affine(const void* x, int dtype, int64_t A, int64_t B, int64_t C, float eps,
                                        uint8_t* q, void* s, void* z, void* workspace, int64_t workspace_bytes,
                                        sqx_stream_t stream) {
  return int8_quantize<1>(x, dtype, A, B, C, eps, q, s, z, workspace, workspace_bytes, stream,
                          "sqx_int8_quantize_affine");
}

template <int OP>
static int int8_dequantize(const uint8_t* q, int64_t A, int64_t B, int64_t C, const void* s, const void* z, int dtype,
                           void* out, sqx_stream_t stream, const char* fn) {
  SQX_REQUIRE(is_float_dtype(dtype), SQX_E_ARG, "%s: unsupported dtype %d", fn, dtype);
  SQX_REQUIRE(A >= 1 && B >= 1 && C >= 1, SQX_E_ARG, "%s: bad view", fn);
  const int64_t n = A * B * C;
  SQX_REQUIRE(q && s && out && (OP == 0 || z), SQX_E_ARG, "%s: null pointer", fn);
  hipStream_t st = as_stream(stream);
  if (dtype == SQX_DTYPE_F32)
    hipLaunchKernelGGL((dequantize_kernel<SQX_DTYPE_F32, OP>), grid_for(n), dim3(256), 0, st, q, n, B, C, s, z, out);
  else if (dtype == SQX_DTYPE_BF16)
    hipLaunchKernelGGL((dequantize_kernel<SQX_DTYPE_BF16, OP>), grid_for(n), dim3(256), 0, st, q, n, B, C, s, z, out);
  else
    hipLaunchKernelGGL((dequantize_kernel<SQX_DTYPE_F16, OP>), grid_for(n), dim3(256), 0, st, q, n, B, C, s, z, out);
  SQX_LAUNCH_CHECK(fn);
  return SQX_OK;
}

extern "C" int sqx_int8_dequantize_sym(const int8_t* q, int64_t A, int64_t B, int64_t C, const void* s, int dtype,
                                       void* out, sqx_stream_t stream) {
  return int8_dequantize<0>(reinterpret_cast<const uint8_t*>(q), A, B, C, s, nullptr, dtype, out, stream,
                            "sqx_int8_dequantize_sym");
}

extern "C" int sqx_int8_dequantize_affine(const uint8_t* q, int64_t A, int64_t B, int64_t C, const void* s,
                                          const void* z, int dtype, void* out, sqx_stream_t stream) {
  return int8_dequantize<1>(q, A, B, C, s, z, dtype, out, stream, "sqx_int8_dequantize_affine");
}

extern "C" int sqx_w8a8_gemm(const int8_t* qx, const void* sx, int sx_dtype, const int8_t* qw, const void* sw,
                             int sw_dtype, float* y, int64_t m, int64_t n, int64_t k, sqx_stream_t stream) {
  SQX_REQUIRE(is_float_dtype(sx_dtype) && is_float_dtype(sw_dtype), SQX_E_ARG, "sqx_w8a8_gemm: bad scale dtype");
  SQX_REQUIRE(m >= 0 && n >= 0 && k >= 1 && m * k < ((int64_t)1 << 31) && n * k < ((int64_t)1 << 31), SQX_E_ARG,
              "sqx_w8a8_gemm: bad shape m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
  SQX_REQUIRE(k <= 131072, SQX_E_ARG, "sqx_w8a8_gemm: k=%lld may overflow the int32 accumulator", (long long)k);
  if (m == 0 || n == 0) return SQX_OK;
  SQX_REQUIRE(qx && sx && qw && sw && y, SQX_E_ARG, "sqx_w8a8_gemm: null pointer");
  SQX_REQUIRE(k % 16 != 0 || (reinterpret_cast<uintptr_t>(qx) % 16 == 0 && reinterpret_cast<uintptr_t>(qw) % 16 == 0),
              SQX_E_ARG, "sqx_w8a8_gemm: qx and qw must be 16-byte aligned");
  // the scale product is taken in the promoted dtype of the two scales (torch type promotion)
  const int pd = sx_dtype == sw_dtype ? sx_dtype : SQX_DTYPE_F32;
  const dim3 grid(static_cast<unsigned>(ceil_div(n, 32)), static_cast<unsigned>(ceil_div(m, 32)));
  hipStream_t st = as_stream(stream);
  const int M = static_cast<int>(m), N = static_cast<int>(n), K = static_cast<int>(k);
  if (pd == SQX_DTYPE_F32)
    hipLaunchKernelGGL(w8a8_kernel<SQX_DTYPE_F32>, grid, dim3(256), 0, st, qx, qw, sx, sx_dtype, sw, sw_dtype, y, M, N, K);
  else if (pd == SQX_DTYPE_BF16)
    hipLaunchKernelGGL(w8a8_kernel<SQX_DTYPE_BF16>, grid, dim3(256), 0, st, qx, qw, sx, sx_dtype, sw, sw_dtype, y, M, N, K);
  else
    hipLaunchKernelGGL(w8a8_kernel<SQX_DTYPE_F16>, grid, dim3(256), 0, st, qx, qw, sx, sx_dtype, sw, sw_dtype, y, M, N, K);
  SQX_LAUNCH_CHECK("sqx_w8a8_gemm");
  return SQX_OK;
}

extern "C" int64_t sqx_int8_tiled_weight_bytes(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0) return -1;
  return ceil_div(rows, 16) * ceil_div(cols, 64) * 1024;
}

extern "C" int sqx_int8_tile(const int8_t* q, int64_t rows, int64_t cols, uint8_t* wt, sqx_stream_t stream) {
  SQX_REQUIRE(rows > 0 && cols > 0 && rows <= ((int64_t)1 << 30) && cols <= ((int64_t)1 << 30), SQX_E_ARG,
              "sqx_int8_tile: bad shape");
  SQX_REQUIRE(q && wt, SQX_E_ARG, "sqx_int8_tile: null pointer");
  const int64_t KB = ceil_div(cols, 64);
  const int64_t nd = ceil_div(rows, 16) * KB * 256;
  hipLaunchKernelGGL(int8_tile_kernel, grid_for(nd), dim3(256), 0, as_stream(stream), q, rows, cols, KB, nd,
                     reinterpret_cast<uint32_t*>(wt));
  SQX_LAUNCH_CHECK("sqx_int8_tile");
  return SQX_OK;
}

extern "C" int sqx_int8_untile(const uint8_t* wt, int64_t rows, int64_t cols, int8_t* q, sqx_stream_t stream) {
  SQX_REQUIRE(rows > 0 && cols > 0 && rows <= ((int64_t)1 << 30) && cols <= ((int64_t)1 << 30), SQX_E_ARG,
              "sqx_int8_untile: bad shape");
  SQX_REQUIRE(q && wt, SQX_E_ARG, "sqx_int8_untile: null pointer");
  const int64_t KB = ceil_div(cols, 64);
  const int64_t nd = ceil_div(rows, 16) * KB * 256;
  hipLaunchKernelGGL(int8_untile_kernel, grid_for(nd), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint32_t*>(wt), rows, cols, KB, nd, q);
  SQX_LAUNCH_CHECK("sqx_int8_untile");
  return SQX_OK;
}

extern "C" int sqx_int8_linear(const uint8_t* wt, const float* scale, const void* x, int act_dtype, void* y,
                               const void* bias, int64_t m, int64_t rows, int64_t cols, int k_slices,
                               sqx_stream_t stream) {
  SQX_REQUIRE(m >= 0 && rows > 0 && cols > 0, SQX_E_ARG, "sqx_int8_linear: bad shape");
  SQX_REQUIRE(act_dtype == SQX_DTYPE_BF16 || act_dtype == SQX_DTYPE_F16, SQX_E_ARG,
              "sqx_int8_linear: activations must be BF16 or F16");
  SQX_REQUIRE(rows < ((int64_t)1 << 31) && ceil_div(cols, 64) * 1024 < ((int64_t)1 << 31) && 64 * cols * 2 < ((int64_t)1 << 31),
              SQX_E_ARG, "sqx_int8_linear: shape too large for 32-bit buffer offsets");
  SQX_REQUIRE(cols % 8 == 0, SQX_E_ARG, "sqx_int8_linear: cols=%lld must be a multiple of 8", (long long)cols);
  SQX_REQUIRE(k_slices <= 16, SQX_E_ARG, "sqx_int8_linear: k_slices %d > 16", k_slices);
  if (m == 0) return SQX_OK;
  SQX_REQUIRE(wt && scale && x && y, SQX_E_ARG, "sqx_int8_linear: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0, SQX_E_ARG,
              "sqx_int8_linear: wt and x must be 16-byte aligned");
  const WInt8::Args a{wt, scale};
  hipError_t e;
  if (act_dtype == SQX_DTYPE_BF16)
    e = gemv_launch<ActBF16, WInt8, 4, 2, false>(a, static_cast<const uint16_t*>(x), y,
                                                 static_cast<const uint16_t*>(bias), nullptr, m, rows, cols, k_slices,
                                                 as_stream(stream));
  else
    e = gemv_launch<ActF16, WInt8, 4, 2, false>(a, static_cast<const uint16_t*>(x), y,
                                                static_cast<const uint16_t*>(bias), nullptr, m, rows, cols, k_slices,
                                                as_stream(stream));
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "sqx_int8_linear: launch failed: %s", hipGetErrorString(e));
  return SQX_OK;
}
