// Prefill / large-batch linears on gfx950: dense contractions on the MFMA units.
//
// MXFP4 x MXFP4 (both operands E2M1 codes with one E8M0 scale per 32 columns, in the tiled FP4
// layout of sqx_fp4.hip): y[m, n] = sum_k X[m, k] W[n, k] on CDNA4's block-scaled
// v_mfma_scale_f32_32x32x64_f8f6f4, which multiplies the E2M1 values, applies each lane's E8M0
// scale to its 32 k-values and accumulates in fp32. This is the config-4 linear
// F.linear(mxfp4_dequantize(x), mxfp4_dequantize(W)) (nvfp4_mxfp4.py:257-272 composed with F.linear)
// without materialising either operand: every product of two dequantized values is exact in fp32.
//
// Tiling. One workgroup (4 waves) owns a 256 (m) x 256 (n) output tile; wave w computes the
// 128 x 128 quarter (w >> 1, w & 1) as 4 x 4 MFMA tiles of 32 x 32 held in 256 accumulation
// registers. A k-step covers one 128-column FP4 block: 16 fragments (1 KiB each, 16 rows x 128
// columns) of X and 16 of W plus their 64-byte scale blocks, 34 KiB, copied global -> LDS by
// buffer loads that write LDS directly (no VGPR round trip) into a ring of NSTAGE stages, NSTAGE-1
// k-steps ahead of the MFMAs. A 32 x 64 MFMA operand (rows 32r.., k-half h) is read from two
// 16-row fragments: lane l takes the 16 bytes of fragment row l & 15 in fragment (l & 31) >> 4 at
// column chunk 2h + (l >> 5), and the matching scale byte.
//
// Grid order. Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2), so
// workgroup b runs on XCD b % 8. Each XCD is given a contiguous range of output tiles, walked in
// groups of kGroupM tile rows, so the workgroups resident on one XCD share X and W fragments in
// that XCD's L2.
#include "sqx_common.h"

namespace sqx {

typedef int i32x8_t __attribute__((__vector_size__(8 * sizeof(int))));
typedef float f32x16_t __attribute__((__vector_size__(16 * sizeof(float))));
typedef __attribute__((address_space(3))) void lds_void;
typedef unsigned u32x2_t __attribute__((__vector_size__(2 * sizeof(unsigned))));

namespace mxg {
constexpr int kTile = 256;                  // output rows and columns per workgroup
constexpr int kFrags = kTile / 16;          // 16-row fragments per operand per k-step
constexpr int kOpBytes = kFrags * 1024;     // one operand's fragments per k-step
constexpr int kScBytes = kFrags * 64;       // one operand's scale bytes per k-step
constexpr int kStage = 2 * kOpBytes + 2 * kScBytes;  // X frags | W frags | X scales | W scales
constexpr int kGroupM = 4;                  // tile rows per group in the walk over output tiles
}  // namespace mxg

// Output tile (tm, tn) of workgroup `bid`.
__device__ inline void mx_tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int lin = bid;
  if ((total & 7) == 0) lin = (bid & 7) * (total >> 3) + (bid >> 3);  // XCD b % 8 gets a contiguous range
  const int per_group = mxg::kGroupM * tiles_n;
  const int g = lin / per_group;
  const int first_m = g * mxg::kGroupM;
  const int gm = min(tiles_m - first_m, mxg::kGroupM);
  const int r = lin - g * per_group;
  tm = first_m + r % gm;
  tn = r / gm;
}

// Issue this wave's share of the global -> LDS copies of k-step kb into `stage`. The 32 fragment
// copies of a step (16 of X, then 16 of W, 1 KiB per instruction) are split evenly over the NW
// waves, and so are the 8 scale copies (256 bytes = 4 fragments' 64-byte blocks per instruction).
// Fragment rows past the operand's last 16-row tile are clamped to it (their outputs are masked).
template <int NW>
__device__ inline void mx_issue_step(uint8_t* stage, int wave, int lane, int kb, int KB, rsrc_t xr, rsrc_t xsr,
                                     rsrc_t wr, rsrc_t wsr, int x_t0, int x_tmax, int w_t0, int w_tmax) {
  constexpr int FPW = 32 / NW, BPW = 8 / NW;
  const int g0 = wave * FPW;  // first fragment of this wave: wave-uniform operand choice
  const bool is_w = g0 >= 16;
  const rsrc_t fr = is_w ? wr : xr;
  const int t0 = is_w ? w_t0 : x_t0;
  const int tmax = is_w ? w_tmax : x_tmax;
  const int f0 = g0 & 15;
  uint8_t* dst = stage + (is_w ? mxg::kOpBytes : 0) + f0 * 1024;
#pragma unroll
  for (int j = 0; j < FPW; ++j) {
    const int t = min(t0 + f0 + j, tmax);
    const uint32_t off = ((uint32_t)t * (uint32_t)KB + (uint32_t)kb) * 1024u + (uint32_t)lane * 16u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(fr, (lds_void*)(dst + j * 1024), 16, off, 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    const int blk = wave * BPW + j;  // 0..7: blocks 0-3 X, 4-7 W
    const bool sw = blk >= 4;
    const int f = (blk & 3) * 4 + (lane >> 4);
    const int t = min((sw ? w_t0 : x_t0) + f, sw ? w_tmax : x_tmax);
    const uint32_t off = ((uint32_t)t * (uint32_t)KB + (uint32_t)kb) * 64u + (uint32_t)(lane & 15) * 4u;
    uint8_t* sdst = stage + 2 * mxg::kOpBytes + (sw ? mxg::kScBytes : 0) + (blk & 3) * 256;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(sw ? wsr : xsr, (lds_void*)sdst, 4, off, 0, 0, 0);
  }
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt[3:0] in bits
// 3:0 and vmcnt[5:4] in bits 15:14; expcnt and lgkmcnt at their maxima).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// WN: waves along n (2: four waves of 128 x 128; 4: eight waves of 128 x 64, two per SIMD).
template <int NSTAGE, int YKIND, int WN>  // YKIND: 0 = bf16, 1 = fp16, 2 = fp32
__global__ __launch_bounds__(128 * WN) void mxfp4_gemm_kernel(const uint8_t* __restrict__ xt,
                                                        const uint8_t* __restrict__ xst,
                                                        const uint8_t* __restrict__ wt,
                                                        const uint8_t* __restrict__ wst, void* __restrict__ y,
                                                        const uint16_t* __restrict__ bias, int m, int n, int KB,
                                                        int tiles_m, int tiles_n, int vec, int lds16) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int NW = 2 * WN;              // waves
  constexpr int CT = 8 / WN;              // 32-column MFMA tiles per wave
  constexpr int kPerStep = 40 / NW;       // buffer->LDS instructions per wave per k-step
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, in an SGPR
  int tm, tn;
  mx_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);

  const int xT = (m + 15) >> 4, wT = (n + 15) >> 4;  // 16-row tiles of each operand
  const rsrc_t xr = make_rsrc(xt, (uint32_t)xT * (uint32_t)KB * 1024u);
  const rsrc_t xsr = make_rsrc(xst, (uint32_t)xT * (uint32_t)KB * 64u);
  const rsrc_t wr = make_rsrc(wt, (uint32_t)wT * (uint32_t)KB * 1024u);
  const rsrc_t wsr = make_rsrc(wst, (uint32_t)wT * (uint32_t)KB * 64u);
  const int x_t0 = tm * mxg::kFrags, w_t0 = tn * mxg::kFrags;

  f32x16_t acc[4][CT];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[r][c][i] = 0.0f;

  // operand read offsets within a stage
  const int wm = wave / WN, wn = wave % WN;
  const uint32_t frag_lane = (uint32_t)((lane & 31) >> 4) * 1024u + (uint32_t)(lane >> 5) * 256u + (uint32_t)(lane & 15) * 16u;
  const uint32_t sc_lane = (uint32_t)((lane & 31) >> 4) * 64u + (uint32_t)(lane >> 5) * 16u + (uint32_t)(lane & 15);
  const uint32_t a_off = (uint32_t)(wm * 8) * 1024u + frag_lane;
  const uint32_t b_off = (uint32_t)mxg::kOpBytes + (uint32_t)(wn * 2 * CT) * 1024u + frag_lane;
  const uint32_t sa_off = 2u * mxg::kOpBytes + (uint32_t)(wm * 8) * 64u + sc_lane;
  const uint32_t sb_off = 2u * mxg::kOpBytes + mxg::kScBytes + (uint32_t)(wn * 2 * CT) * 64u + sc_lane;

  struct Ops {
    i32x8_t a[4], b[CT];
    int sa[4], sb[CT];
  };
  // operands of k-half h of the step held in stage `st`
  auto read_ops = [&](const uint8_t* st, int h, Ops& o) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(st + a_off + r * 2048 + h * 512);
      o.a[r] = i32x8_t{(int)v[0], (int)v[1], (int)v[2], (int)v[3], 0, 0, 0, 0};
      o.sa[r] = st[sa_off + r * 128 + h * 32];
    }
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(st + b_off + c * 2048 + h * 512);
      o.b[c] = i32x8_t{(int)v[0], (int)v[1], (int)v[2], (int)v[3], 0, 0, 0, 0};
      o.sb[c] = st[sb_off + c * 128 + h * 32];
    }
  };
  auto mma = [&](const Ops& o) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < CT; ++c)
        acc[r][c] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(o.b[c], o.a[r], acc[r][c], 4, 4, 0, o.sb[c], 0,
                                                                     o.sa[r]);
  };

  // Pipeline. The copy of step s is issued right after the barrier of iteration s-NSTAGE+1, into
  // the stage of step s-NSTAGE, which every wave finished reading before that barrier. Iteration kb: read operands (kb, 1) | MFMAs (kb, 0) | wait for this wave's
  // copy of step kb+1, barrier | issue the copy of step kb+NSTAGE-1 | read operands (kb+1, 0) |
  // MFMAs (kb, 1). The barrier is a bare s_barrier: each wave has already waited for its own copies
  // (vmcnt), and LDS reads complete before the MFMAs that consume them are issued.
#pragma unroll
  for (int s = 0; s < NSTAGE - 1; ++s)
    if (s < KB)
      mx_issue_step<NW>(smem + s * mxg::kStage, wave, lane, s, KB, xr, xsr, wr, wsr, x_t0, xT - 1, w_t0, wT - 1);
  if (KB - 1 >= NSTAGE - 2) wait_vmcnt<kPerStep * (NSTAGE - 2)>();  // step 0 landed for this wave ...
  else wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();  // ... and for every wave
  Ops o0, o1;
  read_ops(smem, 0, o0);
  // steady state: every iteration issues a copy, and the copies of NSTAGE-3 later steps may stay
  // in flight at the barrier
  int kb = 0;
  for (; kb + NSTAGE - 1 < KB; ++kb) {
    const uint8_t* st = smem + (kb % NSTAGE) * mxg::kStage;
    read_ops(st, 1, o1);
    mma(o0);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<kPerStep * (NSTAGE - 3)>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    mx_issue_step<NW>(smem + ((kb + NSTAGE - 1) % NSTAGE) * mxg::kStage, wave, lane, kb + NSTAGE - 1, KB, xr, xsr, wr,
                  wsr, x_t0, xT - 1, w_t0, wT - 1);
    read_ops(smem + ((kb + 1) % NSTAGE) * mxg::kStage, 0, o0);
    mma(o1);
  }
  // tail: nothing left to issue; wait for everything still in flight
  for (; kb < KB; ++kb) {
    const uint8_t* st = smem + (kb % NSTAGE) * mxg::kStage;
    read_ops(st, 1, o1);
    mma(o0);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (kb + 1 < KB) read_ops(smem + ((kb + 1) % NSTAGE) * mxg::kStage, 0, o0);
    mma(o1);
  }

  // Epilogue. W is the MFMA's first operand, so acc[r][c][i] is
  // y[m0 + 32r + (l & 31)][n0 + 32c + 8(i >> 2) + 4(l >> 5) + (i & 3)]: four consecutive columns of one
  // row per lane and register quad.
  const int m0 = tm * mxg::kTile + wm * 128;
  const int n0 = tn * mxg::kTile + wn * 32 * CT;
  if (YKIND != 2 && lds16) {
    // 16-bit y: each wave converts its 128 x 32CT tile into its own LDS area (rows of kPitch bytes,
    // 8 bytes per lane and register quad), then stores whole rows: kLpr lanes cover one row's
    // 64CT bytes with 16-byte writes, so every store instruction writes 64/kLpr full row segments.
    constexpr int kRowBytes = 64 * CT, kPitch = kRowBytes + 8, kLpr = kRowBytes / 16, kRpp = 64 / kLpr;
    static_assert(NW * 128 * kPitch <= NSTAGE * mxg::kStage, "the epilogue reuses the operand stages");
    __builtin_amdgcn_s_barrier();  // every wave is done reading the operand stages
    uint8_t* ep = smem + wave * 128 * kPitch;
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int cl = 32 * c + 8 * q + 4 * (lane >> 5);  // column within the wave tile
        float badd[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (bias) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (n0 + cl + j < n) badd[j] = YKIND == 1 ? f16_bits_to_f32(bias[n0 + cl + j]) : bf16_bits_to_f32(bias[n0 + cl + j]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int rl = 32 * r + (lane & 31);
          float v[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = acc[r][c][4 * q + j] + badd[j];
          uint32_t lo, hi;
          if (YKIND == 0) {
            lo = f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16);
            hi = f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16);
          } else {
            lo = f32_to_f16_bits(v[0]) | ((uint32_t)f32_to_f16_bits(v[1]) << 16);
            hi = f32_to_f16_bits(v[2]) | ((uint32_t)f32_to_f16_bits(v[3]) << 16);
          }
          *reinterpret_cast<u32x2_t*>(ep + rl * kPitch + cl * 2) = u32x2_t{lo, hi};
        }
      }
    // Each wave reads back only what it wrote. LDS accesses of one wave execute in order; the wave
    // barrier keeps the compiler from moving the reads (other lanes' data) above the writes.
    __builtin_amdgcn_wave_barrier();
    const int cc = (lane % kLpr) * 8;  // 8 columns = 16 bytes per lane
#pragma unroll 4
    for (int p = 0; p < 128 / kRpp; ++p) {
      const int rl = kRpp * p + lane / kLpr;
      const int row = m0 + rl, col = n0 + cc;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ep + rl * kPitch + cc * 2);
      if (row >= m || col >= n) continue;
      uint16_t* dst = static_cast<uint16_t*>(y) + (int64_t)row * n + col;
      if (col + 8 <= n) {
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(dst));
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (col + j < n) dst[j] = static_cast<uint16_t>(v[j >> 1] >> (16 * (j & 1)));
      }
    }
    return;
  }
  // fp32 y, or rows that do not keep 16-byte alignment: direct stores of the four columns
#pragma unroll
  for (int c = 0; c < CT; ++c)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = n0 + 32 * c + 8 * q + 4 * (lane >> 5);
      if (col >= n) continue;
      float badd[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (bias) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (col + j < n) badd[j] = YKIND == 1 ? f16_bits_to_f32(bias[col + j]) : bf16_bits_to_f32(bias[col + j]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + 32 * r + (lane & 31);
        if (row >= m) continue;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = acc[r][c][4 * q + j] + badd[j];
        const int64_t o = (int64_t)row * n + col;
        if (YKIND == 2 && vec && col + 3 < n) {
          *reinterpret_cast<f32x4_t*>(static_cast<float*>(y) + o) = f32x4_t{v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (col + j >= n) break;
            if (YKIND == 0) static_cast<uint16_t*>(y)[o + j] = f32_to_bf16_bits(v[j]);
            else if (YKIND == 1) static_cast<uint16_t*>(y)[o + j] = f32_to_f16_bits(v[j]);
            else static_cast<float*>(y)[o + j] = v[j];
          }
        }
      }
    }
}

}  // namespace sqx

using namespace sqx;

// ==============================================================================================
// extern "C" entry points
// ==============================================================================================
#ifndef SQX_MX_WN
#define SQX_MX_WN 4
#endif
namespace {
constexpr int kMxStages = 4;

template <int YK>
hipError_t launch_mx(const uint8_t* xt, const uint8_t* xst, const uint8_t* wt, const uint8_t* wst, void* y,
                     const uint16_t* bias, int m, int n, int KB, hipStream_t s) {
  const int tiles_m = (m + mxg::kTile - 1) / mxg::kTile, tiles_n = (n + mxg::kTile - 1) / mxg::kTile;
  const size_t lds = (size_t)kMxStages * mxg::kStage;
  auto kern = mxfp4_gemm_kernel<kMxStages, YK, SQX_MX_WN>;
  // more than 64 KiB of dynamic LDS has to be allowed per kernel
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)lds);
  if (e != hipSuccess) return e;
  // four-column vector stores need every row start aligned to the store width
  const int esize = YK == 2 ? 4 : 2;
  const int vec = (n % 4 == 0) && (reinterpret_cast<uintptr_t>(y) % (4 * esize) == 0);
  // the LDS-staged 16-bit epilogue stores 8 columns (16 bytes) per lane
  const int lds16 = YK != 2 && (n % 8 == 0) && (reinterpret_cast<uintptr_t>(y) % 16 == 0);
  hipLaunchKernelGGL(kern, dim3((unsigned)(tiles_m * tiles_n)), dim3(128 * SQX_MX_WN), lds, s, xt, xst, wt, wst, y, bias, m, n,
                     KB, tiles_m, tiles_n, vec, lds16);
  return hipGetLastError();
}
}  // namespace

extern "C" int sqx_mxfp4_gemm(const uint8_t* xt, const uint8_t* xst, const uint8_t* wt, const uint8_t* wst, void* y,
                              int y_dtype, const void* bias, int64_t m, int64_t rows, int64_t cols,
                              sqx_stream_t stream) {
  SQX_REQUIRE(m >= 0 && rows > 0 && cols > 0 && cols % 32 == 0, SQX_E_ARG,
              "sqx_mxfp4_gemm: bad shape m=%lld rows=%lld cols=%lld (cols must be a multiple of 32)", (long long)m,
              (long long)rows, (long long)cols);
  SQX_REQUIRE(y_dtype == SQX_DTYPE_BF16 || y_dtype == SQX_DTYPE_F16 || y_dtype == SQX_DTYPE_F32, SQX_E_ARG,
              "sqx_mxfp4_gemm: bad y_dtype %d", y_dtype);
  SQX_REQUIRE(bias == nullptr || y_dtype != SQX_DTYPE_F32, SQX_E_ARG,
              "sqx_mxfp4_gemm: bias is BF16/F16 and needs y of that dtype");
  const int64_t KB = ceil_div(cols, 128);
  SQX_REQUIRE(ceil_div(m, 16) * KB * 1024 < ((int64_t)1 << 31) && ceil_div(rows, 16) * KB * 1024 < ((int64_t)1 << 31),
              SQX_E_ARG, "sqx_mxfp4_gemm: tiled operand beyond 2 GiB (32-bit buffer offsets)");
  SQX_REQUIRE(m * rows < ((int64_t)1 << 62) && ceil_div(m, 256) * ceil_div(rows, 256) < ((int64_t)1 << 31), SQX_E_ARG,
              "sqx_mxfp4_gemm: too many output tiles");
  if (m == 0) return SQX_OK;
  SQX_REQUIRE(xt && xst && wt && wst && y, SQX_E_ARG, "sqx_mxfp4_gemm: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(xt) % 16 == 0 && reinterpret_cast<uintptr_t>(wt) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(xst) % 4 == 0 && reinterpret_cast<uintptr_t>(wst) % 4 == 0,
              SQX_E_ARG, "sqx_mxfp4_gemm: tiled codes must be 16-byte and scales 4-byte aligned");
  hipStream_t s = as_stream(stream);
  const uint16_t* b16 = static_cast<const uint16_t*>(bias);
  hipError_t e;
  if (y_dtype == SQX_DTYPE_BF16) e = launch_mx<0>(xt, xst, wt, wst, y, b16, (int)m, (int)rows, (int)KB, s);
  else if (y_dtype == SQX_DTYPE_F16) e = launch_mx<1>(xt, xst, wt, wst, y, b16, (int)m, (int)rows, (int)KB, s);
  else e = launch_mx<2>(xt, xst, wt, wst, y, b16, (int)m, (int)rows, (int)KB, s);
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "sqx_mxfp4_gemm: launch failed: %s", hipGetErrorString(e));
  return SQX_OK;
}
