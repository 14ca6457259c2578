// Prefill / large-batch linears on gfx950: dense contractions on the MFMA units.
//
// MXFP4 x MXFP4 (both operands E2M1 codes with one E8M0 scale per 32 columns, in the tiled FP4
// layout of sqx_fp4.hip): y[m, n] = sum_k X[m, k] W[n, k] on CDNA4's block-scaled
// v_mfma_scale_f32_32x32x64_f8f6f4, which multiplies the E2M1 values, applies each lane's E8M0
// scale to its 32 k-values and accumulates in fp32. This is the config-4 linear
// F.linear(mxfp4_dequantize(x), mxfp4_dequantize(W)) (nvfp4_mxfp4.py:257-272 composed with F.linear)
// without materialising either operand: every product of two dequantized values is exact in fp32.
//
// Tiling. One workgroup owns a 256 (m) x 256 (n) output tile. With the default WN = 4 it has eight
// waves (two per SIMD); wave w computes the 128 x 64 part (w / 4, w % 4) as 4 x 2 MFMA tiles of
// 32 x 32 held in 128 accumulation registers (WN = 2: four waves of 128 x 128, 4 x 4 tiles, 256
// registers). A k-step covers one 128-column FP4 block: 16 fragments (1 KiB each, 16 rows x 128
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
// Fragment rows past the operand's last 16-row tile are not read: their copies go past the buffer
// resource, which writes zeros without touching memory (the outputs they feed are masked), so an
// operand of fewer than 256 rows costs only its own bytes.
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
    const int t = t0 + f0 + j;
    const uint32_t off =
        t <= tmax ? ((uint32_t)t * (uint32_t)KB + (uint32_t)kb) * 1024u + (uint32_t)lane * 16u : 0xFFFFFFF0u;
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


// WN: waves along n (2: four waves of 128 x 128; 4: eight waves of 128 x 64, two per SIMD).
// SKIPR: X has at most 128 rows, so the waves of the tile's second 128 rows have nothing to compute.
template <int NSTAGE, int YKIND, int WN, bool SKIPR = false>  // YKIND: 0 = bf16, 1 = fp16, 2 = fp32
__global__ __launch_bounds__(128 * WN) void mxfp4_gemm_kernel(const uint8_t* __restrict__ xt,
                                                        const uint8_t* __restrict__ xst,
                                                        const uint8_t* __restrict__ wt,
                                                        const uint8_t* __restrict__ wst, void* __restrict__ y,
                                                        const uint16_t* __restrict__ bias, int m, int n, int KBall,
                                                        int tiles_m, int tiles_n, int vec, int lds16, int kps,
                                                        int64_t split_stride) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int NW = 2 * WN;              // waves
  constexpr int CT = 8 / WN;              // 32-column MFMA tiles per wave
  constexpr int kPerStep = 40 / NW;       // buffer->LDS instructions per wave per k-step
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, in an SGPR
  int tm, tn;
  mx_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);

  const int xT = (m + 15) >> 4, wT = (n + 15) >> 4;  // 16-row tiles of each operand
  const rsrc_t xr = make_rsrc(xt, (uint32_t)xT * (uint32_t)KBall * 1024u);
  const rsrc_t xsr = make_rsrc(xst, (uint32_t)xT * (uint32_t)KBall * 64u);
  const rsrc_t wr = make_rsrc(wt, (uint32_t)wT * (uint32_t)KBall * 1024u);
  const rsrc_t wsr = make_rsrc(wst, (uint32_t)wT * (uint32_t)KBall * 64u);
  // K split: workgroups with blockIdx.y = j take k-steps [j*kps, (j+1)*kps) and write fp32 partials
  // at y + j*split_stride (YKIND 2)
  const int kbeg = blockIdx.y * kps;
  const int KB = min(KBall, kbeg + kps) - kbeg;
  if (YKIND == 2) y = static_cast<float*>(y) + (int64_t)blockIdx.y * split_stride;
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
      mx_issue_step<NW>(smem + s * mxg::kStage, wave, lane, kbeg + s, KBall, xr, xsr, wr, wsr, x_t0, xT - 1, w_t0,
                        wT - 1);
  if (KB - 1 >= NSTAGE - 2) wait_vmcnt<kPerStep * (NSTAGE - 2)>();  // step 0 landed for this wave ...
  else wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();  // ... and for every wave
  // SKIPR: the waves of rows 128..255 skip their operand reads and MFMAs (they still copy and wait
  // with the others); otherwise every wave computes (no branch in the schedule)
  const bool live = !SKIPR || wm == 0;  // wave-uniform
  Ops o0, o1;
  if (live) read_ops(smem, 0, o0);
  // steady state: every iteration issues a copy, and the copies of NSTAGE-3 later steps may stay
  // in flight at the barrier
  int kb = 0;
  for (; kb + NSTAGE - 1 < KB; ++kb) {
    const uint8_t* st = smem + (kb % NSTAGE) * mxg::kStage;
    if (live) read_ops(st, 1, o1);
    if (live) mma(o0);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<kPerStep * (NSTAGE - 3)>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    mx_issue_step<NW>(smem + ((kb + NSTAGE - 1) % NSTAGE) * mxg::kStage, wave, lane, kbeg + kb + NSTAGE - 1, KBall, xr,
                      xsr, wr,
                  wsr, x_t0, xT - 1, w_t0, wT - 1);
    if (live) read_ops(smem + ((kb + 1) % NSTAGE) * mxg::kStage, 0, o0);
    if (live) mma(o1);
  }
  // tail: nothing left to issue; wait for everything still in flight
  for (; kb < KB; ++kb) {
    const uint8_t* st = smem + (kb % NSTAGE) * mxg::kStage;
    if (live) read_ops(st, 1, o1);
    if (live) mma(o0);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (live && kb + 1 < KB) read_ops(smem + ((kb + 1) % NSTAGE) * mxg::kStage, 0, o0);
    if (live) mma(o1);
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


// ==============================================================================================
// Dequant GEMM: bf16 / fp16 activations x a tiled 4-bit weight (group INT4 or FP4)
// ==============================================================================================
// y[m, n] = sum_k x[m, k] W[n, k] (+ bias[n]) for x [M, K] row-major and W in the tiled layout of
// sqx_int4.hip (group INT4, symmetric or asymmetric) or sqx_fp4.hip (MXFP4 / NVFP4): the prefill
// form of w4a16_linear (int4_group.py:148-164), awq_linear (awq.py:184-192) and the config-4
// FP4-weight linear. Each weight is decoded to the activation dtype in registers exactly as the
// reference's dequantize(...).to(x.dtype) produces it: INT4 as the fp32 (q - z) * s rounded to
// nearest even, FP4 as e2m1 * scale (exact; NVFP4's global scale multiplies the fp32 result).
//
// Tiling. A workgroup of 8 waves owns a 256 x 256 output tile; wave w computes rows
// 128 (w / 4) .. +128 and columns 64 (w % 4) .. +64 as 8 x 4 tiles of v_mfma_f32_16x16x32 with the
// weight as the first operand, so a lane's four accumulators are four consecutive output columns
// of one row. A stage covers 64 k: the 256 activation rows (32 KiB, 16-byte chunks XOR-swizzled
// by row so the operand reads of 8 consecutive rows hit distinct banks), the weight bytes of the
// 16 row tiles for those 64 columns, and their scales; NSTAGE stages form a ring filled by
// buffer -> LDS copies as in the MXFP4 GEMM. Every wave decodes its own 4 weight tiles per 32-k
// MFMA step (the decode is shared by the wave's 8 row tiles).
namespace dqg {
constexpr int kTile = 256;
constexpr int kBK = 64;
constexpr int kXBytes = kTile * kBK * 2;  // activations of one stage
constexpr int kWBytes = 16 * 512;         // 16 weight row tiles x 512 bytes
constexpr int kPBytes = 4096;             // scales / zero-points of one stage
constexpr int kStage = kXBytes + kWBytes + kPBytes;
constexpr int kStages = 3;
constexpr int kEpiPitch = 136;            // LDS bytes per row of a wave's 128 x 64 16-bit output tile
constexpr int kLds = 8 * 128 * kEpiPitch; // 139264 >= kStages * kStage
static_assert(kStages * kStage <= kLds, "stages fit the LDS allocation");
}  // namespace dqg

// Weight formats of the dequant GEMM.
enum : int { kDqInt4 = 0, kDqMx = 1, kDqNv = 2 };

template <int FMT, bool ASYM, bool PBF16, int GROUP>
struct DqW {
  // parameter bytes per stage and tile: INT4 scales (and zero-points) of the stage's groups;
  // MXFP4 32 E8M0 bytes (lanes 32h..32h+31 of the 64-byte block), NVFP4 64 E4M3 bytes
  // asymmetric bf16 INT4 parameters are (scale, zero) pairs in one dword (sqx_int4_tile)
  static constexpr bool PAIR = ASYM && PBF16;
  static constexpr bool ZSEP = ASYM && !PBF16;  // zero-points in a buffer of their own
  static constexpr int PB = (PBF16 && !PAIR) ? 2 : 4;
  static constexpr int kWInstr = FMT == kDqInt4 ? 4 : 1;  // weight copies per wave per stage
  static constexpr int kPInstr = 2;                        // parameter copies per wave per stage
  static constexpr int NGS = GROUP >= 64 ? 1 : 64 / GROUP;  // INT4 groups per stage
  static constexpr int NP = FMT == kDqMx ? 2 : FMT == kDqNv ? 4 : (ZSEP ? 2 : 1) * NGS * 16 * 16 * PB / 256;
  static_assert(NP <= 16, "parameter copies fit two per wave");
};

template <class A, int FMT, bool ASYM, bool PBF16, int GROUP, int YKIND, int TMR = 256>
__global__ __launch_bounds__(512) void dq_gemm_kernel(const uint16_t* __restrict__ x, const uint8_t* __restrict__ wt,
                                                     const void* __restrict__ st, const void* __restrict__ zt,
                                                     const float* __restrict__ s_global, void* __restrict__ y,
                                                     const uint16_t* __restrict__ bias, int m, int n, int K, int KB,
                                                     int tiles_m, int tiles_n, int lds16, int splits,
                                                     float* __restrict__ ws) {
  using P = DqW<FMT, ASYM, PBF16, GROUP>;
  static_assert(TMR == 256 || TMR == 128, "256- or 128-row output tiles");
  constexpr int group = GROUP;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int NS = dqg::kStages;
  constexpr int kXI = TMR / 64;   // activation copies per wave per stage (8 rows each)
  constexpr int RPW = TMR / 8;    // activation rows a wave copies
  constexpr int MT = TMR / 32;    // 16-row MFMA tiles of a wave (it owns TMR / 2 rows)
  constexpr int kPerStage = kXI + P::kWInstr + P::kPInstr;  // buffer -> LDS copies per wave per stage
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int tm, tn;
  // split-K: workgroup b computes split b % splits of tile b / splits (stages s0 .. s0+S-1)
  const int tile = blockIdx.x / splits, split = blockIdx.x - tile * splits;
  mx_tile_of(tile, tiles_m, tiles_n, tm, tn);
  const int S_all = 2 * KB;  // stages of 64 columns (the tiled weight is padded to 128-column blocks)
  const int Sp = (S_all + splits - 1) / splits;
  const int s0 = split * Sp;
  const int S = min(S_all, s0 + Sp) - s0;
  const int wT = (n + 15) >> 4;
  const int w_t0 = tn * 16;
  const int Gp = KB * (128 / (FMT == kDqInt4 ? GROUP : 128));  // INT4 groups per row (padded)

  const rsrc_t xr = make_rsrc(x, (uint32_t)((uint64_t)m * (uint64_t)K * 2u));
  const rsrc_t wr = make_rsrc(wt, (uint32_t)wT * (uint32_t)KB * 1024u);
  uint32_t pbytes;
  if (FMT == kDqInt4) pbytes = (uint32_t)wT * (uint32_t)Gp * 16u * P::PB;
  else pbytes = (uint32_t)wT * (uint32_t)KB * (FMT == kDqMx ? 64u : 128u);
  const rsrc_t sr = make_rsrc(st, pbytes);
  const rsrc_t zr = make_rsrc(ASYM ? zt : st, pbytes);
  constexpr int np = P::NP;

  // ---- copies of stage s into ring slot `slot`
  auto issue = [&](int s, int slot) {
    uint8_t* base = smem + slot * dqg::kStage;
    const int kb = s >> 1, h = s & 1;
    // activations: wave w copies rows RPW*w .. RPW*w + RPW-1 (8 rows of 8 chunks per instruction)
#pragma unroll
    for (int j = 0; j < kXI; ++j) {
      const int r = RPW * wave + 8 * j + (lane >> 3);
      const int c = (lane & 7) ^ (r & 7);
      const int R = tm * TMR + r, col = 64 * s + 8 * c;
      const bool ok = (R < m) & (col < K);  // no short-circuit: a select, not a branch
      const uint32_t off = ok ? ((uint32_t)R * (uint32_t)K + (uint32_t)col) * 2u : 0xFFFFFFF0u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(base + (RPW * wave + 8 * j) * 128), 16, off, 0, 0, 0);
    }
    uint8_t* wbase = base + dqg::kXBytes;
    if (FMT == kDqInt4) {
      // tiles 2w, 2w+1: dwords 2h and 2h+1 of every lane's 16 bytes, 256 bytes per copy
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int f = 2 * wave + (j >> 1), i = 2 * h + (j & 1);
        const int t = min(w_t0 + f, wT - 1);
        const uint32_t off = ((uint32_t)t * (uint32_t)KB + (uint32_t)kb) * 1024u + (uint32_t)lane * 16u + (uint32_t)i * 4u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(wbase + f * 512 + (j & 1) * 256), 4, off, 0, 0, 0);
      }
    } else {
      // tiles 2w (lanes 0-31) and 2w+1 (lanes 32-63): bytes 512h .. 512h+511 of their blocks
      const int f = 2 * wave + (lane >> 5);
      const int t = min(w_t0 + f, wT - 1);
      const uint32_t off = ((uint32_t)t * (uint32_t)KB + (uint32_t)kb) * 1024u + 512u * (uint32_t)h + (uint32_t)(lane & 31) * 16u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(wbase + 2 * wave * 512), 16, off, 0, 0, 0);
    }
    uint8_t* pbase = base + dqg::kXBytes + dqg::kWBytes;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int pi = 2 * wave + j;  // parameter copy index; copies past np land in unused LDS
      const int pr = pi < np ? pi : 0;
      uint32_t off;
      bool zsrc = false;
      if (FMT == kDqInt4) {
        // layout in LDS: [scales | zeros][group gi][tile f][row] of PB bytes; 256 bytes per copy
        constexpr int TPI = 256 / (16 * P::PB);  // tiles per copy
        const int per_kind = np / (P::ZSEP ? 2 : 1);
        zsrc = P::ZSEP && pr >= per_kind;
        const int q = pr - (zsrc ? per_kind : 0);
        const int gi = q / (16 / TPI);
        const int f = TPI * (q % (16 / TPI)) + lane / (64 / TPI);
        const int t = min(w_t0 + f, wT - 1);
        const int g = (64 * s) / group + gi;
        off = ((uint32_t)t * (uint32_t)Gp + (uint32_t)g) * 16u * P::PB + (uint32_t)(lane % (64 / TPI)) * 4u;
      } else if (FMT == kDqMx) {
        const int f = 8 * pr + (lane >> 3);
        const int t = min(w_t0 + f, wT - 1);
        off = ((uint32_t)t * (uint32_t)KB + (uint32_t)kb) * 64u + 32u * (uint32_t)h + (uint32_t)(lane & 7) * 4u;
      } else {
        const int f = 4 * pr + (lane >> 4);
        const int t = min(w_t0 + f, wT - 1);
        off = ((uint32_t)t * (uint32_t)KB + (uint32_t)kb) * 128u + 64u * (uint32_t)h + (uint32_t)(lane & 15) * 4u;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(zsrc ? zr : sr, (lds_void*)(pbase + pi * 256), 4, off, 0, 0, 0);
    }
  };

  f32x4_t acc[MT][4];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int wm = wave >> 2, wn = wave & 3;
  const int nl = lane & 15, jg = lane >> 4;
  // p0: the scale's fp32 bits, or for bf16 INT4 parameters bf16 scale | bf16 zero-point << 16;
  // p1: fp32 zero-points (asymmetric INT4 with fp32 parameters only)
  constexpr int kP1 = (FMT == kDqInt4 && ASYM && !PBF16) ? 4 : 1;
  struct Raw {
    u32x4_t xo[MT];  // activation operands of the wave's row tiles
    uint32_t wd[4];  // weight codes of the 4 column tiles
    uint32_t p0[4], p1[kP1];
  };
  // operands of MFMA step q (32 columns) of the stage in ring slot `slot`
  auto read = [&](int slot, int s, int q, Raw& o) {
    const uint8_t* base = smem + slot * dqg::kStage;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = wm * (TMR / 2) + 16 * mt + nl;
      const int sl = (4 * q + jg) ^ (nl & 7);
      o.xo[mt] = *reinterpret_cast<const u32x4_t*>(base + r * 128 + sl * 16);
    }
    const uint8_t* wb = base + dqg::kXBytes;
    const uint8_t* pb = base + dqg::kXBytes + dqg::kWBytes;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int f = wn * 4 + nt;
      if (FMT == kDqInt4) {
        o.wd[nt] = *reinterpret_cast<const uint32_t*>(wb + f * 512 + q * 256 + lane * 4);
        const int gi = GROUP >= 64 ? 0 : (32 * q) / GROUP;
        constexpr int zoff = P::NGS * 16 * 16 * P::PB;
        const int po = ((gi * 16 + f) * 16 + nl) * P::PB;
        if (P::PAIR) {
          o.p0[nt] = *reinterpret_cast<const uint32_t*>(pb + po);  // bf16 scale | bf16 zero << 16
        } else if (PBF16) {
          o.p0[nt] = *reinterpret_cast<const uint16_t*>(pb + po);
        } else {
          o.p0[nt] = *reinterpret_cast<const uint32_t*>(pb + po);
          if (ASYM) o.p1[nt % kP1] = *reinterpret_cast<const uint32_t*>(pb + zoff + po);
        }
      } else {
        const int ll = 16 * q + nl;  // lane of the 128-column block within the stage's half
        o.wd[nt] = *reinterpret_cast<const uint32_t*>(wb + f * 512 + ll * 16 + jg * 4);
        if (FMT == kDqMx) {
          o.p0[nt] = (uint32_t)pb[f * 32 + ll] << 23;  // the fp32 2**(e - 127)
        } else {
          o.p0[nt] = __builtin_bit_cast(uint32_t, e4m3_value(pb[f * 64 + 2 * ll + (jg >> 1)]));
        }
      }
    }
    (void)s;
  };
  // weight operand of column tile nt: 8 consecutive k of row nl, in the activation dtype
  auto decode = [&](const Raw& o, int nt) -> u32x4_t {
    const uint32_t d = o.wd[nt];
    if (FMT == kDqMx) {
      const float sc = __builtin_bit_cast(float, o.p0[nt]);
      return u32x4_t{A::fp4_pair_scaled(d, sc, 0), A::fp4_pair_scaled(d, sc, 1), A::fp4_pair_scaled(d, sc, 2),
                     A::fp4_pair_scaled(d, sc, 3)};
    }
    float w[8];
    if (FMT == kDqNv) {
      const float sc = __builtin_bit_cast(float, o.p0[nt]);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const f32x2_t f = A::fp4_pair_f32(d, p);
        w[2 * p] = f[0] * sc;
        w[2 * p + 1] = f[1] * sc;
      }
      return u32x4_t{A::pack_exact(w[0], w[1]), A::pack_exact(w[2], w[3]), A::pack_exact(w[4], w[5]),
                     A::pack_exact(w[6], w[7])};
    }
    // INT4: element e in nibble e/2 (even e) or 4 + e/2 (odd e); u as fp32, then fp32 (u - z) * s
    const uint32_t lo = d & 0x0F0F0F0Fu, hi = (d >> 4) & 0x0F0F0F0Fu;
    const float u[8] = {ubyte_f32<0>(lo), ubyte_f32<2>(lo), ubyte_f32<0>(hi), ubyte_f32<2>(hi),
                        ubyte_f32<1>(lo), ubyte_f32<3>(lo), ubyte_f32<1>(hi), ubyte_f32<3>(hi)};
    const float sc = PBF16 ? bf16_bits_to_f32((uint16_t)(o.p0[nt] & 0xffffu)) : __builtin_bit_cast(float, o.p0[nt]);
    if (!ASYM || PBF16) {
      // z * s is exact (z = 8, or z <= 15 and s has at most 8 significant bits), so the fma rounds
      // the exact (u - z) * s once
      const float zf = ASYM ? bf16_bits_to_f32((uint16_t)(o.p0[nt] >> 16)) : 8.0f;
      const float c = -zf * sc;
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = fmaf(u[e], sc, c);
    } else {
      const float zf = __builtin_bit_cast(float, o.p1[nt % kP1]);
#pragma unroll
      for (int e = 0; e < 8; ++e) w[e] = (u[e] - zf) * sc;
    }
    return u32x4_t{A::pack_rne(w[0], w[1]), A::pack_rne(w[2], w[3]), A::pack_rne(w[4], w[5]), A::pack_rne(w[6], w[7])};
  };
  auto mma = [&](const Raw& o) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const u32x4_t b = decode(o, nt);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = A::mfma(b, o.xo[mt], acc[mt][nt]);
    }
  };

  // pipeline (as the MXFP4 GEMM): iteration s: read (s, 1) | MFMAs (s, 0) | wait for stage s+1,
  // barrier | copy stage s+NS-1 into the slot of s-1 | read (s+1, 0) | MFMAs (s, 1)
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < S) issue(s0 + s, s);
  if (S - 1 >= NS - 2) wait_vmcnt<kPerStage * (NS - 2)>();
  else wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  Raw o0, o1;
  read(0, 0, 0, o0);
  int s = 0;
  for (; s + NS - 1 < S; ++s) {
    read(s % NS, s, 1, o1);
    mma(o0);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<kPerStage * (NS - 3)>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(s0 + s + NS - 1, (s + NS - 1) % NS);
    read((s + 1) % NS, s + 1, 0, o0);
    mma(o1);
  }
  for (; s < S; ++s) {
    read(s % NS, s, 1, o1);
    mma(o0);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 < S) read((s + 1) % NS, s + 1, 0, o0);
    mma(o1);
  }

  // epilogue: acc[mt][nt][i] is y[m0 + 16mt + (l & 15)][n0 + 16nt + 4(l >> 4) + i]
  const int m0 = tm * TMR + wm * (TMR / 2);
  const int n0 = tn * dqg::kTile + wn * 64;
  if (splits > 1) {
    // raw fp32 partial sums of this split; dq_reduce_kernel adds the splits in order
    float* part = ws + (int64_t)split * m * n;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int col = n0 + 16 * nt + 4 * jg;
      if (col >= n) continue;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int row = m0 + 16 * mt + nl;
        if (row >= m) continue;
        float* dst = part + (int64_t)row * n + col;
        if ((n & 3) == 0) {
          *reinterpret_cast<f32x4_t*>(dst) = acc[mt][nt];
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (col + j < n) dst[j] = acc[mt][nt][j];
        }
      }
    }
    return;
  }
  const float gs = FMT == kDqNv ? *s_global : 1.0f;
  if (YKIND != 2 && lds16) {
    __builtin_amdgcn_s_barrier();  // every wave is done reading the stages
    uint8_t* ep = smem + wave * 128 * dqg::kEpiPitch;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int cl = 16 * nt + 4 * jg;
      float badd[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (bias) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (n0 + cl + j < n) badd[j] = YKIND == 1 ? f16_bits_to_f32(bias[n0 + cl + j]) : bf16_bits_to_f32(bias[n0 + cl + j]);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int rl = 16 * mt + nl;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = acc[mt][nt][j] * gs + badd[j];
        const uint32_t lo = YKIND == 0 ? ActBF16::pack_rne(v[0], v[1]) : ActF16::pack_rne(v[0], v[1]);
        const uint32_t hi = YKIND == 0 ? ActBF16::pack_rne(v[2], v[3]) : ActF16::pack_rne(v[2], v[3]);
        *reinterpret_cast<u32x2_t*>(ep + rl * dqg::kEpiPitch + cl * 2) = u32x2_t{lo, hi};
      }
    }
    __builtin_amdgcn_wave_barrier();
    const int cc = (lane & 7) * 8;
#pragma unroll 4
    for (int p = 0; p < TMR / 16; ++p) {
      const int rl = 8 * p + (lane >> 3);
      const int row = m0 + rl, col = n0 + cc;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ep + rl * dqg::kEpiPitch + cc * 2);
      if (row >= m || col >= n) continue;
      uint16_t* dst = static_cast<uint16_t*>(y) + (int64_t)row * n + col;
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(dst));
    }
    return;
  }
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int col = n0 + 16 * nt + 4 * jg;
    if (col >= n) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int row = m0 + 16 * mt + nl;
      if (row >= m) continue;
      const int64_t o = (int64_t)row * n + col;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (col + j >= n) break;
        float v = acc[mt][nt][j] * gs;
        if (bias) v += YKIND == 1 ? f16_bits_to_f32(bias[col + j]) : bf16_bits_to_f32(bias[col + j]);
        if (YKIND == 0) static_cast<uint16_t*>(y)[o + j] = f32_to_bf16_bits(v);
        else if (YKIND == 1) static_cast<uint16_t*>(y)[o + j] = f32_to_f16_bits(v);
        else static_cast<float*>(y)[o + j] = v;
      }
    }
  }
}

// y[i] = (sum over splits, in order, of the fp32 partials) * gs (+ bias[i % n]), rounded to y's dtype.
template <int YKIND>
__global__ __launch_bounds__(256) void dq_reduce_kernel(const float* __restrict__ ws, int splits, int64_t mn, int n,
                                                        const float* __restrict__ s_global,
                                                        const uint16_t* __restrict__ bias, void* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= mn) return;
  float v = 0.0f;
  for (int s = 0; s < splits; ++s) v += ws[(int64_t)s * mn + i];
  if (s_global) v *= *s_global;
  if (bias) v += YKIND == 1 ? f16_bits_to_f32(bias[i % n]) : bf16_bits_to_f32(bias[i % n]);
  if (YKIND == 0) static_cast<uint16_t*>(y)[i] = f32_to_bf16_bits(v);
  else if (YKIND == 1) static_cast<uint16_t*>(y)[i] = f32_to_f16_bits(v);
  else static_cast<float*>(y)[i] = v;
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

// K splits of the MXFP4 GEMM for a shape, from a cost model fitted to measurements of 128..512-row
// products at Llama shapes. One 256 x 256 workgroup fills a CU (its four operand stages take 136 KiB
// of LDS), so S splits run in ceil(tiles * S / 256) rounds of ceil(KB / S) k-steps. A k-step takes
// about 0.7 us with the chip nearly idle and 1.25 us with every CU loading (HBM shared); each split
// adds an fp32 partial of the output, written once and read back once (8 bytes per output element
// at about 5 TB/s). S minimises the sum, at most 16.
int mx_splits(int64_t m, int64_t rows, int64_t cols) {
  const int64_t tiles = ceil_div(m, mxg::kTile) * ceil_div(rows, mxg::kTile), KB = ceil_div(cols, 128);
  int best = 1;
  double best_us = 0.0;
  for (int S = 1; S <= 16 && S <= KB; ++S) {
    const int64_t per = ceil_div(KB, S);
    if (ceil_div(KB, per) != S) continue;  // the last split would be empty
    const int64_t wgs = tiles * S, rounds = ceil_div(wgs, 256);
    const double busy = rounds > 1 ? 1.0 : (double)wgs / 256.0;
    double us = (double)rounds * (double)per * (0.7 + 0.55 * busy);
    if (S > 1) us += (double)S * (double)m * (double)rows * 8.0 / 5e6;
    if (S == 1 || us < best_us) best = S, best_us = us;
  }
  return best;
}

// splits > 1: fp32 partials into ws ([splits][m][n], 16-byte aligned, checked by the caller), then
// the in-order reduce adds the splits and the bias and rounds to y's dtype.
template <int YK>
hipError_t launch_mx(const uint8_t* xt, const uint8_t* xst, const uint8_t* wt, const uint8_t* wst, void* y,
                     const uint16_t* bias, int m, int n, int KB, int splits, float* ws, hipStream_t s) {
  const int tiles_m = (m + mxg::kTile - 1) / mxg::kTile, tiles_n = (n + mxg::kTile - 1) / mxg::kTile;
  const size_t lds = (size_t)kMxStages * mxg::kStage;
  const int kps = (KB + splits - 1) / splits;
  auto kern = m <= 128 ? (splits > 1 ? mxfp4_gemm_kernel<kMxStages, 2, SQX_MX_WN, true>
                                     : mxfp4_gemm_kernel<kMxStages, YK, SQX_MX_WN, true>)
                       : (splits > 1 ? mxfp4_gemm_kernel<kMxStages, 2, SQX_MX_WN>
                                     : mxfp4_gemm_kernel<kMxStages, YK, SQX_MX_WN>);
  // more than 64 KiB of dynamic LDS has to be allowed per kernel
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)lds);
  if (e != hipSuccess) return e;
  void* out = splits > 1 ? static_cast<void*>(ws) : y;
  // four-column vector stores need every row start aligned to the store width
  const int esize = (YK == 2 || splits > 1) ? 4 : 2;
  const int vec = (n % 4 == 0) && (reinterpret_cast<uintptr_t>(out) % (4 * esize) == 0);
  // the LDS-staged 16-bit epilogue stores 8 columns (16 bytes) per lane
  const int lds16 = YK != 2 && splits == 1 && (n % 8 == 0) && (reinterpret_cast<uintptr_t>(y) % 16 == 0);
  hipLaunchKernelGGL(kern, dim3((unsigned)(tiles_m * tiles_n), (unsigned)splits), dim3(128 * SQX_MX_WN), lds, s, xt,
                     xst, wt, wst, out, splits > 1 ? nullptr : bias, m, n, KB, tiles_m, tiles_n, vec, lds16, kps,
                     (int64_t)m * n);
  if (splits > 1) {
    const int64_t mn = (int64_t)m * n;
    hipLaunchKernelGGL(dq_reduce_kernel<YK>, dim3((unsigned)ceil_div(mn, 256)), dim3(256), 0, s, ws, splits, mn, n,
                       nullptr, bias, y);
  }
  return hipGetLastError();
}

int mx_check(const char* fn, const uint8_t* xt, const uint8_t* xst, const uint8_t* wt, const uint8_t* wst,
             const void* y, int y_dtype, const void* bias, int64_t m, int64_t rows, int64_t cols) {
  SQX_REQUIRE(m >= 0 && rows > 0 && cols > 0 && cols % 32 == 0, SQX_E_ARG,
              "%s: bad shape m=%lld rows=%lld cols=%lld (cols must be a multiple of 32)", fn, (long long)m,
              (long long)rows, (long long)cols);
  SQX_REQUIRE(y_dtype == SQX_DTYPE_BF16 || y_dtype == SQX_DTYPE_F16 || y_dtype == SQX_DTYPE_F32, SQX_E_ARG,
              "%s: bad y_dtype %d", fn, y_dtype);
  SQX_REQUIRE(bias == nullptr || y_dtype != SQX_DTYPE_F32, SQX_E_ARG, "%s: bias is BF16/F16 and needs y of that dtype",
              fn);
  const int64_t KB = ceil_div(cols, 128);
  SQX_REQUIRE(ceil_div(m, 16) * KB * 1024 < ((int64_t)1 << 31) && ceil_div(rows, 16) * KB * 1024 < ((int64_t)1 << 31),
              SQX_E_ARG, "%s: tiled operand beyond 2 GiB (32-bit buffer offsets)", fn);
  SQX_REQUIRE(m * rows < ((int64_t)1 << 62) && ceil_div(m, 256) * ceil_div(rows, 256) < ((int64_t)1 << 31), SQX_E_ARG,
              "%s: too many output tiles", fn);
  if (m == 0) return SQX_OK;
  SQX_REQUIRE(xt && xst && wt && wst && y, SQX_E_ARG, "%s: null pointer", fn);
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(xt) % 16 == 0 && reinterpret_cast<uintptr_t>(wt) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(xst) % 4 == 0 && reinterpret_cast<uintptr_t>(wst) % 4 == 0,
              SQX_E_ARG, "%s: tiled codes must be 16-byte and scales 4-byte aligned", fn);
  return SQX_OK;
}

int mx_run(const char* fn, const uint8_t* xt, const uint8_t* xst, const uint8_t* wt, const uint8_t* wst, void* y,
           int y_dtype, const void* bias, int64_t m, int64_t rows, int64_t cols, int splits, float* ws,
           hipStream_t s) {
  const uint16_t* b16 = static_cast<const uint16_t*>(bias);
  const int KB = (int)ceil_div(cols, 128);
  hipError_t e;
  if (y_dtype == SQX_DTYPE_BF16) e = launch_mx<0>(xt, xst, wt, wst, y, b16, (int)m, (int)rows, KB, splits, ws, s);
  else if (y_dtype == SQX_DTYPE_F16) e = launch_mx<1>(xt, xst, wt, wst, y, b16, (int)m, (int)rows, KB, splits, ws, s);
  else e = launch_mx<2>(xt, xst, wt, wst, y, b16, (int)m, (int)rows, KB, splits, ws, s);
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return SQX_OK;
}
}  // namespace

extern "C" int sqx_mxfp4_gemm(const uint8_t* xt, const uint8_t* xst, const uint8_t* wt, const uint8_t* wst, void* y,
                              int y_dtype, const void* bias, int64_t m, int64_t rows, int64_t cols,
                              sqx_stream_t stream) {
  if (int rc = mx_check("sqx_mxfp4_gemm", xt, xst, wt, wst, y, y_dtype, bias, m, rows, cols)) return rc;
  if (m == 0) return SQX_OK;
  return mx_run("sqx_mxfp4_gemm", xt, xst, wt, wst, y, y_dtype, bias, m, rows, cols, 1, nullptr, as_stream(stream));
}

extern "C" int64_t sqx_mxfp4_gemm_workspace_bytes(int64_t m, int64_t rows, int64_t cols, int splits) {
  if (m <= 0 || rows <= 0 || cols <= 0) return 0;
  const int sp = splits > 0 ? splits : mx_splits(m, rows, cols);
  return sp > 1 ? (int64_t)sp * m * rows * 4 : 0;
}

extern "C" int sqx_mxfp4_gemm_ws(const uint8_t* xt, const uint8_t* xst, const uint8_t* wt, const uint8_t* wst, void* y,
                                 int y_dtype, const void* bias, int64_t m, int64_t rows, int64_t cols, int splits,
                                 void* ws, int64_t ws_bytes, sqx_stream_t stream) {
  const char* fn = "sqx_mxfp4_gemm_ws";
  if (int rc = mx_check(fn, xt, xst, wt, wst, y, y_dtype, bias, m, rows, cols)) return rc;
  const int64_t KB = ceil_div(cols, 128);
  SQX_REQUIRE(splits <= 16, SQX_E_ARG, "%s: splits %d above 16", fn, splits);
  if (m == 0) return SQX_OK;
  int sp = splits;
  if (sp <= 0) {  // automatic: without a large enough workspace, one pass per tile
    sp = mx_splits(m, rows, cols);
    if (sp > 1 && (ws == nullptr || ws_bytes < (int64_t)sp * m * rows * 4 || reinterpret_cast<uintptr_t>(ws) % 16))
      sp = 1;
  } else {
    SQX_REQUIRE(ceil_div(KB, ceil_div(KB, sp)) == sp, SQX_E_ARG,
                "%s: %d splits of %lld k-steps of 128 columns would leave one empty", fn, sp, (long long)KB);
    if (sp > 1) {
      SQX_REQUIRE(ws && reinterpret_cast<uintptr_t>(ws) % 16 == 0, SQX_E_ARG,
                  "%s: splits > 1 need a 16-byte aligned workspace", fn);
      SQX_REQUIRE(ws_bytes >= (int64_t)sp * m * rows * 4, SQX_E_SPACE, "%s: workspace of %lld bytes, %lld needed", fn,
                  (long long)ws_bytes, (long long)sp * m * rows * 4);
    }
  }
  SQX_REQUIRE(sp == 1 || (int64_t)sp * m * rows < ((int64_t)1 << 40), SQX_E_ARG, "%s: workspace too large", fn);
  return mx_run(fn, xt, xst, wt, wst, y, y_dtype, bias, m, rows, cols, sp, static_cast<float*>(ws),
                as_stream(stream));
}

namespace {
// K splits for a shape: when the output tiles fill less than three quarters of the 256 CUs, as many
// splits as keep the workgroups within one round on the CUs (a second, partial round costs more than
// the splits save, and every split adds M x N fp32 partials to write and reduce), at least 4 stages
// (256 columns) per split, and no empty split.
// Output-tile rows: 128 for M <= 128, where a 256-row tile is at least half padding (config 4's
// bf16 activations at M = 128: 106 -> 74 us and 96 -> 65 us), else 256: a 128-row tile decodes each
// weight for half as many MFMAs, and at M = 512 / 2048 it measured slower on the 14336-wide shapes
// (97 -> 104 us, 298 -> 364 us) and within 6 % elsewhere. Also 128 when 256-row tiles would number
// fewer than 16, where the K splits that fill the CUs are the cost (4096->1024 at M = 512, which
// splits 16 ways either way: 31.9 -> 28.3 us; 4096x4096 at M = 512 has 32 tiles: 44.3 us against
// 43.0 us at its best 128-row split, so it stays).
int dq_tile_rows(int64_t m, int64_t rows) {
  if (m <= 128) return 128;
  return ceil_div(m, 256) * ceil_div(rows, dqg::kTile) < 16 ? 128 : 256;
}

int dq_splits(int64_t m, int64_t rows, int64_t cols) {
  const int64_t tiles = ceil_div(m, dq_tile_rows(m, rows)) * ceil_div(rows, dqg::kTile);
  const int64_t S = 2 * ceil_div(cols, 128);
  if (tiles >= 192) return 1;
  const int64_t want = std::min<int64_t>(std::min<int64_t>(256 / tiles, S / 4), 16);
  if (want < 2) return 1;
  const int64_t per = ceil_div(S, want);
  return (int)ceil_div(S, per);
}

template <class A, int FMT, bool ASYM, bool PBF16, int GROUP, int YK>
hipError_t launch_dq(const uint16_t* x, const uint8_t* wt, const void* st, const void* zt, const float* s_global,
                     void* y, const uint16_t* bias, int m, int n, int K, int KB, float* ws, int64_t ws_bytes,
                     hipStream_t s) {
  const int tmr = dq_tile_rows(m, n);
  const int tiles_m = (m + tmr - 1) / tmr, tiles_n = (n + dqg::kTile - 1) / dqg::kTile;
  int splits = dq_splits(m, n, K);
  if (splits > 1 && (ws == nullptr || ws_bytes < (int64_t)splits * m * n * 4 || reinterpret_cast<uintptr_t>(ws) % 16))
    splits = 1;  // no (or too small a) workspace: one pass per tile
  auto kern = tmr == 128 ? dq_gemm_kernel<A, FMT, ASYM, PBF16, GROUP, YK, 128> : dq_gemm_kernel<A, FMT, ASYM, PBF16, GROUP, YK, 256>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     dqg::kLds);
  if (e != hipSuccess) return e;
  const int lds16 = YK != 2 && (n % 8 == 0) && (reinterpret_cast<uintptr_t>(y) % 16 == 0);
  hipLaunchKernelGGL(kern, dim3((unsigned)(tiles_m * tiles_n * splits)), dim3(512), dqg::kLds, s, x, wt, st, zt,
                     s_global, y, bias, m, n, K, KB, tiles_m, tiles_n, lds16, splits, ws);
  if (splits > 1) {
    const int64_t mn = (int64_t)m * n;
    hipLaunchKernelGGL(dq_reduce_kernel<YK>, dim3((unsigned)ceil_div(mn, 256)), dim3(256), 0, s, ws, splits, mn, n,
                       FMT == kDqNv ? s_global : nullptr, bias, y);
  }
  return hipGetLastError();
}

// shape checks shared by the dequant GEMM entry points
int dq_check(const char* fn, const void* x, const void* wt, const void* y, int64_t m, int64_t rows, int64_t cols) {
  SQX_REQUIRE(m >= 0 && rows > 0 && cols > 0 && cols % 32 == 0, SQX_E_ARG,
              "%s: bad shape m=%lld rows=%lld cols=%lld (cols must be a multiple of 32)", fn, (long long)m,
              (long long)rows, (long long)cols);
  SQX_REQUIRE(m * cols * 2 < ((int64_t)1 << 31) && ceil_div(rows, 16) * ceil_div(cols, 128) * 1024 < ((int64_t)1 << 31) &&
                  ceil_div(m, 256) * ceil_div(rows, 256) < ((int64_t)1 << 31),
              SQX_E_ARG, "%s: operands beyond 2 GiB (32-bit buffer offsets)", fn);
  SQX_REQUIRE(m == 0 || (x && wt && y), SQX_E_ARG, "%s: null pointer", fn);
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(wt) % 16 == 0, SQX_E_ARG,
              "%s: x and the tiled weight must be 16-byte aligned", fn);
  return SQX_OK;
}
}  // namespace

extern "C" int64_t sqx_gemm_workspace_bytes(int64_t m, int64_t rows, int64_t cols) {
  if (m <= 0 || rows <= 0 || cols <= 0) return 0;
  const int sp = dq_splits(m, rows, cols);
  return sp > 1 ? (int64_t)sp * m * rows * 4 : 0;
}

extern "C" int sqx_int4_gemm(const uint8_t* wt, const void* st, const void* zt, int param_dtype, const void* x,
                             int act_dtype, void* y, const void* bias, int64_t m, int64_t rows, int64_t cols,
                             int64_t group, void* ws, int64_t ws_bytes, sqx_stream_t stream) {
  if (int rc = dq_check("sqx_int4_gemm", x, wt, y, m, rows, cols)) return rc;
  SQX_REQUIRE(group == 32 || group == 64 || group == 128, SQX_E_ARG,
              "sqx_int4_gemm: group %lld not one of 32, 64, 128", (long long)group);
  SQX_REQUIRE(cols % group == 0, SQX_E_ARG, "sqx_int4_gemm: cols %lld not a multiple of group %lld", (long long)cols,
              (long long)group);
  SQX_REQUIRE(param_dtype == SQX_DTYPE_F32 || param_dtype == SQX_DTYPE_BF16, SQX_E_ARG,
              "sqx_int4_gemm: param_dtype must be F32 or BF16");
  SQX_REQUIRE(act_dtype == SQX_DTYPE_BF16 || act_dtype == SQX_DTYPE_F16, SQX_E_ARG,
              "sqx_int4_gemm: activations must be BF16 or F16");
  if (m == 0) return SQX_OK;
  SQX_REQUIRE(st, SQX_E_ARG, "sqx_int4_gemm: null scales");
  const bool asym = zt != nullptr, pbf = param_dtype == SQX_DTYPE_BF16;
  const int KB = (int)ceil_div(cols, 128);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* b16 = static_cast<const uint16_t*>(bias);
  hipStream_t s = as_stream(stream);
  hipError_t e;
#define SQX_DQG(ACT, AS, PB, G, YK) \
  e = launch_dq<ACT, kDqInt4, AS, PB, G, YK>(xp, wt, st, zt, nullptr, y, b16, (int)m, (int)rows, (int)cols, KB, \
                                             static_cast<float*>(ws), ws_bytes, s)
#define SQX_DQ(ACT, AS, PB, YK)                               \
  do {                                                        \
    if (group == 32) SQX_DQG(ACT, AS, PB, 32, YK);            \
    else if (group == 64) SQX_DQG(ACT, AS, PB, 64, YK);       \
    else SQX_DQG(ACT, AS, PB, 128, YK);                       \
  } while (0)
  if (act_dtype == SQX_DTYPE_BF16) {
    if (asym) { if (pbf) SQX_DQ(ActBF16, true, true, 0); else SQX_DQ(ActBF16, true, false, 0); }
    else { if (pbf) SQX_DQ(ActBF16, false, true, 0); else SQX_DQ(ActBF16, false, false, 0); }
  } else {
    if (asym) { if (pbf) SQX_DQ(ActF16, true, true, 1); else SQX_DQ(ActF16, true, false, 1); }
    else { if (pbf) SQX_DQ(ActF16, false, true, 1); else SQX_DQ(ActF16, false, false, 1); }
  }
#undef SQX_DQ
#undef SQX_DQG
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "sqx_int4_gemm: launch failed: %s", hipGetErrorString(e));
  return SQX_OK;
}

extern "C" int sqx_fp4_gemm(const uint8_t* wt, const uint8_t* st, int fmt, const float* s_global, const void* x,
                            int act_dtype, void* y, int y_dtype, const void* bias, int64_t m, int64_t rows, int64_t cols,
                            void* ws, int64_t ws_bytes, sqx_stream_t stream) {
  if (int rc = dq_check("sqx_fp4_gemm", x, wt, y, m, rows, cols)) return rc;
  SQX_REQUIRE(fmt == SQX_FP4_MX || fmt == SQX_FP4_NV, SQX_E_ARG, "sqx_fp4_gemm: bad fmt %d", fmt);
  SQX_REQUIRE(act_dtype == SQX_DTYPE_BF16 || act_dtype == SQX_DTYPE_F16, SQX_E_ARG,
              "sqx_fp4_gemm: activations must be BF16 or F16");
  SQX_REQUIRE(y_dtype == act_dtype || y_dtype == SQX_DTYPE_F32, SQX_E_ARG,
              "sqx_fp4_gemm: y_dtype must be the activation dtype or F32");
  SQX_REQUIRE(bias == nullptr || y_dtype == act_dtype, SQX_E_ARG, "sqx_fp4_gemm: bias needs y in act_dtype");
  if (m == 0) return SQX_OK;
  SQX_REQUIRE(st && (fmt == SQX_FP4_MX || s_global), SQX_E_ARG, "sqx_fp4_gemm: null pointer");
  const int KB = (int)ceil_div(cols, 128);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* b16 = static_cast<const uint16_t*>(bias);
  hipStream_t s = as_stream(stream);
  const bool yf = y_dtype == SQX_DTYPE_F32;
  hipError_t e;
#define SQX_DQ(ACT, F, YK) \
  e = launch_dq<ACT, F, false, false, 128, YK>(xp, wt, st, nullptr, s_global, y, b16, (int)m, (int)rows, (int)cols, KB, \
                                              static_cast<float*>(ws), ws_bytes, s)
  if (act_dtype == SQX_DTYPE_BF16) {
    if (fmt == SQX_FP4_MX) { if (yf) SQX_DQ(ActBF16, kDqMx, 2); else SQX_DQ(ActBF16, kDqMx, 0); }
    else { if (yf) SQX_DQ(ActBF16, kDqNv, 2); else SQX_DQ(ActBF16, kDqNv, 0); }
  } else {
    if (fmt == SQX_FP4_MX) { if (yf) SQX_DQ(ActF16, kDqMx, 2); else SQX_DQ(ActF16, kDqMx, 1); }
    else { if (yf) SQX_DQ(ActF16, kDqNv, 2); else SQX_DQ(ActF16, kDqNv, 1); }
  }
#undef SQX_DQ
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "sqx_fp4_gemm: launch failed: %s", hipGetErrorString(e));
  return SQX_OK;
}

// ----------------------------------------------------------------------------------------------
// fp32 activations for the int4 linear (w4a16_linear / awq_linear with x in fp32): x (optionally
// divided by a per-column scale in fp32) splits into three bf16 rows a = bf16(v), b = bf16(v - a),
// c = bf16(v - a - b), whose sum is v exactly for every normal fp32 v (8 significant bits each); the
// 3m rows go through the decode GEMV with fp32 outputs (exact code products, the fp32 group scale
// applied to each group's partial sum, 64 rows per pass over the weight), and
// y = (y_a + y_b) + y_c (+ bias) in fp32. The prefill GEMM is not used here: it decodes each weight
// to bf16, which the fp32 reference does not.
// ----------------------------------------------------------------------------------------------
namespace {
__global__ __launch_bounds__(256) void split3_cols_kernel(const float* __restrict__ x, const float* __restrict__ cs,
                                                          int64_t n, int64_t cols, uint16_t* __restrict__ parts) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = cs ? x[i] / cs[i % cols] : x[i];
  const uint16_t a = f32_to_bf16_bits(v);
  const float r1 = v - bf16_bits_to_f32(a);  // exact (Sterbenz)
  const uint16_t b = f32_to_bf16_bits(r1);
  parts[i] = a;
  parts[n + i] = b;
  parts[2 * n + i] = f32_to_bf16_bits(r1 - bf16_bits_to_f32(b));
}

__global__ __launch_bounds__(256) void sum3_rows_bias_kernel(const float* __restrict__ y3, int64_t n, int64_t cols,
                                                             const float* __restrict__ bias, float* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float v = (y3[i] + y3[n + i]) + y3[2 * n + i];
  if (bias) v += bias[i % cols];
  y[i] = v;
}

constexpr int64_t kAlign = 256;
int64_t align_up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
}  // namespace

// workspace of sqx_int4_linear_f32: the three bf16 parts of x [3m, cols], then y3 [3m, rows] fp32
extern "C" int64_t sqx_int4_linear_f32_workspace_bytes(int64_t m, int64_t rows, int64_t cols) {
  if (m <= 0 || rows <= 0 || cols <= 0) return 0;
  return align_up(3 * m * cols * 2) + align_up(3 * m * rows * 4);
}

extern "C" int sqx_int4_linear_f32(const uint8_t* wt, const void* st, const void* zt, int param_dtype, const float* x,
                                   const float* col_scale, float* y, const float* bias, int64_t m, int64_t rows,
                                   int64_t cols, int64_t group, void* ws, int64_t ws_bytes, sqx_stream_t stream) {
  const char* fn = "sqx_int4_linear_f32";
  SQX_REQUIRE(m >= 0 && rows > 0 && cols > 0, SQX_E_ARG, "%s: bad shape m=%lld rows=%lld cols=%lld", fn, (long long)m,
              (long long)rows, (long long)cols);
  SQX_REQUIRE(group == 32 || group == 64 || group == 128, SQX_E_ARG, "%s: group_size %lld unsupported (32, 64 or 128)",
              fn, (long long)group);
  SQX_REQUIRE(cols % group == 0, SQX_E_ARG, "in_features=%lld not divisible by group_size=%lld", (long long)cols,
              (long long)group);
  SQX_REQUIRE(param_dtype == SQX_DTYPE_F32 || param_dtype == SQX_DTYPE_BF16, SQX_E_ARG,
              "%s: param_dtype must be F32 or BF16", fn);
  SQX_REQUIRE(rows < ((int64_t)1 << 31) && 64 * cols * 2 < ((int64_t)1 << 31) &&
                  ceil_div(cols, 128) * 1024 < ((int64_t)1 << 31),
              SQX_E_ARG, "%s: shape too large for 32-bit buffer offsets", fn);
  if (m == 0) return SQX_OK;
  SQX_REQUIRE(wt && st && x && y && ws, SQX_E_ARG, "%s: null pointer", fn);
  const int64_t need = sqx_int4_linear_f32_workspace_bytes(m, rows, cols);
  SQX_REQUIRE(ws_bytes >= need, SQX_E_SPACE, "%s: workspace of %lld bytes, needs %lld", fn, (long long)ws_bytes,
              (long long)need);
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(wt) % 16 == 0 && reinterpret_cast<uintptr_t>(ws) % kAlign == 0, SQX_E_ARG,
              "%s: wt must be 16-byte and ws 256-byte aligned", fn);
  hipStream_t s = as_stream(stream);
  char* wsb = static_cast<char*>(ws);
  uint16_t* parts = reinterpret_cast<uint16_t*>(wsb);
  float* y3 = reinterpret_cast<float*>(wsb + align_up(3 * m * cols * 2));
  const int64_t nx = m * cols, ny = m * rows;
  hipLaunchKernelGGL(split3_cols_kernel, dim3((unsigned)ceil_div(nx, 256)), dim3(256), 0, s, x, col_scale, nx, cols,
                     parts);
  SQX_LAUNCH_CHECK(fn);
  const hipError_t e =
      int4_gemv_f32out(wt, st, zt, param_dtype == SQX_DTYPE_BF16, parts, y3, 3 * m, rows, cols, (int)group, s);
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: launch failed: %s", fn, hipGetErrorString(e));
  hipLaunchKernelGGL(sum3_rows_bias_kernel, dim3((unsigned)ceil_div(ny, 256)), dim3(256), 0, s, y3, ny, rows, bias, y);
  SQX_LAUNCH_CHECK(fn);
  return SQX_OK;
}
