// The decode-regime linear for 9..64 activation rows (gfx950): y[m, n] = sum_k x[m, k] * W[n, k]
// over the same tiled weights as the GEMV (1 KiB blocks of 16 weight rows; see sqx_gemv.h).
//
// Why a second kernel. The GEMV gives each 16-row tile its own workgroup, so every tile re-reads
// the activation fragments of all M rows: at M = 64 that is 16 KiB of activations per 1 KiB weight
// block, and the offset of the unsigned codes is removed by a second MFMA per tile. Both grow with
// M, and at M = 64 the GEMV runs at a tenth of the weight stream's rate. Here:
//  * a workgroup owns R consecutive row tiles; each wave loads a k-block's activation fragments
//    once and applies them to all R tiles from registers (R times fewer activation loads);
//  * the code offset is removed through the per-row activation sums of each group, one MFMA
//    against a constant all-ones operand per k-block and chunk, shared by the R tiles: the group's
//    MFMA chain starts from C = -offset * sum(x) instead of zero, so a tile costs only its own
//    MFMAs plus one FMA per output element for the group scale;
//  * the waves of a workgroup split the k-blocks (partials summed through LDS in wave order) and,
//    optionally, S workgroups split K further: each writes fp32 partials [S][M][N] to the caller's
//    workspace and skinny_reduce_kernel adds them in split order. Deterministic for a given
//    (R, waves, S).
// The kernels' split_out argument: 0 writes bf16 y [M][N]; 1 the fp32 partials; 2 (no K split, N a
// multiple of 16) SwiGLU pairs for a fused gate|up weight whose rows alternate in groups of 8: each
// output rounded to bf16, then y [M][N / 2] = bf16(silu(g) * u) per pair, as the SiLU kernel does.
//
// Weight policies opt in with these members (WInt4 provides them):
//   W::ctx_tiles(args, t0, nt, KB, lane)   buffer resources covering tiles t0 .. t0+nt-1 (loads of
//                                          tiles past the last one return zero)
//   W::load(ctx, r*KB + kb, w, p)          block kb of tile r (tiles are contiguous in HBM)
//   W::NG, W::MPG                          groups per block, MFMA steps (32 columns) per group
//   W::bfrag<A>(w, i)                      B fragment of step i: activation-type pairs of (offset + code)
//   W::kConstOffset, W::const_offset<A>()  the offset when it is the same for every group
//   W::offset<A>(p, g)                     magic + zero point of group g (lane's weight row)
//   W::scale(p, g)                         group scale (lane's weight row)
// A policy whose codes decode to the weight values themselves (no offset, no group scale) declares
// kPlainBlocks = true instead: its MFMAs chain straight into the output sums. A per-token factor
// (kRowScale, row_scale) is applied in the epilogue as in the GEMV, and with K splits by the reduce,
// which takes the factors from W::row_scales(args) [m] and W::out_scales(args) [n].
#pragma once

#include "sqx_gemv.h"

namespace sqx {

static constexpr int kSkinnyMaxWaves = 8;

template <class W, class = void>
struct plain_blocks : std::false_type {};
template <class W>
struct plain_blocks<W, std::void_t<decltype(W::kPlainBlocks)>> : std::integral_constant<bool, W::kPlainBlocks> {};
// KiB of weights in flight per compute wave of the LDS-staged variant (a ring of this many k-blocks
// over the wave's R tiles)
#ifndef SQX_SKINNY_RING_KIB
#define SQX_SKINNY_RING_KIB 8
#endif
template <int R>
constexpr int skinny_ring() { return SQX_SKINNY_RING_KIB / R > 1 ? SQX_SKINNY_RING_KIB / R : 1; }
// LDS stages of activations in the LDS-staged variant. A wave's loads complete in issue order, so
// the wait for the copy of block s also waits for every weight load issued before it: with the
// copy issued NS-1 steps ahead, a step can take no less than the loaded memory latency / NS. More
// stages (up to the ring depth, within 160 KiB per workgroup) keep more weight bytes in flight.
// (The count of loads a wait may leave outstanding, (NS-1) x R x LOADS + (NS-2) x MCH, stays below
// vmcnt's 64.)
constexpr int kSkinnyLdsBytes = 160 * 1024;
#ifndef SQX_SKINNY_MAX_STAGES
#define SQX_SKINNY_MAX_STAGES 4
#endif
template <int MCH, int R, int D, int KG, int LOADS>
constexpr int skinny_stages() {
  const int fit = kSkinnyLdsBytes / (KG * MCH * 16 * 256);
  int ns = fit < D ? fit : D;
  ns = ns < 3 ? 3 : (ns > SQX_SKINNY_MAX_STAGES ? SQX_SKINNY_MAX_STAGES : ns);
  while (ns > 3 && (ns - 1) * R * LOADS + (ns - 2) * MCH >= 64) --ns;
  return ns;
}

// Waves per workgroup a variant may use: variants that need more than the 256 registers a wave
// gets at two waves per SIMD (4 chunks x 4 tiles; 8 chunk-tiles with several groups per block or
// with per-group zero points) run one wave per SIMD.
constexpr int skinny_max_waves(int mch, int r, int ng, bool const_offset) {
  return (mch * r >= 16 || ((ng >= 2 || !const_offset) && mch * r >= 8)) ? 4 : kSkinnyMaxWaves;
}

// The MFMAs of one k-block for MCH 16-row activation chunks and R weight tiles, ordered so that the
// matrix unit always has independent work: the activation sums of every chunk (independent chains,
// interleaved), then the main chains of every (tile, chunk) pair, interleaved step by step. Each
// group's chain starts from C = -offset * sum(x); the group scale is one FMA per output element.
template <class A, class W, int MCH, int R>
__device__ __forceinline__ void skinny_block(const u32x4_t (&xv)[MCH][W::STEPS], const u32x4_t (&b)[R][W::STEPS],
                                             const typename W::P (&pc)[R], const u32x4_t& onev,
                                             f32x4_t (&yacc)[R][MCH]) {
  constexpr int NG = W::NG;
  constexpr int MPG = W::MPG;
  if constexpr (plain_blocks<W>::value) {
#pragma unroll
    for (int i = 0; i < W::STEPS; ++i)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < MCH; ++c) yacc[r][c] = A::mfma(xv[c][i], b[r][i], yacc[r][c]);
    return;
  }
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    f32x4_t xs[MCH];
#pragma unroll
    for (int c = 0; c < MCH; ++c) xs[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = g * MPG; i < (g + 1) * MPG; ++i)
#pragma unroll
      for (int c = 0; c < MCH; ++c) xs[c] = A::mfma(xv[c][i], onev, xs[c]);
    f32x4_t acc[R][MCH];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float o = W::kConstOffset ? -W::template const_offset<A>() : -W::template offset<A>(pc[r], g);
#pragma unroll
      for (int c = 0; c < MCH; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[r][c][j] = o * xs[c][j];
    }
#pragma unroll
    for (int i = g * MPG; i < (g + 1) * MPG; ++i)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < MCH; ++c) acc[r][c] = A::mfma(xv[c][i], b[r][i], acc[r][c]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float sc = W::scale(pc[r], g);
#pragma unroll
      for (int c = 0; c < MCH; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) yacc[r][c][j] = fmaf(sc, acc[r][c][j], yacc[r][c][j]);
    }
  }
}

template <class A, class W, int MCH, int R>
__global__ __launch_bounds__((64 * skinny_max_waves(MCH, R, W::NG, W::kConstOffset))) void skinny_kernel(const typename W::Args wa,
                                                                       const uint16_t* __restrict__ x,
                                                                       void* __restrict__ out,
                                                                       const uint16_t* __restrict__ bias, int M,
                                                                       int N, int K, int KB, int T, int kbs, int kbw,
                                                                       int split_out) {
  extern __shared__ f32x4_t red[];  // [NW][MCH][64]
  constexpr int KBLK = W::KBLK;
  constexpr int STEPS = W::STEPS;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int t0 = blockIdx.x * R;
  const int nt = min(R, T - t0);
  const int ks0 = blockIdx.y * kbs;
  const int ks1 = min(KB, ks0 + kbs);
  const int kb0 = ks0 + wave * kbw;
  const int kb1 = min(ks1, kb0 + kbw);
  const int nl = lane & 15;
  const int jg = lane >> 4;

  const typename W::Ctx wc = W::ctx_tiles(wa, t0, nt, KB, lane);
  const rsrc_t xr = make_rsrc(x, (uint32_t)M * (uint32_t)K * 2u);  // rows >= M read as zero
  uint32_t xvo[MCH];
#pragma unroll
  for (int c = 0; c < MCH; ++c) xvo[c] = ((uint32_t)(c * 16 + nl) * (uint32_t)K) * 2u;
  const uint32_t ones = A::pair_from_f32(1.0f);
  const u32x4_t onev = u32x4_t{ones, ones, ones, ones};

  f32x4_t yacc[R][MCH];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MCH; ++c) yacc[r][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // The next block's weights and activations are loaded while this block's are used.
  u32x4_t xv[MCH][STEPS];
  u32x4_t w[R];
  typename W::P p[R];
  auto load_x = [&](int kb, u32x4_t (&xo)[MCH][STEPS]) {
#pragma unroll
    for (int c = 0; c < MCH; ++c)
#pragma unroll
      for (int i = 0; i < STEPS; ++i) xo[c][i] = bload128(xr, xvo[c] + 2u * W::xk(i, jg), (uint32_t)(kb * KBLK) * 2u);
  };
  // Each wave walks its k-blocks starting at a rotation set by its workgroup's place on its XCD
  // (workgroup b runs on XCD b % 8): otherwise every workgroup's wave w reads the same activation
  // columns at the same moment, and those rows, a row stride apart, crowd into the same L2 channels.
  const int nblk = kb1 - kb0;
  const int rot = nblk > 0 ? static_cast<int>((blockIdx.x >> 3) % static_cast<unsigned>(nblk)) : 0;
  auto kb_at = [&](int it) {
    int j = it + rot;
    if (j >= nblk) j -= nblk;
    return kb0 + j;
  };
  if (nblk > 0) {
    const int kf = kb_at(0);
#pragma unroll
    for (int r = 0; r < R; ++r) W::load(wc, r * KB + kf, w[r], p[r]);
    load_x(kf, xv);
  }
  for (int it = 0; it < nblk; ++it) {
    const int kb = kb_at(it);
    const bool more = it + 1 < nblk;  // wave-uniform
    const int kn = more ? kb_at(it + 1) : kb;
    u32x4_t b[R][STEPS];
    typename W::P pc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int i = 0; i < STEPS; ++i) b[r][i] = W::template bfrag<A>(w[r], i);
      pc[r] = p[r];
    }
    u32x4_t xn[MCH][STEPS];
    if (more) {
#pragma unroll
      for (int r = 0; r < R; ++r) W::load(wc, r * KB + kn, w[r], p[r]);
      load_x(kn, xn);
    }
    if (kb == KB - 1 && KB * KBLK != K) {  // activations at or beyond K must not enter the sums
#pragma unroll
      for (int i = 0; i < STEPS; ++i) {
        if (kb * KBLK + W::xk(i, jg) >= K) {
#pragma unroll
          for (int c = 0; c < MCH; ++c) xv[c][i] = u32x4_t{0u, 0u, 0u, 0u};
        }
      }
    }
    skinny_block<A, W, MCH, R>(xv, b, pc, onev, yacc);
    if (more) {
#pragma unroll
      for (int c = 0; c < MCH; ++c)
#pragma unroll
        for (int i = 0; i < STEPS; ++i) xv[c][i] = xn[c][i];
    }
  }

  // Per tile: sum the NW partials in wave order. Float j of a wave's block is (chunk c, lane l, row r).
  constexpr int kOut = MCH * 64 * 4;
  const float* rf = reinterpret_cast<const float*>(red);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r > 0) __syncthreads();  // the previous tile's sums are read
#pragma unroll
    for (int c = 0; c < MCH; ++c) red[(wave * MCH + c) * 64 + lane] = yacc[r][c];
    __syncthreads();
    if (r < nt) {
      for (int j = threadIdx.x; j < kOut; j += blockDim.x) {
        float v = 0.0f;
        for (int ww = 0; ww < nw; ++ww) v += rf[ww * kOut + j];
        const int c = j >> 8;
        const int l = (j >> 2) & 63;
        const int m = c * 16 + 4 * (l >> 4) + (j & 3);
        const int n = (t0 + r) * 16 + (l & 15);
        if (split_out == 2) {  // SwiGLU pairs: output n's up row n + 8 is j ^ 32, in this wave and iteration
          const bool ok = m < M && n < N;
          float q = 0.0f;
          if (ok) {
            v *= W::out_scale(wa, n);
            if (bias) v += A::to_f32(bias[n]);
            q = A::to_f32(A::from_f32(v));
          }
          const float u = __shfl_xor(q, 32, 64);
          if (ok && (l & 15) < 8)
            static_cast<uint16_t*>(out)[(int64_t)m * (N / 2) + (t0 + r) * 8 + (l & 15)] =
                static_cast<uint16_t>(A::pack_rne(silu_f32(q) * u, 0.0f));
          continue;
        }
        if (m < M && n < N) {
          if (split_out) {
            static_cast<float*>(out)[((int64_t)blockIdx.y * M + m) * N + n] = v;
          } else {
            if constexpr (has_row_scale<W>::value)
              v = v * W::row_scale(wa, m) * W::out_scale(wa, n);
            else
              v *= W::out_scale(wa, n);
            if (bias) v += A::to_f32(bias[n]);
            static_cast<uint16_t*>(out)[(int64_t)m * N + n] = A::from_f32(v);
          }
        }
      }
    }
  }
}

// Variant with the activations staged through LDS. A workgroup owns 4R row tiles and a range of n
// k-blocks. It has 4 x KG compute waves: wave (kg, tg) owns tiles tg*R .. tg*R+R-1 of the group and
// the kg-th of KG equal parts of the k-range, so KG = 2 puts two compute waves on each SIMD without
// more workgroups; at the end the second k-group's partial sums are added to the first's through
// LDS in a fixed order.
//  * Each k-group stages its k-blocks of activations (all M rows, 256 bytes a row) in its own ring
//    of NS LDS stages, with buffer loads that write LDS directly, 16 bytes a lane in whole row
//    segments; every wave of the group copies MCH of the block's 1 KiB pieces. Slot (row r, chunk
//    q) holds chunk q ^ (r & 15) of the row, so the 16 rows a fragment read touches fall in 16
//    different bank groups. Rows at or beyond M and columns at or beyond K are copied as zeros.
//  * Every wave keeps the weights of the next D k-blocks in flight in a register ring.
//  * Every step issues the same loads in the same order (copy of block s+A with A = NS-1, then the
//    ring refill of block s+D; past the k-group's last block, zero-size buffer resources and
//    out-of-range offsets keep the count without touching memory), so at step s the copy of block s
//    is complete once at most A x (ring loads) + (A-1) x MCH loads are outstanding. After that wait
//    the barrier B_s tells every wave that block s is in LDS and that the slot of block s-1 may be
//    refilled.
template <class A, class W, int MCH, int R, int D, int KG>
__global__ __launch_bounds__(256 * KG) void skinny_lds_kernel(const typename W::Args wa, const uint16_t* __restrict__ x,
                                                              void* __restrict__ out, const uint16_t* __restrict__ bias,
                                                              int M, int N, int K, int KB, int T, int kbs,
                                                              int split_out) {
  constexpr int KBLK = W::KBLK;
  static_assert(KBLK == 128, "an activation row of a block is 16 chunks of 16 bytes");
  static_assert(D >= 2, "the issue order assumes a ring of at least two blocks");
  constexpr int STEPS = W::STEPS;
  constexpr int NG = W::NG;
  constexpr int kStage = MCH * 16 * 256;
  constexpr int NS = skinny_stages<MCH, R, D, KG, W::kLoads>();
  constexpr int AH = NS - 1;  // steps a copy is issued ahead of its use
  static_assert(AH <= D, "the prologue issues the first copies among the first ring loads");
  constexpr int kWaitN = AH * R * W::kLoads + (AH - 1) * MCH;  // loads issued after a block's copy by its step
  static_assert(kWaitN < 64, "vmcnt is 6 bits");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_skinny[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tg = wave & 3;
  const int kg = wave >> 2;
  const int ks0 = blockIdx.y * kbs;
  const int n = min(KB, ks0 + kbs) - ks0;  // k-blocks of this split
  const int nh = (n + KG - 1) / KG;        // steps every wave walks
  const int k0 = ks0 + kg * nh;            // the k-group's first block
  const int nk = max(0, min(nh, n - kg * nh));  // its real blocks; later steps load zeros
  // Step s reads block k0 + s: every workgroup walks its tiles from the k-group's first block (a
  // start rotated per workgroup measured about 10 % slower).
  auto kb_of = [&](int s) { return k0 + s; };
  uint8_t* ring = smem_skinny + kg * NS * kStage;
  const rsrc_t xr = make_rsrc(x, (uint32_t)M * (uint32_t)K * 2u);
  const rsrc_t xnull = make_rsrc(x, 0u);  // zero-size: copies of steps past the range write zeros
  // Per-lane offsets of the copies within a k-block, fixed for the whole walk (the block's column
  // offset goes in the scalar offset). Rows at or beyond M copy row M-1: they only feed output rows
  // that are never stored. Keeping the per-step copies free of vector arithmetic matters: a
  // temporary there takes a register of the weight ring, and the compiler then drains every
  // outstanding load before writing it, once per unrolled round of steps. (A vector, not an array:
  // hipcc drops the host stub of a kernel whose lambda indexes a captured array in this builtin.)
  static_assert(MCH <= 4, "one offset per chunk in a 4-vector");
  u32x4_t xoff = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
  for (int q = 0; q < MCH; ++q) {
    const int r = 4 * (tg + 4 * q) + (lane >> 4);
    xoff[q] = ((uint32_t)min(r, M - 1) * (uint32_t)K + 8u * (uint32_t)((lane & 15) ^ (r & 15))) * 2u;
  }
  auto issue_x = [&](int s, int slot) {  // this wave's MCH copies of step s
    const bool live = s < nk;
    const int kb = live ? kb_of(s) : 0;
    uint8_t* base = ring + slot * kStage;
    if (live && (kb + 1) * KBLK > K) {  // the partial last block: columns at or beyond K copy zeros
#pragma unroll
      for (int q = 0; q < MCH; ++q) {
        const int j = tg + 4 * q;  // rows 4j .. 4j+3
        const int r = 4 * j + (lane >> 4);
        const int col = kb * KBLK + 8 * ((lane & 15) ^ (r & 15));
        const bool ok = (r < M) & (col < K);  // a select, not a branch
        const uint32_t off = ok ? ((uint32_t)r * (uint32_t)K + (uint32_t)col) * 2u : 0xFFFFFFF0u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(base + j * 1024), 16, off, 0, 0, 0);
      }
    } else {
      const rsrc_t& rs = live ? xr : xnull;
      const uint32_t so = (uint32_t)(kb * KBLK) * 2u;
#pragma unroll
      for (int q = 0; q < MCH; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(base + (tg + 4 * q) * 1024), 16, xoff[q], so, 0, 0);
    }
  };

  // the wave's first tile and tile count, pinned to scalar registers (they size buffer resources)
  const int tw0 = __builtin_amdgcn_readfirstlane((blockIdx.x * 4 + tg) * R);
  const int nt = __builtin_amdgcn_readfirstlane(max(0, min(R, T - tw0)));
  const int nl = lane & 15;
  const int jg = lane >> 4;
  const typename W::Ctx wc = W::ctx_tiles(wa, nt > 0 ? tw0 : 0, nt, KB, lane);
  const typename W::Ctx wnull = W::ctx_tiles(wa, 0, 0, KB, lane);  // zero-size: its loads return zero
  const uint32_t ones = A::pair_from_f32(1.0f);
  const u32x4_t onev = u32x4_t{ones, ones, ones, ones};
  // With one offset for every group, the sum chain multiplies by -(magic + 8) directly and its result
  // seeds the main chains; per-group zero points scale the plain sum per tile.
  const uint32_t sumc = W::kConstOffset ? A::pair_from_f32(-W::template const_offset<A>()) : ones;
  const u32x4_t sumv = u32x4_t{sumc, sumc, sumc, sumc};

  f32x4_t yacc[R][MCH];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int c = 0; c < MCH; ++c) yacc[r][c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  u32x4_t wring[D][R];
  typename W::P pring[D][R];
  auto load_step = [&](int s, int slot) {  // exactly R * W::kLoads loads
    const bool live = s < nk;
    const typename W::Ctx& c = live ? wc : wnull;
    const int kb = live ? kb_of(s) : 0;
#pragma unroll
    for (int r = 0; r < R; ++r) W::load(c, r * KB + kb, wring[slot][r], pring[slot][r]);
  };
  // prologue in the steady state's issue order: ring blocks 0 .. D-A-1 first (older than every
  // copy), then copy j and ring D-A+j for j < A
#pragma unroll
  for (int d = 0; d < D - AH; ++d) load_step(d, d);
#pragma unroll
  for (int j = 0; j < AH; ++j) {
    __builtin_amdgcn_sched_barrier(0);
    issue_x(j, j);
    __builtin_amdgcn_sched_barrier(0);
    load_step(D - AH + j, D - AH + j);
  }

  // Software pipeline (one group per block): the weights of step s+1 are decoded while the MFMAs
  // of step s run, so the decode's VALU work issues between independent MFMAs. Blocks with several
  // groups decode each step's weights at its start instead. Ring slot t % D holds step t; it is
  // refilled with step t+D at the start of step t (after its decode).
  constexpr bool PIPE = NG == 1;
  u32x4_t bcur[R][STEPS];
  typename W::P pcur[R];
  if (PIPE) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int i = 0; i < STEPS; ++i) bcur[r][i] = W::template bfrag<A>(wring[0][r], i);
      pcur[r] = pring[0][r];
    }
  }

  for (int s0 = 0; s0 < nh; s0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int s = s0 + d;
      if (s >= nh) break;  // workgroup-uniform: every wave meets nh barriers
      const int dn = (d + 1) % D;  // ring slot of step s+1 (a constant once the loop is unrolled)
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt<kWaitN>();
      lds_barrier();  // B_s: block s is in this k-group's ring
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (!PIPE) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
          for (int i = 0; i < STEPS; ++i) bcur[r][i] = W::template bfrag<A>(wring[d][r], i);
          pcur[r] = pring[d][r];
        }
      }
      issue_x(s + AH, (s + AH) % NS);
      __builtin_amdgcn_sched_barrier(0);
      load_step(s + D, d);
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* st = ring + (s % NS) * kStage;
      u32x4_t xv[MCH][STEPS];
#pragma unroll
      for (int c = 0; c < MCH; ++c) {
        const int row = c * 16 + nl;
#pragma unroll
        for (int i = 0; i < STEPS; ++i) {
          const int q = W::xk(i, jg) >> 3;
          xv[c][i] = *reinterpret_cast<const u32x4_t*>(st + row * 256 + ((q ^ (row & 15)) << 4));
        }
      }
      if constexpr (!PIPE) {
        skinny_block<A, W, MCH, R>(xv, bcur, pcur, onev, yacc);
      } else {
        u32x4_t bnext[R][STEPS];
        typename W::P pnext[R];
        f32x4_t xs[MCH];
#pragma unroll
        for (int c = 0; c < MCH; ++c) xs[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < STEPS; ++i)
#pragma unroll
          for (int c = 0; c < MCH; ++c) xs[c] = A::mfma(xv[c][i], sumv, xs[c]);
        f32x4_t acc[R][MCH];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if constexpr (W::kConstOffset) {
#pragma unroll
            for (int c = 0; c < MCH; ++c) acc[r][c] = xs[c];
          } else {
            const float o = -W::template offset<A>(pcur[r], 0);
#pragma unroll
            for (int c = 0; c < MCH; ++c)
#pragma unroll
              for (int j = 0; j < 4; ++j) acc[r][c][j] = o * xs[c][j];
          }
        }
#pragma unroll
        for (int i = 0; i < STEPS; ++i)
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int c = 0; c < MCH; ++c) acc[r][c] = A::mfma(xv[c][i], bcur[r][i], acc[r][c]);
        // decode step s+1 while the chains run (after the last step the result goes unused)
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
          for (int i = 0; i < STEPS; ++i) bnext[r][i] = W::template bfrag<A>(wring[dn][r], i);
          pnext[r] = pring[dn][r];
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float sc = W::scale(pcur[r], 0);
#pragma unroll
          for (int c = 0; c < MCH; ++c)
#pragma unroll
            for (int j = 0; j < 4; ++j) yacc[r][c][j] = fmaf(sc, acc[r][c][j], yacc[r][c][j]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
          for (int i = 0; i < STEPS; ++i) bcur[r][i] = bnext[r][i];
          pcur[r] = pnext[r];
        }
      }
    }
  }
  // Every copy has landed (nothing may still write LDS) before the ring is reused or freed.
  wait_vmcnt<0>();

  if constexpr (KG == 2) {  // the second k-group's sums join the first's, in that order
    f32x4_t* red = reinterpret_cast<f32x4_t*>(smem_skinny);
    lds_barrier();  // every wave is done with the rings
    if (kg == 1) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < MCH; ++c) red[((tg * R + r) * MCH + c) * 64 + lane] = yacc[r][c];
    }
    lds_barrier();
    if (kg == 1) return;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int c = 0; c < MCH; ++c) {
        const f32x4_t v = red[((tg * R + r) * MCH + c) * 64 + lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) yacc[r][c][j] += v[j];
      }
  }

  // yacc[r][c][j] is y[c*16 + 4(l >> 4) + j][(tw0 + r)*16 + (l & 15)]
  if (split_out == 2) {  // SwiGLU pairs (N a multiple of 16): output n's up row n + 8 is lane ^ 8
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r >= nt) break;
      const int nn = (tw0 + r) * 16 + nl;
      const float os = W::out_scale(wa, nn);
      const float bv = bias ? A::to_f32(bias[nn]) : 0.0f;
#pragma unroll
      for (int c = 0; c < MCH; ++c) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int m = c * 16 + 4 * jg + j;
          const float q = A::to_f32(A::from_f32(yacc[r][c][j] * os + bv));
          const float u = __shfl_xor(q, 8, 64);
          if (m < M && nl < 8)
            static_cast<uint16_t*>(out)[(int64_t)m * (N / 2) + (tw0 + r) * 8 + nl] =
                static_cast<uint16_t>(A::pack_rne(silu_f32(q) * u, 0.0f));
        }
      }
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r >= nt) break;
    const int nn = (tw0 + r) * 16 + nl;
    if (nn >= N) continue;
    const float os = W::out_scale(wa, nn);
    const float bv = bias ? A::to_f32(bias[nn]) : 0.0f;
#pragma unroll
    for (int c = 0; c < MCH; ++c) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = c * 16 + 4 * jg + j;
        if (m < M) {
          if (split_out) {
            static_cast<float*>(out)[((int64_t)blockIdx.y * M + m) * N + nn] = yacc[r][c][j];
          } else {
            static_cast<uint16_t*>(out)[(int64_t)m * N + nn] = A::from_f32(yacc[r][c][j] * os + bv);
          }
        }
      }
    }
  }
}

// y[m, n] = act(sum over s in order of part[s][m][n] (* rs[m] * cs[n] when rs is given) + bias[n]);
// four outputs per thread.
template <class A>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float* __restrict__ part, int S, int M, int N,
                                                            const uint16_t* __restrict__ bias,
                                                            uint16_t* __restrict__ y, const float* __restrict__ rs,
                                                            const float* __restrict__ cs) {
  const int64_t total = (int64_t)M * N;
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= total) return;
  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(part) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(y) & 7) == 0;
  if (vec && i + 4 <= total) {
    f32x4_t v = *reinterpret_cast<const f32x4_t*>(part + i);
    for (int s = 1; s < S; ++s) {
      const f32x4_t q = *reinterpret_cast<const f32x4_t*>(part + (int64_t)s * total + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] += q[j];
    }
    const int n = static_cast<int>(i % N);
    if (rs) {
      const float r = rs[i / N];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = v[j] * r * cs[n + j];
    }
    uint32_t lo, hi;
    float o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = bias ? v[j] + A::to_f32(bias[n + j]) : v[j];
    lo = static_cast<uint32_t>(A::from_f32(o[0])) | (static_cast<uint32_t>(A::from_f32(o[1])) << 16);
    hi = static_cast<uint32_t>(A::from_f32(o[2])) | (static_cast<uint32_t>(A::from_f32(o[3])) << 16);
    *reinterpret_cast<u32x2v_t*>(y + i) = u32x2v_t{lo, hi};
  } else {
    for (int64_t e = i; e < i + 4 && e < total; ++e) {
      float v = part[e];
      for (int s = 1; s < S; ++s) v += part[(int64_t)s * total + e];
      if (rs) v = v * rs[e / N] * cs[e % N];
      if (bias) v += A::to_f32(bias[e % N]);
      y[e] = A::from_f32(v);
    }
  }
}

// The launch shape the library picks for an m-row linear (m <= 64) over rows x cols weights, from
// measured sweeps of the Llama-3-8B shapes (4096 -> 1024..128256, 14336 -> 4096; m = 2..64):
//   m <= 8        the multi-row GEMV (gemv_rows_kernel) on up to 384 row tiles (512 for m <= 4, and
//                 below 4096 for m = 2) where its k-slices fit; otherwise as below;
//   m <= 16       waves splitting K: 4 tiles x 4 waves above 1024 row tiles, 4 x 8 from 640, 2 x 8 from 384; from 4096
//                 tiles the LDS-staged variant (4 tiles, 4 waves); below 384 tiles the decode GEMV,
//                 except for long K (>= 64 blocks) with a workspace (2 x 8 waves, 2 splits);
//   m <= 32       the LDS-staged variant from 1024 tiles (1 tile per wave, 8 compute waves, or 4 from
//                 4096 tiles); below: long K with a workspace -> LDS-staged, 1 tile, 8 waves, K split
//                 to about 192 workgroups; otherwise waves splitting K, 2 x 8 (2 splits from a
//                 workspace when fewer than 384 tiles);
//   m <= 64       the LDS-staged variant with 8 compute waves (4 from 4096 tiles): 2 tiles per wave
//                 from 1024 tiles; below, 1 tile per wave (2 for long K) and, with a workspace, K split
//                 to about 192 workgroups.
struct SkinnyShape {
  int variant;  // 0: waves splitting K (skinny_kernel); 1: LDS-staged (skinny_lds_kernel); 2: gemv_rows_kernel
  int R;        // row tiles per wave: 1, 2 or 4 (the K-split variant: 2 or 4); variant 2: row groups (0 = default)
  int waves;    // K-split: 1..8 waves per workgroup; LDS-staged: 4 or 8 compute waves (1 or 2 k-groups)
  int S;        // workgroups along K (S > 1 needs a workspace of S*m*rows fp32)
  bool gemv;    // the decode GEMV is the better kernel for this shape
};

inline SkinnyShape skinny_default_shape(int64_t m, int64_t rows, int64_t cols, int kblk, bool have_ws) {
  const int64_t T = ceil_div(rows, 16);
  const int64_t KB = ceil_div(cols, kblk);
  SkinnyShape s{0, 2, 8, 1, false};
  auto split_to_192 = [&]() {  // K splits until about 192 workgroups, >= 4 k-blocks per k-group
    if (!have_ws) return;
    const int64_t wgs = ceil_div(T, 4 * s.R);
    const int64_t kg = s.variant == 1 ? s.waves / 4 : 1;
    while (wgs * s.S < 192 && KB / (2 * s.S * kg) >= 4) s.S *= 2;
  };
  if (m <= 1) {
    s.gemv = true;
  } else if (m <= 8 && kblk == 128 && gemv_rows_fits(m, rows, cols) && (T <= 384 || m <= 4)) {
    // the multi-row GEMV (rotating weights, asymmetric bf16 parameters, M = 2 / 4 / 8 against the
    // kernels below): 4096^2 5.13 / 5.30 / 5.84 -> 4.64 / 4.80 / 5.59 us, 4096->1024 4.33 / 4.65 / 5.18 ->
    // 3.94 / 4.14 / 5.12 us, 14336->4096 13.64 / 12.05 -> 10.29 / 10.45 us (M = 2 / 4), 4096->6144
    // 6.69 / 6.78 / 6.89 -> 5.41 / 5.81 / 6.74 us. Its single-round builds (k-slices of at most four
    // blocks: 60-74 VGPRs at 2..4 rows) also take the large grids at 2..4 rows (the row-tiled kernels
    // these grids took before -> the multi-row GEMV): 4096->28672 (symmetric) at M = 3 / 4 16.1 / 15.9
    // -> 13.5 / 13.8 us, 4096->128256 at M = 2 / 3 / 4 52.3 / 52.0 / 52.8 -> 43.2 / 46.7 / 50.6 us,
    // 4096->14336 (asymmetric) at M = 3 / 4 9.6 / 9.7 -> 9.1 / 8.8 us; at 5..8 rows the row-tiled
    // kernel stays ahead on them.
    s = SkinnyShape{2, 0, 0, 1, false};
  } else if (m <= 16) {
    // (sweep of the LDS-staged shapes at M = 16 / 32 / 48 / 64, symmetric int4, rotating weights:
    // the lm_head 62.6 / 73.7 -> 54.1 / 64.7 us with 2 tiles per wave and 4 waves, gate/up at M = 32
    // 23.0 -> 20.5 us with 2 tiles per wave, down at M = 16 15.2 -> 13.4 us with 4 K splits.)
    // 640..1024 tiles: 4 tiles with 8 waves, at most one workgroup per CU (rotating weights, M = 8 /
    // 16, symmetric and asymmetric int4: 4096->16384 13.4 / 13.8 -> 10.1 / 10.9 us, 4096->14336
    // 10.8 / 12.9 -> 9.7 / 10.5 us, 4096->12288 10.7 / 12.9 -> 9.4 / 10.3 us); beyond 1024 tiles
    // (gate/up 4096->28672 15.1 against 17.5 us at M = 8) and below 640 (4096->8192, 4096->6144)
    // the shapes as before stay ahead.
    if (T >= 4096) s = SkinnyShape{1, 2, 4, 1, false};
    else if (T > 1024) s = SkinnyShape{0, 4, 4, 1, false};
    else if (T >= 640) s = SkinnyShape{0, 4, 8, 1, false};
    else if (T >= 384) s = SkinnyShape{0, 2, 8, 1, false};
    else if (have_ws && KB >= 64) s = m == 16 ? SkinnyShape{1, 1, 8, 4, false} : SkinnyShape{0, 2, 8, 2, false};
    else s.gemv = true;
  } else if (m <= 32) {
    if (T >= 4096) {
      s = SkinnyShape{1, 2, 4, 1, false};
    } else if (T >= 1024) {
      s = SkinnyShape{1, 2, 8, 1, false};
    } else if (have_ws && KB >= 64) {
      s = SkinnyShape{1, 1, 8, 1, false};
      split_to_192();
    } else {
      // 64 tiles and fewer (N <= 1024) split K four ways: 4096->1024 at M = 17 / 32, 7.9 / 9.3 us
      // with two splits against 6.9 / 7.8 us with four
      s = SkinnyShape{0, 2, 8, have_ws ? (T <= 64 && KB >= 32 ? 4 : T < 384 ? 2 : 1) : 1, false};
    }
  } else {
    if (T >= 4096) {
      s = SkinnyShape{1, 2, 4, 1, false};
    } else if (T >= 1024) {
      s = SkinnyShape{1, 2, 8, 1, false};
    } else if (have_ws && T <= 64 && KB >= 32) {
      s = SkinnyShape{0, 2, 8, 4, false};  // 4096->1024 at M = 64: 10.9 -> 10.3 us
    } else {
      s = SkinnyShape{1, KB >= 64 ? 2 : 1, 8, 1, false};
      split_to_192();
    }
  }
  return s;
}

inline int64_t skinny_workspace_bytes(int64_t m, int64_t rows, int S) { return S > 1 ? (int64_t)S * m * rows * 4 : 0; }

// The number of K splits a launch actually makes for S requested over KB k-blocks (no empty split).
inline int skinny_splits(int64_t KB, int S) {
  if (S < 1) S = 1;
  if (S > KB) S = static_cast<int>(KB);
  return static_cast<int>(ceil_div(KB, ceil_div(KB, S)));
}

// The LDS-staged variant: R (1, 2 or 4) tiles per wave, 4 waves per workgroup, S splits along K.
template <class A, class W>
hipError_t skinny_lds_launch(const typename W::Args& wa, const uint16_t* x, uint16_t* y, const uint16_t* bias,
                             int64_t m, int64_t rows, int64_t cols, int R, int KG, int S, float* ws, int64_t ws_bytes,
                             hipStream_t stream, bool reduce = true, bool swiglu = false) {
  constexpr int KBLK = W::KBLK;
  if (m < 1 || m > 64 || (R != 1 && R != 2 && R != 4) || (KG != 1 && KG != 2) || S < 1) return hipErrorInvalidValue;
  // per-group zero points with two or four groups per block hold more parameters per tile: fewer
  // tiles per wave keep the registers within two waves per SIMD
  constexpr int kMaxR = (W::NG == 1 || W::kConstOffset) ? 4 : (W::NG == 2 ? 2 : 1);
  if (R > kMaxR) R = kMaxR;
  const int mch = gemv_mch(m);
  // registers at two waves per SIMD: the pipelined form (one group per block) holds two steps of
  // decoded weights, so 2 or 4 chunks take at most 2 tiles; 4 chunks x 4 tiles never fit
  if (mch >= 2 && R > 2) R = 2;
  constexpr bool kWide4 = W::kConstOffset;  // 4 chunks x 2 tiles fits only without per-tile zero points
  if (mch == 4 && !kWide4) R = 1;
  const int64_t T = ceil_div(rows, 16);
  const int64_t KB = ceil_div(cols, KBLK);
  if (S > KB) S = static_cast<int>(KB);
  const int kbs = static_cast<int>(ceil_div(KB, S));
  S = static_cast<int>(ceil_div(KB, kbs));
  const bool split = S > 1;
  if (split && (ws == nullptr || ws_bytes < skinny_workspace_bytes(m, rows, S))) return hipErrorInvalidValue;
  if (swiglu && (split || rows % 16 != 0)) return hipErrorInvalidValue;  // the pairs need whole tiles, one pass
  const int mode = split ? 1 : (swiglu ? 2 : 0);
  const dim3 grid(static_cast<unsigned>(ceil_div(T, 4 * R)), static_cast<unsigned>(S));
  const size_t lds = static_cast<size_t>(KG) * mch * 16 * 256;  // times the kernel's stage count
  void* o = split ? static_cast<void*>(ws) : static_cast<void*>(y);
  const int M = static_cast<int>(m), N = static_cast<int>(rows), K = static_cast<int>(cols), iKB = static_cast<int>(KB),
            iT = static_cast<int>(T);
#define SQX_SL(MCH_, R_)                                                                                            \
  do {                                                                                                              \
    if (KG == 1)                                                                                                    \
      hipLaunchKernelGGL((skinny_lds_kernel<A, W, MCH_, R_, skinny_ring<R_>(), 1>), grid, dim3(256),              \
                         lds * (skinny_stages<MCH_, R_, skinny_ring<R_>(), 1, W::kLoads>()), stream, wa, x, o,     \
                         bias, M, N, K, iKB, iT, kbs, mode);                                                       \
    else                                                                                                            \
      hipLaunchKernelGGL((skinny_lds_kernel<A, W, MCH_, R_, skinny_ring<R_>(), 2>), grid, dim3(512),              \
                         lds * (skinny_stages<MCH_, R_, skinny_ring<R_>(), 2, W::kLoads>()), stream, wa, x, o,     \
                         bias, M, N, K, iKB, iT, kbs, mode);                                                       \
  } while (0)
  if (mch == 1) {
    if (R == 1) SQX_SL(1, 1);
    else if constexpr (kMaxR >= 2) {
      if (R == 2) SQX_SL(1, 2);
      else if constexpr (kMaxR >= 4) SQX_SL(1, 4);
    }
  } else if (mch == 2) {
    if (R == 1) SQX_SL(2, 1);
    else if constexpr (kMaxR >= 2) SQX_SL(2, 2);
  } else {
    if (R == 1) SQX_SL(4, 1);
    else if constexpr (kMaxR >= 2 && kWide4) SQX_SL(4, 2);
  }
#undef SQX_SL
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !split || !reduce) return e;
  const int64_t quads = ceil_div(m * rows, 4);
  hipLaunchKernelGGL(skinny_reduce_kernel<A>, dim3(static_cast<unsigned>(ceil_div(quads, 256))), dim3(256), 0, stream,
                     ws, S, M, N, bias, y, nullptr, nullptr);
  return hipGetLastError();
}

// Launch the skinny linear for m <= 64 rows. Returns hipErrorInvalidValue when the shape does not
// fit (the entry points check first) or the HIP error of a launch.
template <class A, class W>
// reduce = false with K splits: the fp32 partials [S][m][rows] stay in ws (y is not written); the
// consumer adds them in split order as skinny_reduce_kernel does.
hipError_t skinny_launch(const typename W::Args& wa, const uint16_t* x, uint16_t* y, const uint16_t* bias, int64_t m,
                         int64_t rows, int64_t cols, SkinnyShape sh, float* ws, int64_t ws_bytes, hipStream_t stream,
                         bool reduce = true, bool swiglu = false) {
  constexpr int KBLK = W::KBLK;
  if (sh.variant == 1) {
    if constexpr (KBLK == 128 && !has_row_scale<W>::value)
      return skinny_lds_launch<A, W>(wa, x, y, bias, m, rows, cols, sh.R, sh.waves / 4, sh.S, ws, ws_bytes, stream,
                                     reduce, swiglu);
    else
      return hipErrorInvalidValue;
  }
  if (m < 1 || m > 64 || sh.waves < 1 || sh.waves > kSkinnyMaxWaves || (sh.R != 2 && sh.R != 4) || sh.S < 1)
    return hipErrorInvalidValue;
  const int64_t T = ceil_div(rows, 16);
  const int64_t KB = ceil_div(cols, KBLK);
  int S = sh.S;
  if (S > KB) S = static_cast<int>(KB);
  const int kbs = static_cast<int>(ceil_div(KB, S));
  S = static_cast<int>(ceil_div(KB, kbs));  // no empty splits
  int nw = sh.waves;
  const int mch = gemv_mch(m);
  if (W::NG >= 4 && mch * sh.R >= 16) sh.R = 2;  // four groups per block: 4 x 4 does not fit the registers
  const int nwmax = skinny_max_waves(mch, sh.R, W::NG, W::kConstOffset);
  if (nw > nwmax) nw = nwmax;
  if (nw > kbs) nw = kbs;
  const int kbw = static_cast<int>(ceil_div(kbs, nw));
  nw = static_cast<int>(ceil_div(kbs, kbw));
  const bool split = S > 1;
  if (split && (ws == nullptr || ws_bytes < skinny_workspace_bytes(m, rows, S))) return hipErrorInvalidValue;
  if (swiglu && (split || rows % 16 != 0 || has_row_scale<W>::value)) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(ceil_div(T, sh.R)), static_cast<unsigned>(S));
  const dim3 block(static_cast<unsigned>(64 * nw));
  const size_t lds = static_cast<size_t>(nw) * mch * 64 * sizeof(f32x4_t);
  void* o = split ? static_cast<void*>(ws) : static_cast<void*>(y);
  const int M = static_cast<int>(m), N = static_cast<int>(rows), K = static_cast<int>(cols), iKB = static_cast<int>(KB),
            iT = static_cast<int>(T);
#define SQX_SK(MCH_, R_)                                                                                            \
  hipLaunchKernelGGL((skinny_kernel<A, W, MCH_, R_>), grid, block, lds, stream, wa, x, o, bias, M, N, K, iKB, iT, kbs, \
                     kbw, split ? 1 : (swiglu ? 2 : 0))
  if (mch == 1) {
    if (sh.R == 2) SQX_SK(1, 2); else SQX_SK(1, 4);
  } else if (mch == 2) {
    if (sh.R == 2) SQX_SK(2, 2); else SQX_SK(2, 4);
  } else {
    if constexpr (W::NG >= 4) SQX_SK(4, 2);
    else if (sh.R == 2) SQX_SK(4, 2);
    else SQX_SK(4, 4);
  }
#undef SQX_SK
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !split || !reduce) return e;
  const int64_t quads = ceil_div(m * rows, 4);
  const float* rs = nullptr;
  const float* cs = nullptr;
  if constexpr (has_row_scale<W>::value) {
    rs = W::row_scales(wa);
    cs = W::out_scales(wa);
  }
  hipLaunchKernelGGL(skinny_reduce_kernel<A>, dim3(static_cast<unsigned>(ceil_div(quads, 256))), dim3(256), 0, stream,
                     ws, S, M, N, bias, y, rs, cs);
  return hipGetLastError();
}

}  // namespace sqx
