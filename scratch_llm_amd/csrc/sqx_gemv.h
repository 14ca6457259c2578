// The decode linear shared by the weight formats (gfx950): y[m, n] = sum_k x[m, k] * W[n, k].
//
// Tiled weights: T = ceil(N/16) row tiles x KB = ceil(K/W::KBLK) k-blocks; block (t, kb) is 1 KiB
// at byte (t*KB + kb)*1024 and covers W::KBLK columns (128 for 4-bit codes, 64 for 8-bit), and lane
// L of the consuming wave owns its 16 bytes at 16L. What those bytes mean, and which per-block
// parameters go with them, is the weight format's policy W:
//
//   W::KBLK, W::STEPS              columns per block, MFMA steps (of 32 columns) per block
//   W::Args                        device pointers and scalars of one tiled weight (kernel argument)
//   W::Ctx  W::ctx(args, t, KB, lane)   per-wave buffer resources for tile t
//   W::P                           the parameters of one block, held in registers
//   W::load(ctx, kb, w, p)         buffer loads of block kb: 16 weight bytes + parameters
//   W::xk(i, jg)                   column offset within the block of the 8 activations that lane group
//                                  jg (= lane >> 4) feeds to MFMA step i (the B layout decides it)
//   W::mma<A, MCH>(w, p, xv, yacc) the MFMAs of one block for MCH 16-row activation chunks
//   W::out_scale(args, n)          factor applied to output column n (weight row n)
//   W::kSumOffset, W::NG, W::mma_one<A>(w, p, xv, sig, y0)   (optional) formats whose codes carry
//                                  an offset that costs sum(x) per group: the one-row form, given the
//                                  activation sums sig[g] of the block's NG groups
//
// Structure (one workgroup per 16-row tile, all of K):
//  * NW waves split the tile's k-blocks into contiguous slices (wave w owns [w*kbw, (w+1)*kbw));
//    the per-wave partials are summed through LDS in wave order. No inter-workgroup communication,
//    no global fences: results are deterministic for a given NW.
//  * Software pipeline: the next U blocks' weights are in flight while the current U are computed.
//  * XLDS: the workgroup first copies its activation rows (zero-padded to KB*128 columns, optionally
//    divided by a per-column scale) into LDS with full-width loads; MFMA A fragments are LDS reads and
//    rows at or beyond M alias row M-1 (those outputs are dropped). Otherwise fragments are buffer
//    loads (rows >= M read as zero) and KTAIL zeroes activation columns at or beyond K.
//  * ONE (one activation row, formats with kSumOffset): the offset term of each group is
//    -(offset) * sum(x over the group), so the activation sums are formed once per round of four
//    blocks by one MFMA whose 16 A rows hold the round's 16 chunks of 32 activations (against a
//    B of ones; two MFMAs for a round of eight blocks), instead of an MFMA chain per block against
//    the constant offset. R1: waves whose k-slice is a single round keep no registers for a next
//    round (int4 waves of five to eight blocks run one round of eight, FP4 / FP8 waves of nine to
//    sixteen one round of sixteen). ONE = 2 also
//    drops the workgroup's copy of the activations: each wave loads only its own k-slice (issued
//    before its weights) into its own LDS area, so no workgroup barrier precedes the MFMAs; the SiLU
//    gate and the norm from tile sums (kProNormSum) are applied to that slice on the way in. ONE = 3
//    is ONE = 2 held to 64 VGPRs (8 waves per SIMD, a few registers spilled): for grids of more than
//    1024 tiles whose waves make a single round it hides more latency (gate/up 13.1 -> 12.2 us),
//    while for multi-round waves the spills cost more than the occupancy gives.
#pragma once

#include <type_traits>

#include "sqx_common.h"

namespace sqx {

// Largest LDS copy of the activations a workgroup makes (bytes); larger inputs read fragments
// from global memory. 66 KiB holds 8 padded rows of 4096 columns (65,664 bytes): at M = 8 the copy
// made the 4096-column GEMVs 9 % faster than fragments from global memory.
static constexpr int64_t kXldsMax = 66 * 1024;

inline int64_t gemv_xlds_bytes(int64_t m, int64_t KB, int kblk = 128) { return m * (KB * kblk + 8) * 2; }

inline int gemv_mch(int64_t m) { return m <= 16 ? 1 : (m <= 32 ? 2 : 4); }

// Waves per tile the library picks. One row (the one-row forms): one round of four k-blocks per
// wave, at most 16 waves (measured on the Llama shapes: int4 4096->1024 3.71 -> 3.40 us and
// 4096x4096 4.28 -> 4.18 us at 8 waves instead of 16, MXFP4 8192->28672 25.7 -> 22.3 us and
// 28672->8192 28.5 -> 26.0 us at 16 instead of 8; the others unchanged; with the single-round
// builds the int4 lm_head 4096->128256, 8016 tiles, 45.2 -> 44.2 us at 8 waves instead of 4). More
// rows: 16 for up to 256 tiles, 8 up to 2048 tiles, 4 beyond. At least 2 blocks per wave either way.
inline int gemv_default_kslices(int64_t rows, int64_t cols, int kblk = 128, int64_t m = 2) {
  const int64_t T = ceil_div(rows, 16);
  const int64_t KB = ceil_div(cols, kblk);
  int64_t s = T <= 256 ? 16 : (T <= 2048 ? 8 : 4);
  if (m == 1) s = std::min<int64_t>(16, std::max<int64_t>(1, KB / 4));
  int64_t cap = KB / 2;
  if (cap < 1) cap = 1;
  if (s > cap) s = cap;
  return static_cast<int>(s);
}

// Weight policies with a per-row (token) factor of the output declare `kRowScale = true` and
// `row_scale(args, m)`; `rows_from(args, m0)` moves that factor's pointer to the pass starting at row m0.
template <class W, class = void>
struct has_sum_offset : std::false_type {};
template <class W>
struct has_sum_offset<W, std::void_t<decltype(W::kSumOffset)>> : std::integral_constant<bool, W::kSumOffset> {};
// largest k-slice (in blocks) of a wave that loads its own activations (ONE = 2): four 16-byte loads a lane
static constexpr int kOneMaxKbw = 16;
template <class W, class = void>
struct ng_of : std::integral_constant<int, 1> {};
template <class W>
struct ng_of<W, std::void_t<decltype(W::NG)>> : std::integral_constant<int, W::NG> {};
template <class W>
inline constexpr int kNgOf = ng_of<W>::value;

template <class W, class = void>
struct has_row_scale : std::false_type {};
template <class W>
struct has_row_scale<W, std::void_t<decltype(W::kRowScale)>> : std::integral_constant<bool, W::kRowScale> {};

// What the LDS copy of the activations computes on the way in (XLDS only, bf16 activations):
//   kProPlain    x as given (optionally divided by a per-column scale);
//   kProResNorm  the decode step's residual add + RMSNorm: h = bf16(x + delta) (delta optional; workgroup
//                0 writes h to h_out), then bf16(h * (1 / sqrt(mean(h^2) + eps)) * gain). The sums use
//                the thread mapping and order of the standalone RMSNorm kernel (256 threads, 8 columns
//                each per 2048), so the result is bit-identical to running that kernel first;
//   kProSiluGate x is the fused gate|up row [M, 2K]: bf16(silu(g) * u), as the standalone SiLU kernel;
//   kProNormSum  (one row) x is the residual stream h and ss_in[0..nss) the sums of h^2 over its 16-column
//                tiles, as the residual epilogue of the linear that wrote h leaves them:
//                bf16(h * (1 / sqrt(sum(ss_in) / K + eps)) * gain), the standalone kernel's arithmetic
//                with the sum of squares added in another order.
//   kProScaleSum (one row) RMSNorm's row factor moved past the linear: x is bf16(h * gain) as given
//                (the residual epilogue of the linear that wrote h can write it), and the output is
//                r * (x W^T) with r = 1 / sqrt(sum(ss_in) / K + eps), ss_in as for kProNormSum. Wave 0
//                copies the sums straight into LDS (buffer loads that write LDS, issued behind its
//                activation slice, so no registers hold them) and forms r before the epilogue.
// RES (one row): the residual epilogue. The output is res_out = bf16(res + bf16(x W^T)) (the decode
// step's h = x + o_proj(...), model.py:365-372), and ss_out[t] is the sum of its squares over tile t.
// RKV (one row, fewer than 1024 tiles): the fused q|k|v projection's RoPE and cache write. Rows below
// qn are q, rotated (model.py:205-224: interleaved pairs at position lengths[0], separate fp32
// products and sums of the bf16 output, rounded to bf16) into q_out; rows [qn, qn + kn) are k,
// rotated and stored at cache row min(lengths[0], tmax - 1) of k_cache [kn / 128, tmax, 128]
// (kv_cache.py:194-205); the rest are v, stored there in v_cache. Wave 0 requests the length with
// its activation slice and the pair's cos / sin behind it, so the epilogue finds them in registers.
// SWI (one-row forms): the SwiGLU pair epilogue for a fused gate|up weight whose rows alternate in
// groups of 8 (tile t holds gate rows 8t..8t+7 then the matching up rows): each output is rounded to
// bf16 as the GEMV writes it and y[8t + i] = bf16(silu(g_i) * u_i), as the standalone SiLU kernel
// computes it from those bf16 values (model.py:223-237's silu(w1 x) * w3 x). y has N / 2 entries a row.
// kProAttnCombine (one row, two k-blocks per wave, 128-column blocks): x is the attention output of
//                the decode step, formed here from the key-chunk partials that
//                sqx_decode_attention_partials left (o then (m, l) per head and chunk, at most
//                kAttnFoldChunks chunks of pa.chunk keys; the row attends min(lengths[0] + 1, tmax)
//                keys): each lane merges 4 columns of its wave's slice (one head), as the combine
//                kernel does (attn_chunk_weight, ascending chunks, bf16(o / l)), so the result is
//                bit-identical to running that kernel first. Every load of it is unconditional (chunks
//                past nchunk read past the buffer resource: zero, no traffic).
enum { kProPlain = 0, kProResNorm = 1, kProSiluGate = 2, kProNormSum = 3, kProScaleSum = 4, kProAttnCombine = 5 };
static constexpr int kAttnFoldChunks = 8;
static constexpr int kProMaxRows = 8;
static constexpr int kNormSumMax = 512;  // tiles of sums of squares a kProNormSum prologue reads (K <= 8192)

struct ProArgs {
  const uint16_t* delta;  // kProResNorm: residual delta [M, K] or null
  const uint16_t* gain;   // kProResNorm, kProNormSum: RMSNorm gain [K]
  uint16_t* h_out;        // kProResNorm: x + delta [M, K] (written when delta is given)
  float eps;
  const float* ss_in;     // kProNormSum, kProScaleSum: sums of squares of h per 16-column tile [nss]
  int nss;
  const uint16_t* res;    // RES: residual [N]
  uint16_t* res_out;      // RES: res + the linear's output [N] (may be res)
  float* ss_out;          // RES: sum of res_out^2 per 16-row tile [ceil(N / 16)]
  const uint16_t* gain_next;  // RES: when set, hg_out = bf16(res_out * gain_next) [N] as well
  uint16_t* hg_out;
  const int* lengths;         // RKV: lengths[0], the row's position
  const float* cos_t;         // RKV: RoPE tables [rope_rows, 64]
  const float* sin_t;
  int rope_rows, qn, kn, tmax;
  uint16_t* q_out;            // RKV: rotated q [qn]
  uint16_t* k_cache;          // RKV: [kn / 128, tmax, 128] bf16
  uint16_t* v_cache;
  const float* part;          // kProAttnCombine: the attention partials (o [K/128][nchunk][128], then (m, l))
  int nchunk, chunk;          // kProAttnCombine: chunks per head and keys per chunk (tmax, lengths as RKV)
};

template <class A, class W, int MCH, int U, bool KTAIL, bool XLDS, bool YF32, int PRO = kProPlain, int ONE = 0,
          bool RES = false, bool RKV = false, bool SWI = false, bool R1 = false>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(ONE == 3 ? 8 : 1))) void gemv_kernel(const typename W::Args wa, const uint16_t* __restrict__ x,
                                                    void* __restrict__ yv, const uint16_t* __restrict__ bias,
                                                    const float* __restrict__ colscale, int M, int N, int K, int KB,
                                                    int kbw, const ProArgs pa) {
  static_assert(PRO == kProPlain || (XLDS && MCH == 1), "activation prologues need the LDS copy");
  static_assert(ONE == 0 || (XLDS && MCH == 1 && (U == 4 || U == 8 || (U == 16 && !has_sum_offset<W>::value))),
                "the one-row form reads rounds of 4 or 8 blocks (16 without the sum offset) from LDS");
  static_assert(ONE < 2 || PRO == kProPlain || PRO == kProNormSum || PRO == kProSiluGate || PRO == kProScaleSum ||
                    PRO == kProAttnCombine,
                "a prologue over the whole row needs the workgroup's copy of the activations");
  static_assert(PRO != kProAttnCombine || (ONE >= 2 && W::KBLK == 128), "the attention merge runs in each wave's slice");
  static_assert((PRO != kProNormSum && PRO != kProScaleSum) || ONE >= 2,
                "the norm from tile sums runs in each wave's own slice");
  static_assert(!RES || ONE != 0, "the residual epilogue is a one-row form");
  static_assert(!RKV || (ONE >= 2 && !RES), "the RoPE epilogue is a one-row form of its own");
  static_assert(ONE == 0 || !YF32, "the one-row form writes 16-bit outputs");
  static_assert(!SWI || (ONE != 0 && !RES && !RKV), "the SwiGLU pair epilogue is a one-row form of its own");
  extern __shared__ f32x4_t smem[];  // [NW][MCH][64] partial accumulators, then (XLDS) the activations
  f32x4_t* red = smem;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int t = blockIdx.x;
  const int kb0 = wave * kbw;
  const int kb1 = min(KB, kb0 + kbw);
  const int nl = lane & 15;  // weight row within the tile (B column) == A row within a chunk
  const int jg = lane >> 4;

  const typename W::Ctx wc = W::ctx(wa, t, KB, lane);
  const rsrc_t xr = make_rsrc(x, (uint32_t)M * (uint32_t)K * (PRO == kProSiluGate ? 4u : 2u));
  // RES: wave 0 requests its lanes' residual (and next-norm gain) values now, so that the epilogue of
  // small grids (wave 0 finishes the tile) does not wait for them; lanes 16..63 read neighbours or zero.
  [[maybe_unused]] uint32_t res_pre = 0u, gain_pre = 0u;
  [[maybe_unused]] int len_pre = 0;
  [[maybe_unused]] float cos_pre = 0.0f, sin_pre = 0.0f;
  if constexpr (RES) {
    if (wave == 0) {  // wave-uniform
      const uint32_t off = (uint32_t)(t * 16 + (lane & 15)) * 2u;
      res_pre = bload16(make_rsrc(pa.res, (uint32_t)N * 2u), off, 0u);
      if (pa.gain_next != nullptr) gain_pre = bload16(make_rsrc(pa.gain_next, (uint32_t)N * 2u), off, 0u);
    }
  }
  constexpr int KBLK = W::KBLK;
  constexpr int STEPS = W::STEPS;
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem + nw * MCH * 64);
  const int xpitch = KB * KBLK + 8;  // LDS row pitch in elements (16 bytes of padding per row)
  uint32_t xvo[MCH];
  f32x4_t yacc[MCH];
#pragma unroll
  for (int c = 0; c < MCH; ++c) {
    yacc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    xvo[c] = XLDS ? (uint32_t)(min(c * 16 + nl, M - 1) * xpitch) : ((uint32_t)(c * 16 + nl) * (uint32_t)K) * 2u;
  }

  [[maybe_unused]] float y1 = 0.0f;  // ONE: the row's partial for this lane's weight row (lanes 0..15)
  u32x4_t w[U];
  typename W::P p[U];
  auto load_round = [&](int kr, u32x4_t (&wo)[U], typename W::P (&po)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (kr + u < kb1) W::load(wc, kr + u, wo[u], po[u]);  // wave-uniform condition
  };
  // ONE = 2: this wave's activations from column kb0*KBLK of the single row, nx loads of 16 bytes a
  // lane (nx KiB, ceil(kbw*KBLK/512)), requested ahead of the weights. Every load and store of it is
  // wave-uniform and the first weight round is unconditional (blocks past kb1 are clamped to kb1-1 and
  // left unused), so the wait before the LDS store counts exactly the weight loads still in flight.
  // Columns past the wave's slice read the next wave's activations (unused) or, past K, zero.
  constexpr int kXw = ONE >= 2 ? kOneMaxKbw * KBLK / 8 / 64 : 1;
  const int nx = (kbw * (KBLK / 8) + 63) / 64;
  u32x4_t xw[kXw];
  uint16_t* xwave = xs + (ONE >= 2 ? wave * nx * 512 : 0);  // this wave's LDS slice (ONE = 2)
  [[maybe_unused]] u32x4_t gw[PRO == kProNormSum || PRO == kProSiluGate ? kXw : 1];  // gain, or the up half
  [[maybe_unused]] u32x4_t ssv[PRO == kProNormSum ? kNormSumMax / 256 : 1];
  [[maybe_unused]] __shared__ float row_scale_lds;                              // kProScaleSum: r (wave 0)
  [[maybe_unused]] __shared__ __attribute__((aligned(16))) float ss_lds[PRO == kProScaleSum ? kNormSumMax : 4];
  // kProAttnCombine: this lane's head (kb0 + lane / 32, two k-blocks per wave) and 4 dims; the (m, l)
  // pairs of chunks 2i, 2i+1 and the o values of each chunk, requested ahead of the weights
  [[maybe_unused]] u32x4_t cml[PRO == kProAttnCombine ? kAttnFoldChunks / 2 : 1];
  [[maybe_unused]] u32x4_t cov[PRO == kProAttnCombine ? kAttnFoldChunks : 1];
  [[maybe_unused]] int clen = 0;
  if constexpr (PRO == kProAttnCombine) {
    const int H = K / KBLK, nc = pa.nchunk;
    const int h = kb0 + (lane >> 5), d0 = 4 * (lane & 31);
    constexpr uint32_t kPast = 0x40000000u;  // past both resources: the load returns zero
    const rsrc_t ro = make_rsrc(pa.part, (uint32_t)(H * nc * KBLK) * 4u);
    const rsrc_t rml = make_rsrc(pa.part + (int64_t)H * nc * KBLK, (uint32_t)(H * nc) * 8u);
    clen = static_cast<int>(bload32(make_rsrc(pa.lengths, 4u), 0u, 0u));
#pragma unroll
    for (int i = 0; i < kAttnFoldChunks / 2; ++i)
      cml[i] = bload128(rml, 2 * i < nc ? (uint32_t)(h * nc + 2 * i) * 8u : kPast, 0u);
#pragma unroll
    for (int c = 0; c < kAttnFoldChunks; ++c)
      cov[c] = bload128(ro, c < nc ? (uint32_t)((h * nc + c) * KBLK + d0) * 4u : kPast, 0u);
  }
  if constexpr (ONE >= 2) {
#pragma unroll
    for (int i = 0; i < kXw; ++i)
      if (PRO != kProAttnCombine && i < nx) xw[i] = bload128(xr, (uint32_t)(kb0 * KBLK + 8 * (lane + 64 * i)) * 2u, 0u);
    if constexpr (PRO == kProSiluGate) {  // xw holds the gate half [0, K) of the row, gw the up half
#pragma unroll
      for (int i = 0; i < kXw; ++i)
        if (i < nx) gw[i] = bload128(xr, (uint32_t)(K + kb0 * KBLK + 8 * (lane + 64 * i)) * 2u, 0u);
    }
    if constexpr (PRO == kProNormSum) {
      const rsrc_t gr = make_rsrc(pa.gain, (uint32_t)K * 2u);
      const rsrc_t sr = make_rsrc(pa.ss_in, (uint32_t)pa.nss * 4u);
#pragma unroll
      for (int i = 0; i < kXw; ++i)
        if (i < nx) gw[i] = bload128(gr, (uint32_t)(kb0 * KBLK + 8 * (lane + 64 * i)) * 2u, 0u);
#pragma unroll
      for (int i = 0; i < kNormSumMax / 256; ++i)  // four sums a lane per load; past nss the resource reads zero
        if (i * 256 < pa.nss) ssv[i] = bload128(sr, (uint32_t)(lane + 64 * i) * 16u, 0u);
    }
    if constexpr (RKV) {
      if (wave == 0) len_pre = static_cast<int>(bload32(make_rsrc(pa.lengths, 4u), 0u, 0u));  // wave-uniform
    }
    if constexpr (PRO == kProScaleSum) {
      if (wave == 0) {  // wave-uniform: the sums into LDS, behind the activation slice (zero past nss)
        const rsrc_t sr = make_rsrc(pa.ss_in, (uint32_t)pa.nss * 4u);
#pragma unroll
        for (int i = 0; i < kNormSumMax / 256; ++i)
          if (i * 256 < pa.nss)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void*)(ss_lds + 256 * i), 16,
                                                     (uint32_t)(lane + 64 * i) * 16u, 0, 0, 0);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) W::load(wc, min(kb0 + u, kb1 - 1), w[u], p[u]);
    // the attention merge waits for its partials: keep the scheduler from hoisting it above the
    // weight requests
    if constexpr (PRO == kProAttnCombine) __builtin_amdgcn_sched_barrier(0);
  } else {
    if (kb0 < kb1) load_round(kb0, w, p);
  }
  // The first weight round is in flight while the activations are copied into LDS.
  if constexpr (ONE >= 2) {
    if constexpr (PRO == kProSiluGate) {  // bf16(silu(g) * u) as the standalone SiLU kernel; 0 past K
#pragma unroll
      for (int i = 0; i < kXw; ++i)
        if (i < nx) {
          const bool in = kb0 * KBLK + 8 * (lane + 64 * i) < K;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t g2 = xw[i][j], u2 = gw[i][j];
            const float g0 = bf16_lo(g2), g1 = bf16_hi(g2);
            const uint32_t v = ActBF16::pack_rne(silu_f32(g0) * bf16_lo(u2), silu_f32(g1) * bf16_hi(u2));
            xw[i][j] = in ? v : 0u;
          }
        }
    }
    if constexpr (PRO == kProNormSum) {
      // the row's sum of squares from the tile sums: a fixed order, the same in every wave and lane
      float t = 0.0f;
#pragma unroll
      for (int i = 0; i < kNormSumMax / 256; ++i)
        if (i * 256 < pa.nss) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t se = ssv[i][e];
            t += __builtin_bit_cast(float, se);
          }
        }
      t = wave_sum(t);
      const float r = 1.0f / sqrtf(t / static_cast<float>(K) + pa.eps);
#pragma unroll
      for (int i = 0; i < kXw; ++i)
        if (i < nx) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t h2 = xw[i][j], g2 = gw[i][j];
            xw[i][j] = ActBF16::pack_rne(bf16_lo(h2) * r * bf16_lo(g2), bf16_hi(h2) * r * bf16_hi(g2));
          }
        }
    }
    if constexpr (PRO == kProAttnCombine) {
      // the merge of the head's chunks below the row's length, as attn_combine_kernel does
      const int L = min(max(clen, 0) + 1, pa.tmax);
      const int used = (L + pa.chunk - 1) / pa.chunk;  // <= nchunk
      // each element through a scalar: hipcc's bit_cast of a vector element reads element 0
      auto mof = [&](int c) {
        const uint32_t v = cml[c >> 1][2 * (c & 1)];
        return __builtin_bit_cast(float, v);
      };
      auto lof = [&](int c) {
        const uint32_t v = cml[c >> 1][2 * (c & 1) + 1];
        return __builtin_bit_cast(float, v);
      };
      // Every chunk's values are used and the results past `used` dropped by selects (chunks past the
      // length were never written): a branch would let the compiler sink the loads into it, behind
      // the weights, and wait for those as well.
      float M = -INFINITY;
#pragma unroll
      for (int c = 0; c < kAttnFoldChunks; ++c) M = c < used ? fmaxf(M, mof(c)) : M;
      float ls = 0.0f, os[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < kAttnFoldChunks; ++c) {
        const bool u = c < used;
        const float a = attn_chunk_weight(mof(c), M);
        ls = u ? fmaf(lof(c), a, ls) : ls;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t oj = cov[c][j];
          os[j] = u ? fmaf(__builtin_bit_cast(float, oj), a, os[j]) : os[j];
        }
      }
      uint32_t b[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = f32_to_bf16_bits(os[j] / ls);
      *reinterpret_cast<u32x2v_t*>(xwave + 4 * lane) = u32x2v_t{b[0] | (b[1] << 16), b[2] | (b[3] << 16)};
    } else {
#pragma unroll
      for (int i = 0; i < kXw; ++i)
        if (i < nx) *reinterpret_cast<u32x4_t*>(xwave + 8 * (lane + 64 * i)) = xw[i];
    }
    // LDS operations of one wave execute in issue order; only the compiler must not move the
    // fragment reads above the stores
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    if constexpr (RKV) {
      if (wave == 0) {  // the pair's cos / sin at the row's position (needed only in the epilogue)
        // kept in a vector register: moved to a scalar one, it would be waited for where it is loaded,
        // before the wave's weights are requested
        asm volatile("" : "+v"(len_pre));
        const int pos = min(max(len_pre, 0), pa.rope_rows - 1);
        const uint32_t pi = (uint32_t)(pos * 64 + (((t * 16 + (lane & 15)) & 127) >> 1)) * 4u;
        const uint32_t tb = (uint32_t)pa.rope_rows * 64u * 4u;
        cos_pre = __builtin_bit_cast(float, bload32(make_rsrc(pa.cos_t, tb), pi, 0u));
        sin_pre = __builtin_bit_cast(float, bload32(make_rsrc(pa.sin_t, tb), pi, 0u));
      }
    }
  } else if constexpr (PRO == kProResNorm) {
    // The 256 threads of the standalone kernel are emulated by "virtual threads" vt (in passes when
    // the workgroup is smaller; a workgroup is a whole number of waves, so a virtual wave is a real
    // one). Pass 1: h, its sum of squares per row, h -> LDS.
    __shared__ float pro_red[kProMaxRows][4];
    const int tid = threadIdx.x;
    for (int base = 0; base < 256; base += blockDim.x) {
      const int vt = base + tid;
      float ss[kProMaxRows];
#pragma unroll
      for (int r = 0; r < kProMaxRows; ++r) {
        ss[r] = 0.0f;
        if (r < M && vt < 256) {
          for (int c = vt * 8; c < K; c += 256 * 8) {
            u32x4_t v = bload128(xr, (uint32_t)(r * K + c) * 2u, 0u);
            if (pa.delta != nullptr) {
              const u32x4_t dv = *reinterpret_cast<const u32x4_t*>(pa.delta + (int64_t)r * K + c);
#pragma unroll
              for (int j = 0; j < 4; ++j)
                v[j] = ActBF16::pack_rne(bf16_lo(v[j]) + bf16_lo(dv[j]), bf16_hi(v[j]) + bf16_hi(dv[j]));
              if (blockIdx.x == 0) *reinterpret_cast<u32x4_t*>(pa.h_out + (int64_t)r * K + c) = v;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float a0 = bf16_lo(v[j]), a1 = bf16_hi(v[j]);
              ss[r] = fmaf(a0, a0, ss[r]);
              ss[r] = fmaf(a1, a1, ss[r]);
            }
            *reinterpret_cast<u32x4_t*>(xs + r * xpitch + c) = v;
          }
        }
      }
      if (vt < 256) {  // whole waves
#pragma unroll
        for (int r = 0; r < kProMaxRows; ++r) {
          if (r < M) {
            const float t = wave_sum(ss[r]);
            if ((vt & 63) == 0) pro_red[r][vt >> 6] = t;
          }
        }
      }
    }
    // zero the padding columns of the LDS rows
    for (int idx = tid; idx < M * (KB * KBLK - K) / 8; idx += blockDim.x) {
      const int per = (KB * KBLK - K) / 8;
      const int r = idx / per;
      *reinterpret_cast<u32x4_t*>(xs + r * xpitch + K + (idx - r * per) * 8) = u32x4_t{0u, 0u, 0u, 0u};
    }
    __syncthreads();
    // pass 2: normalise in place with the row's factor and the gain
    for (int vt = tid; vt < 256; vt += blockDim.x) {
#pragma unroll
      for (int r = 0; r < kProMaxRows; ++r) {
        if (r < M) {
          const float tot = (pro_red[r][0] + pro_red[r][1]) + (pro_red[r][2] + pro_red[r][3]);
          const float rr = 1.0f / sqrtf(tot / static_cast<float>(K) + pa.eps);
          for (int c = vt * 8; c < K; c += 256 * 8) {
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xs + r * xpitch + c);
            const u32x4_t wv = *reinterpret_cast<const u32x4_t*>(pa.gain + c);
            u32x4_t o;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              o[j] = ActBF16::pack_rne(bf16_lo(v[j]) * rr * bf16_lo(wv[j]), bf16_hi(v[j]) * rr * bf16_hi(wv[j]));
            *reinterpret_cast<u32x4_t*>(xs + r * xpitch + c) = o;
          }
        }
      }
    }
    __syncthreads();
  } else if constexpr (PRO == kProSiluGate) {
    const int chunks_per_row = KB * KBLK / 8;
    for (int idx = threadIdx.x; idx < M * chunks_per_row; idx += blockDim.x) {
      const int r = idx / chunks_per_row;
      const int col = (idx - r * chunks_per_row) * 8;
      u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
      if (col < K) {
        const u32x4_t g2 = bload128(xr, (uint32_t)(r * 2 * K + col) * 2u, 0u);
        const u32x4_t u2 = bload128(xr, (uint32_t)(r * 2 * K + K + col) * 2u, 0u);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float g0 = bf16_lo(g2[j]), g1 = bf16_hi(g2[j]);
          v[j] = ActBF16::pack_rne(silu_f32(g0) * bf16_lo(u2[j]), silu_f32(g1) * bf16_hi(u2[j]));
        }
      }
      *reinterpret_cast<u32x4_t*>(xs + r * xpitch + col) = v;
    }
    __syncthreads();
  } else if (XLDS) {
    const int chunks_per_row = KB * KBLK / 8;  // 16-byte chunks of a padded row
    for (int idx = threadIdx.x; idx < M * chunks_per_row; idx += blockDim.x) {
      const int r = idx / chunks_per_row;
      const int col = (idx - r * chunks_per_row) * 8;
      u32x4_t v = col < K ? bload128(xr, (uint32_t)(r * K + col) * 2u, 0u) : u32x4_t{0u, 0u, 0u, 0u};
      if (colscale != nullptr && col < K) {  // x / s per column, rounded back to the activation type
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = __fdiv_rn(A::to_f32(static_cast<uint16_t>(v[e] & 0xffffu)), colscale[col + 2 * e]);
          const float hi = __fdiv_rn(A::to_f32(static_cast<uint16_t>(v[e] >> 16)), colscale[col + 2 * e + 1]);
          v[e] = static_cast<uint32_t>(A::from_f32(lo)) | (static_cast<uint32_t>(A::from_f32(hi)) << 16);
        }
      }
      *reinterpret_cast<u32x4_t*>(xs + r * xpitch + col) = v;
    }
    __syncthreads();
  }

  for (int kb = kb0; kb < kb1; kb += U) {
    // Global activation fragments of the whole round are requested ahead of the next round's weights:
    // buffer loads retire in issue order, so waiting for them leaves the next weights in flight.
    u32x4_t xg[XLDS ? 1 : U][MCH][STEPS];
    if constexpr (!XLDS) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (kb + u < kb1) {
#pragma unroll
          for (int c = 0; c < MCH; ++c) {
#pragma unroll
            for (int i = 0; i < STEPS; ++i)
              xg[u][c][i] = bload128(xr, xvo[c] + 2u * W::xk(i, jg), (uint32_t)((kb + u) * KBLK) * 2u);
          }
        }
      }
    }
    // R1: every wave's k-slice is a single round (kbw <= U), so no next round is held in registers
    [[maybe_unused]] u32x4_t wn[R1 ? 1 : U];
    [[maybe_unused]] typename W::P pn[R1 ? 1 : U];
    if constexpr (!R1) {
      if (kb + U < kb1) load_round(kb + U, wn, pn);
    }
    // ONE: activation sums of the round's blocks. With CPB chunks of 32 columns per block, one MFMA
    // covers 16 chunks: row r = CPB*b + c of MFMA h holds chunk c of block kb + 16h/CPB + b; lane l
    // receives rows 4(l >> 4) .. +3, i.e. the chunk sums of block u at lane group (CPB*u % 16)/4,
    // elements CPB*u%4 onward, of MFMA CPB*u/16.
    constexpr int CPB = KBLK / 32;
    constexpr int NH = (CPB * U + 15) / 16;  // MFMAs for the round's chunk sums
    static_assert(ONE == 0 || ((CPB * U <= 16 || (CPB * U) % 16 == 0) && 4 % CPB == 0),
                  "a round's chunks fill whole 16-row MFMAs");
    [[maybe_unused]] float sig[U][ONE ? kNgOf<W> : 1];
    if constexpr (ONE != 0 && has_sum_offset<W>::value) {
      const uint16_t* xrow = ONE >= 2 ? xwave + (kb - kb0) * KBLK : xs + kb * KBLK;
      const uint32_t one = A::pair_from_f32(1.0f);
      f32x4_t cs[NH];
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        const int r = lane & 15, b = 16 * h / CPB + r / CPB;
        u32x4_t a2 = u32x4_t{0u, 0u, 0u, 0u};
        if (b < U && kb + b < kb1) a2 = *reinterpret_cast<const u32x4_t*>(xrow + b * KBLK + 32 * (r % CPB) + 8 * jg);
        cs[h] = A::mfma(a2, u32x4_t{one, one, one, one}, f32x4_t{0.f, 0.f, 0.f, 0.f});
      }
      constexpr int NG = kNgOf<W>;
      constexpr int CPG = CPB / NG;  // chunks per group
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          const int h = (CPB * u) / 16, uu = (CPB * u) % 16;
          float v = 0.0f;
#pragma unroll
          for (int i = 0; i < CPG; ++i) v += cs[h][uu % 4 + g * CPG + i];
          sig[u][g] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16 * (uu / 4)));
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (kb + u < kb1) {  // wave-uniform
        const int kk = kb + u;
        u32x4_t xv[MCH][STEPS];
#pragma unroll
        for (int c = 0; c < MCH; ++c) {
#pragma unroll
          for (int i = 0; i < STEPS; ++i) {
            if constexpr (ONE >= 2)
              xv[c][i] = *reinterpret_cast<const u32x4_t*>(xwave + (kk - kb0) * KBLK + W::xk(i, jg));
            else if constexpr (XLDS)
              xv[c][i] = *reinterpret_cast<const u32x4_t*>(xs + xvo[c] + kk * KBLK + W::xk(i, jg));
            else
              xv[c][i] = xg[u][c][i];
          }
        }
        if (KTAIL && !XLDS && kk == KB - 1) {  // activations at or beyond K must not enter the sums
#pragma unroll
          for (int i = 0; i < STEPS; ++i) {
            if (kk * KBLK + W::xk(i, jg) >= K) {
#pragma unroll
              for (int c = 0; c < MCH; ++c) xv[c][i] = u32x4_t{0u, 0u, 0u, 0u};
            }
          }
        }
        if constexpr (ONE != 0) {
          if constexpr (has_sum_offset<W>::value) W::template mma_one<A>(w[u], p[u], xv[0], sig[u], y1);
          else W::template mma<A, MCH>(w[u], p[u], xv, yacc);  // the 16 A rows are copies of the one row
        } else {
          W::template mma<A, MCH>(w[u], p[u], xv, yacc);
        }
      }
    }
    if constexpr (R1) {
      break;
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        w[u] = wn[u];
        p[u] = pn[u];
      }
    }
  }

  // formats without the sum offset: every row of the MFMA output is the one row's, so element 0 of a
  // lane's accumulator is its weight row's partial
  if constexpr (ONE != 0 && !has_sum_offset<W>::value) y1 = yacc[0][0];
  if constexpr (PRO == kProScaleSum) {
    if (wave == 0) {  // the row factor from the sums in LDS, in a fixed order (the same in every workgroup)
      wait_vmcnt<0>();  // the copies into LDS (long done: the weights behind them have been consumed)
      asm volatile("" ::: "memory");
      // the lane index formed afresh here (mbcnt), so that no offset derived from it in the prologue
      // stays live (or spills) through the main loop
      const int ln = static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
      float t = 0.0f;
#pragma unroll
      for (int i = 0; i < kNormSumMax / 256; ++i)
        if (i * 256 < pa.nss) {
          const f32x4_t v4 = *reinterpret_cast<const f32x4_t*>(ss_lds + 256 * i + 4 * ln);
          t += (v4[0] + v4[1]) + (v4[2] + v4[3]);
        }
      t = wave_sum(t);
      if (lane == 0) row_scale_lds = 1.0f / sqrtf(t / static_cast<float>(K) + pa.eps);
    }
  }
  // One row, grids that fit the chip in about one round: lane l < 16 of each wave holds the partial of
  // output t*16 + l, and wave 0 sums them in wave order (the order of the general path below, so the
  // bits are the same) and applies the epilogue. Larger grids measured faster with the general path,
  // where four waves share the sums.
  if (ONE != 0 && gridDim.x < 1024) {
    float* rf1 = reinterpret_cast<float*>(red);
    if (lane < 16) rf1[wave * 16 + lane] = y1;
    __syncthreads();
    if (wave == 0) {
      const int n = t * 16 + lane;
      const bool own = lane < 16 && n < N;
      float v = 0.0f;
      if (lane < 16)
        for (int ww = 0; ww < nw; ++ww) v += rf1[ww * 16 + lane];
      [[maybe_unused]] float hsq = 0.0f;
      if constexpr (RKV) {
#pragma clang fp contract(off)
        if constexpr (PRO == kProScaleSum) v *= row_scale_lds;
        const float xq = A::to_f32(A::from_f32(v));  // the projection's bf16 output
        const float xp = __shfl_xor(xq, 1, 64);      // its RoPE partner (the other dim of the pair)
        if (own) {
          const int slot = min(max(len_pre, 0), pa.tmax - 1);
          if (n < pa.qn + pa.kn) {
            const float r = (n & 1) ? xp * sin_pre + xq * cos_pre : xq * cos_pre - xp * sin_pre;
            if (n < pa.qn) {
              pa.q_out[n] = A::from_f32(r);
            } else {
              const int kd = n - pa.qn;
              pa.k_cache[((int64_t)(kd >> 7) * pa.tmax + slot) * 128 + (kd & 127)] = A::from_f32(r);
            }
          } else {
            const int vd = n - pa.qn - pa.kn;
            pa.v_cache[((int64_t)(vd >> 7) * pa.tmax + slot) * 128 + (vd & 127)] = A::from_f32(xq);
          }
        }
        return;
      }
      if (own) {
        if constexpr (has_row_scale<W>::value)
          v = v * W::row_scale(wa, 0) * W::out_scale(wa, n);
        else
          v *= W::out_scale(wa, n);
        if constexpr (PRO == kProScaleSum) v *= row_scale_lds;
        if (bias) v += A::to_f32(bias[n]);
        if constexpr (SWI) {
          // the pair is formed below, by the whole wave
        } else if constexpr (RES) {
          // opaque until here: otherwise the compiler converts the prefetched values where they are
          // loaded and waits for them there, before wave 0 has issued its weights
          asm volatile("" : "+v"(res_pre), "+v"(gain_pre));
          const float rv = A::to_f32(static_cast<uint16_t>(res_pre));
          const float h = A::to_f32(A::from_f32(rv + A::to_f32(A::from_f32(v))));
          pa.res_out[n] = A::from_f32(h);
          if (pa.gain_next != nullptr) pa.hg_out[n] = A::from_f32(h * A::to_f32(static_cast<uint16_t>(gain_pre)));
          hsq = h * h;
        } else {
          static_cast<uint16_t*>(yv)[n] = A::from_f32(v);
        }
      }
      if constexpr (RES) {
        hsq = wave_sum(hsq);
        if (lane == 0) pa.ss_out[t] = hsq;
      }
      if constexpr (SWI) {
        const float q = own ? A::to_f32(A::from_f32(v)) : 0.0f;  // this row's bf16 output
        const float u = __shfl_xor(q, 8, 64);                     // lane l < 8: its up row (lane l + 8)
        if (own && lane < 8)
          static_cast<uint16_t*>(yv)[t * 8 + lane] = static_cast<uint16_t>(A::pack_rne(silu_f32(q) * u, 0.0f));
      }
    }
    return;
  }
  if constexpr (ONE != 0) yacc[0][0] = y1;
  // Sum the NW partial tiles in wave order. Float j of a wave's block is (chunk c, lane l, row r).
#pragma unroll
  for (int c = 0; c < MCH; ++c) red[(wave * MCH + c) * 64 + lane] = yacc[c];
  __syncthreads();
  constexpr int kOut = MCH * 64 * 4;
  const float* rf = reinterpret_cast<const float*>(red);
  for (int j = threadIdx.x; j < kOut; j += blockDim.x) {
    float v = 0.0f;
    for (int ww = 0; ww < nw; ++ww) v += rf[ww * kOut + j];
    const int c = j >> 8;
    const int l = (j >> 2) & 63;
    const int m = c * 16 + 4 * (l >> 4) + (j & 3);
    const int n = t * 16 + (l & 15);
    [[maybe_unused]] float hsq = 0.0f;
    if (m < M && n < N) {
      if constexpr (has_row_scale<W>::value)
        v = v * W::row_scale(wa, m) * W::out_scale(wa, n);
      else
        v *= W::out_scale(wa, n);
      if constexpr (PRO == kProScaleSum) v *= row_scale_lds;
      if (bias) v += A::to_f32(bias[n]);
      if constexpr (SWI) {
        // below, by the whole wave
      } else if constexpr (RES) {
        const float h = A::to_f32(A::from_f32(A::to_f32(pa.res[n]) + A::to_f32(A::from_f32(v))));
        pa.res_out[n] = A::from_f32(h);
        if (pa.gain_next != nullptr) pa.hg_out[n] = A::from_f32(h * A::to_f32(pa.gain_next[n]));
        hsq = h * h;
      } else if constexpr (YF32) {
        static_cast<float*>(yv)[(int64_t)m * N + n] = v;
      } else {
        static_cast<uint16_t*>(yv)[(int64_t)m * N + n] = A::from_f32(v);
      }
    }
    if constexpr (RES) {
      // the row's 16 outputs sit in wave 0 (j = 4l, l < 16); their squares summed in a fixed order
      if (j < 64) {
        hsq = wave_sum(hsq);
        if (j == 0) pa.ss_out[t] = hsq;
      }
    }
    if constexpr (SWI) {
      // output n's up row n + 8 is output j ^ 32 (l ^ 8, same row m), in this wave and iteration: every
      // iteration covers whole waves (kOut and the block are multiples of 64)
      const bool ok = m < M && n < N;
      const float q = ok ? A::to_f32(A::from_f32(v)) : 0.0f;
      const float u = __shfl_xor(q, 32, 64);
      if (ok && (l & 15) < 8)
        static_cast<uint16_t*>(yv)[(int64_t)m * (N / 2) + t * 8 + (l & 15)] =
            static_cast<uint16_t>(A::pack_rne(silu_f32(q) * u, 0.0f));
    }
  }
}

// Launch the GEMV for every 64-row pass of x. k_slices <= 0 picks the default. Returns 0 or the
// HIP error of the launch.
template <class A, class W, int U1, int U2, bool YF32, int PRO = kProPlain, bool RES = false, bool RKV = false,
          bool SWI = false>
hipError_t gemv_launch(const typename W::Args& wa, const uint16_t* x, void* y, const uint16_t* bias,
                       const float* colscale, int64_t m, int64_t rows, int64_t cols, int k_slices,
                       hipStream_t stream, const ProArgs& pa = ProArgs{nullptr, nullptr, nullptr, 0.0f}) {
  constexpr int KBLK = W::KBLK;
  const int64_t T = ceil_div(rows, 16);
  const int64_t KB = ceil_div(cols, KBLK);
  int nw = k_slices <= 0 ? gemv_default_kslices(rows, cols, KBLK, m) : k_slices;
  if (nw > KB) nw = static_cast<int>(KB);
  const int kbw = static_cast<int>(ceil_div(KB, nw));
  nw = static_cast<int>(ceil_div(KB, kbw));  // no idle waves
  const bool ktail = cols % KBLK != 0;
  const dim3 grid(static_cast<unsigned>(T)), block(static_cast<unsigned>(64 * nw));
  for (int64_t m0 = 0; m0 < m; m0 += 64) {
    const int M = static_cast<int>(m - m0 < 64 ? m - m0 : 64);
    typename W::Args wp = wa;
    if constexpr (has_row_scale<W>::value) wp = W::rows_from(wa, m0);
    const int mch = gemv_mch(M);
    const uint16_t* xp = x + m0 * cols;
    void* yp = static_cast<char*>(y) + m0 * rows * (YF32 ? 4 : 2);
    const int N = static_cast<int>(rows), K = static_cast<int>(cols), iKB = static_cast<int>(KB);
    const size_t red = static_cast<size_t>(nw) * mch * 64 * sizeof(f32x4_t);
    const bool xlds = mch == 1 && gemv_xlds_bytes(M, KB, KBLK) <= kXldsMax;
    if (colscale != nullptr && !xlds) return hipErrorNotSupported;  // column scaling happens in the LDS copy
// the one-row forms have a single-round build (R1) for k-slices of at most one round
#define SQX_GEMV1(MCH_, U_, KT_, XL_, LDS_, ONE_)                                                              \
  do {                                                                                                        \
    if constexpr ((!RKV || ONE_ == 2) && (!SWI || ONE_ >= 2)) {                                              \
      if (ONE_ >= 2 && kbw <= U_)                                                                             \
        hipLaunchKernelGGL((gemv_kernel<A, W, MCH_, U_, KT_, XL_, YF32, PRO, ONE_, RES, RKV, SWI, (ONE_ >= 2)>), grid, \
                           block, LDS_, stream, wp, xp, yp, bias, colscale, M, N, K, iKB, kbw, pa);           \
      else                                                                                                    \
        hipLaunchKernelGGL((gemv_kernel<A, W, MCH_, U_, KT_, XL_, YF32, PRO, ONE_, RES, RKV, SWI>), grid, block, LDS_, \
                           stream, wp, xp, yp, bias, colscale, M, N, K, iKB, kbw, pa);                        \
    }                                                                                                         \
  } while (0)
#define SQX_GEMV(MCH_, U_, KT_, XL_, LDS_) SQX_GEMV1(MCH_, U_, KT_, XL_, LDS_, 0)
// the one-row form 2 in a single round of U_ blocks (int4 tiles: 8 for 5..8 blocks a wave; formats
// without the sum offset: 16 for 9..16 blocks a wave)
#define SQX_GEMVU(U_, KT_, LDS_)                                                                               \
  hipLaunchKernelGGL((gemv_kernel<A, W, 1, U_, KT_, true, YF32, PRO, 2, RES, RKV, SWI, true>), grid, block, LDS_, \
                     stream, wp, xp, yp, bias, colscale, M, N, K, iKB, kbw, pa)
    // the one-row form for formats whose offset costs sum(x) per group: 2 = each wave loads its own
    // k-slice of the activations, 1 = from the workgroup's LDS copy (prologues, column scales)
    // Formats without the sum offset (FP4, FP8) take the per-wave slice form only (their plain MFMA
    // chain on copies of the row); they gain nothing from form 1.
    constexpr bool kOneOk = U1 == 4 && !YF32;
    int one_mode = 0;
    if (kOneOk && M == 1 && xlds) {
      const bool slice = (PRO == kProPlain || PRO == kProNormSum || PRO == kProSiluGate || PRO == kProScaleSum ||
                          PRO == kProAttnCombine) &&
                         colscale == nullptr && kbw <= kOneMaxKbw;
      one_mode = slice ? 2 : (has_sum_offset<W>::value ? 1 : 0);
    }
    if (PRO != kProPlain && (!xlds || m > kProMaxRows || cols % 8 != 0))
      return hipErrorNotSupported;  // the caller checks first
    // one-row forms only: the norm from tile sums, the residual epilogue
    if (((PRO == kProNormSum || PRO == kProScaleSum || PRO == kProAttnCombine) && one_mode != 2) ||
        (RES && one_mode == 0))
      return hipErrorNotSupported;
    // the attention merge: two 128-column k-blocks per wave (4 columns a lane, one head each)
    if (PRO == kProAttnCombine && (kbw != 2 || KBLK != 128 || K % 128 != 0 || pa.nchunk > kAttnFoldChunks))
      return hipErrorNotSupported;
    // the RoPE epilogue: the one-row form 2 with wave 0 finishing each tile (grids under 1024 tiles)
    if (RKV && (one_mode != 2 || T >= 1024)) return hipErrorNotSupported;
    // the SwiGLU pair epilogue: one-row forms over whole 16-row tiles
    if (SWI && (one_mode != 2 || N % 16 != 0)) return hipErrorNotSupported;
    if (one_mode != 0) {
      if constexpr (kOneOk) {
        if (one_mode == 2) {
          const size_t lds = red + static_cast<size_t>(nw) * ((kbw * (KBLK / 8) + 63) / 64) * 1024;
          if constexpr (PRO == kProPlain || PRO == kProScaleSum) {
            if (kbw <= U1 && T > 1024) {  // one round per wave, several rounds of workgroups
              if (ktail) SQX_GEMV1(1, U1, true, true, lds, 3); else SQX_GEMV1(1, U1, false, true, lds, 3);
            } else if (kbw > U1 && kbw <= 2 * U1 && has_sum_offset<W>::value) {
              // 5..8 blocks a wave (the 14336-column down projection): one round of eight blocks
              if constexpr (has_sum_offset<W>::value) {
                if (ktail) SQX_GEMVU(2 * U1, true, lds); else SQX_GEMVU(2 * U1, false, lds);
              }
            } else if (kbw > U1 && kbw <= 4 * U1 && !has_sum_offset<W>::value && PRO == kProPlain && !RES) {
              // FP4 / FP8 waves of 5..16 blocks (MXFP4 28672->8192: 14): one round of sixteen
              if constexpr (!has_sum_offset<W>::value && PRO == kProPlain && !RES) {
                if (ktail) SQX_GEMVU(4 * U1, true, lds); else SQX_GEMVU(4 * U1, false, lds);
              }
            } else {
              if (ktail) SQX_GEMV1(1, U1, true, true, lds, 2); else SQX_GEMV1(1, U1, false, true, lds, 2);
            }
          } else if constexpr (PRO == kProNormSum || PRO == kProSiluGate || PRO == kProAttnCombine) {
            if (ktail) SQX_GEMV1(1, U1, true, true, lds, 2); else SQX_GEMV1(1, U1, false, true, lds, 2);
          }
        } else {
          const size_t lds = red + gemv_xlds_bytes(M, KB, KBLK);
          if constexpr (PRO != kProNormSum && PRO != kProScaleSum && PRO != kProAttnCombine) {
            if (ktail) SQX_GEMV1(1, U1, true, true, lds, 1); else SQX_GEMV1(1, U1, false, true, lds, 1);
          }
        }
      }
    } else if constexpr (RES || PRO == kProNormSum || PRO == kProScaleSum || PRO == kProAttnCombine) {
      return hipErrorNotSupported;
    } else if (PRO != kProPlain || xlds) {
      const size_t lds = red + gemv_xlds_bytes(M, KB, KBLK);
      if (ktail) SQX_GEMV(1, U1, true, true, lds); else SQX_GEMV(1, U1, false, true, lds);
    } else if constexpr (PRO != kProPlain) {
      return hipErrorNotSupported;
    } else if (mch == 1) {
      if (ktail) SQX_GEMV(1, U1, true, false, red); else SQX_GEMV(1, U1, false, false, red);
    } else if (mch == 2) {
      if (ktail) SQX_GEMV(2, U2, true, false, red); else SQX_GEMV(2, U2, false, false, red);
    } else {
      if (ktail) SQX_GEMV(4, 1, true, false, red); else SQX_GEMV(4, 1, false, false, red);
    }
#undef SQX_GEMV
#undef SQX_GEMV1
#undef SQX_GEMVU
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// ---------------------------------------------------------------------------------------------
// Two to eight activation rows (formats whose codes carry an offset charged through sum(x), i.e. the
// int4 tiles): the one-row form carried to M rows. One workgroup per 16-row tile, its waves on
// contiguous k-slices as in the one-row form.
//  * Each wave copies its own k-slice of the M rows (nx 16-byte loads a lane per row, requested
//    ahead of its first weight round) into its own LDS area: no workgroup copy, no barrier before
//    the MFMAs. Columns at or past K read zero (a buffer resource per row).
//  * MFMA A rows are the activation rows (A row r reads row min(r, M - 1); outputs of rows >= M are
//    dropped), B the weight codes as exact (magic + code) bf16 pairs: 4 MFMAs a block for all M
//    rows, as for one row.
//  * The code offset -(magic + zero) * sum(x over the group) is charged per row from activation
//    sums: per round of four blocks one MFMA per row puts the row's 16 chunks of 32 activations in
//    the A rows against a B of ones (lane group u then holds block u's chunk sums), instead of the
//    second MFMA chain per block of the general path. Lane (nl, jg) holds outputs of rows 4 jg + j
//    (j < 4) for weight row nl, so rows 0..3 sit in lane group 0 and rows 4..7 in lane group 1.
//  * The wave partials are summed through LDS in wave order (deterministic for a given wave count).
// MR (2, 4 or 8) is the largest M a build takes; XW the largest nx (k-slices of up to 4 XW blocks).
// The decode step's fusions of the one-row form, per row (layouts [M][...] row after row):
//   PRO = kProSiluGate  x is the fused gate|up activation [M, 2K]; each wave forms bf16(silu(g) * u)
//                       of its slice on the way into LDS, as the standalone SiLU kernel does;
//   PRO = kProScaleSum  RMSNorm's row factor past the linear: x is bf16(h * gain) and row m's output is
//                       r_m * (x W^T), r_m = 1 / sqrt(sum(ss_in[m][0..nss)) / K + eps), the sums copied
//                       into LDS behind the activation slice and added in the one-row form's order;
//   RES                 the residual epilogue: res_out[m] = bf16(res[m] + bf16(y[m])), hg_out[m] =
//                       bf16(res_out[m] * gain_next) when gain_next is given, ss_out[m][t] = sum of
//                       res_out[m]^2 over tile t (16 outputs, summed by a fixed shuffle tree);
//   RKV                 the q|k|v projection's RoPE and cache write at row m's position lengths[m]:
//                       q_out [M][qn], k_cache / v_cache [M][kn / 128][tmax][128];
//   SWI                 the SwiGLU pair epilogue of the one-row form (rows of 8-row gate / up groups):
//                       y [M][N / 2].
// The epilogue's residual, gain and length values are requested at kernel start (cos / sin behind the
// activation slice), by the threads that use them.
// RG = 2 (MR = 4, 5..8 rows): two workgroups per tile, rows 0..3 and 4..7. Workgroups b and b + 8 take
// the same tile: the hardware hands workgroups to the eight XCDs in turn, so both run on one XCD and
// the second finds the tile's weights in that XCD's L2 (the grid covers whole groups of 8 tiles).
template <class A, class W, int MR, int XW, int PRO = kProPlain, bool RES = false, bool RKV = false, int RG = 1,
          bool SWI = false, bool R1 = false>
__global__ __launch_bounds__(1024) void gemv_rows_kernel(const typename W::Args wa, const uint16_t* __restrict__ x_,
                                                         uint16_t* __restrict__ y_, const uint16_t* __restrict__ bias,
                                                         int M_, int N, int K, int KB, int kbw, const ProArgs pa_) {
  static_assert(has_sum_offset<W>::value && W::KBLK == 128 && W::STEPS == 4, "int4 tiles: 128-column blocks");
  static_assert(MR == 2 || MR == 4 || MR == 8, "2, 4 or 8 rows");
  static_assert(PRO == kProPlain || PRO == kProSiluGate || PRO == kProScaleSum, "plain rows, SiLU gate or row factor");
  static_assert(!(RES && RKV) && !(SWI && (RES || RKV)), "one epilogue");
  static_assert(RG == 1 || (RG == 2 && MR == 4), "two groups of four rows");
  constexpr int KBLK = 128, U = 4, NG = kNgOf<W>, CPB = 4, CPG = CPB / NG, MPG = 4 / NG;
  constexpr int kJ = 16 * (MR < 4 ? 4 : MR);  // epilogue threads: output j = (lane l = j / 4, element e = j % 4)
  constexpr int RS = PRO == kProSiluGate ? 2 : 1;  // activation row stride in units of K
  extern __shared__ f32x4_t smem[];  // [NW][64] partial accumulators, then each wave's activation rows
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int T = (N + 15) / 16;
  const int b = static_cast<int>(blockIdx.x);
  const int t = RG == 1 ? b : (((b >> 4) << 3) | (b & 7));
  const int rb = RG == 1 ? 0 : 4 * ((b >> 3) & 1);  // first row of this workgroup
  const int M = RG == 1 ? M_ : min(4, M_ - rb);
  if (RG == 2 && (t >= T || M <= 0)) return;  // the whole workgroup: padding tiles, or rows 4..7 of M <= 4
  const uint16_t* x = x_ + static_cast<int64_t>(rb) * RS * K;
  uint16_t* y = y_ == nullptr ? nullptr : y_ + static_cast<int64_t>(rb) * (SWI ? N / 2 : N);
  ProArgs pa = pa_;
  if (RG == 2 && rb > 0) {  // this workgroup's rows of every row-major array
    if (pa.res) pa.res += static_cast<int64_t>(rb) * N;
    if (pa.res_out) pa.res_out += static_cast<int64_t>(rb) * N;
    if (pa.hg_out) pa.hg_out += static_cast<int64_t>(rb) * N;
    if (pa.ss_out) pa.ss_out += static_cast<int64_t>(rb) * T;
    if (pa.ss_in) pa.ss_in += static_cast<int64_t>(rb) * pa.nss;
    if (pa.lengths) pa.lengths += rb;
    if (pa.q_out) pa.q_out += static_cast<int64_t>(rb) * pa.qn;
    if (pa.k_cache) pa.k_cache += static_cast<int64_t>(rb) * pa.kn * pa.tmax;
    if (pa.v_cache) pa.v_cache += static_cast<int64_t>(rb) * pa.kn * pa.tmax;
  }
  const int kb0 = wave * kbw;
  const int kb1 = min(KB, kb0 + kbw);
  const int nl = lane & 15, jg = lane >> 4;
  const typename W::Ctx wc = W::ctx(wa, t, KB, lane);
  const int nx = (kbw * (KBLK / 8) + 63) / 64;
  // LDS row pitch: nx KiB plus 64 bytes, so that rows start 16 banks apart
  const int pitch = nx * 512 + 32;
  uint16_t* xwave = reinterpret_cast<uint16_t*>(smem + nw * 64) + wave * MR * pitch;
  // the epilogue's output of this thread (at most one, as blockDim >= 64 and kJ <= 128 outputs are
  // spread over the first kJ threads)
  const int jo = threadIdx.x;
  const int mo = 4 * ((jo >> 2) >> 4) + (jo & 3);
  const int no = t * 16 + ((jo >> 2) & 15);
  const bool own = jo < kJ && mo < M && no < N;
  [[maybe_unused]] uint32_t res_pre = 0u, gain_pre = 0u;
  [[maybe_unused]] int len_pre = 0;
  [[maybe_unused]] float cos_pre = 0.0f, sin_pre = 0.0f;
  if constexpr (RES) {
    if (own) {
      res_pre = bload16(make_rsrc(pa.res, (uint32_t)M * N * 2u), (uint32_t)(mo * N + no) * 2u, 0u);
      if (pa.gain_next != nullptr) gain_pre = bload16(make_rsrc(pa.gain_next, (uint32_t)N * 2u), (uint32_t)no * 2u, 0u);
    }
  }
  if constexpr (RKV) {
    if (own) len_pre = static_cast<int>(bload32(make_rsrc(pa.lengths, (uint32_t)M * 4u), (uint32_t)mo * 4u, 0u));
  }

  // this wave's k-slice of every row (and of the up half for the SiLU gate), requested ahead of the
  // weights
  u32x4_t xw[MR][XW];
  [[maybe_unused]] u32x4_t gw[PRO == kProSiluGate ? MR : 1][XW];
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    if (r < M) {  // wave-uniform
      const rsrc_t rr = make_rsrc(x + static_cast<int64_t>(r) * RS * K, static_cast<uint32_t>(K) * 2u);
#pragma unroll
      for (int i = 0; i < XW; ++i)
        if (i < nx) xw[r][i] = bload128(rr, (uint32_t)(kb0 * KBLK + 8 * (lane + 64 * i)) * 2u, 0u);
      if constexpr (PRO == kProSiluGate) {
        const rsrc_t ru = make_rsrc(x + static_cast<int64_t>(r) * RS * K + K, static_cast<uint32_t>(K) * 2u);
#pragma unroll
        for (int i = 0; i < XW; ++i)
          if (i < nx) gw[r][i] = bload128(ru, (uint32_t)(kb0 * KBLK + 8 * (lane + 64 * i)) * 2u, 0u);
      }
    }
  }
  // kProScaleSum: row r's sums of squares into LDS (buffer loads that write LDS), by wave r mod nw
  [[maybe_unused]] __shared__ __attribute__((aligned(16))) float ss_lds[PRO == kProScaleSum ? MR : 1]
                                                                        [PRO == kProScaleSum ? kNormSumMax : 4];
  [[maybe_unused]] __shared__ float row_scale_lds[MR];
  if constexpr (PRO == kProScaleSum) {
    for (int r = wave; r < M; r += nw) {  // wave-uniform
      const rsrc_t sr = make_rsrc(pa.ss_in + static_cast<int64_t>(r) * pa.nss, (uint32_t)pa.nss * 4u);
#pragma unroll
      for (int i = 0; i < kNormSumMax / 256; ++i)
        if (i * 256 < pa.nss)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void*)(&ss_lds[r][256 * i]), 16,
                                                   (uint32_t)(lane + 64 * i) * 16u, 0, 0, 0);
    }
  }
  // the first weight round is unconditional (blocks past kb1 clamped and unused): the wait before the
  // LDS stores then counts exactly the weight loads still in flight
  u32x4_t w[U];
  typename W::P p[U];
#pragma unroll
  for (int u = 0; u < U; ++u) W::load(wc, min(kb0 + u, kb1 - 1), w[u], p[u]);
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    if (r < M) {
#pragma unroll
      for (int i = 0; i < XW; ++i)
        if (i < nx) {
          u32x4_t v = xw[r][i];
          if constexpr (PRO == kProSiluGate) {  // past K both halves read zero, and silu(0) * 0 = 0
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t g2 = v[j], u2 = gw[r][i][j];
              v[j] = ActBF16::pack_rne(silu_f32(bf16_lo(g2)) * bf16_lo(u2), silu_f32(bf16_hi(g2)) * bf16_hi(u2));
            }
          }
          *reinterpret_cast<u32x4_t*>(xwave + r * pitch + 8 * (lane + 64 * i)) = v;
        }
    }
  }
  // LDS operations of one wave execute in issue order; only the compiler must not move the fragment
  // reads above the stores
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
  if constexpr (RKV) {
    if (own) {  // the pair's cos / sin at the row's position (needed only in the epilogue)
      asm volatile("" : "+v"(len_pre));
      const int pos = min(max(len_pre, 0), pa.rope_rows - 1);
      const uint32_t pi = (uint32_t)(pos * 64 + ((no & 127) >> 1)) * 4u;
      const uint32_t tb = (uint32_t)pa.rope_rows * 64u * 4u;
      cos_pre = __builtin_bit_cast(float, bload32(make_rsrc(pa.cos_t, tb), pi, 0u));
      sin_pre = __builtin_bit_cast(float, bload32(make_rsrc(pa.sin_t, tb), pi, 0u));
    }
  }

  const uint16_t* xfrag = xwave + min(nl, M - 1) * pitch;  // this lane's A row
  const uint32_t one = A::pair_from_f32(1.0f);
  const u32x4_t ones = u32x4_t{one, one, one, one};
  float yv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  auto load_round = [&](int kr, u32x4_t (&wo)[U], typename W::P (&po)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (kr + u < kb1) W::load(wc, kr + u, wo[u], po[u]);  // wave-uniform condition
  };
  for (int kb = kb0; kb < kb1; kb += U) {
    // R1: every wave's k-slice is a single round (kbw <= 4), so no next round is held in registers
    [[maybe_unused]] u32x4_t wn[R1 ? 1 : U];
    [[maybe_unused]] typename W::P pn[R1 ? 1 : U];
    if constexpr (!R1) {
      if (kb + U < kb1) load_round(kb + U, wn, pn);
    }
    // the round's chunk sums per row: A row c = chunk c % 4 of block c / 4 (lane l gets the chunk sums
    // of block l >> 4)
    f32x4_t cs[MR];
    {
      const int c = lane & 15, b = c / CPB;
      const bool live = kb + b < kb1;
#pragma unroll
      for (int r = 0; r < MR; ++r) {
        cs[r] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        if (r < M) {  // wave-uniform
          u32x4_t a2 = u32x4_t{0u, 0u, 0u, 0u};
          if (live)
            a2 = *reinterpret_cast<const u32x4_t*>(xwave + r * pitch + (kb - kb0 + b) * KBLK + 32 * (c % CPB) + 8 * jg);
          cs[r] = A::mfma(a2, ones, cs[r]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (kb + u < kb1) {  // wave-uniform
        const int kk = kb + u;
        u32x4_t xv[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xv[i] = *reinterpret_cast<const u32x4_t*>(xfrag + (kk - kb0) * KBLK + W::xk(i, jg));
          b[i] = W::template bfrag<A>(w[u], i);
        }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = g * MPG; i < (g + 1) * MPG; ++i) acc = A::mfma(xv[i], b[i], acc);
          const float off = W::template offset<A>(p[u], g), sc = W::scale(p[u], g);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (j >= MR) break;  // rows past a two-row build (their outputs are dropped)
            // the group's sum of row j (and of row 4 + j for lane group 1), a wave-uniform value
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int i = 0; i < CPG; ++i) s0 += cs[j][g * CPG + i];
            s0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s0), 16 * u));
            if constexpr (MR == 8) {
#pragma unroll
              for (int i = 0; i < CPG; ++i) s1 += cs[4 + j][g * CPG + i];
              s1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s1), 16 * u));
              s0 = jg == 1 ? s1 : s0;
            }
            yv[j] = fmaf(sc, fmaf(-off, s0, acc[j]), yv[j]);
          }
        }
      }
    }
    if constexpr (R1) {
      break;
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        w[u] = wn[u];
        p[u] = pn[u];
      }
    }
  }

  if constexpr (PRO == kProScaleSum) {
    for (int r = wave; r < M; r += nw) {  // wave-uniform: row r's factor, in the one-row form's order
      wait_vmcnt<0>();  // the copies into LDS (long done: the weights behind them have been consumed)
      asm volatile("" ::: "memory");
      const int ln = static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
      float tt = 0.0f;
#pragma unroll
      for (int i = 0; i < kNormSumMax / 256; ++i)
        if (i * 256 < pa.nss) {
          const f32x4_t v4 = *reinterpret_cast<const f32x4_t*>(&ss_lds[r][256 * i + 4 * ln]);
          tt += (v4[0] + v4[1]) + (v4[2] + v4[3]);
        }
      tt = wave_sum(tt);
      if (lane == 0) row_scale_lds[r] = 1.0f / sqrtf(tt / static_cast<float>(K) + pa.eps);
    }
  }
  // Sum the wave partials in wave order. Float j of a wave's block is (lane l, row r).
  f32x4_t* red = smem;
  red[wave * 64 + lane] = f32x4_t{yv[0], yv[1], yv[2], yv[3]};
  __syncthreads();
  if (jo >= kJ) return;  // whole waves
  const float* rf = reinterpret_cast<const float*>(red);
  float v = 0.0f;
  if (own) {
    for (int ww = 0; ww < nw; ++ww) v += rf[ww * 256 + jo];
    v *= W::out_scale(wa, no);
    if constexpr (PRO == kProScaleSum) v *= row_scale_lds[mo];
  }
  if constexpr (RKV) {
#pragma clang fp contract(off)
    const float xq = A::to_f32(A::from_f32(v));  // the projection's bf16 output
    const float xp = __shfl_xor(xq, 4, 64);      // its RoPE partner (the other dim of the pair, lane ^ 4)
    if (own) {
      const int slot = min(max(len_pre, 0), pa.tmax - 1);
      const int nh = pa.kn >> 7;  // kv heads
      if (no < pa.qn + pa.kn) {
        const float r = (no & 1) ? xp * sin_pre + xq * cos_pre : xq * cos_pre - xp * sin_pre;
        if (no < pa.qn) {
          pa.q_out[static_cast<int64_t>(mo) * pa.qn + no] = A::from_f32(r);
        } else {
          const int kd = no - pa.qn;
          pa.k_cache[((static_cast<int64_t>(mo) * nh + (kd >> 7)) * pa.tmax + slot) * 128 + (kd & 127)] = A::from_f32(r);
        }
      } else {
        const int vd = no - pa.qn - pa.kn;
        pa.v_cache[((static_cast<int64_t>(mo) * nh + (vd >> 7)) * pa.tmax + slot) * 128 + (vd & 127)] = A::from_f32(xq);
      }
    }
    return;
  } else if constexpr (RES) {
    float hsq = 0.0f;
    asm volatile("" : "+v"(res_pre), "+v"(gain_pre));
    if (own) {
      if (bias) v += A::to_f32(bias[no]);
      const float rv = A::to_f32(static_cast<uint16_t>(res_pre));
      const float h = A::to_f32(A::from_f32(rv + A::to_f32(A::from_f32(v))));
      pa.res_out[static_cast<int64_t>(mo) * N + no] = A::from_f32(h);
      if (pa.gain_next != nullptr)
        pa.hg_out[static_cast<int64_t>(mo) * N + no] = A::from_f32(h * A::to_f32(static_cast<uint16_t>(gain_pre)));
      hsq = h * h;
    }
    // the tile's 16 outputs of row mo sit in lanes 4 nl + e of this wave: a fixed shuffle tree
    hsq += __shfl_xor(hsq, 4, 64);
    hsq += __shfl_xor(hsq, 8, 64);
    hsq += __shfl_xor(hsq, 16, 64);
    hsq += __shfl_xor(hsq, 32, 64);
    if (((jo >> 2) & 15) == 0 && mo < M) pa.ss_out[static_cast<int64_t>(mo) * T + t] = hsq;
  } else if constexpr (SWI) {
    // output no's up row no + 8 is thread jo ^ 32 (same row mo), in this wave
    if (own && bias) v += A::to_f32(bias[no]);
    const float q = own ? A::to_f32(A::from_f32(v)) : 0.0f;
    const float u = __shfl_xor(q, 32, 64);
    if (own && ((jo >> 2) & 8) == 0)
      y[static_cast<int64_t>(mo) * (N / 2) + t * 8 + ((jo >> 2) & 7)] =
          static_cast<uint16_t>(A::pack_rne(silu_f32(q) * u, 0.0f));
  } else {
    if (own) {
      if (bias) v += A::to_f32(bias[no]);
      y[static_cast<int64_t>(mo) * N + no] = A::from_f32(v);
    }
  }
}

// Waves per tile of the multi-row form: one round of four blocks per wave up to 16 waves (the one-row
// rule), so k-slices grow past four blocks only beyond 64 blocks.
inline int gemv_rows_default_waves(int64_t rows, int64_t cols) {
  const int64_t KB = ceil_div(cols, 128);
  return static_cast<int>(std::min<int64_t>(16, std::max<int64_t>(1, ceil_div(KB, 4))));
}

// LDS bytes of the multi-row form for a launch of nw waves over k-slices of kbw blocks (dynamic, plus
// the row factor's sums in the kProScaleSum form).
inline size_t gemv_rows_lds_bytes(int64_t m, int nw, int kbw, bool scale_sum = false) {
  const int MR = m <= 2 ? 2 : (m <= 4 ? 4 : 8);
  const int nx = (kbw * 16 + 63) / 64;
  return static_cast<size_t>(nw) * 64 * sizeof(f32x4_t) + static_cast<size_t>(nw) * MR * (nx * 512 + 32) * 2 +
         (scale_sum ? static_cast<size_t>(MR) * (kNormSumMax + 1) * 4 : 0);
}

// Row groups of the multi-row form for m rows (groups = 0: the library's choice): 1 (one workgroup per
// tile, MR = 4 for m <= 4, MR = 8 above) or 2 (5..8 rows: two workgroups of four rows per tile).
// Whether it takes m rows of a [rows, cols] weight with nw waves per tile (0: default); scale_sum: the
// row factor's form. Returns the row groups it runs (0 when it does not fit).
inline int gemv_rows_groups(int64_t m, int64_t rows, int64_t cols, int nw = 0, bool scale_sum = false, int groups = 0) {
  if (m < 2 || m > 8 || rows <= 0 || cols <= 0 || groups < 0 || groups > 2) return 0;
  const int64_t KB = ceil_div(cols, 128);
  if (nw <= 0) nw = gemv_rows_default_waves(rows, cols);
  if (nw > 16) return 0;
  if (nw > KB) nw = static_cast<int>(KB);
  const int kbw = static_cast<int>(ceil_div(KB, nw));
  nw = static_cast<int>(ceil_div(KB, kbw));
  // four rows (or two groups of four): k-slices of up to 8 blocks
  const bool four = kbw <= 8 && gemv_rows_lds_bytes(4, nw, kbw, scale_sum) <= 160 * 1024;
  if (m <= 4) return (groups <= 1 && four) ? 1 : 0;
  // eight rows in one workgroup: k-slices of up to 4 blocks, and two waves at least (the epilogue's
  // outputs of rows 4..7 are threads 64..127)
  const bool eight = kbw <= 4 && nw >= 2 && gemv_rows_lds_bytes(8, nw, kbw, scale_sum) <= 160 * 1024;
  if (groups == 1) return eight ? 1 : 0;
  if (groups == 2) return four ? 2 : 0;
  // the library's choice: eight rows in one workgroup where they fit (its single-round build, at
  // most 97 VGPRs, beat two groups of four on 4096->1024 at 6 / 8 rows: 4.39 / 4.42 -> 4.16 / 4.32 us
  // with rotating weights), else two groups on small grids only: 4096->28672 at 6 / 8 rows took
  // 24.9 / 26.5 us in two groups, and 14336->4096 (where eight rows do not fit) 17.6 us against
  // 12.3 us on the row-tiled kernel, as the second workgroup of a tile does not find the weights in
  // L2 often enough on larger grids.
  if (eight) return 1;
  return (four && ceil_div(rows, 16) <= 64) ? 2 : 0;
}

inline bool gemv_rows_fits(int64_t m, int64_t rows, int64_t cols, int nw = 0, bool scale_sum = false) {
  return gemv_rows_groups(m, rows, cols, nw, scale_sum) != 0;
}

template <class A, class W, int PRO = kProPlain, bool RES = false, bool RKV = false, bool SWI = false>
hipError_t gemv_rows_launch(const typename W::Args& wa, const uint16_t* x, uint16_t* y, const uint16_t* bias,
                            int64_t m, int64_t rows, int64_t cols, int waves, hipStream_t stream,
                            const ProArgs& pa = ProArgs{nullptr, nullptr, nullptr, 0.0f}, int groups = 0) {
  const int rgs = gemv_rows_groups(m, rows, cols, waves, PRO == kProScaleSum, groups);
  if (rgs == 0) return hipErrorNotSupported;
  const int64_t T = ceil_div(rows, 16);
  const int64_t KB = ceil_div(cols, 128);
  int nw = waves > 0 ? waves : gemv_rows_default_waves(rows, cols);
  if (nw > KB) nw = static_cast<int>(KB);
  const int kbw = static_cast<int>(ceil_div(KB, nw));
  nw = static_cast<int>(ceil_div(KB, kbw));
  const bool eight = m > 4 && rgs == 1;
  const bool two = m <= 2 && rgs == 1;  // the two-row build: 92-96 VGPRs against 104-112, half the LDS slice
  const size_t lds = gemv_rows_lds_bytes(eight ? 8 : (two ? 2 : 4), nw, kbw);  // the row factor's sums are static LDS
  const dim3 block(static_cast<unsigned>(64 * nw));
  const int M = static_cast<int>(m), N = static_cast<int>(rows), K = static_cast<int>(cols), iKB = static_cast<int>(KB);
  // columns at or past K (a k tail) read zero through the row resources, so the padded blocks need no
  // masking
  if (SWI && rows % 16 != 0) return hipErrorNotSupported;  // whole gate / up tiles
  if (rgs == 2)
    hipLaunchKernelGGL((gemv_rows_kernel<A, W, 4, 2, PRO, RES, RKV, 2, SWI>),
                       dim3(static_cast<unsigned>(ceil_div(T, 8) * 16)), block, lds, stream, wa, x, y, bias, M, N, K, iKB,
                       kbw, pa);
  else if (two && kbw <= 4)
    hipLaunchKernelGGL((gemv_rows_kernel<A, W, 2, 1, PRO, RES, RKV, 1, SWI, true>), dim3(static_cast<unsigned>(T)), block,
                       lds, stream, wa, x, y, bias, M, N, K, iKB, kbw, pa);
  else if (two)
    hipLaunchKernelGGL((gemv_rows_kernel<A, W, 2, 2, PRO, RES, RKV, 1, SWI>), dim3(static_cast<unsigned>(T)), block, lds,
                       stream, wa, x, y, bias, M, N, K, iKB, kbw, pa);
  else if (!eight && kbw <= 4)
    hipLaunchKernelGGL((gemv_rows_kernel<A, W, 4, 1, PRO, RES, RKV, 1, SWI, true>), dim3(static_cast<unsigned>(T)), block,
                       lds, stream, wa, x, y, bias, M, N, K, iKB, kbw, pa);
  else if (!eight)
    hipLaunchKernelGGL((gemv_rows_kernel<A, W, 4, 2, PRO, RES, RKV, 1, SWI>), dim3(static_cast<unsigned>(T)), block, lds,
                       stream, wa, x, y, bias, M, N, K, iKB, kbw, pa);
  else
    hipLaunchKernelGGL((gemv_rows_kernel<A, W, 8, 1, PRO, RES, RKV, 1, SWI, true>), dim3(static_cast<unsigned>(T)), block,
                       lds, stream, wa, x, y, bias, M, N, K, iKB, kbw, pa);
  return hipGetLastError();
}

}  // namespace sqx
