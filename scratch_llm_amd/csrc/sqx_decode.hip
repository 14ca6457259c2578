// The non-linear ops of one Llama-shaped decode step, fused for MI355X. They are
// the callers around the quantized linears in src/scratch_llm/model.py: RMSNorm (:148-162), the
// residual adds of TransformerBlock.forward (:394-403), RoPE (:185-224), SwiGLU's gate (:227-237),
// decode attention against a slot KV cache (:262-366 with kv_cache.py:80-262) and the greedy pick of
// sampling.py:80-86.
//
// Layouts: activation rows are bf16 [B, width]. The KV cache of one layer is two bf16 tensors
// [B, Hkv, Tmax, hd] (kv_cache.py:234-262, BatchedKVCache). lengths[b] (int32) is the number of
// valid positions of slot b before this step's write (kv_cache.py:126): the new key/value lands at
// min(lengths[b], Tmax - 1), RoPE uses position lengths[b], and the row attends keys
// j <= lengths[b] (write-then-mask, model.py:293-305). All arithmetic is fp32; each written tensor
// is rounded to bf16 once (round to nearest even).
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "sqx_common.h"

namespace sqx {

// ---------------------------------------------------------------------------------------------
// Residual add + RMSNorm. With delta: h = bf16(x + delta) is written to h_out and normalised;
// without: h = x. y = bf16(h * (1 / sqrt(mean(h^2) + eps)) * w), the product taken left to right in
// fp32 as model.py:158-162 does. One workgroup of 256 threads per row; d % 8 == 0, d <= 16384.
// PART: delta is the bf16 rounding of the sum, in split order, of S fp32 partials [S][rows][d] at
// part (a K-split linear's workspace), exactly as that linear's own reduce would have written it.
// ---------------------------------------------------------------------------------------------
template <int NCH, bool PART = false, int PS = 0>  // PS: the split count when known at compile time
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ delta,
                                                      const uint16_t* __restrict__ w, float eps, int d,
                                                      uint16_t* __restrict__ h_out, uint16_t* __restrict__ y,
                                                      const float* __restrict__ part = nullptr, int S = 0,
                                                      int64_t pstride = 0) {
  // Thread t owns columns 8t + 2048i (i < NCH): every load of the row, the delta and the gain is
  // issued before the first use, and the row stays in registers between the two passes.
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  u32x4_t v[NCH], wv[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = tid * 8 + i * 2048;
    if (c < d) {
      v[i] = *reinterpret_cast<const u32x4_t*>(x + row * d + c);
      wv[i] = *reinterpret_cast<const u32x4_t*>(w + c);
    }
  }
  if (PART || delta != nullptr) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid * 8 + i * 2048;
      if (c < d) {
        u32x4_t dv;
        if constexpr (PART) {
          const float* p0 = part + row * d + c;
          f32x4_t a = *reinterpret_cast<const f32x4_t*>(p0), b = *reinterpret_cast<const f32x4_t*>(p0 + 4);
          if constexpr (PS > 1) {  // every split's loads in flight together, then the sums in order
            f32x4_t pa[PS - 1], pb[PS - 1];
#pragma unroll
            for (int s = 1; s < PS; ++s) {
              pa[s - 1] = *reinterpret_cast<const f32x4_t*>(p0 + s * pstride);
              pb[s - 1] = *reinterpret_cast<const f32x4_t*>(p0 + s * pstride + 4);
            }
#pragma unroll
            for (int s = 1; s < PS; ++s)
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                a[j] += pa[s - 1][j];
                b[j] += pb[s - 1][j];
              }
          } else {
            for (int s = 1; s < S; ++s) {
              const f32x4_t a2 = *reinterpret_cast<const f32x4_t*>(p0 + s * pstride);
              const f32x4_t b2 = *reinterpret_cast<const f32x4_t*>(p0 + s * pstride + 4);
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                a[j] += a2[j];
                b[j] += b2[j];
              }
            }
          }
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            dv[j] = static_cast<uint32_t>(f32_to_bf16_bits(a[2 * j])) |
                    (static_cast<uint32_t>(f32_to_bf16_bits(a[2 * j + 1])) << 16);
            dv[2 + j] = static_cast<uint32_t>(f32_to_bf16_bits(b[2 * j])) |
                        (static_cast<uint32_t>(f32_to_bf16_bits(b[2 * j + 1])) << 16);
          }
        } else {
          dv = *reinterpret_cast<const u32x4_t*>(delta + row * d + c);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[i][j] = ActBF16::pack_rne(bf16_lo(v[i][j]) + bf16_lo(dv[j]), bf16_hi(v[i][j]) + bf16_hi(dv[j]));
        *reinterpret_cast<u32x4_t*>(h_out + row * d + c) = v[i];
      }
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    if (tid * 8 + i * 2048 < d) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a0 = bf16_lo(v[i][j]), a1 = bf16_hi(v[i][j]);
        ss = fmaf(a0, a0, ss);
        ss = fmaf(a1, a1, ss);
      }
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  const float r = 1.0f / sqrtf(total / static_cast<float>(d) + eps);
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int c = tid * 8 + i * 2048;
    if (c < d) {
      u32x4_t o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = ActBF16::pack_rne(bf16_lo(v[i][j]) * r * bf16_lo(wv[i][j]), bf16_hi(v[i][j]) * r * bf16_hi(wv[i][j]));
      *reinterpret_cast<u32x4_t*>(y + row * d + c) = o;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// RoPE + KV-cache write. The fused projection row is qkv = [q (H*hd) | k (Hkv*hd) | v (Hkv*hd)].
// Pair (x_2i, x_2i+1) of a q or k head becomes (x_2i cos - x_2i+1 sin, x_2i sin + x_2i+1 cos) with
// cos/sin the fp32 tables [rope_rows, hd/2] at position lengths[b] (model.py:196-224; the products
// and sums are separate fp32 roundings, as the reference's tensor ops are). q goes to q_out
// [B, H, hd]; k and v go into the cache at min(lengths[b], Tmax - 1). One thread per pair.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rope_kv_kernel(const uint16_t* __restrict__ qkv, const int* __restrict__ lengths,
                                                      const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                                      int rope_rows, int H, int Hkv, int hd, int tmax,
                                                      uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
                                                      uint16_t* __restrict__ vc) {
#pragma clang fp contract(off)
  const int b = blockIdx.y;
  const int width = (H + 2 * Hkv) * hd;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (2 * i >= width) return;
  const int len = lengths[b];
  const int p = min(max(len, 0), rope_rows - 1);
  const int slot = min(max(len, 0), tmax - 1);
  const uint32_t two = *reinterpret_cast<const uint32_t*>(qkv + static_cast<int64_t>(b) * width + 2 * i);
  const int head = (2 * i) / hd, c = (2 * i) % hd;
  if (head < H + Hkv) {
    const float x0 = bf16_lo(two), x1 = bf16_hi(two);
    const float cs = cos_t[static_cast<int64_t>(p) * (hd / 2) + c / 2];
    const float sn = sin_t[static_cast<int64_t>(p) * (hd / 2) + c / 2];
    const float e = x0 * cs - x1 * sn;
    const float o = x0 * sn + x1 * cs;
    const uint32_t r = ActBF16::pack_rne(e, o);
    if (head < H) {
      *reinterpret_cast<uint32_t*>(q_out + (static_cast<int64_t>(b) * H + head) * hd + c) = r;
    } else {
      const int64_t at = ((static_cast<int64_t>(b) * Hkv + (head - H)) * tmax + slot) * hd + c;
      *reinterpret_cast<uint32_t*>(kc + at) = r;
    }
  } else {
    const int64_t at = ((static_cast<int64_t>(b) * Hkv + (head - H - Hkv)) * tmax + slot) * hd + c;
    *reinterpret_cast<uint32_t*>(vc + at) = two;
  }
}

// ---------------------------------------------------------------------------------------------
// Decode attention, split over the keys (flash decoding). softmax(q k^T / sqrt(hd)) v over the keys
// j <= lengths[b] of kv head kh for its G = H / Hkv query heads (GQA: query head h reads kv head
// h / G, the repeat_interleave of model.py:315-318).
//
// Workgroup (chunk, kh, b) takes keys [chunk*C, chunk*C + C) and writes, per query head, the fp32
// partial (m, l, o[hd]) of that range: m the maximum score (log2 units: scores are scaled by
// log2(e) / sqrt(hd) so that the exponentials are exp2), l = sum 2^(s - m), o = sum 2^(s - m) v.
// The NWV waves (4, or 8 for the o projection's fused merge) take alternate blocks of 16 keys (the
// kernel and its layouts are described at attn_partial_mfma_kernel below); the waves' partials are
// merged at the end. hd must be 128.
//
// Partial layout in the workspace (16-byte aligned rows): o at po[((b*H + h)*nchunk + c)*hd + d], then
// (m, l) at pml[((b*H + h)*nchunk + c)*2 + {0, 1}] with pml = po + B*H*nchunk*hd. The merge of a
// head's chunks follows attn_chunk_weight (sqx_common.h) in ascending chunk order, shared by
// attn_combine_kernel and the o projection's prologue (kProAttnCombine in sqx_gemv.h).
// ---------------------------------------------------------------------------------------------
constexpr int kHd = 128;
constexpr int kKeysPerStep = 16;

// RoPE of one lane's 8 consecutive dims (4 pairs) with the pair's cos/sin, rounded to bf16 as the
// reference's rotated q and k are (separate fp32 products and sums, model.py:218-224).
__device__ inline u32x4_t rope8(u32x4_t v, const float (&cs)[4], const float (&sn)[4]) {
#pragma clang fp contract(off)
  u32x4_t r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float x0 = bf16_lo(v[j]), x1 = bf16_hi(v[j]);
    r[j] = ActBF16::pack_rne(x0 * cs[j] - x1 * sn[j], x0 * sn[j] + x1 * cs[j]);
  }
  return r;
}

// One lane's 8 dims of a cache row: 16 bytes of bf16, or 8 bytes of E4M3 codes (KV8).
template <bool KV8>
struct KvRow;
template <>
struct KvRow<false> {
  using T = u32x4_t;
  static constexpr int kBytes = 2;  // per element
};
template <>
struct KvRow<true> {
  using T = u32x2v_t;
  static constexpr int kBytes = 1;
  __device__ static void to_f32(const T& r, float (&f)[8]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const f32x2_t a = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(r[j]), false);
      const f32x2_t b = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(r[j]), true);
      f[4 * j] = a[0];
      f[4 * j + 1] = a[1];
      f[4 * j + 2] = b[0];
      f[4 * j + 3] = b[1];
    }
  }
  // E4M3 codes of 8 bf16 values divided by the head's scale (quantize_per_head, fp8_kv_per_head.py:93-96)
  __device__ static T encode(const u32x4_t& v, float s) {
    T r;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t c0 = e4m3_encode_sat(__fdiv_rn(bf16_lo(v[2 * j]), s));
      const uint32_t c1 = e4m3_encode_sat(__fdiv_rn(bf16_hi(v[2 * j]), s));
      const uint32_t c2 = e4m3_encode_sat(__fdiv_rn(bf16_lo(v[2 * j + 1]), s));
      const uint32_t c3 = e4m3_encode_sat(__fdiv_rn(bf16_hi(v[2 * j + 1]), s));
      r[j] = c0 | (c1 << 8) | (c2 << 16) | (c3 << 24);
    }
    return r;
  }
};

// 8 E4M3 codes (two dwords, code e in byte e) as 4 dwords of bf16 pairs in the same order; every
// E4M3 value is exact in bf16.
__device__ inline u32x4_t e4m3x8_to_bf16(u32x2v_t c) {
  u32x4_t r;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t w = c[h];  // through a scalar: hipcc's element access of a vector value
    r[2 * h] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
    r[2 * h + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
  }
  return r;
}

// The same partials with the scores on the matrix unit. Per 16 keys a wave computes
// S^T = K Q^T as four v_mfma_f32_16x16x32_bf16 (A: the 16 key rows, lane l holding dims
// 32i + 8 (l / 16) .. +8 of key l % 16; B: the G query heads as columns, zero past G; products exact,
// fp32 sums), so lane l gets the scores of keys 4 (l / 16) + j (j < 4) for head l % 16. The softmax
// runs in that layout: the step maximum of a head is shared by its four lane groups, so m is the
// same in every lane of a head and the running l sums stay per lane until the end. The exponentials
// p go through the wave's own LDS rows to the value layout of the VALU accumulation (lane group kl
// holds value rows base + 4u + kl, each lane 8 dims, fp32 products and sums as above). This moves
// the dot products and most of the softmax off the VALU, which bounds the kernel above at large
// batch (every lane worked every head's scores, 4 fdot2 and 4 row reductions a key).
template <int G, bool ROPE, bool KV8, int NWV, bool QP = false>
__global__ __launch_bounds__(NWV * 64) __attribute__((amdgpu_waves_per_eu(2))) void attn_partial_mfma_kernel(const uint16_t* __restrict__ q, uint8_t* __restrict__ kc,
                                                                uint8_t* __restrict__ vc, const int* __restrict__ lengths,
                                                                const float* __restrict__ cos_t,
                                                                const float* __restrict__ sin_t,
                                                                const float* __restrict__ kscale,
                                                                const float* __restrict__ vscale, int rope_rows, int H,
                                                                int Hkv, int tmax, int chunk, int nchunk, float qscale,
                                                                float* __restrict__ po, float* __restrict__ pml,
                                                                uint16_t* __restrict__ out,
                                                                const float* __restrict__ qpart, int qsplits) {
  static_assert(G >= 1 && G <= 16, "query heads are the 16 columns of the score tile");
  static_assert(NWV == 4 || NWV == 8, "4 or 8 waves per workgroup");
  using R = KvRow<KV8>;
  using Row = typename R::T;          // a lane's 8 dims of a cache row: 16 bytes bf16, 8 bytes E4M3
  constexpr uint32_t ES = R::kBytes;  // bytes per element
  const int ch = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kl = lane >> 4, dl = lane & 15;  // value layout: key group, 8-dim slice; score layout: key quad, head
  const int t0 = ch * chunk;
  // the NWV waves take alternate 16-key blocks of the chunk: the workgroup streams one region
  const int ws = t0 + wave * kKeysPerStep;
  constexpr int kWaveStride = NWV * kKeysPerStep;
  const int64_t head_off = (static_cast<int64_t>(b) * Hkv + kh) * tmax * kHd * ES;  // bytes

  // Two register sets in turn: block base + stride is requested before block base is worked on
  // (loads past the range read zero from the buffer resources, so every iteration issues the same
  // loads and the waits are exact counts)
  auto load_block = [&](const rsrc_t& kr, const rsrc_t& vrs, int lim, int bs, Row (&ko)[4], Row (&vo_)[4]) {
    const int kq = bs + dl;
    const uint32_t kt = kq < lim ? static_cast<uint32_t>(kq) : 0xFFFFFFu;  // past the range: zero rows (score masked)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (KV8) ko[i] = bload64<2>(kr, kt * kHd + 8u * kl, 32u * i);
      else ko[i] = bload128<2>(kr, kt * (kHd * 2u) + 16u * kl, 64u * i);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int tv = bs + 4 * u + kl;  // rows past the wave's range read as zero (weight 0 meets no NaN)
      const uint32_t vo = (tv < lim ? static_cast<uint32_t>(tv) : 0xFFFFFFu) * (kHd * ES) + 8u * ES * dl;
      if constexpr (KV8) vo_[u] = bload64<2>(vrs, vo, 0u);
      else vo_[u] = bload128<2>(vrs, vo, 0u);
    }
  };
  // The wave's first block is requested before the row's length is known, through resources that end
  // at tmax: its rows at or past the length (unwritten cache rows, possibly NaN) are masked where they
  // are used (scores to -inf, value rows to zero). Later blocks read through resources that end at
  // the length, so their rows past it read as zero.
  Row ka[4], va[4], kb[4], vb[4];
  {
    const rsrc_t kt0 = make_rsrc(kc + head_off, static_cast<uint32_t>(tmax) * kHd * ES);
    const rsrc_t vt0 = make_rsrc(vc + head_off, static_cast<uint32_t>(tmax) * kHd * ES);
    load_block(kt0, vt0, min(t0 + chunk, tmax), ws, ka, va);
  }
  const int width = (ROPE ? H + 2 * Hkv : H) * kHd;
  const uint16_t* qrow = q + static_cast<int64_t>(b) * width;
  // rows(cols, v): v[n] = the 8 consecutive values of the row from column cols[n], as bf16 pairs,
  // every load issued before the first use. QP (with ROPE): the q|k|v row is the sum of the qsplits
  // fp32 partials [S][B][width] of a K-split projection, added in split order and rounded to bf16 as
  // skinny_reduce_kernel does (the bits that reduce writes); the first two partials load together
  // with no branch between them (for S = 1 the second, read at stride 0, is dropped by a select), so
  // up to two splits cost one round trip.
  auto rows = [&](const auto& cols, auto& v) {
    constexpr int N = std::extent<std::remove_reference_t<decltype(cols)>>::value;
    if constexpr (!QP) {
#pragma unroll
      for (int n = 0; n < N; ++n) v[n] = *reinterpret_cast<const u32x4_t*>(qrow + cols[n]);
    } else {
      const int64_t stride = static_cast<int64_t>(gridDim.z) * width;
      const float* p = qpart + static_cast<int64_t>(b) * width;
      const bool two = qsplits > 1;
      const float* p1 = p + (two ? stride : 0);
      f32x4_t a[N][2], c[N][2];
#pragma unroll
      for (int n = 0; n < N; ++n)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          a[n][h] = *reinterpret_cast<const f32x4_t*>(p + cols[n] + 4 * h);
          c[n][h] = *reinterpret_cast<const f32x4_t*>(p1 + cols[n] + 4 * h);
        }
#pragma unroll
      for (int n = 0; n < N; ++n)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int j = 0; j < 4; ++j) a[n][h][j] = two ? a[n][h][j] + c[n][h][j] : a[n][h][j];
      for (int sp = 2; sp < qsplits; ++sp) {
#pragma unroll
        for (int n = 0; n < N; ++n)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const f32x4_t d = *reinterpret_cast<const f32x4_t*>(p + sp * stride + cols[n] + 4 * h);
#pragma unroll
            for (int j = 0; j < 4; ++j) a[n][h][j] += d[j];
          }
      }
#pragma unroll
      for (int n = 0; n < N; ++n)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4_t& x = a[n][j >> 1];
          v[n][j] = static_cast<uint32_t>(f32_to_bf16_bits(x[2 * (j & 1)])) |
                    (static_cast<uint32_t>(f32_to_bf16_bits(x[2 * (j & 1) + 1])) << 16);
        }
    }
  };
  // The query slices and (ROPE, wave 0) the new key and value rows are requested with the first block,
  // before the row's length is known; only RoPE's tables depend on it.
  u32x4_t qv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) qv[i] = u32x4_t{0u, 0u, 0u, 0u};
  if (dl < G) {
    int cq[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) cq[i] = (kh * G + dl) * kHd + 32 * i + 8 * kl;
    rows(cq, qv);
  }
  [[maybe_unused]] u32x4_t kv16[2] = {u32x4_t{0u, 0u, 0u, 0u}, u32x4_t{0u, 0u, 0u, 0u}};
  if constexpr (ROPE) {
    if (wave == 0 && kl == 0) {
      const int ckv[2] = {(H + kh) * kHd + dl * 8, (H + Hkv + kh) * kHd + dl * 8};
      rows(ckv, kv16);
    }
  }
  const int len = max(lengths[b], 0);
  const int L = min(len + 1, tmax);
  const int slot = min(len, tmax - 1);
  if (t0 >= L) return;  // the combine reads only chunks below L
  const int we = min(t0 + chunk, L);

  __shared__ float sm[NWV][G], sl[NWV][G];
  __shared__ float so[NWV][G][kHd];
  __shared__ __attribute__((aligned(16))) float sp[NWV][16][G < 4 ? 4 : G];  // per wave: p[key][head]
  __shared__ __attribute__((aligned(16))) float sa[NWV][G < 4 ? 4 : G];      // per wave: the step's rescale

  // E4M3 rows: the K scale folds into the query's scale, the V scale multiplies the partial
  const float ks = KV8 ? kscale[kh] : 1.0f;
  const float vs = KV8 ? vscale[kh] : 1.0f;
  const float qs = qscale * ks;
  const int64_t pr = ROPE ? static_cast<int64_t>(min(len, rope_rows - 1)) * (kHd / 2) : 0;
  // the query heads as the B operand: lane l holds dims 32i + 8 kl .. +8 of head dl (zero past G)
  if (dl < G) {
    if constexpr (ROPE) {
      float cs[4][4], sn[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          cs[i][j] = cos_t[pr + 16 * i + 4 * kl + j];
          sn[i][j] = sin_t[pr + 16 * i + 4 * kl + j];
        }
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = rope8(qv[i], cs[i], sn[i]);
    }
  }
  // ROPE: the new key and value in the value layout (dims 8 dl .. +8); the workgroup holding the
  // slot writes them to the cache; the key and value (kept in LDS, the key as stored) stand in for
  // the slot row below
  __shared__ Row knew_lds[ROPE ? 16 : 1], vnew_lds[ROPE ? 16 : 1];
  if constexpr (ROPE) {
    float cs[4], sn[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      cs[j] = cos_t[pr + dl * 4 + j];
      sn[j] = sin_t[pr + dl * 4 + j];
    }
    if (wave == 0 && kl == 0) {
      const u32x4_t kb16 = rope8(kv16[0], cs, sn);
      const u32x4_t vb16 = kv16[1];
      Row knew, vnew;
      if constexpr (KV8) {  // quantized with the head's scales, as the cache stores them
        knew = R::encode(kb16, ks);
        vnew = R::encode(vb16, vs);
      } else {
        knew = kb16;
        vnew = vb16;
      }
      knew_lds[dl] = knew;
      vnew_lds[dl] = vnew;
      if (ch == slot / chunk) {  // one cache row each, from this workgroup only
        *reinterpret_cast<Row*>(kc + head_off + (static_cast<int64_t>(slot) * kHd + dl * 8) * ES) = knew;
        *reinterpret_cast<Row*>(vc + head_off + (static_cast<int64_t>(slot) * kHd + dl * 8) * ES) = vnew;
      }
    }
    __syncthreads();
  }
  // the rows below L as buffer resources (streaming loads: each row is read once); loads of rows past
  // them return zero
  const rsrc_t kr = make_rsrc(kc + head_off, static_cast<uint32_t>(L) * kHd * ES);
  const rsrc_t vrs = make_rsrc(vc + head_off, static_cast<uint32_t>(L) * kHd * ES);
  float m = -INFINITY, l = 0.0f;  // score layout: head dl's running max (same in its 4 lane groups), lane's l
  float o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) o[g][j] = 0.0f;

  auto process = [&](int base, const Row (&kraw)[4], const Row (&vraw)[4]) {
    const int kk = base + dl;
    u32x4_t kf[4];
    Row vr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (KV8) kf[i] = e4m3x8_to_bf16(kraw[i]);  // E4M3 keys to bf16 pairs (exact) for the MFMA
      else kf[i] = kraw[i];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) vr[u] = vraw[u];
    if (base == ws) {  // wave-uniform: the first block was read up to tmax
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (base + 4 * u + kl >= we) vr[u] = Row{};
    }
    if constexpr (ROPE) {
      if (slot >= base && slot < base + kKeysPerStep) {  // wave-uniform: this step holds the new key
        if (kk == slot) {  // dims 32 i + 8 kl .. +8 of the new key as stored (E4M3: the code, read back)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if constexpr (KV8) kf[i] = e4m3x8_to_bf16(knew_lds[4 * i + kl]);
            else kf[i] = knew_lds[4 * i + kl];
          }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (base + 4 * u + kl == slot) vr[u] = vnew_lds[dl];
      }
    }
    f32x4_t sc{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) sc = ActBF16::mfma(kf[i], qv[i], sc);
    // score layout: keys base + 4 kl + j of head dl
    float s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = base + 4 * kl + j < we ? sc[j] * qs : -INFINITY;
    float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mn = fmaxf(m, mx);
    // a head whose keys are all masked so far keeps m = -inf and adds nothing
    const float a = mn == -INFINITY ? 1.0f : exp2f(m - mn);
    float p[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] = s[j] == -INFINITY ? 0.0f : exp2f(s[j] - mn);
    l = fmaf(l, a, (p[0] + p[1]) + (p[2] + p[3]));
    m = mn;
    if (dl < G) {
#pragma unroll
      for (int j = 0; j < 4; ++j) sp[wave][4 * kl + j][dl] = p[j];
      if (kl == 0) sa[wave][dl] = a;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's own rows are written before it reads them
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    float pv[4][G], av[G];
#pragma unroll
    for (int g = 0; g < G; ++g) av[g] = sa[wave][g];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int g = 0; g < G; ++g) pv[u][g] = sp[wave][4 * u + kl][g];
    __builtin_amdgcn_wave_barrier();  // and the next step's writes after these reads
    asm volatile("" ::: "memory");
    float vf[KV8 ? 4 : 1][8];  // E4M3 values to fp32 once per step (exact)
    if constexpr (KV8) {
#pragma unroll
      for (int u = 0; u < 4; ++u) R::to_f32(vr[u], vf[u]);
    }
    auto vval = [&](int u, int j) -> float {
      if constexpr (KV8) return vf[u][j];
      else return (j & 1) ? bf16_hi(vr[u][j >> 1]) : bf16_lo(vr[u][j >> 1]);
    };
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float e = o[g][j] * av[g];
#pragma unroll
        for (int u = 0; u < 4; ++u) e = fmaf(pv[u][g], vval(u, j), e);
        o[g][j] = e;
      }
    }
  };
  for (int base = ws; base < we; base += 2 * kWaveStride) {
    load_block(kr, vrs, we, base + kWaveStride, kb, vb);
    process(base, ka, va);
    if (base + kWaveStride >= we) break;  // wave-uniform
    load_block(kr, vrs, we, base + 2 * kWaveStride, ka, va);
    process(base + kWaveStride, kb, vb);
  }
  // the lane groups of the wave: m is already common to a head's lanes, so l and o simply add
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o[g][j] += __shfl_xor(o[g][j], 16, 64);
      o[g][j] += __shfl_xor(o[g][j], 32, 64);
    }
  if (kl == 0) {
    if (dl < G) {
      sm[wave][dl] = m;
      sl[wave][dl] = l;
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < 8; ++j) so[wave][g][dl * 8 + j] = o[g][j];
  }
  __syncthreads();
  // merge the NWV waves: thread (g, dd) writes element dd of head g's partial
  for (int idx = threadIdx.x; idx < G * kHd; idx += NWV * 64) {
    const int g = idx / kHd, dd = idx % kHd;
    float M = sm[0][g];
#pragma unroll
    for (int w = 1; w < NWV; ++w) M = fmaxf(M, sm[w][g]);
    float lsum = 0.0f, osum = 0.0f;
#pragma unroll
    for (int w = 0; w < NWV; ++w) {
      const float a = sm[w][g] == -INFINITY ? 0.0f : exp2f(sm[w][g] - M);
      lsum = fmaf(sl[w][g], a, lsum);
      osum = fmaf(so[w][g][dd], a, osum);
    }
    const int64_t row = (static_cast<int64_t>(b) * H + kh * G + g) * nchunk + ch;
    const float ov = KV8 ? osum * vs : osum;
    if (out != nullptr) {
      // one chunk holds every key of the row: attn_combine_kernel's arithmetic for a single chunk
      // (its maximum drops a NaN m for -inf; weight, fma into zero, division), so the output is
      // bit-identical to the partial followed by the combine
      const float a = attn_chunk_weight(M, fmaxf(M, -INFINITY));
      out[row * kHd + dd] = f32_to_bf16_bits(fmaf(ov, a, 0.0f) / fmaf(lsum, a, 0.0f));
    } else {
      if (dd == 0) *reinterpret_cast<f32x2_t*>(pml + row * 2) = f32x2_t{M, lsum};
      po[row * kHd + dd] = ov;
    }
  }
}

// out[b, h*hd + d] = bf16(sum_c 2^(m_c - M) o_c[d] / sum_c 2^(m_c - M) l_c) over the chunks c that
// hold keys of row b, merged as attn_chunk_weight describes, in ascending chunk order. Row layout [B, H*hd] is the
// (B, 1, H*hd) view that o_proj takes (model.py:365). One workgroup of 128 threads per (head, row),
// one output element per thread.
constexpr int kMaxChunks = 1024;

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Every load is requested at the start: the o values of the first kCombineBatch chunks (past nchunk the
// buffer resource reads zero) before the row's length is known, one chunk's (m, l) per thread. The
// chunk weights go through LDS; the sums then run over the chunks in ascending order with the results
// past the length dropped by selects (those chunks were never written).
constexpr int kCombineBatch = 32;
__global__ __launch_bounds__(128) void attn_combine_kernel(const float* __restrict__ po, const float* __restrict__ pml,
                                                           const int* __restrict__ lengths, int H, int tmax, int chunk,
                                                           int nchunk, uint16_t* __restrict__ out) {
  __shared__ float sa[kMaxChunks + kCombineBatch], sl[kMaxChunks + kCombineBatch];  // a batch may read past `used`
  __shared__ float red[2];
  const int h = blockIdx.x, b = blockIdx.y, dd = threadIdx.x, lane = dd & 63, wave = dd >> 6;
  const int64_t row0 = (static_cast<int64_t>(b) * H + h) * nchunk;
  const rsrc_t ro = make_rsrc(po + row0 * kHd, static_cast<uint32_t>(nchunk) * kHd * 4u);
  float ov[kCombineBatch];
#pragma unroll
  for (int i = 0; i < kCombineBatch; ++i)
    ov[i] = __builtin_bit_cast(float, bload32(ro, static_cast<uint32_t>(i * kHd + dd) * 4u, 0u));
  const f32x2_t* ml = reinterpret_cast<const f32x2_t*>(pml + row0 * 2);
  const int L = min(max(lengths[b], 0) + 1, tmax);
  const int used = (L + chunk - 1) / chunk;
  float mx = -INFINITY;
  for (int c = dd; c < used; c += kHd) {
    const f32x2_t v = ml[c];
    sa[c] = v[0];
    sl[c] = v[1];
    mx = fmaxf(mx, v[0]);
  }
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  const float M = fmaxf(red[0], red[1]);
  for (int c = dd; c < used; c += kHd) sa[c] = attn_chunk_weight(sa[c], M);
  __syncthreads();
  float ls = 0.0f, os = 0.0f;
  for (int c0 = 0; c0 < used; c0 += kCombineBatch) {
    if (c0 > 0) {
#pragma unroll
      for (int i = 0; i < kCombineBatch; ++i)
        ov[i] = __builtin_bit_cast(float, bload32(ro, static_cast<uint32_t>((c0 + i) * kHd + dd) * 4u, 0u));
    }
#pragma unroll
    for (int i = 0; i < kCombineBatch; ++i) {
      const bool u = c0 + i < used;
      const float a = sa[c0 + i];
      ls = u ? fmaf(sl[c0 + i], a, ls) : ls;
      os = u ? fmaf(ov[i], a, os) : os;
    }
  }
  out[(static_cast<int64_t>(b) * H + h) * kHd + dd] = f32_to_bf16_bits(os / ls);
}

// ---------------------------------------------------------------------------------------------
// SwiGLU gate: out = bf16(silu(g) * u), silu(g) = g / (1 + e^-g), from the fused projection row
// [g (F) | u (F)] (model.py:227-237 with w1 = gate, w3 = up). Two elements per thread.
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu, int F, int64_t n,
                                                       uint16_t* __restrict__ out) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 2;
  if (i >= n) return;
  const int64_t b = i / F, c = i % F;
  const uint32_t g2 = *reinterpret_cast<const uint32_t*>(gu + b * 2 * F + c);
  const uint32_t u2 = *reinterpret_cast<const uint32_t*>(gu + b * 2 * F + F + c);
  const float g0 = bf16_lo(g2), g1 = bf16_hi(g2);
  const float r0 = silu_f32(g0) * bf16_lo(u2);
  const float r1 = silu_f32(g1) * bf16_hi(u2);
  *reinterpret_cast<uint32_t*>(out + i) = ActBF16::pack_rne(r0, r1);
}

// Eight elements per thread (16-byte loads and stores) when F is a multiple of 8 and the buffers are
// 16-byte aligned, so eight consecutive elements never cross a row; the same arithmetic per element
// as silu_mul_kernel. PAIRS8: the row is laid out in 8-element groups [g 8j .. 8j+7 | u 8j .. 8j+7], as
// a fused gate|up weight with alternating 8-row groups writes it.
template <bool PAIRS8 = false>
__global__ __launch_bounds__(256) void silu_mul8_kernel(const uint16_t* __restrict__ gu, int F, int64_t n,
                                                        uint16_t* __restrict__ out) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  if (i >= n) return;
  const int64_t b = i / F, c = i % F;
  const uint16_t* gp = gu + b * 2 * F + (PAIRS8 ? 2 * c : c);
  const u32x4_t g4 = *reinterpret_cast<const u32x4_t*>(gp);
  const u32x4_t u4 = *reinterpret_cast<const u32x4_t*>(gp + (PAIRS8 ? 8 : F));
  u32x4_t r;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    r[j] = ActBF16::pack_rne(silu_f32(bf16_lo(g4[j])) * bf16_lo(u4[j]), silu_f32(bf16_hi(g4[j])) * bf16_hi(u4[j]));
  *reinterpret_cast<u32x4_t*>(out + i) = r;
}

// Embedding rows out[b] = table[tokens[b]] (model.py:136-145). An id outside [0, V) gives a zero row.
__global__ __launch_bounds__(256) void embed_kernel(const uint16_t* __restrict__ table, const int* __restrict__ tok,
                                                    int64_t V, int d, uint16_t* __restrict__ out) {
  const int b = blockIdx.x;
  const int t = tok[b];
  const bool ok = t >= 0 && t < V;
  const uint16_t* src = table + (ok ? static_cast<int64_t>(t) : 0) * d;
  for (int c = threadIdx.x * 8; c < d; c += 256 * 8) {
    u32x4_t v = *reinterpret_cast<const u32x4_t*>(src + c);
    if (!ok) v = u32x4_t{0, 0, 0, 0};
    *reinterpret_cast<u32x4_t*>(out + static_cast<int64_t>(b) * d + c) = v;
  }
}

// Greedy pick: next_tok[b] = the first index of the maximum of logits[b] (torch.argmax; a NaN
// counts as the maximum, sampling.py:82-83).
__device__ inline bool argmax_takes(float ov, int oi, float cv, int ci) {
  const bool on = ov != ov, cn = cv != cv;
  if (on || cn) return on && (!cn || oi < ci);
  return ov > cv || (ov == cv && oi < ci);
}

// Partial pick over a span of one row: workgroup (blk, b) of 256 threads reduces elements
// [blk * span, blk * span + span) to (value, index) in part[b, blk]. VEC: 16-byte loads (span and
// V multiples of 8, 16-byte aligned rows).
template <bool VEC>
__global__ __launch_bounds__(256) void argmax_partial_kernel(const uint16_t* __restrict__ logits, int64_t V, int span,
                                                             int nblk, float* __restrict__ pv, int* __restrict__ pi) {
  __shared__ float bv[4];
  __shared__ int bi[4];
  const int blk = blockIdx.x, b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint16_t* row = logits + static_cast<int64_t>(b) * V;
  const int64_t e0 = static_cast<int64_t>(blk) * span, e1 = min<int64_t>(V, e0 + span);
  float best = -INFINITY;
  int idx = 0x7fffffff;
  auto take = [&](float x, int v) {
    if (argmax_takes(x, v, best, idx)) {
      best = x;
      idx = v;
    }
  };
  if constexpr (VEC) {
#pragma unroll 2
    for (int64_t c = e0 + 8 * tid; c < e1; c += 8 * 256) {
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(row + c);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        take(bf16_lo(w[j]), static_cast<int>(c + 2 * j));
        take(bf16_hi(w[j]), static_cast<int>(c + 2 * j + 1));
      }
    }
  } else {
    for (int64_t v = e0 + tid; v < e1; v += 256) take(bf16_bits_to_f32(row[v]), static_cast<int>(v));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    take(ov, oi);
  }
  if (lane == 0) {
    bv[wave] = best;
    bi[wave] = idx;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) take(bv[w], bi[w]);
    pv[static_cast<int64_t>(b) * nblk + blk] = best;
    pi[static_cast<int64_t>(b) * nblk + blk] = idx;
  }
}

// next_tok[b] = the pick among row b's nblk (<= 64) partials: one wave per row.
__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ pv, const int* __restrict__ pi,
                                                          int nblk, int* __restrict__ next_tok) {
  const int b = blockIdx.x, lane = threadIdx.x;
  float best = lane < nblk ? pv[static_cast<int64_t>(b) * nblk + lane] : -INFINITY;
  int idx = lane < nblk ? pi[static_cast<int64_t>(b) * nblk + lane] : 0x7fffffff;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (argmax_takes(ov, oi, best, idx)) {
      best = ov;
      idx = oi;
    }
  }
  if (lane == 0) next_tok[b] = idx;
}

// SlotKVCache.advance(1) (kv_cache.py:207-213): lengths[b] += 1 for active rows (all rows when
// active is null).
__global__ void advance_kernel(int* __restrict__ lengths, const uint8_t* __restrict__ active, int B) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < B && (active == nullptr || active[b] != 0)) lengths[b] += 1;
}

}  // namespace sqx

using namespace sqx;

// ==============================================================================================
// extern "C" entry points
// ==============================================================================================
static bool al16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

extern "C" int sqx_rmsnorm(const void* x, const void* delta, const void* w, float eps, int64_t rows, int64_t d,
                           void* h_out, void* y, sqx_stream_t stream) {
  SQX_REQUIRE(rows >= 0 && d > 0 && d % 8 == 0 && rows < (int64_t(1) << 31) && d <= 16384, SQX_E_ARG,
              "sqx_rmsnorm: bad shape [%lld, %lld] (d a multiple of 8, at most 16384)", (long long)rows, (long long)d);
  if (rows == 0) return SQX_OK;
  SQX_REQUIRE(x && w && y && (delta == nullptr || h_out != nullptr), SQX_E_ARG, "sqx_rmsnorm: null pointer");
  SQX_REQUIRE(al16(x) && al16(w) && al16(y) && al16(delta) && al16(h_out), SQX_E_ARG,
              "sqx_rmsnorm: pointers must be 16-byte aligned");
  const int nch = static_cast<int>(ceil_div(d, 2048));
#define SQX_RMS(N_)                                                                                             \
  hipLaunchKernelGGL(rmsnorm_kernel<N_>, dim3(static_cast<unsigned>(rows)), dim3(256), 0, as_stream(stream),     \
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(delta),                       \
                     static_cast<const uint16_t*>(w), eps, static_cast<int>(d), static_cast<uint16_t*>(h_out), \
                     static_cast<uint16_t*>(y))
  if (nch <= 1) SQX_RMS(1);
  else if (nch <= 2) SQX_RMS(2);
  else if (nch <= 4) SQX_RMS(4);
  else SQX_RMS(8);
#undef SQX_RMS
  SQX_LAUNCH_CHECK("sqx_rmsnorm");
  return SQX_OK;
}

extern "C" int sqx_rmsnorm_partials(const void* x, const float* part, int splits, const void* w, float eps,
                                    int64_t rows, int64_t d, void* h_out, void* y, sqx_stream_t stream) {
  const char* fn = "sqx_rmsnorm_partials";
  SQX_REQUIRE(rows >= 0 && d > 0 && d % 8 == 0 && rows < (int64_t(1) << 31) && d <= 16384, SQX_E_ARG,
              "%s: bad shape [%lld, %lld] (d a multiple of 8, at most 16384)", fn, (long long)rows, (long long)d);
  SQX_REQUIRE(splits >= 1 && splits <= 64, SQX_E_ARG, "%s: %d splits (1..64)", fn, splits);
  if (rows == 0) return SQX_OK;
  SQX_REQUIRE(x && part && w && y && h_out, SQX_E_ARG, "%s: null pointer", fn);
  SQX_REQUIRE(al16(x) && al16(part) && al16(w) && al16(y) && al16(h_out), SQX_E_ARG,
              "%s: pointers must be 16-byte aligned", fn);
  const int nch = static_cast<int>(ceil_div(d, 2048));
#define SQX_RMS1(N_, PS_)                                                                                        \
  hipLaunchKernelGGL((rmsnorm_kernel<N_, true, PS_>), dim3(static_cast<unsigned>(rows)), dim3(256), 0,             \
                     as_stream(stream), static_cast<const uint16_t*>(x), nullptr, static_cast<const uint16_t*>(w), eps, \
                     static_cast<int>(d), static_cast<uint16_t*>(h_out), static_cast<uint16_t*>(y), part, splits,   \
                     rows * d)
#define SQX_RMS(N_)                                  \
  do {                                               \
    if (splits == 2) SQX_RMS1(N_, 2);                \
    else if (splits == 4) SQX_RMS1(N_, 4);           \
    else if (splits == 8) SQX_RMS1(N_, 8);           \
    else SQX_RMS1(N_, 0);                            \
  } while (0)
  if (nch <= 1) SQX_RMS(1);
  else if (nch <= 2) SQX_RMS(2);
  else if (nch <= 4) SQX_RMS(4);
  else SQX_RMS(8);
#undef SQX_RMS
#undef SQX_RMS1
  SQX_LAUNCH_CHECK(fn);
  return SQX_OK;
}

extern "C" int sqx_rope_kv(const void* qkv, const int* lengths, const float* cos_t, const float* sin_t,
                           int64_t rope_rows, int64_t B, int64_t H, int64_t Hkv, int64_t hd, int64_t tmax,
                           void* q_out, void* k_cache, void* v_cache, sqx_stream_t stream) {
  SQX_REQUIRE(B >= 0 && H > 0 && Hkv > 0 && H % Hkv == 0 && hd > 0 && hd % 2 == 0 && tmax > 0 && rope_rows > 0,
              SQX_E_ARG, "sqx_rope_kv: bad shape");
  SQX_REQUIRE(B < 65536 && (H + 2 * Hkv) * hd < (int64_t(1) << 30) && rope_rows < (int64_t(1) << 31) &&
                  tmax < (int64_t(1) << 31),
              SQX_E_ARG, "sqx_rope_kv: shape too large");
  if (B == 0) return SQX_OK;
  SQX_REQUIRE(qkv && lengths && cos_t && sin_t && q_out && k_cache && v_cache, SQX_E_ARG, "sqx_rope_kv: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(qkv) % 4 == 0 && reinterpret_cast<uintptr_t>(q_out) % 4 == 0 &&
                  reinterpret_cast<uintptr_t>(k_cache) % 4 == 0 && reinterpret_cast<uintptr_t>(v_cache) % 4 == 0,
              SQX_E_ARG, "sqx_rope_kv: bf16 buffers must be 4-byte aligned");
  const int64_t pairs = (H + 2 * Hkv) * hd / 2;
  hipLaunchKernelGGL(rope_kv_kernel, dim3(static_cast<unsigned>(ceil_div(pairs, 256)), static_cast<unsigned>(B)),
                     dim3(256), 0, as_stream(stream), static_cast<const uint16_t*>(qkv), lengths, cos_t, sin_t,
                     static_cast<int>(rope_rows), static_cast<int>(H), static_cast<int>(Hkv), static_cast<int>(hd),
                     static_cast<int>(tmax), static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache),
                     static_cast<uint16_t*>(v_cache));
  SQX_LAUNCH_CHECK("sqx_rope_kv");
  return SQX_OK;
}

// Keys per workgroup: the smallest of 64..1024 that still gives about SQX_ATTN_TARGET_WG workgroups.
// Long walks per wave amortise each workgroup's set-up and merge, and with the next block's rows in
// flight during each block (two register sets) one workgroup per CU streams well: measured at 2048
// keys (partial + combine), B = 1 / 8 / 32 / 64 take 9.5 / 17.8 / 48.8 / 91.1 us with a 256-workgroup
// target, against 10.2 / 22.5 / 60.4 / 104.9 us for a single register set and a 1024 target.
// When the (row, kv head) pairs alone reach the target, each takes all its keys as one chunk and its
// workgroup writes the output (no combine launch): at 2048 keys the Llama-3-8B decode step at
// B = 32 / 64 went from 3.77 / 5.90 ms to 3.63 / 5.72 ms (5.61 -> 5.26 ms with the E4M3 cache).
#ifndef SQX_ATTN_TARGET_WG
#define SQX_ATTN_TARGET_WG 256
#endif
#ifndef SQX_ATTN_MAX_CHUNK
#define SQX_ATTN_MAX_CHUNK 1024
#endif
#ifndef SQX_ATTN_MIN_CHUNK
#define SQX_ATTN_MIN_CHUNK 64
#endif
extern "C" int sqx_attn_chunk(int64_t B, int64_t Hkv, int64_t tmax) {
  if (B * Hkv >= SQX_ATTN_TARGET_WG && tmax > 0 && tmax < (int64_t(1) << 30))
    return static_cast<int>(std::max<int64_t>(SQX_ATTN_MIN_CHUNK, ceil_div(tmax, 64) * 64));
  int c = SQX_ATTN_MIN_CHUNK;
  while (c < SQX_ATTN_MAX_CHUNK && B * Hkv * ceil_div(tmax, 2 * c) >= SQX_ATTN_TARGET_WG) c *= 2;
  return c;
}

extern "C" int64_t sqx_attn_workspace_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t tmax) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || tmax <= 0) return 0;
  return B * H * ceil_div(tmax, sqx_attn_chunk(B, Hkv, tmax)) * (kHd + 2) * 4;
}

// Keys per workgroup of the partials that the o projection merges in its prologue
// (sqx_decode_attention_partials): 8 waves per workgroup and at most kFoldMaxChunks chunks per head,
// the smallest multiple of 128 keys (one 16-key block per wave) that gets there. Every workgroup of the
// o projection merges every head's chunks, so few chunks keep that merge cheap; eight waves with the
// two-block register ring keep a chunk of 256 keys per workgroup in flight.
constexpr int kFoldMaxChunks = 8;
constexpr int kFoldWaves = 8;
extern "C" int sqx_attn_partials_chunk(int64_t tmax) {
  if (tmax <= 0) return 0;
  const int64_t step = kFoldWaves * kKeysPerStep;
  return static_cast<int>(std::max<int64_t>(step, ceil_div(ceil_div(tmax, kFoldMaxChunks), step) * step));
}

extern "C" int64_t sqx_attn_partials_workspace_bytes(int64_t B, int64_t H, int64_t tmax) {
  if (B <= 0 || H <= 0 || tmax <= 0) return 0;
  return B * H * ceil_div(tmax, sqx_attn_partials_chunk(tmax)) * (kHd + 2) * 4;
}

// chunk > 0 with nwv = 8 and no combine: the partials for the o projection's merge; otherwise the
// library's chunk with 4 waves per workgroup and the combine kernel.
static int decode_attention_impl(const void* q, void* k_cache, void* v_cache, const int* lengths, const float* cos_t,
                                 const float* sin_t, int64_t rope_rows, const float* kscale, const float* vscale,
                                 int64_t B, int64_t H, int64_t Hkv, int64_t hd, int64_t tmax, void* out, void* ws,
                                 int64_t ws_bytes, sqx_stream_t stream, const char* fn, bool partials_only = false,
                                 const float* qpart = nullptr, int qsplits = 0) {
  const bool rope = cos_t != nullptr;
  const bool kv8 = kscale != nullptr;
  SQX_REQUIRE(!kv8 || vscale != nullptr, SQX_E_ARG, "%s: null V scale", fn);
  SQX_REQUIRE(hd == kHd, SQX_E_ARG, "%s: head_dim %lld is not supported (128)", fn, (long long)hd);
  SQX_REQUIRE(B >= 0 && H > 0 && Hkv > 0 && H % Hkv == 0 && tmax > 0, SQX_E_ARG, "%s: bad shape", fn);
  SQX_REQUIRE(B < 65536 && Hkv < 65536 && tmax < (int64_t(1) << 30) && (H + 2 * Hkv) * hd < (int64_t(1) << 30),
              SQX_E_ARG, "%s: shape too large", fn);
  const int G = static_cast<int>(H / Hkv);
  SQX_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, SQX_E_ARG, "%s: %d query heads per kv head (1, 2, 4 or 8 are built)",
              fn, G);
  SQX_REQUIRE(!rope || (sin_t != nullptr && rope_rows > 0 && rope_rows < (int64_t(1) << 31)), SQX_E_ARG,
              "%s: bad RoPE tables", fn);
  if (B == 0) return SQX_OK;
  SQX_REQUIRE(q && k_cache && v_cache && lengths && ws && (out || partials_only), SQX_E_ARG, "%s: null pointer", fn);
  const int64_t need = partials_only ? sqx_attn_partials_workspace_bytes(B, H, tmax)
                                     : sqx_attn_workspace_bytes(B, H, Hkv, tmax);
  SQX_REQUIRE(ws_bytes >= need, SQX_E_SPACE, "%s: workspace of %lld bytes, %lld needed", fn, (long long)ws_bytes,
              (long long)need);
  SQX_REQUIRE(al16(q) && al16(k_cache) && al16(v_cache) && al16(ws), SQX_E_ARG,
              "%s: q, caches and workspace must be 16-byte aligned", fn);
  const int chunk = partials_only ? sqx_attn_partials_chunk(tmax) : sqx_attn_chunk(B, Hkv, tmax);
  const int nchunk = static_cast<int>(ceil_div(tmax, chunk));
  SQX_REQUIRE(nchunk <= kMaxChunks, SQX_E_ARG, "%s: %d key chunks of %d (at most %d)", fn, nchunk, chunk, kMaxChunks);
  hipStream_t s = as_stream(stream);
  const float qscale = 1.4426950408889634f / sqrtf(static_cast<float>(hd));  // log2(e) / sqrt(hd)
  const dim3 grid(static_cast<unsigned>(nchunk), static_cast<unsigned>(Hkv), static_cast<unsigned>(B));
  const auto* qp = static_cast<const uint16_t*>(q);
  auto* kp = static_cast<uint8_t*>(k_cache);
  auto* vp = static_cast<uint8_t*>(v_cache);
  float* po = static_cast<float*>(ws);
  float* pml = po + B * H * nchunk * kHd;
  // one chunk per row: the partial kernel writes the output itself and no combine runs
  uint16_t* direct = !partials_only && nchunk == 1 ? static_cast<uint16_t*>(out) : nullptr;
  const int iH = static_cast<int>(H), iK = static_cast<int>(Hkv), iT = static_cast<int>(tmax);
  const int rr = static_cast<int>(rope_rows);
#define SQX_ATTN_M(G_, R_, K8_)                                                                                     \
  do {                                                                                                             \
    if (partials_only)                                                                                             \
      hipLaunchKernelGGL((attn_partial_mfma_kernel<G_, R_, K8_, kFoldWaves>), grid, dim3(kFoldWaves * 64), 0, s, qp, \
                         kp, vp, lengths, cos_t, sin_t, kscale, vscale, rr, iH, iK, iT, chunk, nchunk, qscale, po,  \
                         pml, nullptr, nullptr, 0);                                                                \
    else                                                                                                           \
      hipLaunchKernelGGL((attn_partial_mfma_kernel<G_, R_, K8_, 4>), grid, dim3(256), 0, s, qp, kp, vp, lengths,    \
                         cos_t, sin_t, kscale, vscale, rr, iH, iK, iT, chunk, nchunk, qscale, po, pml, direct,      \
                         nullptr, 0);                                                                              \
  } while (0)
#define SQX_ATTN_MQ(G_, K8_)                                                                                        \
  hipLaunchKernelGGL((attn_partial_mfma_kernel<G_, true, K8_, 4, true>), grid, dim3(256), 0, s, qp, kp, vp, lengths, \
                     cos_t, sin_t, kscale, vscale, rr, iH, iK, iT, chunk, nchunk, qscale, po, pml, direct, qpart,     \
                     qsplits)
#define SQX_ATTN_MG(M_, ...)                      \
  switch (G) {                                    \
    case 1: M_(1, __VA_ARGS__); break;            \
    case 2: M_(2, __VA_ARGS__); break;            \
    case 4: M_(4, __VA_ARGS__); break;            \
    default: M_(8, __VA_ARGS__); break;           \
  }
  // scores on the matrix unit (E4M3 keys decoded to bf16 pairs on the way in)
  if (rope && qsplits > 0) {
    if (kv8) { SQX_ATTN_MG(SQX_ATTN_MQ, true) } else { SQX_ATTN_MG(SQX_ATTN_MQ, false) }
  } else if (rope) {
    if (kv8) { SQX_ATTN_MG(SQX_ATTN_M, true, true) } else { SQX_ATTN_MG(SQX_ATTN_M, true, false) }
  } else {
    if (kv8) { SQX_ATTN_MG(SQX_ATTN_M, false, true) } else { SQX_ATTN_MG(SQX_ATTN_M, false, false) }
  }
#undef SQX_ATTN_MG
#undef SQX_ATTN_MQ
#undef SQX_ATTN_M
  SQX_LAUNCH_CHECK(fn);
  if (partials_only || direct != nullptr) return SQX_OK;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(static_cast<unsigned>(H), static_cast<unsigned>(B)), dim3(kHd), 0, s, po,
                     pml, lengths, iH, iT, chunk, nchunk, static_cast<uint16_t*>(out));
  SQX_LAUNCH_CHECK(fn);
  return SQX_OK;
}

extern "C" int sqx_decode_attention_partials(const void* q, const int* lengths, const float* cos_t, const float* sin_t,
                                             int64_t rope_rows, void* k_cache, void* v_cache, const float* k_scale,
                                             const float* v_scale, int64_t B, int64_t H, int64_t Hkv, int64_t hd,
                                             int64_t tmax, void* ws, int64_t ws_bytes, sqx_stream_t stream) {
  const char* fn = "sqx_decode_attention_partials";
  SQX_REQUIRE((k_scale == nullptr) == (v_scale == nullptr), SQX_E_ARG, "%s: give both scales or neither", fn);
  return decode_attention_impl(q, k_cache, v_cache, lengths, cos_t, sin_t, rope_rows, k_scale, v_scale, B, H, Hkv, hd,
                               tmax, nullptr, ws, ws_bytes, stream, fn, true);
}

extern "C" int sqx_attn_partials_combine(const void* ws, const int* lengths, int64_t B, int64_t H, int64_t tmax,
                                         void* out, sqx_stream_t stream) {
  const char* fn = "sqx_attn_partials_combine";
  SQX_REQUIRE(B >= 0 && B < 65536 && H > 0 && H < 65536 && tmax > 0 && tmax < (int64_t(1) << 30), SQX_E_ARG,
              "%s: bad shape", fn);
  if (B == 0) return SQX_OK;
  SQX_REQUIRE(ws && lengths && out, SQX_E_ARG, "%s: null pointer", fn);
  const int chunk = sqx_attn_partials_chunk(tmax);
  const int nchunk = static_cast<int>(ceil_div(tmax, chunk));
  const float* po = static_cast<const float*>(ws);
  const float* pml = po + B * H * nchunk * kHd;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(static_cast<unsigned>(H), static_cast<unsigned>(B)), dim3(kHd), 0,
                     as_stream(stream), po, pml, lengths, static_cast<int>(H), static_cast<int>(tmax), chunk, nchunk,
                     static_cast<uint16_t*>(out));
  SQX_LAUNCH_CHECK(fn);
  return SQX_OK;
}

extern "C" int sqx_decode_attention(const void* q, const void* k_cache, const void* v_cache, const int* lengths,
                                    int64_t B, int64_t H, int64_t Hkv, int64_t hd, int64_t tmax, void* out,
                                    void* ws, int64_t ws_bytes, sqx_stream_t stream) {
  return decode_attention_impl(q, const_cast<void*>(k_cache), const_cast<void*>(v_cache), lengths, nullptr, nullptr, 0,
                               nullptr, nullptr, B, H, Hkv, hd, tmax, out, ws, ws_bytes, stream, "sqx_decode_attention");
}

extern "C" int sqx_decode_attention_rope(const void* qkv, const int* lengths, const float* cos_t, const float* sin_t,
                                         int64_t rope_rows, void* k_cache, void* v_cache, int64_t B, int64_t H,
                                         int64_t Hkv, int64_t hd, int64_t tmax, void* out, void* ws, int64_t ws_bytes,
                                         sqx_stream_t stream) {
  SQX_REQUIRE(cos_t != nullptr, SQX_E_ARG, "sqx_decode_attention_rope: null cos table");
  return decode_attention_impl(qkv, k_cache, v_cache, lengths, cos_t, sin_t, rope_rows, nullptr, nullptr, B, H, Hkv, hd,
                               tmax, out, ws, ws_bytes, stream, "sqx_decode_attention_rope");
}

// ---------------------------------------------------------------------------------------------
// The allocation-free form of sqx_decode_attention_rope, for callers that cannot allocate (code under
// HIP graph capture, tight serving loops): the key-split partials go to `scratch`, a file-scope device
// array of kNoAllocScratchBytes, instead of a caller workspace. Every GPU the library runs on holds its
// own copy until the process ends. In host code the array's name is not a device address: its address
// on the current device comes from hipGetSymbolAddress, looked up once per device on the first call
// with that device current and kept in scratch_ptr[]. Each call writes every partial the combine
// reads (the chunks below the row's length), so nothing has to start cleared; calls that overlap on
// one GPU share the array and race.
// ---------------------------------------------------------------------------------------------
constexpr int64_t kNoAllocScratchBytes = int64_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kScratchDevices = 64;
std::mutex scratch_mu;
void* scratch_ptr[kScratchDevices] = {};

int scratch_on_current_device(void** out, const char* fn) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  SQX_REQUIRE(e == hipSuccess, SQX_E_HIP, "%s: hipGetDevice failed: %s", fn, hipGetErrorString(e));
  SQX_REQUIRE(dev >= 0 && dev < kScratchDevices, SQX_E_ARG, "%s: device %d out of range", fn, dev);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    SQX_REQUIRE(e == hipSuccess && p != nullptr, SQX_E_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev,
                hipGetErrorString(e));
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return SQX_OK;
}
}  // namespace

extern "C" int sqx_decode_attention_rope_noalloc(const void* qkv, const int* lengths, const float* cos_t,
                                                 const float* sin_t, int64_t rope_rows, void* k_cache, void* v_cache,
                                                 int64_t B, int64_t H, int64_t Hkv, int64_t hd, int64_t tmax,
                                                 void* out, sqx_stream_t stream) {
  const char* fn = "sqx_decode_attention_rope_noalloc";
  SQX_REQUIRE(cos_t != nullptr, SQX_E_ARG, "%s: null cos table", fn);
  const int64_t need = sqx_attn_workspace_bytes(B, H, Hkv, tmax);
  SQX_REQUIRE(need <= kNoAllocScratchBytes, SQX_E_SPACE,
              "%s: B=%lld H=%lld Hkv=%lld tmax=%lld needs %lld bytes of partials, more than the fixed %lld bytes of "
              "scratch (use sqx_decode_attention_rope with a workspace)",
              fn, (long long)B, (long long)H, (long long)Hkv, (long long)tmax, (long long)need,
              (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  if (int rc = scratch_on_current_device(&ws, fn)) return rc;
  return decode_attention_impl(qkv, k_cache, v_cache, lengths, cos_t, sin_t, rope_rows, nullptr, nullptr, B, H, Hkv, hd,
                               tmax, out, ws, kNoAllocScratchBytes, stream, fn);
}

extern "C" int sqx_decode_attention_fp8kv(const void* q, const void* k_codes, const void* v_codes, const float* k_scale,
                                          const float* v_scale, const int* lengths, int64_t B, int64_t H, int64_t Hkv,
                                          int64_t hd, int64_t tmax, void* out, void* ws, int64_t ws_bytes,
                                          sqx_stream_t stream) {
  SQX_REQUIRE(k_scale != nullptr && v_scale != nullptr, SQX_E_ARG, "sqx_decode_attention_fp8kv: null scale");
  return decode_attention_impl(q, const_cast<void*>(k_codes), const_cast<void*>(v_codes), lengths, nullptr, nullptr, 0,
                               k_scale, v_scale, B, H, Hkv, hd, tmax, out, ws, ws_bytes, stream,
                               "sqx_decode_attention_fp8kv");
}

// sqx_decode_attention_rope[_fp8kv] reading the q|k|v rows as the fp32 partials of a K-split
// projection (sqx_int4_skinny_partials), which it adds as that projection's reduce would.
extern "C" int sqx_decode_attention_rope_parts(const float* qkv_parts, int64_t splits, const int* lengths,
                                               const float* cos_t, const float* sin_t, int64_t rope_rows,
                                               void* k_cache, void* v_cache, const float* k_scale,
                                               const float* v_scale, int64_t B, int64_t H, int64_t Hkv, int64_t hd,
                                               int64_t tmax, void* out, void* ws, int64_t ws_bytes,
                                               sqx_stream_t stream) {
  const char* fn = "sqx_decode_attention_rope_parts";
  SQX_REQUIRE(cos_t != nullptr, SQX_E_ARG, "%s: null cos table", fn);
  SQX_REQUIRE((k_scale == nullptr) == (v_scale == nullptr), SQX_E_ARG, "%s: give both scales or neither", fn);
  SQX_REQUIRE(splits >= 1 && splits <= 64, SQX_E_ARG, "%s: %lld splits (1 to 64)", fn, (long long)splits);
  return decode_attention_impl(qkv_parts, k_cache, v_cache, lengths, cos_t, sin_t, rope_rows, k_scale, v_scale, B, H,
                               Hkv, hd, tmax, out, ws, ws_bytes, stream, fn, false, qkv_parts,
                               static_cast<int>(splits));
}

extern "C" int sqx_decode_attention_rope_fp8kv(const void* qkv, const int* lengths, const float* cos_t,
                                               const float* sin_t, int64_t rope_rows, void* k_codes, void* v_codes,
                                               const float* k_scale, const float* v_scale, int64_t B, int64_t H,
                                               int64_t Hkv, int64_t hd, int64_t tmax, void* out, void* ws,
                                               int64_t ws_bytes, sqx_stream_t stream) {
  SQX_REQUIRE(cos_t != nullptr && k_scale != nullptr && v_scale != nullptr, SQX_E_ARG,
              "sqx_decode_attention_rope_fp8kv: null table or scale");
  return decode_attention_impl(qkv, k_codes, v_codes, lengths, cos_t, sin_t, rope_rows, k_scale, v_scale, B, H, Hkv, hd,
                               tmax, out, ws, ws_bytes, stream, "sqx_decode_attention_rope_fp8kv");
}

extern "C" int sqx_silu_mul(const void* gate_up, int64_t B, int64_t F, void* out, sqx_stream_t stream) {
  SQX_REQUIRE(B >= 0 && F > 0 && F % 2 == 0 && B * F < (int64_t(1) << 40), SQX_E_ARG,
              "sqx_silu_mul: bad shape (F must be even)");
  if (B == 0) return SQX_OK;
  SQX_REQUIRE(gate_up && out, SQX_E_ARG, "sqx_silu_mul: null pointer");
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(gate_up) % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 4 == 0, SQX_E_ARG,
              "sqx_silu_mul: pointers must be 4-byte aligned");
  const int64_t n = B * F;
  if (F % 8 == 0 && reinterpret_cast<uintptr_t>(gate_up) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0)
    hipLaunchKernelGGL(silu_mul8_kernel<false>, dim3(static_cast<unsigned>(ceil_div(n / 8, 256))), dim3(256), 0,
                       as_stream(stream), static_cast<const uint16_t*>(gate_up), static_cast<int>(F), n,
                       static_cast<uint16_t*>(out));
  else
    hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(ceil_div(n / 2, 256))), dim3(256), 0,
                       as_stream(stream), static_cast<const uint16_t*>(gate_up), static_cast<int>(F), n,
                       static_cast<uint16_t*>(out));
  SQX_LAUNCH_CHECK("sqx_silu_mul");
  return SQX_OK;
}

extern "C" int sqx_silu_mul_pairs8(const void* gate_up, int64_t B, int64_t F, void* out, sqx_stream_t stream) {
  const char* fn = "sqx_silu_mul_pairs8";
  SQX_REQUIRE(B >= 0 && F > 0 && F % 8 == 0 && B * F < (int64_t(1) << 40), SQX_E_ARG,
              "%s: bad shape (F must be a multiple of 8)", fn);
  if (B == 0) return SQX_OK;
  SQX_REQUIRE(gate_up && out, SQX_E_ARG, "%s: null pointer", fn);
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(gate_up) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0, SQX_E_ARG,
              "%s: pointers must be 16-byte aligned", fn);
  const int64_t n = B * F;
  hipLaunchKernelGGL(silu_mul8_kernel<true>, dim3(static_cast<unsigned>(ceil_div(n / 8, 256))), dim3(256), 0,
                     as_stream(stream), static_cast<const uint16_t*>(gate_up), static_cast<int>(F), n,
                     static_cast<uint16_t*>(out));
  SQX_LAUNCH_CHECK(fn);
  return SQX_OK;
}

extern "C" int sqx_embed(const void* table, int64_t V, const int* tokens, int64_t B, int64_t d, void* out,
                         sqx_stream_t stream) {
  SQX_REQUIRE(B >= 0 && V > 0 && d > 0 && d % 8 == 0 && B < (int64_t(1) << 31) && d < (int64_t(1) << 30), SQX_E_ARG,
              "sqx_embed: bad shape (d must be a multiple of 8)");
  if (B == 0) return SQX_OK;
  SQX_REQUIRE(table && tokens && out, SQX_E_ARG, "sqx_embed: null pointer");
  SQX_REQUIRE(al16(table) && al16(out), SQX_E_ARG, "sqx_embed: table and out must be 16-byte aligned");
  hipLaunchKernelGGL(embed_kernel, dim3(static_cast<unsigned>(B)), dim3(256), 0, as_stream(stream),
                     static_cast<const uint16_t*>(table), tokens, V, static_cast<int>(d), static_cast<uint16_t*>(out));
  SQX_LAUNCH_CHECK("sqx_embed");
  return SQX_OK;
}

static int argmax_blocks(int64_t V) { return static_cast<int>(std::min<int64_t>(64, ceil_div(V, 4096))); }

extern "C" int64_t sqx_argmax_workspace_bytes(int64_t B, int64_t V) {
  if (B <= 0 || V <= 0) return 0;
  return B * argmax_blocks(V) * 8;
}

extern "C" int sqx_argmax(const void* logits, int64_t B, int64_t V, int* next_tok, void* ws, int64_t ws_bytes,
                          sqx_stream_t stream) {
  SQX_REQUIRE(B >= 0 && V > 0 && B < 65536 && V < (int64_t(1) << 31), SQX_E_ARG, "sqx_argmax: bad shape");
  if (B == 0) return SQX_OK;
  SQX_REQUIRE(logits && next_tok && ws, SQX_E_ARG, "sqx_argmax: null pointer");
  SQX_REQUIRE(ws_bytes >= sqx_argmax_workspace_bytes(B, V), SQX_E_SPACE, "sqx_argmax: workspace of %lld bytes, %lld needed",
              (long long)ws_bytes, (long long)sqx_argmax_workspace_bytes(B, V));
  SQX_REQUIRE(reinterpret_cast<uintptr_t>(ws) % 4 == 0, SQX_E_ARG, "sqx_argmax: workspace must be 4-byte aligned");
  const int nblk = argmax_blocks(V);
  const bool vec = V % 8 == 0 && al16(logits);
  int span = static_cast<int>(ceil_div(V, nblk));
  if (vec) span = (span + 7) / 8 * 8;
  float* pv = static_cast<float*>(ws);
  int* pi = reinterpret_cast<int*>(pv + B * nblk);
  const auto* lp = static_cast<const uint16_t*>(logits);
  const dim3 grid(static_cast<unsigned>(nblk), static_cast<unsigned>(B));
  if (vec)
    hipLaunchKernelGGL(argmax_partial_kernel<true>, grid, dim3(256), 0, as_stream(stream), lp, V, span, nblk, pv, pi);
  else
    hipLaunchKernelGGL(argmax_partial_kernel<false>, grid, dim3(256), 0, as_stream(stream), lp, V, span, nblk, pv, pi);
  SQX_LAUNCH_CHECK("sqx_argmax");
  hipLaunchKernelGGL(argmax_final_kernel, dim3(static_cast<unsigned>(B)), dim3(64), 0, as_stream(stream), pv, pi, nblk,
                     next_tok);
  SQX_LAUNCH_CHECK("sqx_argmax");
  return SQX_OK;
}

extern "C" int sqx_advance(int* lengths, const uint8_t* active, int64_t B, sqx_stream_t stream) {
  SQX_REQUIRE(B >= 0 && B < (int64_t(1) << 31), SQX_E_ARG, "sqx_advance: bad B");
  if (B == 0) return SQX_OK;
  SQX_REQUIRE(lengths != nullptr, SQX_E_ARG, "sqx_advance: null lengths");
  hipLaunchKernelGGL(advance_kernel, dim3(static_cast<unsigned>(ceil_div(B, 256))), dim3(256), 0, as_stream(stream),
                     lengths, active, static_cast<int>(B));
  SQX_LAUNCH_CHECK("sqx_advance");
  return SQX_OK;
}
