// decode_int4.hip — single-query paged attention that dequantizes INT4 pages
// just in time (the fused form of the reference's dequantize_kv_cache_int4 ->
// dynamic_sparse_attention composition; TheRadDani/memopt-transformer-runtime
// src/csrc/quantization.cu:232-270 and src/csrc/attention.cu:98-339).
//
// HBM-bound design for gfx950 (wave64), two kernels:
//  * decode_int4_pages_kernel reads this build's INT4 page pool: one wave
//    streams one (page, head) block per step (16 tokens x D/2 bytes of K
//    codes and of V codes, 1 KiB each at D=128, plus the fp16 scales);
//    lane l = 8p + c owns tokens p and p + 8 and dims [c*D/8, (c+1)*D/8),
//    one 16-byte load each for K and V. The loads carry the non-temporal
//    cache-policy bit: each instruction covers whole 128-byte lines that no
//    later step reads again;
//  * decode_int4_kernel reads the reference's token-major codes [nb, bs, H,
//    D/2] with separate scales: lane l owns token l/4 and dims
//    [(l%4)*D/4, (l%4+1)*D/4), inside one 64-dim scale group;
//  * each wave keeps U pages in flight (the next batch's loads are issued
//    before the current one is consumed) and a workgroup runs NW waves over
//    interleaved pages of one (b, h);
//  * K nibbles become fp16 (1024 + code or 64 + code) with one v_bfi_b32
//    against the fp16 exponent patterns 0x6400 / 0x5400 and feed
//    v_dot2_f32_f16 directly; the constant bias sum q . (bias) is taken off
//    once per token, which leaves q . (code - 8);
//  * V nibbles are unpacked the same way and the bias is subtracted per pair
//    (exact fp16 code - 8). The row-layout kernel accumulates in fp32; the
//    page-layout kernel accumulates with v_dot2_f32_f16 over a token pair
//    against fp16 weights p * (V scale), kept <= 2^15 by raising the softmax
//    reference point. No bias is carried in the accumulators: removing
//    1032 * (sum of weights) at the end cost ~1e-2 absolute on output dims
//    near zero next to a token with a V scale in the hundreds;
//  * the softmax running max is wave-uniform and lazily raised: it is updated
//    (with a wave max and a rescale of the accumulators) only when some score
//    exceeds it by more than 8 in log2 units, so the common page costs no
//    cross-lane reduction; the partial dots of a token are summed with DPP
//    moves (3 over the 8 lanes of a token pair in the page kernel);
//  * only pages that intersect the sink range or the window are visited,
//    block-table entries < 0 or >= num_kv_blocks are skipped, and split-K
//    partials (m, l, o) are merged by the last split of each (b, h) to
//    finish (decode_epilogue).
#include <atomic>
#include <cstdlib>

#include "attention.hpp"

namespace memopt {

template <typename ST>
__device__ __forceinline__ float load_scale(const void *p, int64_t i) {
  return (float)reinterpret_cast<const ST *>(p)[i];
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Raw buffer descriptor over one (page, head) block: scalar base, 32-bit
// per-lane byte offsets (buffer_load ... offen), no per-lane 64-bit math.
// dword3 0x00020000 = 32-bit data format, the untyped raw-buffer setting.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t block_rsrc(const uint8_t *blk) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)blk, (short)0, 0x7FFFFFFF, 0x00020000);
}

template <int D>
struct LaneChunk;
template <>
struct LaneChunk<128> {
  uint4 w;
  static constexpr int kWords = 4;
  __device__ __forceinline__ void load(const uint8_t *p) { w = *reinterpret_cast<const uint4 *>(p); }
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kStreamLoad);
    w = make_uint4(v.x, v.y, v.z, v.w);
  }
  __device__ __forceinline__ uint32_t word(int i) const {
    return i == 0 ? w.x : (i == 1 ? w.y : (i == 2 ? w.z : w.w));
  }
};
template <>
struct LaneChunk<64> {
  uint2 w;
  static constexpr int kWords = 2;
  __device__ __forceinline__ void load(const uint8_t *p) { w = *reinterpret_cast<const uint2 *>(p); }
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kStreamLoad);
    w = make_uint2(v.x, v.y);
  }
  __device__ __forceinline__ uint32_t word(int i) const { return i == 0 ? w.x : w.y; }
};

static constexpr uint32_t kLoMask = 0x000F000Fu, kHiMask = 0x00F000F0u;
static constexpr uint32_t kMagic1024 = 0x64006400u, kMagic64 = 0x54005400u;

// Biased fp16 pairs of the 8 nibbles of a word, order (e0,e4), (e1,e5),
// (e2,e6), (e3,e7) with e_i = bits 4i..4i+3: values 1024+e for the first and
// third pair, 64+e for the second and fourth.
__device__ __forceinline__ void unpack_biased(uint32_t w, uint32_t r[4]) {
  const uint32_t w8 = w >> 8;
  r[0] = bfi(kLoMask, w, kMagic1024);
  r[1] = bfi(kHiMask, w, kMagic64);
  r[2] = bfi(kLoMask, w8, kMagic1024);
  r[3] = bfi(kHiMask, w8, kMagic64);
}

// The same pairs all biased by 64: (e0,e4) and (e2,e6) are shifted into bits
// 4-7 / 20-23 first. Two shifts more than unpack_biased, and a bias sum of
// 72 * sum(q) instead of up to 1032 * sum(q): the K dot products start from
// minus that sum, so a 14x smaller bias keeps 14x more of the fp32 mantissa
// for the score itself at large |q|.
__device__ __forceinline__ void unpack_biased64(uint32_t w, uint32_t r[4]) {
  r[0] = bfi(kHiMask, w << 4, kMagic64);
  r[1] = bfi(kHiMask, w, kMagic64);
  r[2] = bfi(kHiMask, w >> 4, kMagic64);
  r[3] = bfi(kHiMask, w >> 8, kMagic64);
}

// Same pairs as exact (code - 8) values.
__device__ __forceinline__ void unpack_exact(uint32_t w, half2_t h[4]) {
  uint32_t r[4];
  unpack_biased(w, r);
  const half2_t b1032 = {(half_t)1032.0f, (half_t)1032.0f};
  const half2_t b72 = {(half_t)72.0f, (half_t)72.0f};
  h[0] = as_half2(r[0]) - b1032;
  h[1] = as_half2(r[1]) - b72;
  h[2] = as_half2(r[2]) - b1032;
  h[3] = as_half2(r[3]) - b72;
}

// Slot s of a lane's accumulator holds dim base + kSlotDim[s % 8] + 8*(s / 8).
__device__ __constant__ int kSlotDim[8] = {0, 4, 1, 5, 2, 6, 3, 7};

template <int D, typename ST, int NW, int U>
__global__ __launch_bounds__(NW * 64) void decode_int4_kernel(const DecodeParams p) {
  constexpr int BPL = D / 8;   // code bytes per lane per page
  constexpr int DPL = D / 4;   // dims per lane
  constexpr int NWORD = BPL / 4;
  using Chunk = LaneChunk<D>;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int32_t b = blockIdx.z, h = blockIdx.y, split = blockIdx.x;
  const int t = lane >> 2, c = lane & 3;
  const int g = (c * DPL) / 64;  // scale group of this lane's dims

  __shared__ float s_acc[NW][D];
  __shared__ float s_ml[NW][2];

  const int32_t ctx = p.ctx[b];
  const KeyRange kr = key_range(ctx, ctx - 1, p.W, p.sinks, false);

  // Visited logical pages: sink pages then window pages (deduplicated).
  const int32_t last_page = min((kr.hi + 15) >> 4, p.M);
  const int32_t sink_pages = min((kr.sink_end + 15) >> 4, last_page);
  const int32_t win_page0 = max(kr.win_lo >> 4, sink_pages);
  const int32_t n_win = max(0, last_page - win_page0);
  const int64_t n_vis = (int64_t)sink_pages + n_win;
  const SplitRange sr = split_range((int32_t)n_vis, split, p.splits);
  const int32_t begin = sr.begin, end = sr.end;

  // q as fp16 pairs in unpack order + the bias sum q . (bias + 8).
  half2_t qp[NWORD][4];
  float bias = 0.0f;
  {
    const half_t *qrow = p.q + ((int64_t)b * p.H + h) * D + c * DPL;
#pragma unroll
    for (int k = 0; k < NWORD; ++k) {
      const uint4 u = *reinterpret_cast<const uint4 *>(qrow + 8 * k);
      const half2_t e01 = as_half2(u.x), e23 = as_half2(u.y), e45 = as_half2(u.z), e67 = as_half2(u.w);
      qp[k][0] = half2_t{e01.x, e45.x};
      qp[k][1] = half2_t{e01.y, e45.y};
      qp[k][2] = half2_t{e23.x, e67.x};
      qp[k][3] = half2_t{e23.y, e67.y};
      bias = fmaf(72.0f, ((float)e01.x + (float)e45.x) + ((float)e23.x + (float)e67.x), bias);
      bias = fmaf(72.0f, ((float)e01.y + (float)e45.y) + ((float)e23.y + (float)e67.y), bias);
    }
  }

  float m = -INFINITY, l = 0.0f;
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.0f;

  const int32_t *btrow = p.bt + (int64_t)b * p.M;
  const uint8_t *kbase = p.kc + (int64_t)h * p.kv_hs;
  const uint8_t *vbase = p.vc + (int64_t)h * p.kv_hs;
  const int64_t sbase = (int64_t)h * p.sc_hs;
  const uint32_t koff = (uint32_t)(t * p.kv_ts + c * BPL);
  const uint32_t soff = (uint32_t)(t * p.sc_ts + g);

  for (int32_t base = begin + wave * U; base < end; base += NW * U) {
    int32_t lp[U];
    bool ok[U];
    Chunk kw[U], vw[U];
    float sk[U], sv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int32_t i = base + u;
      lp[u] = (i < sink_pages) ? i : win_page0 + (i - sink_pages);
      const int32_t phys = btrow[(i < end) ? lp[u] : 0];  // lp < M whenever i < end
      ok[u] = (i < end) && phys >= 0 && phys < p.nb;
      // Invalid pages read page 0 of this head (always mapped) and are masked.
      const int64_t pg = ok[u] ? (int64_t)phys : 0;
      kw[u].load(kbase + pg * p.kv_ps + koff);
      vw[u].load(vbase + pg * p.kv_ps + koff);
      sk[u] = load_scale<ST>(p.ks, sbase + pg * p.sc_ps + soff);
      sv[u] = load_scale<ST>(p.vs, sbase + pg * p.sc_ps + soff);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float dot = 0.0f;
#pragma unroll
      for (int k = 0; k < NWORD; ++k) {
        uint32_t r[4];
        unpack_biased64(kw[u].word(k), r);
#pragma unroll
        for (int j = 0; j < 4; ++j) dot = __builtin_amdgcn_fdot2(as_half2(r[j]), qp[k][j], dot, false);
      }
      float s = (dot - bias) * sk[u];
      s += xor1(s);
      s += xor2(s);
      const int32_t tok = lp[u] * 16 + t;
      const bool valid = ok[u] && tok < kr.hi && (tok >= kr.win_lo || tok < kr.sink_end);
      s = valid ? s * p.qk_scale_log2 : -INFINITY;

      if (__any(s > m + 8.0f)) {  // wave-uniform, rare after the first pages
        const float mn = fmaxf(m, wave_max(s));
        const float alpha = (mn == m) ? 1.0f : fast_exp2(m - mn);
        l *= alpha;
#pragma unroll
        for (int d = 0; d < DPL; ++d) acc[d] *= alpha;
        m = mn;
      }
      const float pw = valid ? fast_exp2(s - m) : 0.0f;
      l += pw;
      const float wv = valid ? pw * sv[u] : 0.0f;  // a scale past the context may be NaN
#pragma unroll
      for (int k = 0; k < NWORD; ++k) {
        half2_t hv[4];
        unpack_exact(vw[u].word(k), hv);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[8 * k + 2 * j] = fmaf(wv, (float)hv[j].x, acc[8 * k + 2 * j]);
          acc[8 * k + 2 * j + 1] = fmaf(wv, (float)hv[j].y, acc[8 * k + 2 * j + 1]);
        }
      }
    }
  }

  // Sum the 16 token slots sharing this lane's dims (lanes c, c+4, ..., c+60);
  // m is wave-uniform, so partials add directly. l counts each token once per c.
  l += dpp_f32<0x124>(l);  // row_ror:4
  l += dpp_f32<0x128>(l);  // row_ror:8
  l = xor16_sum(l);
  l = xor32_sum(l);
#pragma unroll
  for (int d = 0; d < DPL; ++d) {
    float v = acc[d];
    v += dpp_f32<0x124>(v);
    v += dpp_f32<0x128>(v);
    v = xor16_sum(v);
    v = xor32_sum(v);
    acc[d] = v;
  }
  if (t == 0) {
#pragma unroll
    for (int s = 0; s < DPL; ++s) s_acc[wave][c * DPL + 8 * (s >> 3) + kSlotDim[s & 7]] = acc[s];
    if (c == 0) {
      s_ml[wave][0] = m;
      s_ml[wave][1] = l;
    }
  }
  __syncthreads();
  decode_epilogue<D, NW>(p, (int64_t)b * p.H + h, split, s_acc, s_ml);
}

// Decode over this build's INT4 page format (page_format.hpp): lane l = 8p + c
// owns tokens (p, p+8) and dims [c*D/8, (c+1)*D/8) of a (page, head) block.
// The two partial dots of a lane reduce over its 8-lane group with 3 DPP
// moves; V accumulates both tokens per instruction with v_dot2_f32_f16
// against the fp16 pair of softmax weights (times V scales).
template <int D, int NW, int U>
__global__ __launch_bounds__(NW * 64) void decode_int4_pages_kernel(const DecodeParams p) {
  constexpr int BPL = D / 8;     // bytes per lane per code region
  constexpr int DPL = D / 8;     // dims per lane
  constexpr int KW = BPL / 8;    // K words per token
  constexpr int VW = BPL / 4;    // V words (4 dims x 2 tokens each)
  using Chunk = LaneChunk<D>;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int32_t b = blockIdx.z, h = blockIdx.y, split = blockIdx.x;
  const int pp = lane >> 3, c = lane & 7;
  const int g = (c * DPL) / 64;

  __shared__ float s_acc[NW][D];
  __shared__ float s_ml[NW][2];

  const int32_t ctx = p.ctx[b];
  const KeyRange kr = key_range(ctx, ctx - 1, p.W, p.sinks, false);
  const int32_t last_page = min((kr.hi + 15) >> 4, p.M);
  const int32_t sink_pages = min((kr.sink_end + 15) >> 4, last_page);
  const int32_t win_page0 = max(kr.win_lo >> 4, sink_pages);
  const int32_t n_win = max(0, last_page - win_page0);
  const int64_t n_vis = (int64_t)sink_pages + n_win;
  const SplitRange sr = split_range((int32_t)n_vis, split, p.splits);
  const int32_t begin = sr.begin, end = sr.end;

  // q for this lane's dims as fp16 pairs in unpack order; the dot products
  // start from -q . (bias + 8) so they end at q . (code - 8).
  half2_t qp[KW][4];
  float bias = 0.0f;
  {
    const half_t *qrow = p.q + ((int64_t)b * p.H + h) * D + c * DPL;
#pragma unroll
    for (int k = 0; k < KW; ++k) {
      const uint4 u = *reinterpret_cast<const uint4 *>(qrow + 8 * k);
      const half2_t e01 = as_half2(u.x), e23 = as_half2(u.y), e45 = as_half2(u.z), e67 = as_half2(u.w);
      qp[k][0] = half2_t{e01.x, e45.x};
      qp[k][1] = half2_t{e01.y, e45.y};
      qp[k][2] = half2_t{e23.x, e67.x};
      qp[k][3] = half2_t{e23.y, e67.y};
      bias = fmaf(1032.0f, ((float)e01.x + (float)e45.x) + ((float)e23.x + (float)e67.x), bias);
      bias = fmaf(72.0f, ((float)e01.y + (float)e45.y) + ((float)e23.y + (float)e67.y), bias);
    }
  }

  // acc accumulates weight * (code - 8) over exact fp16 code values: no bias
  // rides along, so a heavy token adds nothing to dims where its code is 8,
  // and the fp32 rounding of each v_dot2 stays relative to the output itself.
  // m starts finite so that exp2(-inf - m) = 0 needs no select for masked
  // tokens; the first visible score raises it.
  float m = -3.0e38f, l = 0.0f;
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.0f;

  const int32_t *btrow = p.bt + (int64_t)b * p.M;
  // Uniform (scalar) block base per page + 32-bit per-lane byte offsets.
  const uint8_t *hbase = p.kc + (int64_t)h * p.kv_hs;
  const uint32_t koff = lane * BPL;
  const uint32_t voff = (uint32_t)(p.vc - p.kc) + lane * BPL;
  const uint32_t ksoff = (uint32_t)((const uint8_t *)p.ks - p.kc) + 2 * (g * 16 + 2 * pp);
  const uint32_t vsoff = (uint32_t)((const uint8_t *)p.vs - p.kc) + 2 * (g * 16 + 2 * pp);
  const int32_t nb32 = (int32_t)min(p.nb, (int64_t)INT32_MAX);

  // Page batches of U pages are double-buffered: the loads of batch n+1 are
  // in flight while batch n is consumed. Slots past their limit (and
  // unlinked pages) load page 0 of this head, which is always mapped and
  // L2-resident after the first touch, and are masked out.
  struct Batch {
    Chunk kw[U], vw[U];
    half2_t sk[U], sv[U];
    int32_t lp[U];
    bool ok[U];
  };
  auto issue_lim = [&](Batch &bt, int32_t base, int32_t lim) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int32_t i = base + u;
      bt.lp[u] = (i < sink_pages) ? i : win_page0 + (i - sink_pages);
      const int32_t phys = btrow[(i < lim) ? bt.lp[u] : 0];  // lp < M whenever i < lim <= end
      bt.ok[u] = (i < lim) && phys >= 0 && phys < nb32;
      const int64_t pg = bt.ok[u] ? (int64_t)phys : 0;
      const __amdgpu_buffer_rsrc_t r = block_rsrc(uniform_ptr(hbase + pg * p.kv_ps));
      bt.kw[u].load(r, koff);
      bt.vw[u].load(r, voff);
      bt.sk[u] = as_half2(__builtin_amdgcn_raw_buffer_load_b32(r, (int)ksoff, 0, kStreamLoad));
      bt.sv[u] = as_half2(__builtin_amdgcn_raw_buffer_load_b32(r, (int)vsoff, 0, kStreamLoad));
    }
  };
  auto issue = [&](Batch &bt, int32_t base) { issue_lim(bt, base, end); };
  auto consume = [&](const Batch &bt) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float d0 = -bias, d1 = -bias;
#pragma unroll
      for (int k = 0; k < KW; ++k) {
        uint32_t r0[4], r1[4];
        unpack_biased(bt.kw[u].word(k), r0);
        unpack_biased(bt.kw[u].word(KW + k), r1);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          d0 = __builtin_amdgcn_fdot2(as_half2(r0[j]), qp[k][j], d0, false);
          d1 = __builtin_amdgcn_fdot2(as_half2(r1[j]), qp[k][j], d1, false);
        }
      }
      float s0 = d0 * (float)bt.sk[u].x, s1 = d1 * (float)bt.sk[u].y;
      s0 += xor1(s0);
      s1 += xor1(s1);
      s0 += xor2(s0);
      s1 += xor2(s1);
      s0 += half_mirror(s0);
      s1 += half_mirror(s1);
      s0 *= p.qk_scale_log2;
      s1 *= p.qk_scale_log2;
      // Whole page inside the window (the common case): no per-token mask.
      const int32_t tok0 = bt.lp[u] * 16;
      half2_t sv = bt.sv[u];
      if (!(bt.ok[u] && tok0 >= kr.win_lo && tok0 + 16 <= kr.hi)) {  // wave-uniform
        const int32_t t0 = tok0 + pp, t1 = t0 + 8;
        const bool v0 = bt.ok[u] && t0 < kr.hi && (t0 >= kr.win_lo || t0 < kr.sink_end);
        const bool v1 = bt.ok[u] && t1 < kr.hi && (t1 >= kr.win_lo || t1 < kr.sink_end);
        s0 = v0 ? s0 : -INFINITY;
        s1 = v1 ? s1 : -INFINITY;
        // Masked tokens may carry any scale bits (NaN past the context).
        sv = half2_t{v0 ? sv.x : (half_t)0.0f, v1 ? sv.y : (half_t)0.0f};
      }
      const float smax = fmaxf(s0, s1);
      if (__any(smax > m + 8.0f)) {  // wave-uniform, rare after the first pages
        const float mn = fmaxf(m, wave_max(smax));
        const float alpha = (mn == m) ? 1.0f : fast_exp2(m - mn);
        l *= alpha;
#pragma unroll
        for (int d = 0; d < DPL; ++d) acc[d] *= alpha;
        m = mn;
      }
      float p0 = fast_exp2(s0 - m);  // masked tokens: s = -inf, p = 0
      float p1 = fast_exp2(s1 - m);
      // The V weights p * (V scale) enter the accumulation as fp16, so they
      // must stay finite: p reaches 2^8 under the lazy max and a V scale
      // reaches 9352, past 65504. When a weight of the wave exceeds 2^15
      // (possible only for V scales above 128), the reference point m is
      // raised by the integer e that brings the largest weight to <= 2^14,
      // and everything accumulated so far is scaled by 2^-e. The softmax is
      // unchanged (m cancels in o / l); weights far below the largest one
      // lose nothing that shows in the output.
      const float sv0 = (float)sv.x, sv1 = (float)sv.y;
      float x0 = p0 * sv0, x1 = p1 * sv1;
      if (__any(fmaxf(x0, x1) > 32768.0f)) {  // wave-uniform
        const float e = ceilf(__log2f(wave_max(fmaxf(x0, x1)))) - 14.0f;
        const float alpha = fast_exp2(-e);
        l *= alpha;
#pragma unroll
        for (int d = 0; d < DPL; ++d) acc[d] *= alpha;
        m += e;
        p0 *= alpha;
        p1 *= alpha;
        x0 *= alpha;
        x1 *= alpha;
      }
      l += p0 + p1;
      const half2_t wpair = {(half_t)x0, (half_t)x1};
#pragma unroll
      for (int k = 0; k < VW; ++k) {
        half2_t hv[4];
        unpack_exact(bt.vw[u].word(k), hv);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[4 * k + j] = __builtin_amdgcn_fdot2(hv[j], wpair, acc[4 * k + j], false);
      }
    }
  };

  // The (end - begin) % kStep pages left over by whole steps come first,
  // one batch to each of the first waves, issued together with that wave's
  // first regular batch: every wave then runs the same number of steps, and
  // a leftover page does not cost the workgroup a last step of its own.
  constexpr int32_t kStep = NW * U;
  const int32_t rem = (end - begin) % kStep, rbeg = begin + rem;
  const bool extra = wave * U < rem;  // wave-uniform
  Batch ba, bb;
  int32_t base = rbeg + wave * U;
  if (extra) issue_lim(bb, begin + wave * U, rbeg);
  issue(ba, base);
  if (extra) consume(bb);
  while (base < end) {
    issue(bb, base + kStep);
    consume(ba);
    base += kStep;
    if (base >= end) break;
    issue(ba, base + kStep);
    consume(bb);
    base += kStep;
  }

  // Sum the 8 token-pair lanes sharing this lane's dims (lanes c, c+8, ...).
  l += dpp_f32<0x128>(l);  // row_ror:8
  l = xor16_sum(l);
  l = xor32_sum(l);
#pragma unroll
  for (int d = 0; d < DPL; ++d) {
    float v = acc[d];
    v += dpp_f32<0x128>(v);
    v = xor16_sum(v);
    v = xor32_sum(v);
    acc[d] = v;
  }
  if (pp == 0) {
#pragma unroll
    for (int d = 0; d < DPL; ++d) s_acc[wave][c * DPL + d] = acc[d];
    if (c == 0) {
      s_ml[wave][0] = m;
      s_ml[wave][1] = l;
    }
  }
  __syncthreads();
  decode_epilogue<D, NW>(p, (int64_t)b * p.H + h, split, s_acc, s_ml);
}

static int device_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
      cus = prop.multiProcessorCount;
    if (cus <= 0) cus = 256;
  }
  return cus;
}

// Launch shape (waves per workgroup, pages per double-buffered batch). The
// default (8, 1) measured fastest on MI355X for 16 x 32 heads x 4096 tokens
// with streaming loads: 47.6-48.8 us against 49.0-49.7 for (4, 2) and 51-55
// for shapes with more pages in flight per CU ((4, 4), (8, 2), (8, 4),
// (16, 2), triple buffering), which lose more to the memory system than
// they hide; MEMOPT_DECODE_SHAPE="NW,U" selects another compiled shape.
struct DecodeShape {
  int nw, u;
};
static DecodeShape decode_shape() {
  DecodeShape s = {8, 1};
  if (const char *e = std::getenv("MEMOPT_DECODE_SHAPE")) {
    int a = 0, c = 0;
    if (std::sscanf(e, "%d,%d", &a, &c) == 2 &&
        ((a == 4 && c == 2) || (a == 8 && c == 1) || (a == 8 && c == 2) || (a == 8 && c == 4) ||
         (a == 16 && c == 2) || (a == 4 && c == 4)))
      s = {a, c};
  }
  return s;
}

int decode_splits(int32_t batch, int32_t heads, int32_t max_pages_visited) {
  const int64_t units = (int64_t)batch * heads;
  if (units <= 0) return 1;
  const DecodeShape sh = decode_shape();
  // About 2 workgroups per CU; 3 when the batch has fewer (b, h) units than
  // CUs (config 5's 128 units: 6 splits measured 1.5 % faster than 4, and
  // 2, 3 or 8 slower).
  const int64_t target_wgs = (units < device_cus() ? 3LL : 2LL) * device_cus();
  int64_t s = (target_wgs + units - 1) / units;
  // Keep at least 4 page batches per wave.
  const int64_t cap = max_pages_visited / (4LL * sh.nw * sh.u);
  if (s > cap) s = cap;
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  if (const char *e = std::getenv("MEMOPT_DECODE_SPLITS")) {
    const int v = std::atoi(e);
    if (v >= 1 && v <= 64) s = v;
  }
  return (int)s;
}

template <int D, typename ST>
static void launch_shape(const DecodeParams &p, dim3 grid, DecodeShape sh, hipStream_t stream) {
#define MEMOPT_DECODE_CASE(NW_, U_)                                                                   \
  if (sh.nw == NW_ && sh.u == U_) {                                                                   \
    if (p.pages)                                                                                      \
      hipLaunchKernelGGL((decode_int4_pages_kernel<D, NW_, U_>), grid, dim3(NW_ * 64), 0, stream, p); \
    else                                                                                              \
      hipLaunchKernelGGL((decode_int4_kernel<D, ST, NW_, U_>), grid, dim3(NW_ * 64), 0, stream, p);  \
    return;                                                                                           \
  }
  MEMOPT_DECODE_CASE(4, 2)
  MEMOPT_DECODE_CASE(8, 2)
  MEMOPT_DECODE_CASE(8, 1)
  MEMOPT_DECODE_CASE(8, 4)
  MEMOPT_DECODE_CASE(4, 4)
  MEMOPT_DECODE_CASE(16, 2)
#undef MEMOPT_DECODE_CASE
}

int launch_decode_int4(const DecodeParams &p, int32_t batch, int32_t D, int32_t scale_dtype,
                       hipStream_t stream) {
  const DecodeShape sh = decode_shape();
  const dim3 grid(p.splits, p.H, batch);
  if (D == 128 && scale_dtype == MEMOPT_SCALE_F16)
    launch_shape<128, half_t>(p, grid, sh, stream);
  else if (D == 128)
    launch_shape<128, float>(p, grid, sh, stream);
  else if (scale_dtype == MEMOPT_SCALE_F16)
    launch_shape<64, half_t>(p, grid, sh, stream);
  else
    launch_shape<64, float>(p, grid, sh, stream);
  return check_launch("paged_attention(decode_int4)");
}

unsigned long long next_decode_tag() {
  static std::atomic<unsigned long long> calls{0};
  return (calls.fetch_add(1, std::memory_order_relaxed) % ((1ull << 56) - 1)) + 1;
}

}  // namespace memopt
