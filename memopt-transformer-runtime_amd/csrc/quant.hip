// quant.hip — group-64 INT4 quantize / dequantize and the paged write path.
//
// Reference semantics: TheRadDani/memopt-transformer-runtime
//   src/csrc/quantization.cu:104-203 (quantize), :232-270 (dequantize),
//   src/csrc/kv_cache.cu:228-260   (write_cache scatter).
//
// gfx950 mapping: a 64-element group is 128 contiguous bytes of fp16, read as
// one 16-byte load by each of 8 consecutive lanes; the group absmax is a
// 3-step DPP max inside those 8 lanes (no LDS, no barrier); each lane packs its
// 8 codes into one 32-bit word, so a wave reads 1 KiB and writes 256 B of codes
// per step, fully coalesced. The same device routine quantizes token rows
// straight into INT4 pages in write_cache (fused write + quantize).
#include "common.hpp"
#include "page_format.hpp"

namespace memopt {

static constexpr int kThreads = 256;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Workgroups for work_items (one per thread) up to `cap`. The surface
// quantize, dequantize and fp16 scatter launch one item (quantize and
// dequantize: four chunks) per thread with no practical cap: a grid-stride
// loop capped at 16384 workgroups kept one 16-byte load per thread in flight
// at a time (config 2's pool tensor: quantize 0.67 -> 0.72 of HBM with one
// chunk per thread, dequantize 0.77 -> 0.85).
static inline unsigned grid_for(int64_t work_items, int64_t cap = 16384) {
  int64_t g = (work_items + kThreads - 1) / kThreads;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned)g;
}

template <bool VEC>
__device__ __forceinline__ void load8(const half_t *p, float f[8]) {
  if (VEC) {
    unpack_half8(*reinterpret_cast<const uint4 *>(p), f);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)p[i];
  }
}

// One lane = 8 consecutive elements; chunk i covers elements [8i, 8i+8).
// VEC: four chunks per thread, i0 + r * stride, all four non-temporal loads
// issued before any is used (indices past the end load the last chunk and
// store nothing; a group's 8 chunks are all in range or all out, as n_chunks
// is a multiple of 8). With one chunk per thread, a launch of config 2's
// pool tensor had four times the workgroups and ran at 0.72 of HBM, with
// four 0.77 (eight 0.67).
static constexpr int kQuantChunks = 4;
template <bool VEC>
__global__ __launch_bounds__(kThreads) void quantize_kernel(const half_t *__restrict__ in,
                                                            uint8_t *__restrict__ packed,
                                                            float *__restrict__ scales,
                                                            int64_t n_chunks) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  if constexpr (VEC) {
    constexpr int R = kQuantChunks;
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    for (int64_t i0 = (int64_t)blockIdx.x * kThreads + threadIdx.x; i0 < n_chunks; i0 += R * stride) {
      u4v x[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t i = min(i0 + r * stride, n_chunks - 1);
        x[r] = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(in + i * 8));
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t i = i0 + r * stride;
        float v[8];
        unpack_half8(make_uint4(x[r].x, x[r].y, x[r].z, x[r].w), v);
        float s;
        const uint32_t w = quantize8(v, s);  // every lane of a group takes part (DPP absmax)
        if (i < n_chunks) {
          reinterpret_cast<uint32_t *>(packed)[i] = w;
          if ((i & 7) == 0) scales[i >> 3] = s;
        }
      }
    }
  } else {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n_chunks; i += stride) {
      float v[8];
      load8<VEC>(in + i * 8, v);
      float s;
      const uint32_t w = quantize8(v, s);
#pragma unroll
      for (int b = 0; b < 4; ++b) packed[i * 4 + b] = (uint8_t)(w >> (8 * b));
      if ((i & 7) == 0) scales[i >> 3] = s;
    }
  }
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void dequantize_kernel(const uint8_t *__restrict__ packed,
                                                              const float *__restrict__ scales,
                                                              half_t *__restrict__ out,
                                                              int64_t n_chunks) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  auto expand = [](uint32_t w, float s) {
    half_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (half_t)((float)((int)((w >> (4 * e)) & 0xF) - 8) * s);
    return make_uint4(as_u32(half2_t{h[0], h[1]}), as_u32(half2_t{h[2], h[3]}), as_u32(half2_t{h[4], h[5]}),
                      as_u32(half2_t{h[6], h[7]}));
  };
  if constexpr (VEC) {
    // Four chunks per trip, all loads issued before any is used: one 4-byte
    // load per trip left too few bytes in flight to cover HBM latency.
    constexpr int R = 4;
    for (int64_t i0 = (int64_t)blockIdx.x * kThreads + threadIdx.x; i0 < n_chunks; i0 += R * stride) {
      uint32_t w[R];
      float sc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t i = min(i0 + r * stride, n_chunks - 1);
        w[r] = reinterpret_cast<const uint32_t *>(packed)[i];
        sc[r] = scales[i >> 3];
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int64_t i = i0 + r * stride;
        if (i < n_chunks) {
          const uint4 o = expand(w[r], sc[r]);
          typedef uint32_t u4v __attribute__((ext_vector_type(4)));
          __builtin_nontemporal_store((u4v){o.x, o.y, o.z, o.w}, reinterpret_cast<u4v *>(out + i * 8));
        }
      }
    }
  } else {
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n_chunks; i += stride) {
      uint32_t w = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) w |= (uint32_t)packed[i * 4 + b] << (8 * b);
      const uint4 o = expand(w, scales[i >> 3]);
      const uint32_t ow[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) out[i * 8 + e] = as_half2(ow[e >> 1])[e & 1];
    }
  }
}

// fp16 pool scatter: chunk i = 8 halves of token (i / cpr); cpr = H*D/8.
__global__ __launch_bounds__(kThreads) void write_fp16_kernel(
    const uint4 *__restrict__ keys, const uint4 *__restrict__ values, uint4 *__restrict__ kpool,
    uint4 *__restrict__ vpool, const int32_t *__restrict__ slots, int64_t n_chunks, int64_t cpr,
    int64_t n_slots) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  // 32-bit token index when it fits (a 64-bit division expands to a long
  // sequence); the pool rows are written with non-temporal stores (nothing
  // reads them back soon): 79 us per launch, 0.85 of HBM, on 16384 tokens x
  // 32 x 128 (non-temporal loads as well: slower).
  if (n_chunks < (1LL << 31) && cpr < (1LL << 31)) {
    const uint32_t cp = (uint32_t)cpr;
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n_chunks; i += stride) {
      const uint32_t t = (uint32_t)i / cp, c = (uint32_t)i - t * cp;
      const int64_t slot = slots[t];
      if (slot < 0 || slot >= n_slots) continue;
      const u4v kx = *reinterpret_cast<const u4v *>(keys + i);
      const u4v vx = *reinterpret_cast<const u4v *>(values + i);
      __builtin_nontemporal_store(kx, reinterpret_cast<u4v *>(kpool + slot * cpr + c));
      __builtin_nontemporal_store(vx, reinterpret_cast<u4v *>(vpool + slot * cpr + c));
    }
    return;
  }
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n_chunks; i += stride) {
    const int64_t t = i / cpr, c = i - t * cpr;
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= n_slots) continue;
    kpool[slot * cpr + c] = keys[i];
    vpool[slot * cpr + c] = values[i];
  }
}

__global__ __launch_bounds__(kThreads) void write_fp16_scalar_kernel(
    const half_t *__restrict__ keys, const half_t *__restrict__ values, half_t *__restrict__ kpool,
    half_t *__restrict__ vpool, const int32_t *__restrict__ slots, int64_t n, int64_t row,
    int64_t n_slots) {
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
    const int64_t t = i / row, c = i - t * row;
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= n_slots) continue;
    kpool[slot * row + c] = keys[i];
    vpool[slot * row + c] = values[i];
  }
}

// Fused write + quantize into the INT4 page pool (page_format.hpp). Chunk i =
// 8 elements (dims 8cc..8cc+7) of the (token, head) row; all 8 lanes of a
// 64-element group take the same branch, as quantize8's DPP reduction needs.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void write_int4_kernel(
    const half_t *__restrict__ keys, const half_t *__restrict__ values, uint8_t *__restrict__ pool,
    const int32_t *__restrict__ slots, int64_t n_chunks, int32_t H, int32_t D, int64_t n_slots) {
  const Int4Page f(D);
  const int64_t stride = (int64_t)gridDim.x * kThreads;
  const int32_t cpr = D / 8;  // chunks per (token, head) row
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n_chunks; i += stride) {
    const int64_t th = i / cpr;
    const int32_t cc = (int32_t)(i - th * cpr);
    const int64_t t = th / H;
    const int32_t h = (int32_t)(th - t * H);
    const int64_t slot = slots[t];
    float kv[8], vv[8];
    load8<VEC>(keys + i * 8, kv);
    load8<VEC>(values + i * 8, vv);
    float s_k, s_v;
    const uint32_t wk = quantize8(kv, s_k);
    const uint32_t wv = quantize8(vv, s_v);
    if (slot < 0 || slot >= n_slots) continue;
    const int64_t page = slot >> 4;
    const int32_t pos = (int32_t)(slot & 15), d0 = 8 * cc;
    uint8_t *blk = pool + (page * H + h) * f.block;
    *reinterpret_cast<uint32_t *>(blk + f.kcodes + f.k_byte(pos, d0)) = wk;
    uint8_t *vb = blk + f.vcodes + f.v_byte(pos, d0);
    *reinterpret_cast<uint16_t *>(vb) = (uint16_t)(wv & 0xFFFFu);
    *reinterpret_cast<uint16_t *>(vb + 4) = (uint16_t)(wv >> 16);
    if ((d0 & 63) == 0) {
      reinterpret_cast<half_t *>(blk + f.kscales)[f.scale_idx(pos, d0 >> 6)] = page_scale(s_k);
      reinterpret_cast<half_t *>(blk + f.vscales)[f.scale_idx(pos, d0 >> 6)] = page_scale(s_v);
    }
  }
}

// Fused write + quantize, one wave per (group of 16 tokens, head, K or V).
//  * Full page: when the group's 16 slots are one aligned page (slot of token
//    t0 + i = 16 P + i), the wave builds the (page, head) block in its page
//    layout: lane l = 8p + c quantizes tokens p and p + 8 over the dims
//    [c*D/8, (c+1)*D/8) and stores exactly the bytes it owns, K and V codes as
//    one 16-byte (D = 128) or 8-byte (D = 64) store each, the group scales as
//    one 4-byte store per token pair. 64-groups span 4 (D = 128) or 8 (D = 64)
//    lanes.
//  * Otherwise (decode appends, ragged tails, arbitrary slots) it scatters
//    8-element chunks like write_int4_kernel.
// 32-bit indexing: requires T * H * D < 2^31 (checked by the caller).
template <int D>
__global__ __launch_bounds__(kThreads) void write_int4_pages_kernel(
    const half_t *__restrict__ keys, const half_t *__restrict__ values, uint8_t *__restrict__ pool,
    const int32_t *__restrict__ slots, uint32_t T, uint32_t H, int64_t n_slots) {
  constexpr int DPL = D / 8;    // dims per lane per token in the page layout
  constexpr int GL = 64 / DPL;  // lanes per 64-group
  constexpr int CPR = D / 8;    // 8-element chunks per (token, head) row
  constexpr int KW = DPL / 8;   // packed words per token and lane
  const Int4Page f(D);
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t wid2 = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  const bool is_v = wid2 & 1;  // wave-uniform
  const uint32_t wid = wid2 >> 1;
  const uint32_t g = wid / H, h = wid - g * H;
  const uint32_t t0 = g * 16;
  if (t0 >= T) return;  // wave-uniform
  const size_t rowstride = (size_t)H * D;  // elements per token
  const half_t *__restrict__ src = is_v ? values : keys;
  const int64_t codes_off = is_v ? f.vcodes : f.kcodes, scales_off = is_v ? f.vscales : f.kscales;

  // The full-page path's loads do not depend on the slots, so they are issued
  // before the slot check (rows clamped to T - 1; unused when the group
  // scatters) and overlap its round trip: 2 x [16384, 32, 128] went from
  // 0.80 to 0.84-0.86 of HBM.
  const int p = lane >> 3, c = lane & 7;
  uint4 raw[2][KW];
#pragma unroll
  for (int tk = 0; tk < 2; ++tk) {
    const uint32_t row = min(t0 + p + 8 * tk, T - 1);
    const size_t o = (size_t)row * rowstride + (size_t)h * D + c * DPL;
#pragma unroll
    for (int k = 0; k < KW; ++k) raw[tk][k] = *reinterpret_cast<const uint4 *>(src + o + 8 * k);
  }
  int32_t sl = -1;
  if (lane < 16 && t0 + lane < T) sl = slots[t0 + lane];
  const int32_t s0 = __builtin_amdgcn_readfirstlane(sl);
  const bool mine = lane >= 16 || sl == s0 + (int32_t)lane;
  const bool full = __all(mine) && s0 >= 0 && (s0 & 15) == 0 && (int64_t)s0 + 16 <= n_slots;

  if (full) {
    float x[2][DPL];
#pragma unroll
    for (int tk = 0; tk < 2; ++tk)
#pragma unroll
      for (int k = 0; k < KW; ++k) unpack_half8(raw[tk][k], &x[tk][8 * k]);
    float am[2];
#pragma unroll
    for (int tk = 0; tk < 2; ++tk) {
      float a = 0.0f;
#pragma unroll
      for (int i = 0; i < DPL; ++i) a = fmaxf(a, fabsf(x[tk][i]));
      am[tk] = group_absmax<GL>(a);
    }
    // One reciprocal for both tokens: the group's lanes hold both absmaxes,
    // even lanes take token p's and odd lanes token p + 8's, and lane pairs
    // swap their results.
    const bool odd = lane & 1;
    const float s_own = scale_of(odd ? am[1] : am[0]);
    const float y_own = 1.0f / s_own;
    const float s_oth = xor1(s_own), y_oth = xor1(y_own);
    const float sc[2] = {odd ? s_oth : s_own, odd ? s_own : s_oth};
    const float yy[2] = {odd ? y_oth : y_own, odd ? y_own : y_oth};
    uint32_t wd[2][KW];
#pragma unroll
    for (int tk = 0; tk < 2; ++tk) int4_pack<DPL>(x[tk], sc[tk], yy[tk], wd[tk]);
    uint8_t *blk = pool + ((int64_t)(s0 >> 4) * H + h) * f.block;
    uint32_t out[2 * KW];
    if (!is_v) {
      // K: token p's bytes, then token p + 8's
#pragma unroll
      for (int k = 0; k < KW; ++k) {
        out[k] = wd[0][k];
        out[KW + k] = wd[1][k];
      }
    } else {
      // V unit u (4 dims) = 2 bytes of token p, then 2 bytes of token p + 8
#pragma unroll
      for (int u = 0; u < 2 * KW; ++u) {
        const uint32_t lo = wd[0][u >> 1] >> (16 * (u & 1)), hi = wd[1][u >> 1] >> (16 * (u & 1));
        out[u] = (lo & 0xFFFFu) | (hi << 16);
      }
    }
    // Streaming stores (codes here, scales below): nothing in this launch
    // re-reads them; measured 13% faster than plain stores.
    if constexpr (D == 128) {
      const u32x4_t w = {out[0], out[1], out[2], out[3]};
      __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t *>(blk + codes_off + lane * f.BPL));
    } else {
      const u32x2_t w = {out[0], out[1]};
      __builtin_nontemporal_store(w, reinterpret_cast<u32x2_t *>(blk + codes_off + lane * f.BPL));
    }
    if (c % GL == 0)
      __builtin_nontemporal_store(as_u32(half2_t{page_scale(sc[0]), page_scale(sc[1])}),
                                  reinterpret_cast<uint32_t *>(blk + scales_off + 2 * f.scale_idx(p, (c * DPL) / 64)));
    return;
  }

#pragma unroll
  for (int u = 0; u < 16 * CPR / 64; ++u) {
    const uint32_t j = u * 64 + lane;
    const uint32_t t = t0 + j / CPR, cc = j % CPR;
    if (t >= T) continue;  // a token's CPR (>= 8) chunks leave together: 64-groups stay whole
    float x[8];
    unpack_half8(*reinterpret_cast<const uint4 *>(src + (size_t)t * rowstride + (size_t)h * D + cc * 8), x);
    float sc;
    const uint32_t w = quantize8(x, sc);
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= n_slots) continue;
    const int32_t pos = (int32_t)(slot & 15), d0 = 8 * (int32_t)cc;
    uint8_t *blk = pool + ((slot >> 4) * H + h) * f.block;
    if (!is_v) {
      *reinterpret_cast<uint32_t *>(blk + f.kcodes + f.k_byte(pos, d0)) = w;
    } else {
      uint8_t *vb = blk + f.vcodes + f.v_byte(pos, d0);
      *reinterpret_cast<uint16_t *>(vb) = (uint16_t)(w & 0xFFFFu);
      *reinterpret_cast<uint16_t *>(vb + 4) = (uint16_t)(w >> 16);
    }
    if ((d0 & 63) == 0) reinterpret_cast<half_t *>(blk + scales_off)[f.scale_idx(pos, d0 >> 6)] = page_scale(sc);
  }
}

// INT4 page pool -> fp16 pools [nb, 16, H, D] (K and V): one wave per
// (page, head), lane l = 8p + c decodes tokens p and p + 8 over dims
// [c D/8, (c+1) D/8) (page_format.hpp). value = fp16(RN(float(code - 8) *
// scale)) with the page's fp16 scale, the values the attention kernels use.
template <int D>
__global__ __launch_bounds__(256) void int4_pages_to_fp16_kernel(const uint8_t *__restrict__ pages, int64_t units,
                                                                 int32_t H, half_t *__restrict__ kout,
                                                                 half_t *__restrict__ vout) {
  constexpr int DPL = D / 8;
  const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (unit >= units) return;
  const Int4Page f(D);
  const int lane = threadIdx.x & 63, p = lane >> 3, c = lane & 7, g = (c * DPL) / 64;
  const int64_t page = unit / H;
  const int32_t h = (int32_t)(unit % H);
  const uint8_t *blk = pages + unit * f.block;
  const half_t *ksc = reinterpret_cast<const half_t *>(blk + f.kscales);
  const half_t *vsc = reinterpret_cast<const half_t *>(blk + f.vscales);
  const uint8_t *kb = blk + f.kcodes + lane * DPL, *vb = blk + f.vcodes + lane * DPL;
#pragma unroll
  for (int tok = 0; tok < 2; ++tok) {
    const float sk = (float)ksc[g * 16 + 2 * p + tok], sv = (float)vsc[g * 16 + 2 * p + tok];
    half_t ko[DPL], vo[DPL];
#pragma unroll
    for (int i = 0; i < DPL / 2; ++i) {
      const uint32_t byte = kb[tok * (DPL / 2) + i];
      ko[2 * i] = (half_t)((float)((int)(byte & 15u) - 8) * sk);
      ko[2 * i + 1] = (half_t)((float)((int)(byte >> 4) - 8) * sk);
    }
#pragma unroll
    for (int u = 0; u < DPL / 4; ++u) {
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const uint32_t byte = vb[4 * u + 2 * tok + b];
        vo[4 * u + 2 * b] = (half_t)((float)((int)(byte & 15u) - 8) * sv);
        vo[4 * u + 2 * b + 1] = (half_t)((float)((int)(byte >> 4) - 8) * sv);
      }
    }
    const int64_t row = ((page * 16 + p + 8 * tok) * H + h) * (int64_t)D + c * DPL;
#pragma unroll
    for (int i = 0; i < DPL / 8; ++i) {
      *reinterpret_cast<uint4 *>(kout + row + 8 * i) = *reinterpret_cast<const uint4 *>(ko + 8 * i);
      *reinterpret_cast<uint4 *>(vout + row + 8 * i) = *reinterpret_cast<const uint4 *>(vo + 8 * i);
    }
  }
}

}  // namespace memopt

using namespace memopt;

static inline bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

extern "C" {

int memopt_quantize_kv_cache_int4(const void *cache, int64_t numel, int64_t last_dim,
                                  int32_t group_size, uint8_t *packed_out, float *scales_out,
                                  void *stream) {
  MEMOPT_REQUIRE(group_size == 64, MEMOPT_ERR_INVALID,
                 "quantize_kv_cache_int4: group_size must equal 64 (got " + std::to_string(group_size) + ")");
  MEMOPT_REQUIRE(numel % 64 == 0, MEMOPT_ERR_INVALID,
                 "quantize_kv_cache_int4: total_elements (" + std::to_string(numel) +
                     ") must be divisible by group_size (64)");
  MEMOPT_REQUIRE(last_dim % 2 == 0, MEMOPT_ERR_INVALID,
                 "quantize_kv_cache_int4: last dimension (" + std::to_string(last_dim) +
                     ") must be even for INT4 packing");
  if (numel == 0) return MEMOPT_OK;
  MEMOPT_REQUIRE(cache && packed_out && scales_out, MEMOPT_ERR_INVALID, "quantize_kv_cache_int4: null pointer");
  const int64_t n_chunks = numel / 8;
  hipStream_t s = (hipStream_t)stream;
  const bool vec = aligned(cache, 16) && aligned(packed_out, 4);
  if (vec)
    hipLaunchKernelGGL(quantize_kernel<true>,
                       dim3(grid_for((n_chunks + kQuantChunks - 1) / kQuantChunks, 1LL << 30)), dim3(kThreads), 0, s,
                       (const half_t *)cache, packed_out, scales_out, n_chunks);
  else
    hipLaunchKernelGGL(quantize_kernel<false>, dim3(grid_for(n_chunks)), dim3(kThreads), 0, s,
                       (const half_t *)cache, packed_out, scales_out, n_chunks);
  return check_launch("quantize_kv_cache_int4");
}

int memopt_dequantize_kv_cache_int4(const uint8_t *packed, int64_t packed_numel, const float *scales,
                                    int64_t num_scales, int32_t group_size, void *out, void *stream) {
  MEMOPT_REQUIRE(group_size == 64, MEMOPT_ERR_INVALID,
                 "dequantize_kv_cache_int4: group_size must equal 64");
  const int64_t total = packed_numel * 2;
  MEMOPT_REQUIRE(total % 64 == 0 && num_scales == total / 64, MEMOPT_ERR_INVALID,
                 "dequantize_kv_cache_int4: scales length (" + std::to_string(num_scales) +
                     ") != expected num_groups (" + std::to_string(total / 64) + ")");
  if (total == 0) return MEMOPT_OK;
  MEMOPT_REQUIRE(packed && scales && out, MEMOPT_ERR_INVALID, "dequantize_kv_cache_int4: null pointer");
  const int64_t n_chunks = total / 8;
  hipStream_t s = (hipStream_t)stream;
  const bool vec = aligned(packed, 4) && aligned(out, 16);
  if (vec)
    hipLaunchKernelGGL(dequantize_kernel<true>, dim3(grid_for((n_chunks + 3) / 4, 1LL << 30)), dim3(kThreads), 0,
                       s, packed, scales, (half_t *)out, n_chunks);
  else
    hipLaunchKernelGGL(dequantize_kernel<false>, dim3(grid_for(n_chunks)), dim3(kThreads), 0, s, packed,
                       scales, (half_t *)out, n_chunks);
  return check_launch("dequantize_kv_cache_int4");
}

int memopt_write_cache(const void *keys, const void *values, int64_t num_tokens, int32_t num_heads,
                       int32_t head_dim, const int32_t *slot_mapping, void *stream) {
  const PoolView p = pool_snapshot();
  MEMOPT_REQUIRE(p.initialized, MEMOPT_ERR_STATE, "write_cache: pool not initialized; call init_pool first");
  MEMOPT_REQUIRE(num_heads == p.num_heads, MEMOPT_ERR_INVALID, "write_cache: num_heads != pool.num_heads");
  MEMOPT_REQUIRE(head_dim == p.head_dim, MEMOPT_ERR_INVALID, "write_cache: head_dim != pool.head_dim");
  if (num_tokens == 0) return MEMOPT_OK;
  MEMOPT_REQUIRE(keys && values && slot_mapping, MEMOPT_ERR_INVALID, "write_cache: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const int64_t n_slots = p.num_blocks * p.block_size;
  const int64_t row = (int64_t)num_heads * head_dim;
  if (p.kv_format == MEMOPT_KV_FP16) {
    const bool vec = row % 8 == 0 && aligned(keys, 16) && aligned(values, 16) && aligned(p.key, 16) &&
                     aligned(p.value, 16);
    if (vec) {
      const int64_t cpr = row / 8, n = num_tokens * cpr;
      hipLaunchKernelGGL(write_fp16_kernel, dim3(grid_for(n, 1LL << 30)), dim3(kThreads), 0, s,
                         (const uint4 *)keys, (const uint4 *)values, (uint4 *)p.key, (uint4 *)p.value, slot_mapping,
                         n, cpr, n_slots);
    } else {
      const int64_t n = num_tokens * row;
      hipLaunchKernelGGL(write_fp16_scalar_kernel, dim3(grid_for(n)), dim3(kThreads), 0, s,
                         (const half_t *)keys, (const half_t *)values, (half_t *)p.key, (half_t *)p.value,
                         slot_mapping, n, row, n_slots);
    }
  } else {
    const int64_t n = num_tokens * row / 8;
    const bool vec = aligned(keys, 16) && aligned(values, 16);
    // (64-bit element offsets, 32-bit token indices and wave ids: a whole
    // fp16 pool of config 5, 2.4e9 elements per K, converts through this
    // kernel too)
    const int64_t waves = (num_tokens + 15) / 16 * num_heads * 2;
    if (vec && waves < (1LL << 32) && num_tokens < (1LL << 31) && (head_dim == 64 || head_dim == 128)) {
      const unsigned grid = (unsigned)((waves + kThreads / 64 - 1) / (kThreads / 64));
      if (head_dim == 128)
        hipLaunchKernelGGL(write_int4_pages_kernel<128>, dim3(grid), dim3(kThreads), 0, s, (const half_t *)keys,
                           (const half_t *)values, (uint8_t *)p.key, slot_mapping, (uint32_t)num_tokens,
                           (uint32_t)num_heads, n_slots);
      else
        hipLaunchKernelGGL(write_int4_pages_kernel<64>, dim3(grid), dim3(kThreads), 0, s, (const half_t *)keys,
                           (const half_t *)values, (uint8_t *)p.key, slot_mapping, (uint32_t)num_tokens,
                           (uint32_t)num_heads, n_slots);
    } else if (vec)
      hipLaunchKernelGGL(write_int4_kernel<true>, dim3(grid_for(n)), dim3(kThreads), 0, s,
                         (const half_t *)keys, (const half_t *)values, (uint8_t *)p.key, slot_mapping, n,
                         num_heads, head_dim, n_slots);
    else
      hipLaunchKernelGGL(write_int4_kernel<false>, dim3(grid_for(n)), dim3(kThreads), 0, s,
                         (const half_t *)keys, (const half_t *)values, (uint8_t *)p.key, slot_mapping, n,
                         num_heads, head_dim, n_slots);
  }
  return check_launch("write_cache");
}

int memopt_int4_pages_to_fp16(const uint8_t *pages, int64_t num_blocks, int32_t num_heads, int32_t head_dim,
                              void *key_out, void *value_out, void *stream) {
  MEMOPT_REQUIRE(num_blocks >= 0 && num_heads > 0, MEMOPT_ERR_INVALID, "int4_pages_to_fp16: bad sizes");
  MEMOPT_REQUIRE(head_dim == 64 || head_dim == 128, MEMOPT_ERR_UNSUPPORTED,
                 "int4_pages_to_fp16: head_dim must be 64 or 128");
  if (num_blocks == 0) return MEMOPT_OK;
  MEMOPT_REQUIRE(pages && key_out && value_out, MEMOPT_ERR_INVALID, "int4_pages_to_fp16: null pointer");
  const int64_t units = num_blocks * num_heads;
  const dim3 grid((unsigned)((units + 3) / 4));
  if (head_dim == 128)
    hipLaunchKernelGGL(int4_pages_to_fp16_kernel<128>, grid, dim3(256), 0, (hipStream_t)stream, pages, units,
                       num_heads, (half_t *)key_out, (half_t *)value_out);
  else
    hipLaunchKernelGGL(int4_pages_to_fp16_kernel<64>, grid, dim3(256), 0, (hipStream_t)stream, pages, units,
                       num_heads, (half_t *)key_out, (half_t *)value_out);
  return check_launch("int4_pages_to_fp16");
}

}  // extern "C"
