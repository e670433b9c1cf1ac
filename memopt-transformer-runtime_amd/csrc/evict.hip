// evict.hip — Ada-KV token eviction on the paged pool (fp16 or INT4 pages).
//
// evict_tokens: TheRadDani/memopt-transformer-runtime src/csrc/kv_cache.cu:640-1156,
// implemented to the documented intent rather than the literal kernel:
//   * the keep-th largest (sink-boosted) score per (seq, head) is found exactly
//     by a 4-pass 8-bit radix select over order-preserving uint32 keys (the
//     reference's 32-step bisection starts from bounds that include the 1e38
//     sink boost and never leaves them, so it evicts nothing when sinks > 0);
//   * whole (token, head) rows are zeroed (the reference zeroes 1 dim in 32);
//   * every evicted token is counted toward its block's vote (the reference
//     counts one token per 32-token run, so no block is ever freed);
//   * no seq_len cap (the reference rejects seq_len > 4096).
// evict_cache: src/csrc/kv_cache.cu:379-483 (per (block, head) selection).
#include <string>

#include "common.hpp"
#include "page_format.hpp"

namespace memopt {

template <int N>
struct IntC {
  static constexpr int value = N;
};

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct RowZero {
  int32_t kv_format, H, D, bs;
  void *k, *v, *ks, *vs;
};

// Zero (page, pos, head) in both K and V. fp16: D halves. INT4 pages: the
// row's D/64 fp16 scales in K and V set to 0 and its codes left in place:
// every element then dequantizes to (code - 8) * 0 = 0 (-0 for codes below
// 8), so attention sees exactly a zeroed row (score 0, no V contribution),
// and an evicted token costs 8 written bytes instead of D + 4 D/64.
__device__ void zero_row(const RowZero &z, int64_t page, int32_t pos, int32_t head) {
  if (z.kv_format == MEMOPT_KV_FP16) {
    const int64_t off = ((page * z.bs + pos) * z.H + head) * (int64_t)z.D;
    half_t *k = (half_t *)z.k + off, *v = (half_t *)z.v + off;
    if ((z.D & 7) == 0) {  // rows are 16-byte aligned: 2*D*(row index) with D % 8 == 0
      const uint4 zero = {0u, 0u, 0u, 0u};
      for (int d = 0; d < z.D; d += 8) {
        *reinterpret_cast<uint4 *>(k + d) = zero;
        *reinterpret_cast<uint4 *>(v + d) = zero;
      }
    } else {
      for (int d = 0; d < z.D; ++d) {
        k[d] = (half_t)0.0f;
        v[d] = (half_t)0.0f;
      }
    }
  } else {
    const Int4Page f(z.D);
    uint8_t *blk = (uint8_t *)z.k + (page * z.H + head) * f.block;
    for (int g = 0; g < f.G; ++g) {
      reinterpret_cast<half_t *>(blk + f.kscales)[f.scale_idx(pos, g)] = (half_t)0.0f;
      reinterpret_cast<half_t *>(blk + f.vscales)[f.scale_idx(pos, g)] = (half_t)0.0f;
    }
  }
}

// Zeroes the evicted tokens of one (page, head) block of the INT4 page pool
// (scales to 0, as zero_row), one wave per block, with 2- and 4-byte stores
// (the path for pools that zero_int4_scale_lines does not take): lane
// l = 8p + c writes the K and V scales of groups c, c + 8, ... for tokens p
// and p + 8, the two halves of one 32-bit scale word. Rewriting the codes as
// well (8 to 16 bytes per token interleaved with kept tokens) cost 1.8-2x:
// those partial lines become read-modify-writes in memory.
__device__ __forceinline__ void zero_int4_block(uint8_t *blk, int32_t D, int lane, bool e0, bool e1) {
  if (!(e0 || e1)) return;
  const Int4Page f(D);
  const int32_t p = lane >> 3, c = lane & 7;
  half_t *ksc = reinterpret_cast<half_t *>(blk + f.kscales), *vsc = reinterpret_cast<half_t *>(blk + f.vscales);
  for (int32_t g = c; g < f.G; g += 8) {
    const int32_t i0 = g * 16 + 2 * p;  // scale_idx(p, g); scale_idx(p + 8, g) = i0 + 1
    if (e0 && e1) {
      *reinterpret_cast<uint32_t *>(ksc + i0) = 0u;
      *reinterpret_cast<uint32_t *>(vsc + i0) = 0u;
    } else {
      const int32_t i = i0 + (e0 ? 0 : 1);
      ksc[i] = (half_t)0.0f;
      vsc[i] = (half_t)0.0f;
    }
  }
}

// Zeroes the evicted tokens of a row's INT4 blocks (scales to 0, as
// zero_row) by rewriting whole scale regions. A block's K scales and V
// scales are one contiguous run of 64 G bytes (16 tokens x G groups x 2 B,
// twice), so a wave covers 64 / (4 G) blocks per step, 4 G lanes each with
// one 16-byte chunk: load the chunk, clear the evicted tokens' halves, store
// it back. Writing full lines instead of single 2- or 4-byte scales avoids
// the memory side's read-modify-write of partial lines: 1.6x faster on
// config 3's shape. The steps are unrolled UL deep so the block-table and
// scale loads of UL steps are in flight together.
//   The read-modify-write is not atomic: a physical page must appear at most
// once in the block tables of one call (one sequence owns a page, as the
// pool's allocator hands them out). Requires G <= 16 and a 16-byte aligned
// pool; the caller uses zero_int4_block otherwise.
template <int NW>
__device__ __forceinline__ void zero_int4_scale_lines(uint8_t *pool, const Int4Page &f, int32_t H, int32_t h,
                                                      const int32_t *bt, const uint32_t *evbits, int32_t nlb,
                                                      int64_t total_pool_blocks, int32_t wave, int32_t lane) {
  constexpr int UL = 8;
  const int32_t lpb = 4 * f.G, bpw = 64 / lpb, jb = lane / lpb, q = lane % lpb;
  const int32_t gmask = 16 * f.G - 1;  // scale index inside the K (or V) run
  for (int32_t lb0 = wave * bpw * UL; lb0 < nlb; lb0 += NW * bpw * UL) {
    uint32_t mm[UL];  // evicted tokens of the lane's block, 0 if none or unmapped
    int32_t ph[UL];
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      const int32_t lb = lb0 + u * bpw + jb;
      mm[u] = (jb < bpw && lb < nlb) ? (evbits[lb >> 1] >> ((lb & 1) * 16)) & 0xFFFFu : 0u;
      ph[u] = mm[u] ? bt[lb] : -1;
    }
    uint4 v[UL];
    uint4 *w[UL];
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      if (!(ph[u] >= 0 && ph[u] < total_pool_blocks)) mm[u] = 0;
      w[u] = reinterpret_cast<uint4 *>(pool + ((int64_t)(mm[u] ? ph[u] : 0) * H + h) * f.block + f.kscales) + q;
      if (mm[u]) v[u] = *w[u];
    }
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      if (!mm[u]) continue;
      uint32_t x[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {  // half 8 q + k of the run; scale_idx(t, g) = 16 g + 2 (t & 7) + (t >> 3)
        const int32_t i = (8 * q + k) & gmask;
        const int32_t t = 8 * (i & 1) + ((i & 15) >> 1);
        if ((mm[u] >> t) & 1) x[k >> 1] &= (k & 1) ? 0x0000FFFFu : 0xFFFF0000u;
      }
      *w[u] = (uint4){x[0], x[1], x[2], x[3]};
    }
  }
}

// Longest score row handled (the evicted-token bitmask lives in LDS).
static constexpr int32_t kEvictMaxLen = 1 << 19;
// Keys kept in LDS for the last radix pass of a streamed row (24 KB).
static constexpr int32_t kEvictCand = 6144;

// One workgroup of NT threads per (seq, head): blockIdx.x = seq, blockIdx.y = head.
// Thread tid owns tokens t = tid + i NT; with R > 0 their keys stay in
// registers (rows up to R NT tokens are read once), with R == 0 the row is
// streamed from memory in batches of 8 loads per pass.
//  A. tau = key of the keep-th largest sink-boosted score, by a 4-pass 8-bit
//     radix select (MSB first): per-wave LDS histograms of the digit among
//     keys matching the prefix so far, then a parallel suffix sum over the
//     256 bins picks the digit.
//  B. evicted-token bitmask in LDS (key < tau, sinks excluded), then zero the
//     evicted (token, head) rows.
//  C. block votes: a full logical block whose every token is evicted votes
//     is_block_free[phys] += 1; the vote that reaches H unlinks it. A head
//     votes only after its own zeroing, so the H-th vote (the unlink) comes
//     after every head has read the block-table entry.
template <int NT, int R, bool V4 = false>
__global__ __launch_bounds__(NT) void evict_tokens_kernel(
    const float *__restrict__ scores, int32_t *__restrict__ block_tables, int32_t *__restrict__ is_block_free,
    int32_t H, int32_t L, int32_t M, int64_t total_pool_blocks, int32_t keep, int32_t sinks, RowZero z) {
  constexpr int NW = NT / 64;
  const int32_t n = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const int32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const float *row = scores + ((int64_t)n * H + h) * L;
  __shared__ uint32_t hist[NW][256];
  __shared__ uint32_t suf[257];
  __shared__ uint32_t s_prefix, s_k;
  extern __shared__ uint32_t evbits[];  // (L + 63) / 64 * 2 words

  const uint32_t sink_key = order_key(1e38f);
  // All loads of a batch are issued first (index clamped into the row),
  // then turned into keys: a load placed under the sink test would be waited
  // on before the next one is issued.
  auto keys_of = [&](int32_t t0, auto nc, uint32_t *kout) __attribute__((always_inline)) {
    constexpr int N = decltype(nc)::value;
    float v[N];
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = row[min(t0 + j * NT, L - 1)];
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const uint32_t kv = order_key(v[j]);
      kout[j] = t0 + j * NT < sinks ? sink_key : kv;
    }
  };
  uint32_t kreg[R > 0 ? R : 1];
  if constexpr (R > 0) keys_of(tid, IntC<R>{}, kreg);
  // Calls f(t, key) for every token of this thread.
  auto for_keys = [&](auto f) __attribute__((always_inline)) {
    if constexpr (R > 0) {
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const int32_t t = tid + i * NT;
        if (t < L) f(t, kreg[i]);
      }
    } else {
      for (int32_t base = 0; base < L; base += 8 * NT) {
        uint32_t kb[8];
        keys_of(base + tid, IntC<8>{}, kb);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int32_t t = base + tid + j * NT;
          if (t < L) f(t, kb[j]);
        }
      }
    }
  };

  // Radix-pass visitor: streamed rows whose length is a multiple of 4 (and a
  // 16-byte aligned base) are read as float4, a quarter of the load
  // instructions of the token-per-lane order; the histograms do not depend
  // on the visiting order.
  auto for_keys_hist = [&](auto f) __attribute__((always_inline)) {
    if constexpr (R == 0 && V4) {
      for (int32_t base = 0; base < L; base += 32 * NT) {
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          v[j] = *reinterpret_cast<const float4 *>(row + min(base + 4 * (tid + j * NT), L - 4));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int32_t t = base + 4 * (tid + j * NT);
          auto one = [&](int32_t tq, float x) __attribute__((always_inline)) {
            if (tq < L) f(tq, tq < sinks ? sink_key : order_key(x));
          };
          one(t, v[j].x);
          one(t + 1, v[j].y);
          one(t + 2, v[j].z);
          one(t + 3, v[j].w);
        }
      }
    } else {
      for_keys(f);
    }
  };

  // ---- A: radix select ----
  // Streamed rows (R == 0) copy the keys that match the 16-bit prefix into
  // LDS (cand, after the bitmask words) during the third pass, and the last
  // pass reads them from there when they fit: four streamed passes over the
  // row instead of five. After two 8-bit digits the matching keys are
  // typically a fraction of a percent of the row.
  __shared__ uint32_t s_cnt;
  uint32_t *cand = evbits + (L + 63) / 64 * 2;
  uint32_t ncand = 0xFFFFFFFFu;
  uint32_t prefix = 0, pmask = 0, k = (uint32_t)keep;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < NW * 256; i += NT) (&hist[0][0])[i] = 0;
    if (tid == 0) {
      suf[256] = 0;
      s_cnt = 0;
    }
    __syncthreads();
    auto bump = [&](int32_t, uint32_t key) {
      if ((key & pmask) == prefix) atomicAdd(&hist[wave][(key >> shift) & 0xFF], 1u);
    };
    if (R == 0 && shift == 8) {
      // Counts the key's digit and appends it to cand; every lane is active.
      auto push = [&](int32_t t, uint32_t key) __attribute__((always_inline)) {
        const bool m = t < L && (key & pmask) == prefix;
        if (m) atomicAdd(&hist[wave][(key >> 8) & 0xFF], 1u);
        const uint64_t bal = __ballot(m);
        if (bal) {  // wave-uniform
          uint32_t b0 = 0;
          if (lane == 0) b0 = atomicAdd(&s_cnt, (uint32_t)__popcll(bal));
          b0 = __builtin_amdgcn_readfirstlane(b0);
          const uint32_t pos =
              b0 + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
          if (m && pos < (uint32_t)kEvictCand) cand[pos] = key;
        }
      };
      if constexpr (V4) {  // the float4 order of for_keys_hist
        for (int32_t base = 0; base < L; base += 32 * NT) {
          float4 v[8];
#pragma unroll
          for (int j = 0; j < 8; ++j)
            v[j] = *reinterpret_cast<const float4 *>(row + min(base + 4 * (tid + j * NT), L - 4));
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int32_t t = base + 4 * (tid + j * NT);
            push(t, t < sinks ? sink_key : order_key(v[j].x));
            push(t + 1, t + 1 < sinks ? sink_key : order_key(v[j].y));
            push(t + 2, t + 2 < sinks ? sink_key : order_key(v[j].z));
            push(t + 3, t + 3 < sinks ? sink_key : order_key(v[j].w));
          }
        }
      } else {
        for (int32_t base = 0; base < L; base += 8 * NT) {
          uint32_t kb[8];
          keys_of(base + tid, IntC<8>{}, kb);
#pragma unroll
          for (int j = 0; j < 8; ++j) push(base + tid + j * NT, kb[j]);
        }
      }
    } else if (R == 0 && shift == 0 && ncand <= (uint32_t)kEvictCand) {
      for (uint32_t i = tid; i < ncand; i += NT) bump(0, cand[i]);
    } else {
      for_keys_hist(bump);
    }
    __syncthreads();
    if (R == 0 && shift == 8) ncand = s_cnt;
    if (tid < 256) {
      uint32_t c = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) c += hist[w][tid];
      suf[tid] = c;
    }
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {  // suf[i] := sum of bins >= i
      const uint32_t v = (tid < 256 && tid + off < 256) ? suf[tid + off] : 0u;
      __syncthreads();
      if (tid < 256) suf[tid] += v;
      __syncthreads();
    }
    if (tid < 256 && suf[tid] >= k && suf[tid + 1] < k) {
      s_prefix = prefix | ((uint32_t)tid << shift);
      s_k = k - suf[tid + 1];
    }
    __syncthreads();
    prefix = s_prefix;
    k = s_k;
    pmask |= 0xFFu << shift;
  }
  const uint32_t tau = prefix;

  // ---- B: evicted bitmask (the 64 lanes of a wave hold 64 consecutive tokens) ----
  const int32_t nwords = (L + 63) / 64 * 2;
  for (int i = tid; i < nwords; i += NT) evbits[i] = 0;
  __syncthreads();
  for_keys([&](int32_t t, uint32_t key) {
    const uint64_t m = __ballot(t >= sinks && key < tau);
    if (lane == 0 && m) {
      evbits[t / 32] = (uint32_t)m;
      evbits[t / 32 + 1] = (uint32_t)(m >> 32);
    }
  });
  __syncthreads();
  auto ev = [&](int32_t t) { return (evbits[t >> 5] >> (t & 31)) & 1u; };

  const int32_t *bt = block_tables + (int64_t)n * M;
  if (z.kv_format == MEMOPT_KV_INT4) {
    const Int4Page f(z.D);
    const int32_t nlb = min((L + 15) / 16, M);
    const int32_t p = lane >> 3;
    if (f.G <= 16 && (reinterpret_cast<uintptr_t>(z.k) & 15) == 0) {
      zero_int4_scale_lines<NW>((uint8_t *)z.k, f, z.H, h, bt, evbits, nlb, total_pool_blocks, wave, lane);
    } else {
      for (int32_t lb0 = wave * 64; lb0 < nlb; lb0 += NW * 64) {
        const int32_t phys_l = lb0 + lane < nlb ? bt[lb0 + lane] : -1;
        const int32_t cnt = min(64, nlb - lb0);
        for (int i = 0; i < cnt; ++i) {
          const int32_t lb = lb0 + i;
          const uint32_t m16 = (evbits[lb >> 1] >> ((lb & 1) * 16)) & 0xFFFFu;  // tokens 16 lb .. 16 lb + 15
          const int32_t phys = __builtin_amdgcn_readlane(phys_l, i);
          if (m16 == 0 || phys < 0 || phys >= total_pool_blocks) continue;  // wave-uniform
          zero_int4_block((uint8_t *)z.k + ((int64_t)phys * z.H + h) * f.block, z.D, lane, (m16 >> p) & 1,
                          (m16 >> (p + 8)) & 1);
        }
      }
    }
  } else {
    for (int32_t t0 = wave * 64; t0 < L; t0 += NW * 64) {
      const int32_t t = t0 + lane, lb = t / z.bs;
      bool e = t < L && ev(t) && lb < M;
      int32_t phys = -1;
      if (e) {
        phys = bt[lb];
        e = phys >= 0 && phys < total_pool_blocks;
      }
      uint64_t mask = __ballot(e);
      while (mask) {  // the wave zeroes each evicted row, 16 bytes per lane
        const int j = __builtin_ctzll(mask);
        mask &= mask - 1;
        const int32_t tj = t0 + j, pj = __shfl(phys, j, 64), lbj = tj / z.bs;
        const int64_t off = (((int64_t)pj * z.bs + (tj - lbj * z.bs)) * z.H + h) * (int64_t)z.D;
        half_t *kr = (half_t *)z.k + off, *vr = (half_t *)z.v + off;
        if ((z.D & 7) == 0) {
          const uint4 zero = {0u, 0u, 0u, 0u};
          for (int d = 8 * lane; d < z.D; d += 512) {
            *reinterpret_cast<uint4 *>(kr + d) = zero;
            *reinterpret_cast<uint4 *>(vr + d) = zero;
          }
        } else {
          for (int d = lane; d < z.D; d += 64) {
            kr[d] = (half_t)0.0f;
            vr[d] = (half_t)0.0f;
          }
        }
      }
    }
  }
  __syncthreads();

  // ---- C: block votes ----
  const int32_t nlb_full = min(L / z.bs, M);
  for (int32_t lb = tid; lb < nlb_full; lb += NT) {
    bool all = true;
    for (int j = 0; j < z.bs && all; ++j) all = ev(lb * z.bs + j);
    if (!all) continue;
    const int32_t phys = bt[lb];
    if (phys < 0 || phys >= total_pool_blocks) continue;
    const int prev = atomicAdd(&is_block_free[phys], 1);
    if (prev + 1 == H) block_tables[(int64_t)n * M + lb] = -1;
  }
}

// One wave per (block, head): lane i owns position i (bs <= 64).
__global__ __launch_bounds__(64) void evict_cache_kernel(const float *__restrict__ scores, int32_t bs,
                                                         int32_t H, int32_t keep, RowZero z) {
  const int64_t blk = blockIdx.x;
  const int32_t h = blockIdx.y, i = threadIdx.x;
  if (i >= bs) return;
  const float si = scores[(blk * bs + i) * H + h];
  int greater = 0;
  for (int j = 0; j < bs; ++j) greater += scores[(blk * bs + j) * H + h] > si ? 1 : 0;
  // Score below the keep-th largest <=> at least `keep` scores strictly above it.
  if (greater >= keep) zero_row(z, blk, i, h);
}

}  // namespace memopt

using namespace memopt;

extern "C" {

int memopt_evict_tokens(const float *attention_scores, int32_t num_seqs, int32_t num_heads, int32_t seq_len,
                        int32_t *block_tables, int32_t max_blocks_per_seq, int32_t *is_block_free,
                        int64_t total_pool_blocks, float retain_ratio, int32_t num_sink_tokens, void *stream) {
  const PoolView p = pool_snapshot();
  MEMOPT_REQUIRE(p.initialized, MEMOPT_ERR_STATE, "evict_tokens: pool not initialized");
  MEMOPT_REQUIRE(retain_ratio > 0.f && retain_ratio <= 1.f, MEMOPT_ERR_INVALID,
                 "evict_tokens: retain_ratio must be in (0, 1]");
  MEMOPT_REQUIRE(num_heads == p.num_heads, MEMOPT_ERR_INVALID,
                 "evict_tokens: attention_scores num_heads != pool.num_heads");
  MEMOPT_REQUIRE(total_pool_blocks <= p.num_blocks, MEMOPT_ERR_INVALID,
                 "evict_tokens: is_block_free size > pool.num_blocks");
  if (num_seqs == 0 || seq_len == 0) return MEMOPT_OK;
  MEMOPT_REQUIRE(attention_scores && block_tables && is_block_free, MEMOPT_ERR_INVALID,
                 "evict_tokens: null pointer");
  // keep = clamp((int)ceilf(r * L), 1, L), in fp32 as src/csrc/kv_cache.cu:754-755.
  int keep = (int)ceilf(retain_ratio * (float)seq_len);
  keep = keep < 1 ? 1 : (keep > seq_len ? seq_len : keep);
  RowZero z{p.kv_format, p.num_heads, p.head_dim, p.block_size, p.key, p.value, p.key_scales, p.value_scales};
  const int32_t sinks = num_sink_tokens < 0 ? 0 : (num_sink_tokens > seq_len ? seq_len : num_sink_tokens);
  MEMOPT_REQUIRE(p.kv_format != MEMOPT_KV_INT4 || p.block_size == 16, MEMOPT_ERR_UNSUPPORTED,
                 "evict_tokens: INT4 page pools use 16-token pages");
  MEMOPT_REQUIRE(seq_len <= kEvictMaxLen, MEMOPT_ERR_UNSUPPORTED,
                 "evict_tokens: seq_len > " + std::to_string(kEvictMaxLen) + " not supported");
  const size_t lds = (size_t)((seq_len + 63) / 64 * 2) * sizeof(uint32_t);
  const size_t lds_cand = lds + kEvictCand * sizeof(uint32_t);  // streamed rows: + the candidate keys
  const dim3 grid(num_seqs, num_heads);
  hipStream_t st = (hipStream_t)stream;
  // Rows up to 8192 (32768) tokens keep their keys in registers with 256
  // (1024) threads; longer rows stream with 1024 threads.
  if (seq_len <= 256 * 32)
    hipLaunchKernelGGL((evict_tokens_kernel<256, 32>), grid, dim3(256), lds, st, attention_scores, block_tables,
                       is_block_free, num_heads, seq_len, max_blocks_per_seq, total_pool_blocks, keep, sinks, z);
  else if (seq_len <= 1024 * 32)
    hipLaunchKernelGGL((evict_tokens_kernel<1024, 32>), grid, dim3(1024), lds, st, attention_scores, block_tables,
                       is_block_free, num_heads, seq_len, max_blocks_per_seq, total_pool_blocks, keep, sinks, z);
  else if (seq_len % 4 == 0 && ((uintptr_t)attention_scores & 15) == 0)
    hipLaunchKernelGGL((evict_tokens_kernel<1024, 0, true>), grid, dim3(1024), lds_cand, st, attention_scores,
                       block_tables, is_block_free, num_heads, seq_len, max_blocks_per_seq, total_pool_blocks, keep,
                       sinks, z);
  else
    hipLaunchKernelGGL((evict_tokens_kernel<1024, 0>), grid, dim3(1024), lds_cand, st, attention_scores, block_tables,
                       is_block_free, num_heads, seq_len, max_blocks_per_seq, total_pool_blocks, keep, sinks, z);
  return check_launch("evict_tokens");
}

int memopt_evict_cache(const float *attention_scores, int64_t num_blocks, float retain_ratio,
                       int32_t num_sink_tokens, void *stream) {
  (void)num_sink_tokens;  // ignored by the reference too (src/csrc/kv_cache.cu:392-393)
  const PoolView p = pool_snapshot();
  MEMOPT_REQUIRE(p.initialized, MEMOPT_ERR_STATE, "evict_cache: pool not initialized");
  MEMOPT_REQUIRE(retain_ratio > 0.f && retain_ratio <= 1.f, MEMOPT_ERR_INVALID,
                 "evict_cache: retain_ratio must be in (0, 1]");
  MEMOPT_REQUIRE(num_blocks <= p.num_blocks, MEMOPT_ERR_INVALID,
                 "evict_cache: attention_scores num_blocks > pool.num_blocks");
  MEMOPT_REQUIRE(p.block_size <= 64, MEMOPT_ERR_UNSUPPORTED, "evict_cache: block_size > 64 not supported");
  if (num_blocks == 0) return MEMOPT_OK;
  int keep = (int)(retain_ratio * (float)p.block_size);  // truncation, src/csrc/kv_cache.cu:426
  keep = keep < 1 ? 1 : (keep > p.block_size ? p.block_size : keep);
  RowZero z{p.kv_format, p.num_heads, p.head_dim, p.block_size, p.key, p.value, p.key_scales, p.value_scales};
  hipLaunchKernelGGL(evict_cache_kernel, dim3((unsigned)num_blocks, p.num_heads), dim3(64), 0,
                     (hipStream_t)stream, attention_scores, p.block_size, p.num_heads, keep, z);
  return check_launch("evict_cache");
}

}  // extern "C"
