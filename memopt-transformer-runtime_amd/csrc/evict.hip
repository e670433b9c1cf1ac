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
#include "common.hpp"
#include "page_format.hpp"

namespace memopt {

static constexpr int kEvictThreads = 256;

__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct RowZero {
  int32_t kv_format, H, D, bs;
  void *k, *v, *ks, *vs;
};

// Zero (page, pos, head) in both K and V. fp16: D halves; INT4 pages: the
// row's codes set to 8 (value 0) and its D/64 fp16 scales to 1.0, which is exactly
// what quantizing a zero row produces (scale 1.0 for an all-zero group,
// src/csrc/quantization.cu:168).
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
    const int32_t dpl = z.D / 8;
    for (int c = 0; c < 8; ++c) {
      uint8_t *kb = blk + f.kcodes + f.k_byte(pos, c * dpl);
      for (int w = 0; w < dpl / 8; ++w) reinterpret_cast<uint32_t *>(kb)[w] = 0x88888888u;
      for (int u = 0; u < dpl / 4; ++u)
        *reinterpret_cast<uint16_t *>(blk + f.vcodes + f.v_byte(pos, c * dpl + 4 * u)) = 0x8888u;
    }
    for (int g = 0; g < f.G; ++g) {
      reinterpret_cast<half_t *>(blk + f.kscales)[f.scale_idx(pos, g)] = (half_t)1.0f;
      reinterpret_cast<half_t *>(blk + f.vscales)[f.scale_idx(pos, g)] = (half_t)1.0f;
    }
  }
}

// One workgroup per (seq, head). blockIdx.x = seq, blockIdx.y = head.
__global__ __launch_bounds__(kEvictThreads) void evict_tokens_kernel(
    const float *__restrict__ scores, int32_t *__restrict__ block_tables, int32_t *__restrict__ is_block_free,
    int32_t H, int32_t L, int32_t M, int64_t total_pool_blocks, int32_t keep, int32_t sinks, RowZero z) {
  const int32_t n = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const float *row = scores + ((int64_t)n * H + h) * L;
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_prefix, s_k;

  // ---- Phase A: exact keep-th largest key (radix select, MSB first) ----
  uint32_t prefix = 0, pmask = 0;
  uint32_t k = (uint32_t)keep;  // rank (1-based) inside the current prefix class
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += kEvictThreads) hist[i] = 0;
    __syncthreads();
    for (int t = tid; t < L; t += kEvictThreads) {
      const uint32_t key = (t < sinks) ? order_key(1e38f) : order_key(row[t]);
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 0xFF], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t acc = 0;
      int b = 255;
      for (; b > 0; --b) {
        if (acc + hist[b] >= k) break;
        acc += hist[b];
      }
      s_prefix = prefix | ((uint32_t)b << shift);
      s_k = k - acc;
    }
    __syncthreads();
    prefix = s_prefix;
    k = s_k;
    pmask |= 0xFFu << shift;
    __syncthreads();
  }
  const uint32_t tau = prefix;  // key of the keep-th largest boosted score

  // ---- Phase B: zero evicted (token, head) rows ----
  const int32_t *bt = block_tables + (int64_t)n * M;
  for (int t = tid; t < L; t += kEvictThreads) {
    if (t < sinks) continue;
    if (order_key(row[t]) >= tau) continue;
    const int32_t lb = t / z.bs;
    if (lb >= M) continue;
    const int32_t phys = bt[lb];
    if (phys < 0 || phys >= total_pool_blocks) continue;
    zero_row(z, phys, t - lb * z.bs, h);
  }
  __syncthreads();

  // ---- Phase C: block votes (full blocks whose every position is evicted) ----
  const int32_t nlb = min(L / z.bs, M);
  for (int lb = tid; lb < nlb; lb += kEvictThreads) {
    bool all = true;
    for (int j = 0; j < z.bs && all; ++j) {
      const int t = lb * z.bs + j;
      all = (t >= sinks) && (order_key(row[t]) < tau);
    }
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
  hipLaunchKernelGGL(evict_tokens_kernel, dim3(num_seqs, num_heads), dim3(kEvictThreads), 0,
                     (hipStream_t)stream, attention_scores, block_tables, is_block_free, num_heads, seq_len,
                     max_blocks_per_seq, total_pool_blocks, keep, sinks, z);
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
