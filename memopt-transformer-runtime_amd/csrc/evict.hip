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
#include <algorithm>
#include <atomic>
#include <string>

#include "common.hpp"
#include "page_format.hpp"

namespace memopt {

template <int N>
struct IntC {
  static constexpr int value = N;
};

// Order-preserving uint32 key of a float: negative values have every bit
// flipped, others the sign bit set; -0 takes the key of +0 (f + 0 turns -0
// into +0 and leaves every other value as it is), since the two compare
// equal: a -0 score ties with a +0 tau, as in float compares. A NaN of
// either sign gets key 0, which no other float has (-inf's key is
// 0x007FFFFF): the reference's selection counts and evicts by float
// compares, which a NaN never passes, so a NaN ranks below every score and
// is never evicted (kNanKey is excluded wherever a key < tau evicts).
static constexpr uint32_t kNanKey = 0u;
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f + 0.0f);
  const uint32_t k = u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
  return f != f ? kNanKey : k;
}

// Set in a page mark when two or more live block-table entries of one call
// name the page.
static constexpr uint32_t kMarkShared = 0x80000000u;

struct RowZero {
  int32_t kv_format, H, D, bs;
  void *k, *v, *ks, *vs;
  // *alias_flag == tag (this call's id) when some physical page appears
  // more than once in this call's block tables, and marks[page] then tells
  // which (set by mark_pages_kernel or the long-row classify launch).
  const uint32_t *alias_flag;
  const uint32_t *marks;
  uint32_t tag;
};

// Whether this call's block tables alias a physical page (wave-uniform).
__device__ __forceinline__ bool pages_aliased(const RowZero &z) {
  return z.alias_flag != nullptr && *z.alias_flag == z.tag;
}

// A page named by more than one live block-table entry of this call is
// shared between sequences (prefix sharing): it receives the union of their
// evictions but never a free vote, so no sequence unlinks it and the free
// sweep never returns a page that another table still maps. Per-(sequence,
// head) votes from two sequences would otherwise add up to H while heads
// still hold live rows.
__device__ __forceinline__ bool page_shared(const RowZero &z, int32_t phys) {
  return pages_aliased(z) && (z.marks[phys] & kMarkShared) != 0;
}

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
//   The plain read-modify-write assumes a physical page appears once in the
// call's block tables (one sequence owns a page, as the pool's allocator
// hands them out). When mark_pages_kernel found a page listed twice, the
// chunk's words are cleared with atomic ANDs instead, so evictions of every
// row that lists the page survive (their union). Requires G <= 16 and a
// 16-byte aligned pool; the caller uses zero_int4_block otherwise. Logical
// blocks [lb_begin, lb_end) of the row, waves wave, wave + NW, ...
template <int NW>
__device__ __forceinline__ void zero_int4_scale_lines(uint8_t *pool, const Int4Page &f, int32_t H, int32_t h,
                                                      const int32_t *bt, const uint32_t *evbits, int32_t lb_begin,
                                                      int32_t lb_end, int64_t total_pool_blocks, int32_t wave,
                                                      int32_t lane, bool aliased) {
  constexpr int UL = 8;
  const int32_t lpb = 4 * f.G, bpw = 64 / lpb, jb = lane / lpb, q = lane % lpb;
  const int32_t gmask = 16 * f.G - 1;  // scale index inside the K (or V) run
  const int32_t nlb = lb_end;
  for (int32_t lb0 = lb_begin + wave * bpw * UL; lb0 < nlb; lb0 += NW * bpw * UL) {
    uint32_t mm[UL];  // evicted tokens of the lane's block, 0 if none or unmapped
    int32_t ph[UL];
    // All loads are unconditional, so that the steps' loads are in flight
    // together: blocks past the end read the last block's entry, and a lane
    // with nothing to clear reads the line of (page 0, head h), which every
    // such lane shares, and stores nothing.
#pragma unroll
    for (int u = 0; u < UL; ++u) ph[u] = bt[min(lb0 + u * bpw + jb, nlb - 1)];
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      const int32_t lb = lb0 + u * bpw + jb;
      const bool in = jb < bpw && lb < nlb;  // 64 % lpb lanes idle when G is no power of 2
      mm[u] = in ? (evbits[lb >> 1] >> ((lb & 1) * 16)) & 0xFFFFu : 0u;
      if (!in) ph[u] = -1;
    }
    uint4 v[UL];
    uint4 *w[UL];
    const uint4 *idle = reinterpret_cast<const uint4 *>(pool + (int64_t)h * f.block + f.kscales) + q;
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      if (!(ph[u] >= 0 && ph[u] < total_pool_blocks)) mm[u] = 0;
      w[u] = reinterpret_cast<uint4 *>(pool + ((int64_t)(mm[u] ? ph[u] : 0) * H + h) * f.block + f.kscales) + q;
      v[u] = *(mm[u] && !aliased ? w[u] : idle);
    }
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      if (!mm[u]) continue;
      uint32_t keepm[4] = {~0u, ~0u, ~0u, ~0u};
#pragma unroll
      for (int k = 0; k < 8; ++k) {  // half 8 q + k of the run; scale_idx(t, g) = 16 g + 2 (t & 7) + (t >> 3)
        const int32_t i = (8 * q + k) & gmask;
        const int32_t t = 8 * (i & 1) + ((i & 15) >> 1);
        if ((mm[u] >> t) & 1) keepm[k >> 1] &= (k & 1) ? 0x0000FFFFu : 0xFFFF0000u;
      }
      if (aliased) {
        uint32_t *wd = reinterpret_cast<uint32_t *>(w[u]);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (keepm[k] != ~0u) atomicAnd(wd + k, keepm[k]);
      } else {
        *w[u] = (uint4){v[u].x & keepm[0], v[u].y & keepm[1], v[u].z & keepm[2], v[u].w & keepm[3]};
      }
    }
  }
}

// Rows up to kShortRow tokens run evict_tokens_kernel (one workgroup per
// row, keys in registers); longer rows run the split kernels below.
static constexpr int32_t kShortRow = 1024 * 32;

// hist[digit] += 1 for the lanes with m. Keys of one row often share their
// leading digits (and a bracket's candidates share more), so most lanes of
// a wave can hit one bin, and same-address LDS atomics serialize: the digit
// of the wave's first matching lane is added with one atomic by one lane
// when 16 or more lanes share it; only the other lanes issue their own.
__device__ __forceinline__ void hist_add_agg(uint32_t *hist, uint32_t digit, bool m) {
  const uint64_t act = __ballot(m);
  if (act) {  // wave-uniform
    const int lead = __builtin_ctzll(act);
    const uint32_t d0 = __builtin_amdgcn_readlane(digit, lead);
    const uint64_t same = __ballot(m && digit == d0);
    const uint32_t n_same = (uint32_t)__popcll(same);
    if (n_same >= 16) {
      if ((int)(threadIdx.x & 63) == lead) atomicAdd(&hist[d0], n_same);
      m = m && digit != d0;
    }
  }
  if (m) atomicAdd(&hist[digit], 1u);
}

template <int NT>
struct SelectShared {
  uint32_t hist[NT / 64][256];
  uint32_t tot[256];  // bin totals over the waves (NT >= 512)
  uint32_t prefix, k;
};

// Key of the k-th largest (1 <= k <= number of keys) of the keys handed out
// by visit(f), which calls f(key) for every key of the calling thread. Four
// 8-bit radix passes (MSB first): per-wave LDS histograms of the digit among
// keys matching the prefix so far; then wave 0 sums the waves' bins (4 per
// lane; with 8 or more waves, 256 threads form the bin totals first), forms
// suffix sums with a wave scan and picks the digit, so a pass costs two
// workgroup barriers (three with the totals). AGG: histogram through hist_add_agg
// (for keys that mostly share their leading digits). Every thread of the
// workgroup calls it.
template <int NT, bool AGG, typename Visit>
__device__ uint32_t radix_select(Visit visit, uint32_t k, SelectShared<NT> &sh, uint32_t fixed = 0,
                                 int fixed_bytes = 0) {
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // The top fixed_bytes bytes of every visited key equal those of `fixed`:
  // those passes are skipped.
  uint32_t pmask = fixed_bytes > 0 ? ~0u << (32 - 8 * fixed_bytes) : 0u;
  uint32_t prefix = fixed & pmask;
  for (int shift = 24 - 8 * fixed_bytes; shift >= 0; shift -= 8) {
    for (int i = tid; i < NW * 256; i += NT) (&sh.hist[0][0])[i] = 0;
    __syncthreads();
    visit([&](uint32_t key) {
      const bool m = (key & pmask) == prefix;
      const uint32_t digit = (key >> shift) & 0xFF;
      if constexpr (AGG) {
        hist_add_agg(sh.hist[wave], digit, m);
      } else if (m) {
        atomicAdd(&sh.hist[wave][digit], 1u);
      }
    });
    __syncthreads();
    if constexpr (NW >= 8) {  // the bin totals by 256 threads, not by wave 0 alone
      if (tid < 256) {
        uint32_t v = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += sh.hist[w][tid];
        sh.tot[tid] = v;
      }
      __syncthreads();
    }
    if (wave == 0) {
      // lane owns bins 4 lane .. 4 lane + 3
      uint32_t c[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t v = 0;
        if constexpr (NW >= 8) {
          v = sh.tot[4 * lane + j];
        } else {
#pragma unroll
          for (int w = 0; w < NW; ++w) v += sh.hist[w][4 * lane + j];
        }
        c[j] = v;
      }
      const uint32_t tot = c[0] + c[1] + c[2] + c[3];
      // above = sum of the totals of lanes > lane (exclusive suffix scan)
      uint32_t inc = tot;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_down(inc, off, 64);
        if (lane + off < 64) inc += o;
      }
      uint32_t above = inc - tot;
      // suffix count of bin 4 lane + j = above + c[j] + ... + c[3]
#pragma unroll
      for (int j = 3; j >= 0; --j) {
        const uint32_t upto = above + c[j];  // keys with digit >= 4 lane + j
        if (upto >= k && above < k) {
          sh.prefix = prefix | ((uint32_t)(4 * lane + j) << shift);
          sh.k = k - above;
        }
        above = upto;
      }
    }
    __syncthreads();
    prefix = sh.prefix;
    k = sh.k;
    pmask |= 0xFFu << shift;
  }
  return prefix;
}

__device__ __forceinline__ uint32_t token_key(const float *row, int32_t t, int32_t sinks) {
  return t < sinks ? order_key(1e38f) : order_key(row[t]);
}

// One workgroup of NT threads per (seq, head): blockIdx.x = seq, blockIdx.y = head.
// Thread tid owns tokens t = tid + i NT, i < R; their keys stay in registers,
// so the row is read once (rows up to R NT tokens).
//  A. tau = key of the keep-th largest sink-boosted score, by radix_select.
//  B. evicted-token bitmask in LDS (key < tau, sinks and NaN excluded), then zero the
//     evicted (token, head) rows.
//  C. block votes: a full logical block whose every token is evicted votes
//     is_block_free[phys] += 1; the vote that reaches H unlinks it. A head
//     votes only after its own zeroing, so the H-th vote (the unlink) comes
//     after every head has read the block-table entry.
template <int NT, int R>
__global__ __launch_bounds__(NT) void evict_tokens_kernel(
    const float *__restrict__ scores, int32_t *__restrict__ block_tables, int32_t *__restrict__ is_block_free,
    int32_t H, int32_t L, int32_t M, int64_t total_pool_blocks, int32_t keep, int32_t sinks, RowZero z) {
  constexpr int NW = NT / 64;
  const int32_t n = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const int32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const float *row = scores + ((int64_t)n * H + h) * L;
  __shared__ SelectShared<NT> sh;
  extern __shared__ uint32_t evbits[];  // (L + 63) / 64 * 2 words

  // All loads are issued first (index clamped into the row), then turned
  // into keys: a load placed under the sink test would be waited on before
  // the next one is issued. They are non-temporal (the scores are read
  // once; the INT4 scale runs the zeroing rewrites stay cached instead:
  // config 3 28.6 against 29.9 us).
  uint32_t kreg[R];
  {
    float v[R];
#pragma unroll
    for (int j = 0; j < R; ++j) v[j] = __builtin_nontemporal_load(&row[min(tid + j * NT, L - 1)]);
#pragma unroll
    for (int j = 0; j < R; ++j) kreg[j] = tid + j * NT < sinks ? order_key(1e38f) : order_key(v[j]);
  }
  // Calls f(t, key) for every token of this thread.
  auto for_keys = [&](auto f) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int32_t t = tid + i * NT;
      if (t < L) f(t, kreg[i]);
    }
  };

  // ---- A: radix select ----
  const uint32_t tau = radix_select<NT, false>([&](auto f) { for_keys([&](int32_t, uint32_t key) { f(key); }); },
                                               (uint32_t)keep, sh);

  // ---- B: evicted bitmask (the 64 lanes of a wave hold 64 consecutive tokens) ----
  const int32_t nwords = (L + 63) / 64 * 2;
  for (int i = tid; i < nwords; i += NT) evbits[i] = 0;
  __syncthreads();
  for_keys([&](int32_t t, uint32_t key) {
    const uint64_t m = __ballot(t >= sinks && key < tau && key != kNanKey);
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
      zero_int4_scale_lines<NW>((uint8_t *)z.k, f, z.H, h, bt, evbits, 0, nlb, total_pool_blocks, wave, lane,
                                pages_aliased(z));
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
    if (phys < 0 || phys >= total_pool_blocks || page_shared(z, phys)) continue;
    const int prev = atomicAdd(&is_block_free[phys], 1);
    if (prev + 1 == H) block_tables[(int64_t)n * M + lb] = -1;
  }
}

// ---------------------------------------------------------------------------
// Aliased physical pages
// ---------------------------------------------------------------------------
// Each live block-table entry e (logical block lb < nlb of its row, a page
// inside the pool) exchanges marks[phys] for e + 1. The value it takes out
// is the previous entry that marked the page: in this call, or left from an
// earlier call or any earlier content of the memory. The page is shared in
// this call exactly when some exchange takes out an entry e' != e that is a
// live entry naming the same page in the current block tables: with k >= 2
// live entries on a page, every exchange after the first takes out one of
// them; with k = 1, a live entry e' naming the page would be a second one.
// So stale or arbitrary marks are harmless and nothing is cleared between
// calls. The detecting entry ORs kMarkShared into the mark (the last
// exchange of a shared page detects and ORs after it, so the final mark
// carries the bit exactly when k >= 2) and sets *flag = tag, this call's id
// (a stale flag only selects the atomic scale rewrite, which gives the same
// result as the plain one). Block tables do not change during the mark pass.
struct MarkArgs {
  const int32_t *bt;
  int64_t entries;  // num_seqs * max_blocks_per_seq (0: nothing to mark)
  int32_t M, nlb;
  int64_t total_pool_blocks;
  uint32_t *marks;
  uint32_t *flag;
  uint32_t tag;
};

// mark_entry in steps, so that its dependent memory round trips overlap
// other work: the block-table value of entry e, loaded whatever e (index
// clamped, so the load needs no branch and nothing waits for it until the
// value is used) ...
__device__ __forceinline__ int32_t mark_load(const MarkArgs &a, int64_t e) {
  return a.entries > 0 ? a.bt[min(e, a.entries - 1)] : -1;
}
// ... the page of entry e (or -1) from that value ...
__device__ __forceinline__ int32_t mark_page(const MarkArgs &a, int64_t e, int32_t phys) {
  if (e >= a.entries || (int32_t)(e % a.M) >= a.nlb) return -1;
  return phys >= 0 && phys < a.total_pool_blocks ? phys : -1;
}
// ... the exchange (its result, only read by mark_check and only where
// phys >= 0, is left unset elsewhere, so that nothing waits for it) ...
__device__ __forceinline__ void mark_swap(const MarkArgs &a, int64_t e, int32_t phys, uint32_t &old) {
  if (phys >= 0) old = atomicExch(&a.marks[phys], (uint32_t)(e + 1));
}
// ... and the alias check: the entry taken out must still name the page.
__device__ __forceinline__ void mark_check(const MarkArgs &a, int64_t e, int32_t phys, uint32_t old) {
  const int64_t o = (int64_t)(old & ~kMarkShared) - 1;
  if (phys < 0 || o < 0 || o == e || o >= a.entries || (int32_t)(o % a.M) >= a.nlb) return;
  if (a.bt[o] != phys) return;
  atomicOr(&a.marks[phys], kMarkShared);
  atomicExch(a.flag, a.tag);
}

__device__ __forceinline__ void mark_entry(const MarkArgs &a, int64_t e) {
  const int32_t phys = mark_page(a, e, a.bt[e]);
  uint32_t old = 0;
  mark_swap(a, e, phys, old);
  mark_check(a, e, phys, old);
}

__global__ __launch_bounds__(256) void mark_pages_kernel(const MarkArgs a) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e < a.entries) mark_entry(a, e);
}

// ---------------------------------------------------------------------------
// Long rows (L > 32768): several workgroups per (seq, head)
// ---------------------------------------------------------------------------
// A row is cut into spans of kSpan tokens and takes three kernels:
//  K1 evict_classify_long_kernel, one workgroup per span: it loads a
//     16 x 512-key sample spread over the row and computes a bracket
//     [lo, hi] around the row's keep-th largest key from it (every span of
//     a row derives the same bracket from the same sample), then streams
//     its span through a window of loads per thread. Each token is then
//     kept (key > hi, counted), evicted (key < lo, a bit of the row's
//     bitmask) or a candidate ((score, token) appended to its wave's list
//     in LDS; the lists are copied to the span's list at the end). The
//     same launch marks the block-table entries (alias check, INT4 pools)
//     over its whole grid;
//  K2 evict_resolve_long_kernel, one workgroup per row: when the bracket
//     holds the keep-th key (fewer than keep keys above hi, at least keep
//     at or above lo) and the candidates fit in LDS, it gathers the spans'
//     lists, takes tau = the exact (keep - above)-th largest candidate and
//     ORs the evicted ones into the bitmask; otherwise (a miss, heavy ties,
//     too many candidates, a wave list that overflowed) an exact radix
//     select over the whole row and a full bitmask;
//  K3 zero the evicted rows and vote for fully evicted blocks: for INT4
//     pools, workgroups over (sequence, range of logical blocks) covering
//     all heads of each page (evict_apply_pages_kernel); otherwise
//     kApplySplit workgroups per row, each over a range of logical blocks.
// The result is the same exact top-k as the single-workgroup kernel.
static constexpr int32_t kClsNT = 1024, kClsPer = 16;  // K1 threads per workgroup, float4 loads per thread
static constexpr int32_t kClsWin = 2;  // K1 loads in flight per thread (2 to 10 measured: 2 is fastest)
static constexpr int32_t kClsPre = 2;  // of which issued before the bracket
static constexpr int32_t kSpan = kClsNT * kClsPer * 4;  // tokens per K1 workgroup (65536)
static constexpr int32_t kSampleChunks = 16, kSampleChunk = 512, kSample = kSampleChunks * kSampleChunk;
static constexpr int32_t kResNT = 1024;     // K2 threads per workgroup
static constexpr int32_t kResCand = 8192;   // candidates K2 gathers in LDS
static constexpr int32_t kLdsWords = 4096;  // bitmask words K2 merges per LDS round
static constexpr int32_t kApplySplit = 32;  // apply workgroups per row (non-INT4 pools)
static constexpr int32_t kRep = 16;         // copies of each first-byte bin of the bracket histogram
static constexpr int32_t kWaveCand = 512;   // candidate list slots per K1 wave
static constexpr int32_t kSpanCand = kWaveCand * (kClsNT / 64);  // per span (8192)

struct LongRows {
  const float *scores;
  int32_t H, L, keep, sinks;
  int32_t words;    // bitmask words per row ((L + 63) / 64 * 2)
  int32_t spans;    // K1 workgroups per row (ceil(L / kSpan))
  uint4 *slot;      // [rows][spans] (kept count, candidate count | kListLost, lo, hi)
  uint32_t *bits;   // [rows][words] evicted tokens
  uint2 *cand;      // [rows][spans][kSpanCand] (score bits, token) candidate lists
};
// Set in a slot's candidate count when a wave's list overflowed: the span's
// list is incomplete, and the resolve selects over the whole row instead.
static constexpr uint32_t kListLost = 0x80000000u;

// Workgroup barrier that orders LDS accesses only: it does not wait for the
// caller's outstanding global loads and stores.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

struct ClassifyLds {
  uint32_t skeys[kSample];
  uint32_t h1[256][kRep];  // first-byte histogram, lane l adds to copy l % kRep
  uint32_t tot[256];       // its bin totals
  uint32_t h2[2][256];     // second-byte histograms under the two picked first bytes
  uint32_t pick[2][2];     // [hi, lo] x (digit, remaining rank)
  uint32_t above, ncand;
  uint32_t wcount[kClsNT / 64];
  uint2 wcand[kClsNT / 64][kWaveCand];  // per-wave candidate lists
};

// Bracket of the keep-th largest key from the sample keys in sm.skeys:
// sample rank ks = keep * kSample / L, the bracket spans ks -+ (4 binomial
// sigmas + 8) sample ranks. The bounds only need to bracket tau, so 16 bits
// of each suffice: the bin (top 16 bits) holding the sample key of rank
// r_hi, resp. r_lo, found with one histogram of the first byte for both
// ranks and one of the second byte per rank; hi = the top of its bin, lo =
// the bottom of its. Scores share few leading bytes (a first-byte bin can
// hold most of a wave's keys, and same-address LDS atomics serialize), so
// each first-byte bin has kRep copies, lane l adding to copy l % kRep.
// Returns (lo, hi) to every thread. sm.h1 and sm.h2 must be zero and
// sm.skeys complete (after a barrier) on entry; ends with a barrier. Its
// barriers order LDS only: the caller's span loads stay in flight.
template <int NT>
__device__ __forceinline__ uint2 sample_bracket(const LongRows &lr, ClassifyLds &sm) {
  constexpr int PER = kSample / NT;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const float ks = (float)lr.keep * (float)kSample / (float)lr.L;
  const float margin = 4.0f * sqrtf(fmaxf(ks * (1.0f - ks / (float)kSample), 0.0f)) + 8.0f;
  const int32_t r_hi = (int32_t)floorf(ks - margin), r_lo = (int32_t)ceilf(ks + margin);
  const int32_t want[2] = {r_hi, r_lo};
  // wave 0: the digit holding the k-th largest key of hist[256] and the rank left in it
  auto pick = [&](const uint32_t *hist, int which, uint32_t k) {
    if (wave == 0) {
      uint32_t c[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = hist[4 * lane + j];
      const uint32_t tot = c[0] + c[1] + c[2] + c[3];
      uint32_t inc = tot;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_down(inc, off, 64);
        if (lane + off < 64) inc += o;
      }
      uint32_t above = inc - tot;
#pragma unroll
      for (int j = 3; j >= 0; --j) {
        const uint32_t upto = above + c[j];
        if (upto >= k && above < k) {
          sm.pick[which][0] = 4 * lane + j;
          sm.pick[which][1] = k - above;
        }
        above = upto;
      }
    }
  };
#pragma unroll
  for (int j = 0; j < PER; ++j) atomicAdd(&sm.h1[sm.skeys[tid + j * NT] >> 24][lane % kRep], 1u);
  lds_barrier();
  if (tid < 256) {
    uint32_t t = 0;
#pragma unroll
    for (int i = 0; i < kRep; ++i) t += sm.h1[tid][(i + tid) % kRep];
    sm.tot[tid] = t;
  }
  lds_barrier();
  for (int which = 0; which < 2; ++which)
    if (want[which] >= 1 && want[which] <= kSample) pick(sm.tot, which, (uint32_t)want[which]);
  lds_barrier();
  const uint32_t d1[2] = {sm.pick[0][0], sm.pick[1][0]};
  const uint32_t k1[2] = {sm.pick[0][1], sm.pick[1][1]};
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint32_t key = sm.skeys[tid + j * NT];
#pragma unroll
    for (int which = 0; which < 2; ++which)
      if ((key >> 24) == d1[which]) atomicAdd(&sm.h2[which][(key >> 16) & 0xFF], 1u);
  }
  lds_barrier();
  for (int which = 0; which < 2; ++which)
    if (want[which] >= 1 && want[which] <= kSample) pick(sm.h2[which], which, k1[which]);
  lds_barrier();
  const uint32_t hi = r_hi < 1 ? 0xFFFFFFFFu : (((d1[0] << 8) | sm.pick[0][0]) << 16) | 0xFFFFu;
  const uint32_t lo = r_lo > kSample ? 0u : ((d1[1] << 8) | sm.pick[1][0]) << 16;
  return make_uint2(lo, hi);
}

// K1, workgroup (r, s): span s of row r. The sample is loaded and the
// bracket computed first, with the first kClsPre span loads per thread in
// flight; the rest of the span streams through a window of kClsWin loads
// per thread, each float4 classified as it arrives. V4: the row base is
// 16-byte aligned and L % 4 == 0, so a lane's 4 tokens are one float4;
// otherwise four scalar loads. Lane l of wave w holds tokens t_span + 4096 j + 256 w + 4 l .. + 3
// for j < kClsPer; bitmask word t / 32 gets the nibbles of lanes 8g .. 8g
// + 7, OR-ed together by 3 DPP steps.
template <bool V4>
__global__ __launch_bounds__(kClsNT) void evict_classify_long_kernel(const LongRows lr, const MarkArgs ma) {
  constexpr int NT = kClsNT, NW = NT / 64, PER = kClsPer, SPER = kSample / NT;
  const int32_t r = blockIdx.x, s = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const int32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int32_t L = lr.L;
  const float *row = lr.scores + (int64_t)r * L;
  __shared__ ClassifyLds sm;
  auto sample_token = [&](int32_t i) {
    const int32_t c = i / kSampleChunk;
    return (int32_t)((int64_t)c * (L - kSampleChunk) / (kSampleChunks - 1)) + i % kSampleChunk;
  };
  // The sample, and this thread's first page-mark entry: its block-table
  // load travels with the sample, the exchange is issued among the span's
  // loads (a barrier would wait for it) and its result is checked at the
  // end.
  const int64_t nthr = (int64_t)gridDim.x * gridDim.y * NT;
  const int64_t e0 = ((int64_t)s * gridDim.x + r) * NT + tid;
  float sv[SPER];
#pragma unroll
  for (int j = 0; j < SPER; ++j) sv[j] = row[sample_token(tid + j * NT)];
  const int32_t mraw = mark_load(ma, e0);
  // The span is read through a window of kClsWin loads per thread: the
  // first kClsPre are issued right behind the sample (before anything
  // waits for it) and fly during the bracket, whose barriers do not wait
  // for them, and each later one is issued as a float4 is classified, so
  // the data of all waves arrives interleaved with the classification
  // instead of one wave's whole share after another's. With all 16 loads
  // issued before the bracket K1 took 29 us on config 5, with a window of 6
  // 25.4-27.4 us, of 2 23.5 us: a wave stalls at issue while the memory
  // pipeline is full, which holds back the bracket. The loads are
  // non-temporal: the scores are read once, and kept out of the caches they
  // leave the INT4 scale runs there for the apply launch (config 5 apply
  // 50.3 -> 44.7 us over repeated calls).
  const int32_t t_span = s * kSpan;
  auto load4 = [&](int j) __attribute__((always_inline)) {
    const int32_t t = t_span + 4 * (j * NT + tid);
    const float *p4 = row + min(t, L - 4);
    if constexpr (V4) {
      typedef float f4v __attribute__((ext_vector_type(4)));
      const f4v x = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(p4));
      return make_float4(x.x, x.y, x.z, x.w);
    } else {
      return make_float4(__builtin_nontemporal_load(p4), __builtin_nontemporal_load(p4 + 1),
                         __builtin_nontemporal_load(p4 + 2), __builtin_nontemporal_load(p4 + 3));
    }
  };
  float4 v[kClsWin];
#pragma unroll
  for (int j = 0; j < kClsPre; ++j) v[j] = load4(j);
  // keeps the loads above in front of the first wait for the sample
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t sink_key = order_key(1e38f);
#pragma unroll
  for (int j = 0; j < SPER; ++j) {
    const int32_t i = tid + j * NT;
    const uint32_t k = order_key(sv[j]);
    sm.skeys[i] = sample_token(i) < lr.sinks ? sink_key : k;
  }
  const int32_t mphys = mark_page(ma, e0, mraw);
  for (int i = tid; i < 256 * kRep; i += NT) (&sm.h1[0][0])[i] = 0;
  for (int i = tid; i < 2 * 256; i += NT) (&sm.h2[0][0])[i] = 0;
  if (tid == 0) sm.above = sm.ncand = 0;
  lds_barrier();
  const uint2 br = sample_bracket<NT>(lr, sm);
  const uint32_t lo = br.x, hi = br.y;
#pragma unroll
  for (int j = kClsPre; j < kClsWin; ++j) v[j] = load4(j);
  uint32_t *bits = lr.bits + (int64_t)r * lr.words;
  const __amdgpu_buffer_rsrc_t brow = __builtin_amdgcn_make_buffer_rsrc(bits, (short)0, lr.words * 4, 0x00020000);
  // Sink tokens count with the key of a 1e38 score and are never evicted.
  const uint32_t sink_gt = sink_key > hi ? 0xFu : 0u, sink_in = sink_key >= lo && sink_key <= hi ? 0xFu : 0u;
  // The scores are compared with the floats whose keys are lo and hi: x <
  // flo implies key(x) < lo and x > fhi implies key(x) > hi, and a token
  // the float compare cannot place (a NaN, -0 against a +0 bound, a NaN
  // bound) becomes a candidate, which the resolve places exactly.
  const float flo = __builtin_bit_cast(float, (lo & 0x80000000u) ? lo ^ 0x80000000u : ~lo);
  const float fhi = __builtin_bit_cast(float, (hi & 0x80000000u) ? hi ^ 0x80000000u : ~hi);
  const uint32_t sink_bits = __builtin_bit_cast(uint32_t, 1e38f);
  uint32_t above = 0, ncand = 0;
  uint32_t mold;  // set by mark_swap where mphys >= 0
  uint32_t wcnt = 0;     // this wave's list length (wave-uniform)
  bool wlost = false;    // the wave's list overflowed (wave-uniform)
  // One float4 of the span: plain = the wave's 256 tokens of this step are
  // all inside the row and past the sinks (every step but the row's first
  // and last), which drops the per-token masks.
  auto step = [&](const float4 &v4, int32_t t0, int32_t word, auto plain) __attribute__((always_inline)) {
    float x[4] = {v4.x, v4.y, v4.z, v4.w};
    uint32_t in_row = 0xFu, sinkm = 0u;
    if constexpr (!plain.value) {
      // nibble masks of the lane's 4 tokens: inside the row, and sinks
      in_row = 0xFu >> (4 - min(4, max(0, L - t0)));
      sinkm = 0xFu >> (4 - min(4, max(0, lr.sinks - t0)));
      if constexpr (!V4) {
        // the slot holding the row's last token was loaded from L - 4:
        // shift it down by d so that x[k] is token t0 + k again (k + d <= 3
        // for every token of the row)
        const int32_t d = min(3, max(0, t0 - (L - 4)));
        if (d >= 1) x[0] = x[1], x[1] = x[2], x[2] = x[3];
        if (d >= 2) x[0] = x[1], x[1] = x[2];
        if (d >= 3) x[0] = x[1];
      }
    }
    uint32_t lt = 0, gt = 0, raw[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      raw[k] = __builtin_bit_cast(uint32_t, x[k]);
      lt |= x[k] < flo ? 1u << k : 0u;
      gt |= x[k] > fhi ? 1u << k : 0u;
    }
    uint32_t cand = ~(lt | gt) & 0xFu, nib = lt;
    if constexpr (!plain.value) {
      gt = ((gt & ~sinkm) | (sink_gt & sinkm)) & in_row;
      cand = ((cand & ~sinkm) | (sink_in & sinkm)) & in_row;
      nib = lt & ~sinkm & in_row;
#pragma unroll
      for (int k = 0; k < 4; ++k) raw[k] = (sinkm >> k) & 1 ? sink_bits : raw[k];
    }
    above += __builtin_popcount(gt);
    const uint32_t nc = __builtin_popcount(cand);
    ncand += nc;
    {  // append the candidates (score bits, token) to the wave's list:
       // offsets from a wave prefix of the lanes' counts (0..4, three bit
       // planes)
      uint32_t pre = 0, tot = 0;
#pragma unroll
      for (int b = 0; b < 3; ++b) {
        const uint64_t bb = __ballot((nc >> b) & 1);
        pre += __builtin_amdgcn_mbcnt_hi((uint32_t)(bb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bb, 0u)) << b;
        tot += (uint32_t)__popcll(bb) << b;
      }
      if (wcnt + tot <= (uint32_t)kWaveCand) {  // wave-uniform
        uint32_t pos = wcnt + pre;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t is = (cand >> k) & 1;
          if (is) sm.wcand[wave][pos] = make_uint2(raw[k], (uint32_t)(t0 + k));
          pos += is;
        }
      } else {
        wlost = true;
      }
      wcnt += tot;
    }
    uint32_t e = nib << (4 * (lane & 7));
    e |= __builtin_bit_cast(uint32_t, dpp_f32<0xB1>(__builtin_bit_cast(float, e)));   // quad_perm [1,0,3,2]
    e |= __builtin_bit_cast(uint32_t, dpp_f32<0x4E>(__builtin_bit_cast(float, e)));   // quad_perm [2,3,0,1]
    e |= __builtin_bit_cast(uint32_t, dpp_f32<0x141>(__builtin_bit_cast(float, e)));  // row_half_mirror
    // Every lane of the group of 8 holds the group's word, and all 8 store
    // it (one write per address) through a buffer resource bounded by the
    // row's words, which drops the words past the row: with no lane mask,
    // every step issues exactly one store, so the compiler can count the
    // window's loads exactly (a store under a lane mask may be skipped, and
    // it would then wait for the newer load of the window as well).
    __builtin_amdgcn_raw_buffer_store_b32(e, brow, word * 4, 0, 0);
  };
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int32_t t0 = t_span + 4 * (j * NT + tid);
    const int32_t tw = t_span + 4 * j * NT + 256 * wave;  // the wave's first token of this step
    const int32_t word = (t_span >> 5) + 8 * (j * NW + wave) + (lane >> 3);
    const float4 cur = v[j % kClsWin];
    if (j + kClsWin < PER) v[j % kClsWin] = load4(j + kClsWin);
    if (j == 0) mark_swap(ma, e0, mphys, mold);
    if (tw >= lr.sinks && tw + 256 <= L)  // wave-uniform
      step(cur, t0, word, IntC<1>{});
    else
      step(cur, t0, word, IntC<0>{});
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    above += __shfl_xor(above, off, 64);
    ncand += __shfl_xor(ncand, off, 64);
  }
  if (lane == 0) {
    if (above) atomicAdd(&sm.above, above);
    if (ncand) atomicAdd(&sm.ncand, ncand);
    sm.wcount[wave] = wlost ? kWaveCand + 1u : wcnt;
  }
  // the page marks: this thread's first entry, then any further ones
  mark_check(ma, e0, mphys, mold);
  for (int64_t e = e0 + nthr; e < ma.entries; e += nthr) mark_entry(ma, e);
  // (the bitmask stores need not be complete for the list copy)
  lds_barrier();
  // The wave lists, concatenated into the span's list.
  uint32_t off = 0, lost = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const uint32_t c = sm.wcount[w];
    off += w < wave ? c : 0u;
    lost |= c > (uint32_t)kWaveCand ? kListLost : 0u;
  }
  uint2 *gl = lr.cand + ((int64_t)r * lr.spans + s) * kSpanCand;
  if (!lost)
    for (uint32_t i = lane; i < wcnt; i += 64) gl[off + i] = sm.wcand[wave][i];
  if (tid == 0) lr.slot[(int64_t)r * lr.spans + s] = make_uint4(sm.above, sm.ncand | lost, lo, hi);
}

static constexpr int32_t kSpanLds = 64;   // spans whose list offsets K2 keeps in LDS
static constexpr int32_t kSpecSpans = 8;  // spans whose lists K2 loads before their counts

struct ResolveLds {
  uint32_t lkey[kResCand], lpos[kResCand];
  SelectShared<kResNT> sh;
  uint32_t hist12[4096], wsum[kResNT / 64], pick[3];  // select12: digit, rank left, bin count
  uint32_t small[64], nsmall;                         // select12: the values of a small bin
  uint32_t lbits[kLdsWords];
  uint32_t cpre[kSpanLds + 1];  // list offsets of the spans (spans <= kSpanLds)
  uint32_t above, ncand, lost;
  uint32_t xabove, xin;  // listed keys above hi, resp. inside [lo, hi]
};

// d of the k-th largest (1 <= k <= number of values) of the values d in
// [0, range] handed out by visit(f) (every thread of the workgroup calls
// it): 12-bit radix passes from the top bit of range. The first pass's
// histogram (bin (d >> shift) for shift = max(bits(range) - 12, 0)) is
// built by the caller in sm.hist12 and visible to all threads on entry.
// When the bin a pass picks holds at most 64 values, they are gathered and
// one wave ranks them (the k-th largest among them is the result) instead
// of a further pass. sm.nsmall must be zero on entry. Thread t owns bins
// 4t .. 4t + 3 of the suffix scan (NT = 1024).
template <int NT, typename Visit>
__device__ uint32_t select12(Visit visit, uint32_t k, uint32_t range, ResolveLds &sm) {
  static_assert(NT * 4 == 4096, "select12 takes 1024 threads");
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nbits = range ? 32 - __builtin_clz(range) : 1;
  uint32_t prefix = 0, pmask = 0;
  for (int shift = max(nbits - 12, 0), first = 1;; shift = max(shift - 12, 0), first = 0) {
    if (!first) {
      if (sm.pick[2] <= 64u) {
        // the picked bin's values (d & pmask == prefix), ranked by wave 0
        visit([&](uint32_t d) {
          if ((d & pmask) == prefix) sm.small[atomicAdd(&sm.nsmall, 1u)] = d;
        });
        __syncthreads();
        if (wave == 0) {
          const uint32_t c = sm.pick[2];
          const uint32_t mine = (uint32_t)lane < c ? sm.small[lane] : 0u;
          uint32_t gt = 0, ge = 0;  // values above, resp. at or above, this lane's
          for (uint32_t j = 0; j < c; ++j) {
            const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)mine, (int)j);
            gt += o > mine;
            ge += o >= mine;
          }
          const uint64_t b = __ballot((uint32_t)lane < c && gt < k && k <= ge);
          if (lane == 0) sm.pick[0] = (uint32_t)__builtin_amdgcn_readlane((int)mine, (int)__builtin_ctzll(b));
        }
        __syncthreads();
        return sm.pick[0];
      }
      for (int i = tid; i < 4096; i += NT) sm.hist12[i] = 0;
      __syncthreads();
      visit([&](uint32_t d) {
        if ((d & pmask) == prefix) atomicAdd(&sm.hist12[(d >> shift) & 0xFFFu], 1u);
      });
      __syncthreads();
    }
    uint32_t c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] = sm.hist12[4 * tid + j];
    const uint32_t tot = c[0] + c[1] + c[2] + c[3];
    uint32_t inc = tot;  // sum of tot over lanes >= lane of the wave
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = __shfl_down(inc, off, 64);
      if (lane + off < 64) inc += o;
    }
    if (lane == 0) sm.wsum[wave] = inc;
    __syncthreads();
    uint32_t above = inc - tot;
#pragma unroll
    for (int w = 0; w < NW; ++w) above += w > wave ? sm.wsum[w] : 0u;
#pragma unroll
    for (int j = 3; j >= 0; --j) {
      const uint32_t upto = above + c[j];  // values with digit >= 4 tid + j
      if (upto >= k && above < k) {
        sm.pick[0] = 4 * tid + j;
        sm.pick[1] = k - above;
        sm.pick[2] = c[j];
      }
      above = upto;
    }
    __syncthreads();
    prefix |= sm.pick[0] << shift;
    pmask |= 0xFFFu << shift;
    k = sm.pick[1];
    if (shift == 0) break;
  }
  return prefix;
}

// K2: one workgroup per row.
__global__ __launch_bounds__(kResNT) void evict_resolve_long_kernel(const LongRows lr) {
  constexpr int NT = kResNT, NW = NT / 64;
  const int32_t r = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int32_t L = lr.L;
  const float *row = lr.scores + (int64_t)r * L;
  uint32_t *bits = lr.bits + (int64_t)r * lr.words;
  const uint4 *slot = lr.slot + (int64_t)r * lr.spans;
  __shared__ ResolveLds sm;
  const uint32_t sink_key = order_key(1e38f);
  if (tid == 0) sm.xabove = sm.xin = sm.nsmall = 0;
  // The first 64 spans' slots, loaded first (wave 0 scans them as soon as
  // they arrive; a later load would have it wait for the ones below too).
  const uint4 sl0 = slot[min(lane, lr.spans - 1)];
  // The row's first kLdsWords bitmask words (written by the classify
  // launch) are read now, for the merge at the end, and the merge's LDS
  // copy and the first select pass's histogram are cleared now.
  constexpr int PW = kLdsWords / NT;
  uint32_t bw[PW];
#pragma unroll
  for (int k = 0; k < PW; ++k) bw[k] = bits[min(k * NT + tid, lr.words - 1)];
  // With up to kSpecSpans spans, the first nq = kResCand / spans entries of
  // every span's list are loaded now, with the counts (entries past a
  // span's count are dropped), so the gather does not wait for the counts
  // first. Entry v = k NT + tid of that sequence is entry v % nq of span
  // v / nq.
  const uint2 *gl0 = lr.cand + (int64_t)r * lr.spans * kSpanCand;
  constexpr int KS = kResCand / NT;
  const bool spec = lr.spans <= kSpecSpans;
  const uint32_t nq = spec ? (uint32_t)(kResCand / lr.spans) : 1u;
  // (loaded whatever spans is, in bounds, so that no branch joins them)
  uint2 sc[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    const uint32_t v = k * NT + tid, q = min(v / nq, (uint32_t)lr.spans - 1);
    sc[k] = gl0[(int64_t)q * kSpanCand + min(v - q * nq, (uint32_t)kSpanCand - 1)];
  }
  for (int i = tid; i < kLdsWords; i += NT) sm.lbits[i] = 0;
  for (int i = tid; i < 4096; i += NT) sm.hist12[i] = 0;
  if (wave == 0) {  // the spans' counts, and their lists' offsets, 64 spans per step
    uint32_t a = 0, off = 0, l = 0;
    for (int32_t q0 = 0; q0 < lr.spans; q0 += 64) {
      const int32_t q = q0 + lane;
      const uint4 sl = q0 == 0 ? sl0 : slot[min(q, lr.spans - 1)];
      const uint32_t c = q < lr.spans ? sl.y & ~kListLost : 0u;
      a += q < lr.spans ? sl.x : 0u;
      l |= q < lr.spans ? sl.y & kListLost : 0u;
      uint32_t inc = c;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(inc, o, 64);
        if (lane >= o) inc += v;
      }
      if (q < kSpanLds) sm.cpre[q] = off + inc - c;
      off += __shfl(inc, 63, 64);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      a += __shfl_xor(a, o, 64);
      l |= __shfl_xor(l, o, 64);
    }
    if (lane == 0) {
      sm.above = a;
      sm.ncand = off;
      sm.lost = l;
      if (lr.spans <= kSpanLds) sm.cpre[lr.spans] = off;
    }
  }
  const uint4 s0 = slot[0];  // every span holds the row's bracket
  const uint32_t lo = s0.z, hi = s0.w;
  lds_barrier();
  const uint32_t above = sm.above, nc = sm.ncand, keep = (uint32_t)lr.keep;
  // first select pass: bins of (key - lo) >> shift1
  const uint32_t range = hi - lo;
  const int shift1 = max((range ? 32 - __builtin_clz(range) : 1) - 12, 0);
  if (above < keep && above + nc >= keep && nc <= (uint32_t)kResCand && !sm.lost) {
    // The spans' candidate lists. The classify launch places a token by
    // float compares with the floats of lo and hi; a score the compares
    // cannot place (a NaN) is listed whatever its key: listed keys above
    // hi count as kept, keys below lo are evicted (a NaN's never is), and the select runs over
    // the keys in [lo, hi], whose first-pass histogram is built here.
    uint32_t xa = 0, xi = 0;
    auto take = [&](uint32_t e, uint2 c) {
      const uint32_t key = order_key(__builtin_bit_cast(float, c.x));
      sm.lkey[e] = key;
      sm.lpos[e] = c.y;
      xa += key > hi;
      const bool in = key >= lo && key <= hi;
      xi += in;
      if (in) atomicAdd(&sm.hist12[(key - lo) >> shift1], 1u);
    };
    if (spec) {
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        // (keeps the key computation here, after the barrier: hoisted to
        // the loads, it would make the code wait for them there)
        asm volatile("" : "+v"(sc[k]));
        const uint32_t v = k * NT + tid, q = v / nq, i = v - q * nq;
        if (q < (uint32_t)lr.spans && i < sm.cpre[q + 1] - sm.cpre[q]) take(sm.cpre[q] + i, sc[k]);
      }
      // a span with more than nq candidates: the rest of its list
      for (int32_t q = 0; q < lr.spans; ++q) {
        const uint32_t cnt = sm.cpre[q + 1] - sm.cpre[q];
        for (uint32_t i = nq + tid; i < cnt; i += NT) take(sm.cpre[q] + i, gl0[(int64_t)q * kSpanCand + i]);
      }
    } else if (lr.spans <= kSpanLds) {
      // all spans' entries as one sequence e = cpre[q] + i: unconditional
      // loads (index clamped), all in flight together
      for (uint32_t e0 = 0; e0 < nc; e0 += 8 * NT) {
        uint2 c[8];
        int32_t q = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t e = min(e0 + k * NT + tid, nc - 1);
          while (q + 1 < lr.spans && sm.cpre[q + 1] <= e) ++q;  // e grows with k
          c[k] = gl0[(int64_t)q * kSpanCand + (e - sm.cpre[q])];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (e0 + k * NT + tid < nc) take(e0 + k * NT + tid, c[k]);
      }
    } else {
      uint32_t base = 0;
      for (int32_t q = 0; q < lr.spans; ++q) {
        const uint32_t cnt = slot[q].y;
        const uint2 *gl = gl0 + (int64_t)q * kSpanCand;
        for (uint32_t i0 = 0; i0 < cnt; i0 += 8 * NT) {
          uint2 c[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) c[k] = gl[min(i0 + k * NT + tid, cnt - 1)];
#pragma unroll
          for (int k = 0; k < 8; ++k)
            if (i0 + k * NT + tid < cnt) take(base + i0 + k * NT + tid, c[k]);
        }
        base += cnt;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      xa += __shfl_xor(xa, off, 64);
      xi += __shfl_xor(xi, off, 64);
    }
    if (lane == 0 && (xa | xi)) {
      atomicAdd(&sm.xabove, xa);
      atomicAdd(&sm.xin, xi);
    }
    __syncthreads();
  }
  const uint32_t above_all = above + sm.xabove;
  const bool listed = above < keep && above + nc >= keep && nc <= (uint32_t)kResCand && !sm.lost &&
                      above_all < keep && above_all + sm.xin >= keep;
  if (listed) {
    // tau - lo = the (keep - above_all)-th largest of key - lo over the
    // candidates in [lo, hi].
    const uint32_t tau = lo + select12<NT>(
                                  [&](auto f) {
                                    for (uint32_t i = tid; i < nc; i += NT) {
                                      const uint32_t k = sm.lkey[i];
                                      if (k >= lo && k <= hi) f(k - lo);
                                    }
                                  },
                                  keep - above_all, hi - lo, sm);
    // The evicted candidates' bits: OR-ed into an LDS copy of a range of
    // kLdsWords bitmask words, then merged into the row's words (the first
    // range's words were read at the start).
    for (int32_t w0 = 0; w0 < lr.words; w0 += kLdsWords) {
      if (w0 > 0) {
        for (int i = tid; i < kLdsWords; i += NT) sm.lbits[i] = 0;
        __syncthreads();
      }
      for (uint32_t i = tid; i < nc; i += NT) {
        const int32_t t = (int32_t)sm.lpos[i], w = (t >> 5) - w0;
        const uint32_t k = sm.lkey[i];
        if (k < tau && k != kNanKey && t >= lr.sinks && w >= 0 && w < kLdsWords) atomicOr(&sm.lbits[w], 1u << (t & 31));
      }
      __syncthreads();
      uint32_t lb[PW], gw[PW];
#pragma unroll
      for (int k = 0; k < PW; ++k) {
        const int32_t i = k * NT + tid;
        lb[k] = w0 + i < lr.words ? sm.lbits[i] : 0u;
        gw[k] = w0 == 0 ? bw[k] : lb[k] ? bits[w0 + i] : 0u;
      }
#pragma unroll
      for (int k = 0; k < PW; ++k)
        if (lb[k]) bits[w0 + k * NT + tid] = gw[k] | lb[k];
      __syncthreads();
    }
    return;
  }
  // Bracket missed (or too many ties or candidates, or a list overflowed):
  // exact select over the whole row, then every bitmask word rewritten.
  const uint32_t tau = radix_select<NT, true>(
      [&](auto f) {
        for (int32_t t0 = 0; t0 < L; t0 += 8 * NT) {
          float x[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) x[j] = row[min(t0 + tid + j * NT, L - 1)];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int32_t t = t0 + tid + j * NT;
            if (t < L) f(t < lr.sinks ? sink_key : order_key(x[j]));
          }
        }
      },
      keep, sm.sh);
  const int32_t nw64 = (L + 63) / 64;
  for (int32_t w = wave; w < nw64; w += NW) {
    const int32_t t = w * 64 + lane;
    const uint32_t key = token_key(row, min(t, L - 1), lr.sinks);
    const bool e = t < L && t >= lr.sinks && key < tau && key != kNanKey;
    const uint64_t b = __ballot(e);
    if (lane == 0) {
      bits[2 * w] = (uint32_t)b;
      bits[2 * w + 1] = (uint32_t)(b >> 32);
    }
  }
}

// K3: zero the evicted rows of logical blocks [lb_begin, lb_end) of row
// (seq n, head h), then vote for the fully evicted ones (after this
// workgroup's own zeroing, so the H-th vote, the unlink, follows every
// head's reads of the block-table entry).
__global__ __launch_bounds__(256) void evict_apply_kernel(const LongRows lr, int32_t *__restrict__ block_tables,
                                                          int32_t *__restrict__ is_block_free, int32_t M,
                                                          int64_t total_pool_blocks, RowZero z) {
  constexpr int NT = 256, NW = NT / 64;
  const int32_t r = blockIdx.x, n = r / lr.H, h = r % lr.H, tid = threadIdx.x, lane = tid & 63;
  const int32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t *evbits = lr.bits + (int64_t)r * lr.words;
  const int32_t *bt = block_tables + (int64_t)n * M;
  const int32_t nlb = min((lr.L + z.bs - 1) / z.bs, M);
  const int32_t per = (nlb + kApplySplit - 1) / kApplySplit;
  const int32_t lb_begin = blockIdx.y * per, lb_end = min(nlb, lb_begin + per);
  auto ev = [&](int32_t t) { return (evbits[t >> 5] >> (t & 31)) & 1u; };
  if (lb_begin < lb_end) {
    if (z.kv_format == MEMOPT_KV_INT4) {
      const Int4Page f(z.D);
      if (f.G <= 16 && (reinterpret_cast<uintptr_t>(z.k) & 15) == 0) {
        zero_int4_scale_lines<NW>((uint8_t *)z.k, f, z.H, h, bt, evbits, lb_begin, lb_end, total_pool_blocks, wave,
                                  lane, pages_aliased(z));
      } else {
        const int32_t p = lane >> 3;
        for (int32_t lb = lb_begin + wave; lb < lb_end; lb += NW) {
          const uint32_t m16 = (evbits[lb >> 1] >> ((lb & 1) * 16)) & 0xFFFFu;
          const int32_t phys = bt[lb];
          if (m16 == 0 || phys < 0 || phys >= total_pool_blocks) continue;  // wave-uniform
          zero_int4_block((uint8_t *)z.k + ((int64_t)phys * z.H + h) * f.block, z.D, lane, (m16 >> p) & 1,
                          (m16 >> (p + 8)) & 1);
        }
      }
    } else {
      const int32_t t_end = min(lr.L, lb_end * z.bs);
      for (int32_t t0 = lb_begin * z.bs + wave * 64; t0 < t_end; t0 += NW * 64) {
        const int32_t t = t0 + lane, lb = t / z.bs;
        bool e = t < t_end && ev(t);
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
  }
  __syncthreads();
  const int32_t full_end = min(lb_end, min(lr.L / z.bs, M));
  for (int32_t lb = lb_begin + tid; lb < full_end; lb += NT) {
    bool all = true;
    for (int j = 0; j < z.bs && all; ++j) all = ev(lb * z.bs + j);
    if (!all) continue;
    const int32_t phys = bt[lb];
    if (phys < 0 || phys >= total_pool_blocks || page_shared(z, phys)) continue;
    const int prev = atomicAdd(&is_block_free[phys], 1);
    if (prev + 1 == lr.H) block_tables[(int64_t)n * M + lb] = -1;
  }
}

// K3 for INT4 pools on the scale-line path (G <= 16, 16-byte aligned pool):
// work items are (logical block, head) pairs of one sequence in page-major
// order, so the H scale runs of a physical page (one per head, a block
// apart) are rewritten together instead of one head's runs spread over the
// whole pool: evicting a quarter of the tokens touches nearly every run, and
// the rewrite is bound by random accesses to memory rows. Workgroup
// (n, y) owns logical blocks [y * per, (y + 1) * per) of sequence n for all
// heads; per * H is about 256 items, one pass of its 4 waves. The votes
// follow the workgroup's own zeroing; a page's H votes of this sequence all
// come from this workgroup, and the unlink writes only this sequence's entry.
// i / H for 0 <= i < 2^24 and 1 <= H < 2^16 as (i * hm) >> 40 with
// hm = ceil(2^40 / H): hm = 2^40 / H + e (0 <= e < 1) adds i e / 2^40 <
// 2^-16 <= 1 / H to the exact quotient, which never reaches the next
// integer.
__device__ __forceinline__ int32_t div_h(int32_t i, uint64_t hm) { return (int32_t)(((uint64_t)(uint32_t)i * hm) >> 40); }

__global__ __launch_bounds__(256) void evict_apply_pages_kernel(const LongRows lr, int32_t *__restrict__ block_tables,
                                                                int32_t *__restrict__ is_block_free, int32_t M,
                                                                int64_t total_pool_blocks, RowZero z, int32_t nlb,
                                                                int32_t per, uint64_t hm) {
  constexpr int NT = 256, NW = NT / 64, UL = 8;
  const int32_t n = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int32_t H = lr.H;
  const uint32_t *bits = lr.bits + (int64_t)n * H * lr.words;  // row (n, h) at h * words
  const int32_t *bt = block_tables + (int64_t)n * M;
  const int32_t lb_begin = blockIdx.y * per, lb_end = min(nlb, lb_begin + per);
  const int32_t items = max(0, lb_end - lb_begin) * H;
  auto mask16 = [&](int32_t lb, int32_t h) { return (bits[(int64_t)h * lr.words + (lb >> 1)] >> ((lb & 1) * 16)) & 0xFFFFu; };
  const Int4Page f(z.D);
  uint8_t *pool = (uint8_t *)z.k;
  // Same line rewrite as zero_int4_scale_lines: 4 G lanes per 16-token
  // block, one 16-byte chunk each, UL steps of 64 / (4 G) blocks in flight.
  const int32_t lpb = 4 * f.G, bpw = 64 / lpb, jb = lane / lpb, q = lane % lpb;
  const int32_t gmask = 16 * f.G - 1;
  const int32_t full_end = min(lb_end, min(lr.L / 16, M));
  // Fully evicted (block, head) items found during the rewrite, voted after
  // one barrier: (logical block, page), a list per wave (each wave clears
  // its own count, so no barrier is needed before the rewrite).
  constexpr int kVotes = 64;
  __shared__ int2 s_vote[NW][kVotes];
  __shared__ uint32_t s_nvote[NW];
  if (lane == 0) s_nvote[wave] = 0;
  for (int32_t i0 = wave * bpw * UL; i0 < items; i0 += NW * bpw * UL) {
    uint32_t mm[UL];
    int32_t ph[UL], hh[UL], ll[UL];
    // All loads are unconditional, so that the steps' loads are in flight
    // together: items past the end read the last item's mask and page, and
    // a lane with nothing to clear reads the line of (page 0, head 0),
    // which every such lane shares, and stores nothing.
    uint32_t wd[UL];
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      const int32_t i = min(i0 + u * bpw + jb, items - 1), q = div_h(i, hm);
      ll[u] = lb_begin + q;
      hh[u] = i - q * H;
    }
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      wd[u] = bits[(int64_t)hh[u] * lr.words + (ll[u] >> 1)];
      ph[u] = bt[ll[u]];
    }
    const bool aliased = pages_aliased(z);  // loaded with the masks and pages
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      const bool in = jb < bpw && i0 + u * bpw + jb < items;  // 64 % lpb lanes idle when G is no power of 2
      mm[u] = in ? (wd[u] >> ((ll[u] & 1) * 16)) & 0xFFFFu : 0u;
      if (!in) ph[u] = -1;
    }
    uint4 v[UL];
    uint4 *w[UL];
    const uint4 *idle = reinterpret_cast<const uint4 *>(pool + f.kscales) + q;
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      if (!(ph[u] >= 0 && ph[u] < total_pool_blocks)) mm[u] = 0;
      w[u] = reinterpret_cast<uint4 *>(pool + ((int64_t)(mm[u] ? ph[u] : 0) * H + hh[u]) * f.block + f.kscales) + q;
      v[u] = *(mm[u] && !aliased ? w[u] : idle);
    }
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      if (q == 0 && mm[u] == 0xFFFFu && ll[u] < full_end) {
        const uint32_t slot = atomicAdd(&s_nvote[wave], 1u);
        if (slot < (uint32_t)kVotes) s_vote[wave][slot] = make_int2(ll[u], ph[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < UL; ++u) {
      if (!mm[u]) continue;
      uint32_t keepm[4] = {~0u, ~0u, ~0u, ~0u};
#pragma unroll
      for (int k = 0; k < 8; ++k) {  // half 8 q + k of the run; scale_idx(t, g) = 16 g + 2 (t & 7) + (t >> 3)
        const int32_t i = (8 * q + k) & gmask;
        const int32_t t = 8 * (i & 1) + ((i & 15) >> 1);
        if ((mm[u] >> t) & 1) keepm[k >> 1] &= (k & 1) ? 0x0000FFFFu : 0xFFFF0000u;
      }
      if (aliased) {
        uint32_t *wd = reinterpret_cast<uint32_t *>(w[u]);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (keepm[k] != ~0u) atomicAnd(wd + k, keepm[k]);
      } else {
        *w[u] = (uint4){v[u].x & keepm[0], v[u].y & keepm[1], v[u].z & keepm[2], v[u].w & keepm[3]};
      }
    }
  }
  // Every wave's block-table reads are done (their values were used) once
  // it reaches the barrier, so an unlink after it cannot hide an entry from
  // a head of this call; the barrier does not wait for the stores.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  auto vote = [&](int32_t lb, int32_t phys) {
    if (page_shared(z, phys)) return;
    const int prev = atomicAdd(&is_block_free[phys], 1);
    if (prev + 1 == H) block_tables[(int64_t)n * M + lb] = -1;
  };
  bool over = false;
#pragma unroll
  for (int w = 0; w < NW; ++w) over = over || s_nvote[w] > (uint32_t)kVotes;
  if (!over) {
    for (uint32_t i = lane; i < s_nvote[wave]; i += 64) vote(s_vote[wave][i].x, s_vote[wave][i].y);
  } else {  // more fully evicted items than a list holds: find them again
    const int32_t vitems = max(0, full_end - lb_begin) * H;
    for (int32_t i = tid; i < vitems; i += NT) {
      const int32_t q = div_h(i, hm), lb = lb_begin + q, h = i - q * H;
      if (mask16(lb, h) != 0xFFFFu) continue;
      const int32_t phys = bt[lb];
      if (phys < 0 || phys >= total_pool_blocks) continue;
      vote(lb, phys);
    }
  }
}

// evict_cache, src/csrc/kv_cache.cu:379-483: one workgroup per (block, head)
// and any block_size up to kEvictCacheMaxBs (the scores of a block live in
// LDS). The reference selects keep = max(1, (int)(r * bs)) times the largest
// remaining score above -1e38 and evicts scores below the last one selected
// (-1e38 when fewer than keep scores exceed it). Here: tau is the keep-th
// largest of the scores above -1e38 when there are at least keep of them,
// else -1e38, and position i is evicted when s_i < tau, i.e. when at least
// keep scores above -1e38 exceed s_i (or, in the short case, s_i < -1e38).
static constexpr int32_t kEvictCacheMaxBs = 8192;

__global__ __launch_bounds__(256) void evict_cache_kernel(const float *__restrict__ scores, int32_t bs, int32_t H,
                                                          int32_t keep, RowZero z) {
  const int64_t blk = blockIdx.x;
  const int32_t h = blockIdx.y;
  extern __shared__ float ssc[];
  __shared__ int32_t s_valid;
  if (threadIdx.x == 0) s_valid = 0;
  __syncthreads();
  int32_t nv = 0;
  for (int32_t i = threadIdx.x; i < bs; i += 256) {
    const float v = scores[(blk * bs + i) * H + h];
    ssc[i] = v;
    nv += v > -1e38f ? 1 : 0;
  }
  if (nv) atomicAdd(&s_valid, nv);
  __syncthreads();
  const bool enough = s_valid >= keep;
  // Pages of more than 256 tokens: tau = the key of the keep-th largest
  // score above -1e38 (a radix select over the block's scores in LDS), and a
  // score above -1e38 is evicted when its key is below tau, the same set as
  // the count below, in O(bs) instead of O(bs^2) per (block, head).
  __shared__ SelectShared<256> sh;
  uint32_t tau = 0;
  if (bs > 256 && enough)  // workgroup-uniform
    tau = radix_select<256, false>(
        [&](auto f) {
          for (int32_t i = threadIdx.x; i < bs; i += 256)
            if (ssc[i] > -1e38f) f(order_key(ssc[i]));
        },
        (uint32_t)keep, sh);
  for (int32_t i = threadIdx.x; i < bs; i += 256) {
    const float si = ssc[i];
    bool evict;
    if (enough) {
      if (bs > 256) {
        // a NaN score has no key order: no score exceeds it (not evicted);
        // one at or below -1e38 is exceeded by every score above -1e38
        evict = !(si != si) && (si > -1e38f ? order_key(si) < tau : true);
      } else {
        int32_t greater = 0;
        for (int32_t j = 0; j < bs; ++j) greater += (ssc[j] > -1e38f && ssc[j] > si) ? 1 : 0;
        evict = greater >= keep;
      }
    } else {
      evict = si < -1e38f;
    }
    if (evict) zero_row(z, blk, i, h);
  }
}

// ---------------------------------------------------------------------------
// evict_tokens workspace (allocated by the caller, see
// memopt_evict_workspace_size; any content, nothing persists between calls):
//   [0, 256)                 alias flag (u32);
//   [256, 256 + marks)       page marks, one u32 per pool block;
//   then (256-aligned)       long-row state: span slots, candidate lists and
//                            row bitmasks (rows longer than kShortRow only).
// ---------------------------------------------------------------------------
static constexpr int64_t kEvictHeader = 256;

static int64_t evict_marks_bytes(int64_t total_pool_blocks) {
  return (4 * total_pool_blocks + 255) / 256 * 256;
}

static int64_t evict_long_bytes(int64_t num_seqs, int32_t num_heads, int32_t seq_len) {
  if (seq_len <= kShortRow) return 0;
  const int64_t rows = num_seqs * num_heads;
  const int64_t words = ((int64_t)seq_len + 63) / 64 * 2;
  const int64_t spans = ((int64_t)seq_len + kSpan - 1) / kSpan;
  return rows * (spans * ((int64_t)sizeof(uint4) + kSpanCand * (int64_t)sizeof(uint2)) +
                 words * (int64_t)sizeof(uint32_t));
}

// Call ids for the alias flag: distinct for 2^32 - 1 consecutive calls.
static std::atomic<uint32_t> g_evict_calls{0};

static uint32_t evict_tag() {
  uint32_t t = g_evict_calls.fetch_add(1, std::memory_order_relaxed) + 1;
  while (t == 0) t = g_evict_calls.fetch_add(1, std::memory_order_relaxed) + 1;
  return t;
}

}  // namespace memopt

using namespace memopt;

extern "C" {

int memopt_evict_workspace_size(int32_t num_seqs, int32_t num_heads, int32_t seq_len,
                                int32_t max_blocks_per_seq, int64_t total_pool_blocks, int64_t *bytes) {
  (void)max_blocks_per_seq;
  MEMOPT_REQUIRE(bytes, MEMOPT_ERR_INVALID, "evict_workspace_size: null output");
  MEMOPT_REQUIRE(num_seqs >= 0 && num_heads >= 0 && seq_len >= 0 && total_pool_blocks >= 0, MEMOPT_ERR_INVALID,
                 "evict_workspace_size: negative size");
  *bytes = kEvictHeader + evict_marks_bytes(total_pool_blocks) + evict_long_bytes(num_seqs, num_heads, seq_len);
  return MEMOPT_OK;
}

int memopt_evict_tokens(const float *attention_scores, int32_t num_seqs, int32_t num_heads, int32_t seq_len,
                        int32_t *block_tables, int32_t max_blocks_per_seq, int32_t *is_block_free,
                        int64_t total_pool_blocks, float retain_ratio, int32_t num_sink_tokens, void *workspace,
                        int64_t workspace_bytes, void *stream) {
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
  int64_t need = 0;
  (void)memopt_evict_workspace_size(num_seqs, num_heads, seq_len, max_blocks_per_seq, total_pool_blocks, &need);
  MEMOPT_REQUIRE(workspace && workspace_bytes >= need, MEMOPT_ERR_INVALID,
                 "evict_tokens: workspace too small (memopt_evict_workspace_size gives " + std::to_string(need) +
                     " bytes)");
  MEMOPT_REQUIRE(((uintptr_t)workspace & 15) == 0, MEMOPT_ERR_INVALID,
                 "evict_tokens: workspace must be 16-byte aligned");
  MEMOPT_REQUIRE((int64_t)num_seqs * max_blocks_per_seq < (1LL << 31), MEMOPT_ERR_UNSUPPORTED,
                 "evict_tokens: block tables too large");
  // keep = clamp((int)ceilf(r * L), 1, L), in fp32 as src/csrc/kv_cache.cu:754-755.
  int keep = (int)ceilf(retain_ratio * (float)seq_len);
  keep = keep < 1 ? 1 : (keep > seq_len ? seq_len : keep);
  const int32_t sinks = num_sink_tokens < 0 ? 0 : (num_sink_tokens > seq_len ? seq_len : num_sink_tokens);
  MEMOPT_REQUIRE(p.kv_format != MEMOPT_KV_INT4 || p.block_size == 16, MEMOPT_ERR_UNSUPPORTED,
                 "evict_tokens: INT4 page pools use 16-token pages");
  MEMOPT_REQUIRE((int64_t)seq_len + kSpan < (1LL << 31), MEMOPT_ERR_UNSUPPORTED,
                 "evict_tokens: seq_len too large");
  const bool int4 = p.kv_format == MEMOPT_KV_INT4;
  const bool long_rows = seq_len > kShortRow;
  const int64_t rows = (int64_t)num_seqs * num_heads;
  const int32_t words = (seq_len + 63) / 64 * 2;
  const int32_t spans = (seq_len + kSpan - 1) / kSpan;
  hipStream_t st = (hipStream_t)stream;
  const uint32_t tag = evict_tag();
  uint8_t *ws = (uint8_t *)workspace;
  uint32_t *flag = (uint32_t *)ws;
  uint32_t *marks = (uint32_t *)(ws + kEvictHeader);
  uint8_t *long_ws = ws + kEvictHeader + evict_marks_bytes(total_pool_blocks);
  RowZero z{p.kv_format, p.num_heads, p.head_dim, p.block_size, p.key, p.value, p.key_scales, p.value_scales,
            flag, marks, tag};
  // Pages listed more than once in the block tables: INT4 pools switch the
  // scale rewrite to atomics, and no format votes for them.
  MarkArgs ma{block_tables, 0, max_blocks_per_seq,
              (int32_t)std::min<int64_t>(((int64_t)seq_len + p.block_size - 1) / p.block_size, max_blocks_per_seq),
              total_pool_blocks, marks, flag, tag};
  if (ma.nlb > 0) ma.entries = (int64_t)num_seqs * max_blocks_per_seq;
  int rc = MEMOPT_OK;
  if (!long_rows && ma.entries > 0) {
    hipLaunchKernelGGL(mark_pages_kernel, dim3((unsigned)((ma.entries + 255) / 256)), dim3(256), 0, st, ma);
    rc = check_launch("evict_tokens(mark_pages)");
    if (rc != MEMOPT_OK) return rc;
  }
  if (long_rows) {
    LongRows lr;
    lr.scores = attention_scores;
    lr.H = num_heads;
    lr.L = seq_len;
    lr.keep = keep;
    lr.sinks = sinks;
    lr.words = words;
    lr.spans = spans;
    lr.slot = reinterpret_cast<uint4 *>(long_ws);
    lr.cand = reinterpret_cast<uint2 *>(lr.slot + rows * spans);
    lr.bits = reinterpret_cast<uint32_t *>(lr.cand + rows * spans * (int64_t)kSpanCand);
    MEMOPT_REQUIRE(rows < (1LL << 31), MEMOPT_ERR_UNSUPPORTED, "evict_tokens: too many (seq, head) rows");
    if (seq_len % 4 == 0 && ((uintptr_t)attention_scores & 15) == 0)
      hipLaunchKernelGGL(evict_classify_long_kernel<true>, dim3((unsigned)rows, (unsigned)spans), dim3(kClsNT), 0, st,
                         lr, ma);
    else
      hipLaunchKernelGGL(evict_classify_long_kernel<false>, dim3((unsigned)rows, (unsigned)spans), dim3(kClsNT), 0,
                         st, lr, ma);
    hipLaunchKernelGGL(evict_resolve_long_kernel, dim3((unsigned)rows), dim3(kResNT), 0, st, lr);
    const int32_t nlb = std::min((seq_len + p.block_size - 1) / p.block_size, max_blocks_per_seq);
    if (int4 && p.head_dim / 64 <= 16 && ((uintptr_t)p.key & 15) == 0 && num_heads < 65536) {
      const int32_t per = std::max(1, 256 / num_heads);
      const uint64_t hm = ((1ULL << 40) + (uint64_t)num_heads - 1) / (uint64_t)num_heads;
      hipLaunchKernelGGL(evict_apply_pages_kernel, dim3((unsigned)num_seqs, (unsigned)((nlb + per - 1) / per)),
                         dim3(256), 0, st, lr, block_tables, is_block_free, max_blocks_per_seq, total_pool_blocks, z,
                         nlb, per, hm);
    } else {
      hipLaunchKernelGGL(evict_apply_kernel, dim3((unsigned)rows, kApplySplit), dim3(256), 0, st, lr, block_tables,
                         is_block_free, max_blocks_per_seq, total_pool_blocks, z);
    }
    return check_launch("evict_tokens(long rows)");
  }
  const size_t lds = (size_t)words * sizeof(uint32_t);
  const dim3 grid(num_seqs, num_heads);
  // Rows up to 8192 (32768) tokens keep their keys in registers with 512
  // (1024) threads (config 3, 8192 tokens: 512 threads x 16 keys 28.8-29.0
  // us per call, 256 x 32 32.7, 1024 x 8 36.4).
  if (seq_len <= 512 * 16)
    hipLaunchKernelGGL((evict_tokens_kernel<512, 16>), grid, dim3(512), lds, st, attention_scores, block_tables,
                       is_block_free, num_heads, seq_len, max_blocks_per_seq, total_pool_blocks, keep, sinks, z);
  else
    hipLaunchKernelGGL((evict_tokens_kernel<1024, 32>), grid, dim3(1024), lds, st, attention_scores, block_tables,
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
  MEMOPT_REQUIRE(p.block_size <= kEvictCacheMaxBs, MEMOPT_ERR_UNSUPPORTED,
                 "evict_cache: block_size > " + std::to_string(kEvictCacheMaxBs) + " not supported");
  if (num_blocks == 0) return MEMOPT_OK;
  int keep = (int)(retain_ratio * (float)p.block_size);  // truncation, src/csrc/kv_cache.cu:426
  keep = keep < 1 ? 1 : (keep > p.block_size ? p.block_size : keep);
  RowZero z{p.kv_format, p.num_heads, p.head_dim, p.block_size, p.key, p.value, p.key_scales, p.value_scales,
            nullptr, nullptr, 0};
  MEMOPT_REQUIRE(num_blocks < (1LL << 31), MEMOPT_ERR_UNSUPPORTED, "evict_cache: too many blocks");
  hipLaunchKernelGGL(evict_cache_kernel, dim3((unsigned)num_blocks, p.num_heads), dim3(256),
                     (size_t)p.block_size * sizeof(float), (hipStream_t)stream, attention_scores, p.block_size,
                     p.num_heads, keep, z);
  return check_launch("evict_cache");
}

}  // extern "C"
