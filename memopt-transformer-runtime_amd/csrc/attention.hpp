// attention.hpp — shared declarations of the paged-attention kernels.
#pragma once
#include "common.hpp"

namespace memopt {

// Key-visibility rule of one query, resolved to two token ranges:
// sinks [0, sink_end) and the window [win_lo, hi) (win_lo >= sink_end when
// the ranges are disjoint; they may overlap, the union is what counts).
struct KeyRange {
  int32_t sink_end, win_lo, hi;
};

// Non-causal (reference dynamic_sparse_attention, src/csrc/attention.cu:158-186,
// plus sinks): every query sees [max(0, ctx-W), ctx) U [0, min(sinks, ctx)).
// Causal (scripts/bench_accuracy.py:271-275): query at absolute position
// pos sees j <= pos && (j < sinks || j >= pos - W + 1).
__host__ __device__ inline KeyRange key_range(int32_t ctx, int32_t pos, int32_t W, int32_t sinks,
                                               bool causal) {
  KeyRange r;
  r.hi = causal ? (pos + 1 < ctx ? pos + 1 : ctx) : ctx;
  if (r.hi < 0) r.hi = 0;
  const int32_t top = causal ? pos + 1 : ctx;  // window anchored at pos (causal) or ctx
  r.win_lo = top - W;
  if (r.win_lo < 0) r.win_lo = 0;
  r.sink_end = sinks < r.hi ? sinks : r.hi;
  if (r.sink_end < 0) r.sink_end = 0;
  return r;
}

// Window of the reference signature: W <= 0 or W > max_seq_len means
// max_seq_len (src/csrc/attention.cu:453-455).
inline int32_t effective_window(int32_t window, int32_t max_seq_len) {
  return (window <= 0 || window > max_seq_len) ? max_seq_len : window;
}

// Visible pages (or 16-token chunks) [begin, end) of split `split` of
// `splits` over n of them, in 32-bit arithmetic: a 64-bit division expands
// to a long scalar sequence that sits on every decode launch's critical path.
struct SplitRange {
  int32_t begin, end;
};
__device__ __forceinline__ SplitRange split_range(int32_t n, int32_t split, int32_t splits) {
  if (splits <= 1) return {0, n};
  const int32_t q = n / splits, r = n - q * splits;
  const int32_t begin = split * q + (split < r ? split : r);
  return {begin, begin + q + (split < r ? 1 : 0)};
}

struct DecodeParams {
  const half_t *q;
  half_t *out;
  const uint8_t *kc, *vc;
  const void *ks, *vs;
  int64_t kv_ps, kv_hs, kv_ts;  // code strides, bytes
  int64_t sc_ps, sc_hs, sc_ts;  // scale strides, elements
  const int32_t *bt;
  const int32_t *ctx;
  int64_t nb;                   // pages in the pool (entries >= nb are skipped)
  int32_t pages;                // 1: this build's INT4 page format (page_format.hpp)
  int32_t M, H, W, sinks, splits;
  int32_t bs;           // tokens per page (fp16 pools; a multiple of 16)
  float qk_scale_log2;  // (1/sqrt(D)) * log2(e)
  float *ws_o;          // [B, H, splits, D] (splits > 1)
  float *ws_ml;         // [B, H, splits, 2]
  unsigned long long *ws_cnt;  // [B, H] arrival counters (splits > 1)
  unsigned long long tag;      // this launch's id, 1 .. 2^56 - 1
};

// Bytes of a decode call's split-K workspace: partials (o[D], m, l) per
// (b, h, split) and one arrival counter per (b, h).
inline int64_t decode_workspace_bytes(int64_t batch, int64_t heads, int64_t splits, int64_t D) {
  return splits > 1 ? batch * heads * (splits * (D + 2) * 4 + 8) : 0;
}

// Id of the next decode launch (for the arrival counters).
unsigned long long next_decode_tag();

// Epilogue of a decode workgroup of NW waves over (b, h, split): merges the
// waves' (m, l, acc[D]) held in LDS. Unsplit: writes the output row. Split:
// writes this split's partial to the workspace with agent-scope stores
// (they bypass the per-XCD L2s, as the splits of one (b, h) run on
// different XCDs), waits for them, and counts its arrival on (b, h) with a
// compare-and-swap on (tag << 8 | count): a counter left by an earlier
// launch (other tag) or zero restarts at 1, so a workspace zeroed once needs
// no clearing between launches (a fresh one must be zero: a stale word equal
// to this launch's (tag << 8 | count) would stop the merge). The split that
// brings the count to `splits` merges every
// partial (log-sum-exp, agent-scope loads) into the output row. No
// workgroup waits for another.
template <int D, int NW>
__device__ __forceinline__ void decode_epilogue(const DecodeParams &p, int64_t bh, int32_t split,
                                                const float (*s_acc)[D], const float (*s_ml)[2]) {
  for (int d = threadIdx.x; d < D; d += NW * 64) {
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) mx = fmaxf(mx, s_ml[w][0]);
    float lt = 0.0f, o = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = (s_ml[w][0] == -INFINITY) ? 0.0f : fast_exp2(s_ml[w][0] - mx);
      lt += s_ml[w][1] * f;
      o += s_acc[w][d] * f;
    }
    if (p.splits == 1) {
      p.out[bh * D + d] = (half_t)(lt > 0.0f ? o / lt : 0.0f);
    } else {
      const int64_t slot = bh * p.splits + split;
      __hip_atomic_store(&p.ws_o[slot * D + d], o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (d == 0) {
        __hip_atomic_store(&p.ws_ml[slot * 2], mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&p.ws_ml[slot * 2 + 1], lt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (p.splits == 1) return;
  __shared__ int s_last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores are complete
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long *cnt = p.ws_cnt + bh;
    unsigned long long e = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), nv;
    do {
      nv = (e >> 8) == p.tag ? e + 1 : (p.tag << 8) | 1;
    } while (!__hip_atomic_compare_exchange_strong(cnt, &e, nv, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT));
    s_last = (int)(nv & 0xFF) == p.splits;
  }
  __syncthreads();
  if (!s_last) return;
  const float *ml = p.ws_ml + bh * p.splits * 2;
  for (int d = threadIdx.x; d < D; d += NW * 64) {
    float mx = -INFINITY;
    for (int s = 0; s < p.splits; ++s)
      mx = fmaxf(mx, __hip_atomic_load(&ml[2 * s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    float lt = 0.0f, o = 0.0f;
    for (int s = 0; s < p.splits; ++s) {
      const float ms = __hip_atomic_load(&ml[2 * s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const float ls = __hip_atomic_load(&ml[2 * s + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const float os = __hip_atomic_load(&p.ws_o[(bh * p.splits + s) * D + d], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
      const float f = ms == -INFINITY ? 0.0f : fast_exp2(ms - mx);
      lt += ls * f;
      o += os * f;
    }
    p.out[bh * D + d] = (half_t)(lt > 0.0f ? o / lt : 0.0f);
  }
}

// Split count used by the INT4 decode kernel for this launch shape.
int decode_splits(int32_t batch, int32_t heads, int32_t max_pages_visited);
// Launches the split-K INT4 decode kernel (splits merged in-kernel).
int launch_decode_int4(const DecodeParams &p, int32_t batch, int32_t D, int32_t scale_dtype,
                       hipStream_t stream);

// Launches the split-K fp16-pool decode kernel (splits merged in-kernel).
int launch_decode_fp16(const DecodeParams &p, int32_t batch, int32_t D, hipStream_t stream);

// Multi-query (q_len >= 2) MFMA kernel over INT4 page pools or contiguous
// fp16 pools with 16-multiple pages and D in {64, 128}.
bool prefill_supported(const memopt_attn_desc &d);
// Workspace of the staged prefill path (0: the path stages in-kernel).
int64_t prefill_workspace_bytes(const memopt_attn_desc &d);
int launch_prefill(const memopt_attn_desc &d, int32_t W, float qk_scale_log2, hipStream_t stream);

}  // namespace memopt
