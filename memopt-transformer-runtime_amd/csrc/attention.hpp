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
};

// Split count used by the INT4 decode kernel for this launch shape.
int decode_splits(int32_t batch, int32_t heads, int32_t max_pages_visited);
// Launches the split-K INT4 decode kernel (+ combine when splits > 1).
int launch_decode_int4(const DecodeParams &p, int32_t batch, int32_t D, int32_t scale_dtype,
                       hipStream_t stream);

// Launches the split-K fp16-pool decode kernel (+ combine when splits > 1).
int launch_decode_fp16(const DecodeParams &p, int32_t batch, int32_t D, hipStream_t stream);
// Log-sum-exp merge of the split partials in p.ws_o / p.ws_ml into p.out.
int launch_decode_combine(const DecodeParams &p, int32_t batch, int32_t D, hipStream_t stream);

// Multi-query (q_len >= 2) MFMA kernel over INT4 page pools or contiguous
// fp16 pools with 16-multiple pages and D in {64, 128}.
bool prefill_supported(const memopt_attn_desc &d);
// Workspace of the staged prefill path (0: the path stages in-kernel).
int64_t prefill_workspace_bytes(const memopt_attn_desc &d);
int launch_prefill(const memopt_attn_desc &d, int32_t W, float qk_scale_log2, hipStream_t stream);

}  // namespace memopt
