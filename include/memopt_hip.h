/*
 * memopt_hip.h — C ABI of the MI355X (gfx950) INT4 KV-cache data plane.
 *
 * Every entry point takes plain device pointers, 64-bit sizes and a
 * hipStream_t (passed as void*), returns an int status (MEMOPT_OK == 0) and
 * records a human-readable message retrievable with memopt_last_error()
 * (thread-local). No libtorch types cross this boundary: callers allocate
 * device memory themselves (the Python `memopt_C` shim uses torch tensors)
 * and keep it alive while the library uses it.
 *
 * Each declaration names the reference interface it replaces:
 * TheRadDani/memopt-transformer-runtime, pybind11 module `memopt_C`
 * (src/csrc/extension.cpp) and the C++ functions it binds.
 *
 * Kernel entry points are asynchronous on `stream`; launch errors are
 * reported through the status code.
 */
#ifndef MEMOPT_HIP_H
#define MEMOPT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Status codes                                                             */
/* ------------------------------------------------------------------------ */
#define MEMOPT_OK               0
#define MEMOPT_ERR_INVALID      1  /* contract violation (shape/dtype/range) */
#define MEMOPT_ERR_STATE        2  /* pool not initialized                    */
#define MEMOPT_ERR_HIP          3  /* HIP runtime / launch error              */
#define MEMOPT_ERR_UNSUPPORTED  4  /* configuration not compiled in           */

/* KV storage formats (memopt_init_pool `kv_format`, memopt_attn_desc.kv_format). */
#define MEMOPT_KV_FP16       0  /* fp16 [num_blocks, block_size, H, D] (reference layout)  */
#define MEMOPT_KV_INT4       1  /* INT4 page pool, one u8 buffer [num_blocks, H, B] with    *
                                 * B = 16*D + 64*(D/64) bytes per (page, head):             *
                                 *   K codes (8*D) | V codes (8*D) | K scales | V scales    *
                                 * (fp16 scales, 32*(D/64) bytes each); 16-token pages;     *
                                 * codes laid out for the wave64 decode kernel: lane 8p+c   *
                                 * owns tokens (p, p+8) x dims [c*D/8, (c+1)*D/8); see      *
                                 * memopt-transformer-runtime_amd/csrc/page_format.hpp.     */
#define MEMOPT_KV_INT4_ROWS  2  /* attention input only: INT4 codes in the reference's      *
                                 * quantize_kv_cache_int4 byte order with arbitrary         *
                                 * page/head/token strides + separate f32/f16 scales        */

/* Scale element types for INT4 caches passed to attention. */
#define MEMOPT_SCALE_F32 0
#define MEMOPT_SCALE_F16 1

/* Message of the last failed call on this thread ("" if none). */
const char *memopt_last_error(void);

/* Replaces get_hello() — src/csrc/extension.cpp:6-8. */
const char *memopt_get_hello(void);

/* ------------------------------------------------------------------------ */
/* Paged pool (host free list + registered device storage)                 */
/* ------------------------------------------------------------------------ */

/* Replaces init_pool(num_blocks, block_size, num_heads, head_dim) —
 * src/csrc/kv_cache.cu:112-153, bound at src/csrc/extension.cpp:20-26.
 * The caller allocates the storage, filled with the empty-row pattern, and
 * passes it in:
 *   MEMOPT_KV_FP16: key/value = fp16 [nb, bs, H, D] zeros; scale pointers unused.
 *   MEMOPT_KV_INT4: key_pool = the page buffer (codes 0x88, scales 1.0);
 *                   value_pool / key_scales / value_scales unused (NULL);
 *                   block_size must be 16 and head_dim a multiple of 64.
 * The free list is reseeded FIFO 0..nb-1. Invalid parameters tear the pool
 * down and return MEMOPT_ERR_INVALID. */
int memopt_init_pool(int64_t num_blocks, int32_t block_size, int32_t num_heads,
                     int32_t head_dim, int32_t kv_format, void *key_pool,
                     void *value_pool, void *key_scales, void *value_scales);

/* Reports the live pool's parameters; returns 1 if a pool is initialized,
 * 0 otherwise (outputs untouched). Used for init_pool's idempotency
 * (src/csrc/kv_cache.cu:115-122). */
int memopt_pool_info(int64_t *num_blocks, int32_t *block_size, int32_t *num_heads,
                     int32_t *head_dim, int32_t *kv_format);

/* Drops the pool (storage pointers are forgotten; the caller frees them). */
int memopt_reset_pool(void);

/* Swaps the live pool's storage and format (fp16 <-> INT4 pages) for the same
 * geometry, keeping the free list, so block tables stay valid across the
 * switch. No counterpart in the reference: it serves the policy forward
 * wrapper that applies MemoryScheduler.use_int4 (src/memopt/scheduler.py:15-18
 * documents the switch; no reference code performs it). The caller fills the
 * new storage (memopt_write_cache into INT4 pages, memopt_int4_pages_to_fp16
 * into fp16 pools) on the stream before using the pool. */
int memopt_pool_set_storage(int32_t kv_format, void *key_pool, void *value_pool);

/* Replaces allocate_block() — src/csrc/kv_cache.cu:163-172. *block_idx = -1
 * when exhausted (not an error). */
int memopt_allocate_block(int64_t *block_idx);

/* Replaces free_block(block_idx) — src/csrc/kv_cache.cu:179-185. */
int memopt_free_block(int64_t block_idx);

/* Replaces free_blocks_count() — src/csrc/kv_cache.cu:198-201. */
int memopt_free_blocks_count(int64_t *count);

/* Replaces write_cache(keys, values, block_tables, slot_mapping) —
 * src/csrc/kv_cache.cu:282-348. keys/values: fp16 [num_tokens, H, D]
 * contiguous; slot_mapping: int32 [num_tokens], slot = block*bs + pos.
 * FP16 pools get a scatter copy; INT4 pools get a fused group-64 quantize
 * into the page (codes bit-exact with memopt_quantize_kv_cache_int4, scales
 * stored as RNE fp16 of the fp32 scale, 9360 = RNE(65504/7) stored as 9352
 * so that 7 * scale stays finite). Slots outside the pool are skipped
 * on device; the caller validates them beforehand. */
int memopt_write_cache(const void *keys, const void *values, int64_t num_tokens,
                       int32_t num_heads, int32_t head_dim,
                       const int32_t *slot_mapping, void *stream);

/* Replaces evict_cache(block_tables, attention_scores, retain_ratio,
 * num_sink_tokens) — src/csrc/kv_cache.cu:379-559. scores: f32
 * [num_blocks, block_size, H]. Per (block, head): keep = max(1,
 * floor(r*bs)); rows scoring below the keep-th largest of the scores above
 * -1e38 (below -1e38 itself when fewer than keep exceed it) are zeroed: the
 * reference's selection with its -1e38 sentinel. Sinks ignored, as in the
 * reference. block_size up to 8192. */
int memopt_evict_cache(const float *attention_scores, int64_t num_blocks,
                       float retain_ratio, int32_t num_sink_tokens, void *stream);

/* Replaces evict_tokens(attention_scores, block_tables, is_block_free,
 * retain_ratio, num_sink_tokens) — src/csrc/kv_cache.cu:640-1156.
 * scores f32 [num_seqs, H, seq_len]; block_tables i32 [num_seqs, max_blocks]
 * (mutated); is_block_free i32 [total_pool_blocks] (mutated, caller zeroes).
 * Per (seq, head): sinks t < num_sink_tokens always kept; keep =
 * clamp(ceilf(r*L), 1, L); tokens scoring below the exact keep-th largest
 * (sink-boosted) score are evicted; their (token, head) rows are zeroed
 * (INT4: every group scale of the row set to 0, codes kept, so the row
 * dequantizes to zeros). A logical block with all block_size positions
 * evicted votes is_block_free[phys] += 1; the vote reaching H unlinks
 * block_tables[seq, lb] = -1. No seq_len cap (rows longer than 32768
 * tokens run as several workgroups per row). A physical page named by more
 * than one live entry of block_tables (shared between sequences) receives
 * the union of their evictions and no votes: it is never unlinked or
 * counted free by this call.
 * `workspace` is device scratch of at least memopt_evict_workspace_size
 * bytes, 16-byte aligned, of any content; nothing in it is kept between
 * calls. The call allocates no device memory. Calls sharing a workspace
 * must not overlap (nor may calls on one pool: they mutate it). */
int memopt_evict_tokens(const float *attention_scores, int32_t num_seqs,
                        int32_t num_heads, int32_t seq_len, int32_t *block_tables,
                        int32_t max_blocks_per_seq, int32_t *is_block_free,
                        int64_t total_pool_blocks, float retain_ratio,
                        int32_t num_sink_tokens, void *workspace,
                        int64_t workspace_bytes, void *stream);

/* Workspace bytes memopt_evict_tokens needs for these sizes: page marks for
 * total_pool_blocks pages plus, for seq_len > 32768, the long-row
 * selection state. No counterpart in the reference, whose kernels keep this
 * state in shared memory (it caps seq_len at 4096). */
int memopt_evict_workspace_size(int32_t num_seqs, int32_t num_heads, int32_t seq_len,
                                int32_t max_blocks_per_seq, int64_t total_pool_blocks,
                                int64_t *bytes);

/* ------------------------------------------------------------------------ */
/* Quantization (surface, whole-tensor)                                     */
/* ------------------------------------------------------------------------ */

/* Replaces quantize_kv_cache_int4(cache, group_size) —
 * src/csrc/quantization.cu:104-203, :294-353. cache: fp16, numel elements,
 * contiguous; packed_out: u8 [numel/2]; scales_out: f32 [numel/64].
 * scale = absmax>0 ? absmax/7 : 1 (IEEE fp32); code = clamp(roundf(v/scale)
 * + 8, 0, 15); byte = code[2i] | code[2i+1] << 4. */
int memopt_quantize_kv_cache_int4(const void *cache, int64_t numel, int64_t last_dim,
                                  int32_t group_size, uint8_t *packed_out,
                                  float *scales_out, void *stream);

/* Replaces dequantize_kv_cache_int4(q_cache, scales, group_size) —
 * src/csrc/quantization.cu:232-270, :371-428. out: fp16 [2*packed_numel],
 * value = fp16(RNE(float(code-8) * scale)). */
int memopt_dequantize_kv_cache_int4(const uint8_t *packed, int64_t packed_numel,
                                    const float *scales, int64_t num_scales,
                                    int32_t group_size, void *out, void *stream);

/* Dequantizes an INT4 page pool [num_blocks, H, B] into fp16 pools
 * key_out/value_out [num_blocks, 16, H, D]: value = fp16(RN(float(code-8) *
 * page scale)), the dequantize_kv_cache_int4 arithmetic of
 * src/csrc/quantization.cu:232-270 applied to this build's page layout
 * (fp16 page scales). head_dim 64 or 128. */
int memopt_int4_pages_to_fp16(const uint8_t *pages, int64_t num_blocks, int32_t num_heads,
                              int32_t head_dim, void *key_out, void *value_out, void *stream);

/* ------------------------------------------------------------------------ */
/* Paged attention                                                          */
/* ------------------------------------------------------------------------ */

/* Replaces dynamic_sparse_attention(query, key_cache, value_cache,
 * block_tables, context_lens, max_seq_len, window_size) —
 * src/csrc/attention.cu:98-339, :371-521 — with reference semantics:
 * non-causal, keys j in [max(0, ctx-W), ctx) for every query, pages with
 * block_tables < 0 skipped, W <= 0 or W > max_seq_len -> max_seq_len,
 * scale 1/sqrtf(D), empty key set -> 0. fp16 pool [nb, bs, H, D]. */
int memopt_dynamic_sparse_attention(const void *query, int32_t batch, int32_t q_len,
                                    int32_t num_heads, int32_t head_dim,
                                    const void *key_cache, const void *value_cache,
                                    int64_t num_kv_blocks, int32_t block_size,
                                    const int32_t *block_tables,
                                    int32_t max_blocks_per_seq,
                                    const int32_t *context_lens, int32_t max_seq_len,
                                    int32_t window_size, void *out, void *stream);

/* Extended paged attention: the reference semantics above plus
 *   - INT4 caches — the INT4 page pool, or reference-order codes with
 *     f32/f16 group-64 scales and arbitrary page/head/token strides —
 *     dequantized just in time; replaces the reference's
 *     dequantize_kv_cache_int4 -> dynamic_sparse_attention composition;
 *   - attention sinks (keys j < num_sink_tokens always visible, the token
 *     rule of src/memopt/triton_attention.py:523-532);
 *   - causal mode (query i at absolute position ctx-q_len+i sees
 *     j <= pos && (j < sinks || j >= pos-W+1), scripts/bench_accuracy.py:253-280).
 * With num_sink_tokens == 0, causal == 0 and an fp16 cache it computes the
 * same function as memopt_dynamic_sparse_attention.
 * `workspace` (device, >= memopt_attention_workspace_size bytes) holds the
 * decode's split-K partials and arrival counters, or the prefill's staged
 * K/V and staging flags; it may be NULL when that size is 0. A decode
 * (q_len == 1) workspace must be zero before its first use; later calls may
 * reuse it without clearing (each call's counters carry the call's id, so
 * what an earlier call left is never taken for its own). A multi-query
 * workspace may hold anything (the call clears its flags itself). */
typedef struct memopt_attn_desc {
  const void *query;          /* fp16 [batch, q_len, H, D] contiguous        */
  void *out;                  /* fp16 [batch, q_len, H, D] contiguous        */
  int32_t batch, q_len, num_heads, head_dim;
  int32_t kv_format;          /* MEMOPT_KV_FP16 / _INT4 (page pool) / _INT4_ROWS */
  const void *key_cache;      /* fp16 elements, INT4 page buffer, or u8 codes */
  const void *value_cache;    /* unused for MEMOPT_KV_INT4                   */
  const void *key_scales;     /* MEMOPT_KV_INT4_ROWS only                    */
  const void *value_scales;
  int32_t scale_dtype;        /* MEMOPT_SCALE_F32 / MEMOPT_SCALE_F16 (ROWS)  */
  int32_t block_size;         /* tokens per page                             */
  int64_t num_kv_blocks;
  /* Strides (FP16 / INT4_ROWS only; derived for INT4 pages): fp16 cache in
   * elements, INT4 codes in bytes, scales in elements. */
  int64_t kv_page_stride, kv_head_stride, kv_token_stride;
  int64_t sc_page_stride, sc_head_stride, sc_token_stride;
  const int32_t *block_tables; /* [batch, max_blocks_per_seq]                */
  int32_t max_blocks_per_seq;
  const int32_t *context_lens; /* [batch]                                    */
  int32_t max_seq_len, window_size, num_sink_tokens, causal;
  void *workspace;
  int64_t workspace_bytes;
} memopt_attn_desc;

int memopt_attention_workspace_size(const memopt_attn_desc *desc, int64_t *bytes);
/* `workspace` must hold at least memopt_attention_workspace_size bytes;
 * a smaller one is an error (MEMOPT_ERR_INVALID). Only
 * memopt_dynamic_sparse_attention, whose reference signature has no
 * workspace, runs a decode that would split unsplit instead. */
int memopt_paged_attention(const memopt_attn_desc *desc, void *stream);

/* Bytes of the per-GPU static scratch of memopt_paged_attention_noalloc. */
#define MEMOPT_NOALLOC_SCRATCH_BYTES (4LL << 20)

/* No counterpart in the reference. For callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc. Computes what memopt_paged_attention computes for the
 * same descriptor (desc->workspace is ignored) and allocates nothing: the
 * decode kernels' split-K partials, and the staged K/V of a multi-query call
 * when they fit, live in a static device array of
 * MEMOPT_NOALLOC_SCRATCH_BYTES (4 MiB) per GPU, held until the process ends;
 * its last 64 KiB hold the decode's arrival counters (zero at load, then
 * only ever counters) and the rest the partials or staged K/V.
 * Results are bit-identical to memopt_paged_attention's except for
 * multi-query calls whose staging does not fit: those run the in-kernel
 * staging kernel, which needs no scratch and agrees with the staged one to
 * within fp16 attention tolerance, not bit for bit. A decode whose partials exceed the rest
 * (B * H * splits * (head_dim + 2) * 4 + 8 * B * H bytes; splits grow only
 * while B * H is below two workgroups per CU) returns MEMOPT_ERR_INVALID. Every call on
 * a GPU shares that GPU's array, so calls that overlap on one GPU (other
 * streams or host threads) race: the caller serializes them. The first call
 * on each device resolves the array's device address there. */
int memopt_paged_attention_noalloc(const memopt_attn_desc *desc, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MEMOPT_HIP_H */
