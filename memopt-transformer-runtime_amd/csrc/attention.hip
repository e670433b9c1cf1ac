// attention.hip — paged attention entry points and the generic kernel.
//
// Reference: TheRadDani/memopt-transformer-runtime src/csrc/attention.cu:371-521
// (dynamic_sparse_attention host checks, window clamp :453-455, scale
// 1/sqrtf(D) :460, kernel semantics :158-186 and :333-338).
//
// Dispatch:
//   * INT4 cache, q_len == 1, 16-token pages, D in {64, 128}, aligned
//     strides -> decode_int4 (split-K, HBM-streaming; decode_int4.hip);
//   * fp16 cache, q_len == 1, pages of 16 * 2^k tokens, D in {64, 128},
//     16-byte aligned rows -> decode_fp16 (split-K, HBM-streaming;
//     decode_fp16.hip);
//   * fp16 or INT4 cache, q_len >= 2, D in {64, 128}, 16-token pages ->
//     prefill (fp16 MFMA; prefill.hip);
//   * anything else -> generic_attention_kernel below: one wave per
//     (b, query, head), lanes over head dims, keys visited in order with an
//     online softmax. INT4 elements are dequantized to fp16 exactly as the
//     reference's dequantize kernel would (fp16(RNE((code-8)*scale))) before
//     use, so it computes the reference composition.
#include <mutex>
#include <string>

#include "attention.hpp"
#include "page_format.hpp"

namespace memopt {

struct GenericParams {
  const half_t *q;
  half_t *out;
  int32_t B, Lq, H, D;
  int32_t fmt, scale_f16;  // fmt: MEMOPT_KV_FP16 / _INT4 (page pool) / _INT4_ROWS
  const void *kc, *vc, *ks, *vs;
  int64_t kv_ps, kv_hs, kv_ts, sc_ps, sc_hs, sc_ts;
  int32_t bs;
  int64_t nb;
  const int32_t *bt;
  int32_t M;
  const int32_t *ctx;
  int32_t W, sinks, causal;
  float scale;
};

__device__ __forceinline__ float kv_elem(const GenericParams &p, bool is_v, int64_t page, int32_t pos,
                                         int32_t head, int32_t d) {
  const void *cache = is_v ? p.vc : p.kc;
  if (p.fmt == MEMOPT_KV_FP16) {
    const half_t *c = (const half_t *)cache;
    return (float)c[page * p.kv_ps + (int64_t)pos * p.kv_ts + (int64_t)head * p.kv_hs + d];
  }
  uint8_t byte;
  float s;
  if (p.fmt == MEMOPT_KV_INT4) {
    const Int4Page f(p.D);
    const uint8_t *blk = (const uint8_t *)p.kc + (page * p.H + head) * f.block;
    byte = is_v ? blk[f.vcodes + f.v_byte(pos, d)] : blk[f.kcodes + f.k_byte(pos, d)];
    s = (float)reinterpret_cast<const half_t *>(blk + (is_v ? f.vscales : f.kscales))[f.scale_idx(pos, d >> 6)];
  } else {
    const uint8_t *c = (const uint8_t *)cache;
    byte = c[page * p.kv_ps + (int64_t)pos * p.kv_ts + (int64_t)head * p.kv_hs + (d >> 1)];
    const void *scales = is_v ? p.vs : p.ks;
    const int64_t si = page * p.sc_ps + (int64_t)pos * p.sc_ts + (int64_t)head * p.sc_hs + (d >> 6);
    s = p.scale_f16 ? (float)((const half_t *)scales)[si] : ((const float *)scales)[si];
  }
  const int code = (d & 1) ? (byte >> 4) : (byte & 0xF);
  return (float)(half_t)((float)(code - 8) * s);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += shfl_xor(v, off);
  return v;
}

constexpr int kMaxDimPerLane = 4;  // D <= 256

__global__ __launch_bounds__(64) void generic_attention_kernel(const GenericParams p) {
  const int32_t h = blockIdx.x, qi = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
  const int32_t ctx = p.ctx[b];
  const int32_t pos = ctx - p.Lq + qi;
  const KeyRange kr = key_range(ctx, pos, p.W, p.sinks, p.causal != 0);
  float qv[kMaxDimPerLane], acc[kMaxDimPerLane];
  const half_t *qrow = p.q + (((int64_t)b * p.Lq + qi) * p.H + h) * p.D;
#pragma unroll
  for (int i = 0; i < kMaxDimPerLane; ++i) {
    const int d = lane + 64 * i;
    qv[i] = d < p.D ? (float)qrow[d] : 0.0f;
    acc[i] = 0.0f;
  }
  float m = -INFINITY, l = 0.0f;
  const int32_t lim = min(kr.hi, p.M * p.bs);
  const int32_t w0 = max(kr.win_lo, kr.sink_end);
  for (int pass = 0; pass < 2; ++pass) {
    const int32_t j0 = pass == 0 ? 0 : w0;
    const int32_t j1 = pass == 0 ? min(kr.sink_end, lim) : lim;
    for (int32_t j = j0; j < j1; ++j) {
      const int32_t page = p.bt[(int64_t)b * p.M + j / p.bs];
      if (page < 0 || page >= p.nb) continue;
      const int32_t ps = j % p.bs;
      float part = 0.0f;
#pragma unroll
      for (int i = 0; i < kMaxDimPerLane; ++i) {
        const int d = lane + 64 * i;
        if (d < p.D) part += qv[i] * kv_elem(p, false, page, ps, h, d);
      }
      const float s = wave_sum(part) * p.scale;
      const float mn = fmaxf(m, s);
      const float alpha = (mn == m) ? 1.0f : __expf(m - mn);
      const float pw = __expf(s - mn);
      l = l * alpha + pw;
#pragma unroll
      for (int i = 0; i < kMaxDimPerLane; ++i) {
        const int d = lane + 64 * i;
        if (d < p.D) acc[i] = acc[i] * alpha + pw * kv_elem(p, true, page, ps, h, d);
      }
      m = mn;
    }
  }
  half_t *orow = p.out + (((int64_t)b * p.Lq + qi) * p.H + h) * p.D;
#pragma unroll
  for (int i = 0; i < kMaxDimPerLane; ++i) {
    const int d = lane + 64 * i;
    if (d < p.D) orow[d] = (half_t)(l > 0.0f ? acc[i] / l : 0.0f);
  }
}

static bool aligned_to(const void *p, int64_t a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }


// Upper bound of pages one sequence visits (sizes the split count).
static int32_t max_pages_visited(const memopt_attn_desc &d) {
  const int32_t W = effective_window(d.window_size, d.max_seq_len);
  int64_t win = (int64_t)W / d.block_size + 2;
  int64_t sink = (int64_t)(d.num_sink_tokens + d.block_size - 1) / d.block_size;
  int64_t v = win + sink;
  if (v > d.max_blocks_per_seq) v = d.max_blocks_per_seq;
  return (int32_t)v;
}

static bool use_decode_int4(const memopt_attn_desc &d) {
  if (d.q_len != 1 || d.block_size != 16 || d.num_kv_blocks <= 0) return false;
  if (d.head_dim != 64 && d.head_dim != 128) return false;
  if (!aligned_to(d.query, 16)) return false;
  if (d.kv_format == MEMOPT_KV_INT4) return aligned_to(d.key_cache, 16);
  if (d.kv_format != MEMOPT_KV_INT4_ROWS) return false;
  // Per-lane offsets inside a (page, head) block are 32-bit.
  if (15 * d.kv_token_stride + d.head_dim / 2 >= (1LL << 31)) return false;
  if (15 * d.sc_token_stride + d.head_dim / 64 >= (1LL << 31)) return false;
  const int64_t bpl = d.head_dim / 8;
  if (!aligned_to(d.key_cache, bpl) || !aligned_to(d.value_cache, bpl)) return false;
  if (d.kv_page_stride % bpl || d.kv_head_stride % bpl || d.kv_token_stride % bpl) return false;
  return true;
}

// fp16 pools: 16-token chunks of pages whose token count is 16 times a power
// of two, 16-byte aligned rows, 32-bit per-lane offsets inside a chunk.
static bool use_decode_fp16(const memopt_attn_desc &d) {
  if (d.kv_format != MEMOPT_KV_FP16 || d.q_len != 1 || d.num_kv_blocks <= 0) return false;
  if (d.head_dim != 64 && d.head_dim != 128) return false;
  if (d.block_size % 16 != 0) return false;
  const int32_t cpp = d.block_size / 16;
  if ((cpp & (cpp - 1)) != 0) return false;
  if (!aligned_to(d.query, 16) || !aligned_to(d.key_cache, 16) || !aligned_to(d.value_cache, 16)) return false;
  if ((d.kv_page_stride * 2) % 16 || (d.kv_head_stride * 2) % 16 || (d.kv_token_stride * 2) % 16) return false;
  if (15 * d.kv_token_stride * 2 + d.head_dim * 2 >= (1LL << 31)) return false;
  return true;
}

static int validate(const memopt_attn_desc &d) {
  MEMOPT_REQUIRE(d.batch >= 0 && d.q_len >= 0 && d.num_heads >= 0 && d.head_dim >= 0, MEMOPT_ERR_INVALID,
                 "paged_attention: negative dimension");
  MEMOPT_REQUIRE(d.head_dim % 2 == 0 && d.head_dim <= 64 * kMaxDimPerLane, MEMOPT_ERR_INVALID,
                 "paged_attention: head_dim must be even and <= 256");
  MEMOPT_REQUIRE(d.block_size > 0, MEMOPT_ERR_INVALID, "paged_attention: block_size must be > 0");
  MEMOPT_REQUIRE(d.max_blocks_per_seq >= 0, MEMOPT_ERR_INVALID, "paged_attention: bad max_blocks_per_seq");
  MEMOPT_REQUIRE(d.kv_format == MEMOPT_KV_FP16 || d.kv_format == MEMOPT_KV_INT4 ||
                     d.kv_format == MEMOPT_KV_INT4_ROWS,
                 MEMOPT_ERR_INVALID, "paged_attention: unknown kv_format");
  if (d.kv_format != MEMOPT_KV_FP16) {
    MEMOPT_REQUIRE(d.head_dim % 64 == 0, MEMOPT_ERR_INVALID,
                   "paged_attention: INT4 caches need head_dim % 64 == 0");
  }
  if (d.kv_format == MEMOPT_KV_INT4) {
    MEMOPT_REQUIRE(d.block_size == 16, MEMOPT_ERR_INVALID, "paged_attention: INT4 page pools use 16-token pages");
  }
  if (d.kv_format == MEMOPT_KV_INT4_ROWS) {
    MEMOPT_REQUIRE(d.key_scales && d.value_scales, MEMOPT_ERR_INVALID, "paged_attention: INT4 needs scales");
    MEMOPT_REQUIRE(d.scale_dtype == MEMOPT_SCALE_F32 || d.scale_dtype == MEMOPT_SCALE_F16, MEMOPT_ERR_INVALID,
                   "paged_attention: unknown scale dtype");
  }
  return MEMOPT_OK;
}

static int decode_workspace(const memopt_attn_desc &d, int32_t *splits, int64_t *bytes) {
  // Splits are sized in the kernels' 16-token units.
  *splits = decode_splits(d.batch, d.num_heads, max_pages_visited(d) * (d.block_size / 16));
  *bytes = decode_workspace_bytes(d.batch, d.num_heads, *splits, d.head_dim);
  return MEMOPT_OK;
}

// Split count and partials buffer of a decode call: the caller's workspace
// when the shape splits. `unsplit_ok`: the entry point has no workspace
// argument (the reference signature, memopt_dynamic_sparse_attention), so a
// call that passes none runs unsplit; memopt_paged_attention callers must
// pass the workspace memopt_attention_workspace_size asks for.
static int decode_plan(const memopt_attn_desc &d, bool unsplit_ok, int32_t *splits) {
  int64_t need;
  decode_workspace(d, splits, &need);
  if (need > 0 && unsplit_ok && d.workspace == nullptr && d.workspace_bytes == 0) {
    *splits = 1;
    return MEMOPT_OK;
  }
  MEMOPT_REQUIRE(need == 0 || (d.workspace && d.workspace_bytes >= need), MEMOPT_ERR_INVALID,
                 "paged_attention: workspace too small (need " + std::to_string(need) + " bytes)");
  return MEMOPT_OK;
}

// Scratch of memopt_paged_attention_noalloc: split-K partials (and staged
// K/V of small multi-query calls) for callers that cannot allocate. Each GPU
// holds its own copy until the process ends; every noalloc call on a GPU
// shares it. Host code never passes `scratch` itself to a kernel (on the host
// it names a stand-in, not device memory): it resolves the device address
// once per device with hipGetSymbolAddress and passes that.
// Its last kNoallocCounterBytes hold the split-K arrival counters and
// nothing else: zero when the program loads, afterwards only ever holding a
// decode call's (tag, count), so a later call's tag never meets a stale
// match (staged K/V and partials stay below them).
static __device__ __align__(256) uint8_t scratch[MEMOPT_NOALLOC_SCRATCH_BYTES];
static constexpr int64_t kNoallocCounterBytes = 64 << 10;
static constexpr int64_t kNoallocDataBytes = MEMOPT_NOALLOC_SCRATCH_BYTES - kNoallocCounterBytes;

static constexpr int kMaxDevices = 64;

// Device address of `scratch` on the current device (nullptr + error set on
// failure). Resolved on the first call per device, with that device current.
static void *scratch_address() {
  static std::mutex mu;
  static void *addr[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    set_error("paged_attention_noalloc: no usable current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      (void)hipGetLastError();
      set_error(std::string("paged_attention_noalloc: hipGetSymbolAddress(scratch) failed: ") +
                hipGetErrorString(e));
      return nullptr;
    }
    addr[dev] = ptr;
  }
  return addr[dev];
}

}  // namespace memopt

using namespace memopt;

extern "C" {

int memopt_attention_workspace_size(const memopt_attn_desc *desc, int64_t *bytes) {
  MEMOPT_REQUIRE(desc && bytes, MEMOPT_ERR_INVALID, "attention_workspace_size: null argument");
  int rc = validate(*desc);
  if (rc != MEMOPT_OK) return rc;
  *bytes = 0;
  if (use_decode_int4(*desc) || use_decode_fp16(*desc)) {
    int32_t splits;
    return decode_workspace(*desc, &splits, bytes);
  }
  if (desc->batch > 0 && prefill_supported(*desc)) *bytes = prefill_workspace_bytes(*desc);
  return MEMOPT_OK;
}

}  // extern "C"

namespace memopt {

// `cnt`: the split-K arrival counters (one per (b, h)); nullptr places
// them after the partials in d.workspace.
static int paged_attention(const memopt_attn_desc &d, bool unsplit_ok, void *stream,
                           unsigned long long *cnt = nullptr) {
  int rc = validate(d);
  if (rc != MEMOPT_OK) return rc;
  if (d.batch == 0 || d.q_len == 0 || d.num_heads == 0 || d.head_dim == 0) return MEMOPT_OK;
  MEMOPT_REQUIRE(d.query && d.out && d.key_cache && (d.value_cache || d.kv_format == MEMOPT_KV_INT4) &&
                     d.block_tables && d.context_lens,
                 MEMOPT_ERR_INVALID, "paged_attention: null pointer");
  const int32_t W = effective_window(d.window_size, d.max_seq_len);
  const float scale = 1.0f / sqrtf((float)d.head_dim);
  hipStream_t s = (hipStream_t)stream;

  if (use_decode_int4(d)) {
    int32_t splits;
    rc = decode_plan(d, unsplit_ok, &splits);
    if (rc != MEMOPT_OK) return rc;
    DecodeParams p;
    p.q = (const half_t *)d.query;
    p.out = (half_t *)d.out;
    if (d.kv_format == MEMOPT_KV_INT4) {
      const Int4Page f(d.head_dim);
      const uint8_t *base = (const uint8_t *)d.key_cache;
      p.pages = 1;
      p.kc = base + f.kcodes;
      p.vc = base + f.vcodes;
      p.ks = base + f.kscales;
      p.vs = base + f.vscales;
      p.kv_ps = d.num_heads * f.block;   // bytes
      p.kv_hs = f.block;
      p.kv_ts = 0;
      p.sc_ps = d.num_heads * f.block / 2;  // fp16 elements
      p.sc_hs = f.block / 2;
      p.sc_ts = 0;
    } else {
      p.pages = 0;
      p.kc = (const uint8_t *)d.key_cache;
      p.vc = (const uint8_t *)d.value_cache;
      p.ks = d.key_scales;
      p.vs = d.value_scales;
      p.kv_ps = d.kv_page_stride;
      p.kv_hs = d.kv_head_stride;
      p.kv_ts = d.kv_token_stride;
      p.sc_ps = d.sc_page_stride;
      p.sc_hs = d.sc_head_stride;
      p.sc_ts = d.sc_token_stride;
    }
    p.bt = d.block_tables;
    p.ctx = d.context_lens;
    p.nb = d.num_kv_blocks;
    p.M = d.max_blocks_per_seq;
    p.H = d.num_heads;
    p.W = W;
    p.sinks = d.num_sink_tokens < 0 ? 0 : d.num_sink_tokens;
    p.splits = splits;
    p.bs = d.block_size;
    p.qk_scale_log2 = scale * 1.4426950408889634f;
    p.ws_o = (float *)d.workspace;
    p.ws_ml = splits > 1 ? p.ws_o + (int64_t)d.batch * d.num_heads * splits * d.head_dim : nullptr;
    p.ws_cnt = splits <= 1 ? nullptr
               : cnt       ? cnt
                           : (unsigned long long *)(p.ws_ml + (int64_t)d.batch * d.num_heads * splits * 2);
    p.tag = next_decode_tag();
    return launch_decode_int4(p, d.batch, d.head_dim, d.kv_format == MEMOPT_KV_INT4 ? MEMOPT_SCALE_F16 : d.scale_dtype, s);
  }

  if (use_decode_fp16(d)) {
    int32_t splits;
    rc = decode_plan(d, unsplit_ok, &splits);
    if (rc != MEMOPT_OK) return rc;
    DecodeParams p;
    p.q = (const half_t *)d.query;
    p.out = (half_t *)d.out;
    p.pages = 0;
    p.kc = (const uint8_t *)d.key_cache;
    p.vc = (const uint8_t *)d.value_cache;
    p.ks = p.vs = nullptr;
    p.kv_ps = d.kv_page_stride * 2;  // bytes
    p.kv_hs = d.kv_head_stride * 2;
    p.kv_ts = d.kv_token_stride * 2;
    p.sc_ps = p.sc_hs = p.sc_ts = 0;
    p.bt = d.block_tables;
    p.ctx = d.context_lens;
    p.nb = d.num_kv_blocks;
    p.M = d.max_blocks_per_seq;
    p.H = d.num_heads;
    p.W = W;
    p.sinks = d.num_sink_tokens < 0 ? 0 : d.num_sink_tokens;
    p.splits = splits;
    p.bs = d.block_size;
    p.qk_scale_log2 = scale * 1.4426950408889634f;
    p.ws_o = (float *)d.workspace;
    p.ws_ml = splits > 1 ? p.ws_o + (int64_t)d.batch * d.num_heads * splits * d.head_dim : nullptr;
    p.ws_cnt = splits <= 1 ? nullptr
               : cnt       ? cnt
                           : (unsigned long long *)(p.ws_ml + (int64_t)d.batch * d.num_heads * splits * 2);
    p.tag = next_decode_tag();
    return launch_decode_fp16(p, d.batch, d.head_dim, s);
  }

  if (prefill_supported(d)) return launch_prefill(d, W, scale * 1.4426950408889634f, s);

  GenericParams g;
  g.q = (const half_t *)d.query;
  g.out = (half_t *)d.out;
  g.B = d.batch;
  g.Lq = d.q_len;
  g.H = d.num_heads;
  g.D = d.head_dim;
  g.fmt = d.kv_format;
  g.scale_f16 = d.scale_dtype == MEMOPT_SCALE_F16;
  g.kc = d.key_cache;
  g.vc = d.value_cache;
  g.ks = d.key_scales;
  g.vs = d.value_scales;
  g.kv_ps = d.kv_page_stride;
  g.kv_hs = d.kv_head_stride;
  g.kv_ts = d.kv_token_stride;
  g.sc_ps = d.sc_page_stride;
  g.sc_hs = d.sc_head_stride;
  g.sc_ts = d.sc_token_stride;
  g.bs = d.block_size;
  g.nb = d.num_kv_blocks;
  g.bt = d.block_tables;
  g.M = d.max_blocks_per_seq;
  g.ctx = d.context_lens;
  g.W = W;
  g.sinks = d.num_sink_tokens < 0 ? 0 : d.num_sink_tokens;
  g.causal = d.causal;
  g.scale = scale;
  MEMOPT_REQUIRE(d.q_len <= 65535 && d.batch <= 65535, MEMOPT_ERR_UNSUPPORTED,
                 "paged_attention: q_len/batch > 65535 not supported by the generic kernel");
  hipLaunchKernelGGL(generic_attention_kernel, dim3(d.num_heads, d.q_len, d.batch), dim3(64), 0, s, g);
  return check_launch("paged_attention(generic)");
}

}  // namespace memopt

extern "C" {

int memopt_paged_attention(const memopt_attn_desc *desc, void *stream) {
  MEMOPT_REQUIRE(desc, MEMOPT_ERR_INVALID, "paged_attention: null descriptor");
  return paged_attention(*desc, false, stream);
}

int memopt_paged_attention_noalloc(const memopt_attn_desc *desc, void *stream) {
  MEMOPT_REQUIRE(desc, MEMOPT_ERR_INVALID, "paged_attention_noalloc: null descriptor");
  memopt_attn_desc d = *desc;
  d.workspace = nullptr;
  d.workspace_bytes = 0;
  int rc = validate(d);
  if (rc != MEMOPT_OK) return rc;
  if (d.batch == 0 || d.q_len == 0 || d.num_heads == 0 || d.head_dim == 0) return MEMOPT_OK;
  int64_t need = 0;
  const bool decode = use_decode_int4(d) || use_decode_fp16(d);
  if (decode) {
    int32_t splits;
    decode_workspace(d, &splits, &need);
    const int64_t units = (int64_t)d.batch * d.num_heads;
    MEMOPT_REQUIRE(need <= kNoallocDataBytes && (need == 0 || units * 8 <= kNoallocCounterBytes),
                   MEMOPT_ERR_INVALID,
                   "paged_attention_noalloc: the split-K partials need " + std::to_string(need) +
                       " bytes, more than the " + std::to_string((long long)kNoallocDataBytes) +
                       " bytes of the static scratch they may use");
  } else if (prefill_supported(d)) {
    need = prefill_workspace_bytes(d);
    if (need > kNoallocDataBytes) need = 0;  // in-kernel staging: no scratch
  }
  if (need > 0) {
    uint8_t *ws = (uint8_t *)scratch_address();
    if (ws == nullptr) return MEMOPT_ERR_HIP;
    d.workspace = ws;
    d.workspace_bytes = kNoallocDataBytes;
    if (decode) return paged_attention(d, false, stream, (unsigned long long *)(ws + kNoallocDataBytes));
  }
  return memopt_paged_attention(&d, stream);
}

int memopt_dynamic_sparse_attention(const void *query, int32_t batch, int32_t q_len, int32_t num_heads,
                                    int32_t head_dim, const void *key_cache, const void *value_cache,
                                    int64_t num_kv_blocks, int32_t block_size, const int32_t *block_tables,
                                    int32_t max_blocks_per_seq, const int32_t *context_lens,
                                    int32_t max_seq_len, int32_t window_size, void *out, void *stream) {
  memopt_attn_desc d = {};
  d.query = query;
  d.out = out;
  d.batch = batch;
  d.q_len = q_len;
  d.num_heads = num_heads;
  d.head_dim = head_dim;
  d.kv_format = MEMOPT_KV_FP16;
  d.key_cache = key_cache;
  d.value_cache = value_cache;
  d.block_size = block_size;
  d.num_kv_blocks = num_kv_blocks;
  d.kv_head_stride = head_dim;
  d.kv_token_stride = (int64_t)num_heads * head_dim;
  d.kv_page_stride = (int64_t)block_size * num_heads * head_dim;
  d.block_tables = block_tables;
  d.max_blocks_per_seq = max_blocks_per_seq;
  d.context_lens = context_lens;
  d.max_seq_len = max_seq_len;
  d.window_size = window_size;
  return paged_attention(d, true, stream);
}

}  // extern "C"
