// prefill.hip — multi-query paged attention on fp16 MFMA (gfx950), over the
// INT4 page pool (dequantized just in time into LDS) or the fp16 pool.
//
// Semantics: TheRadDani/memopt-transformer-runtime src/csrc/attention.cu:98-339
// (paged K/V through block tables, pages < 0 skipped, empty key set -> 0)
// with the window/sink/causal rule of scripts/bench_accuracy.py:253-280
// (causal) or src/csrc/attention.cu:158-186 plus sinks (non-causal).
//
// Layout of the work (wave64, v_mfma_f32_32x32x16_f16):
//  * a workgroup owns 32*NW queries of one (batch, head); wave w owns 32 of
//    them, one query per lane column (lanes l and l+32 share query l%32);
//  * keys advance in tiles of 64 (four 16-token chunks). All threads of the
//    workgroup stage a tile in LDS: K as 64 rows x D dims (fp16), V
//    transposed as D rows x 64 keys. INT4 pages are unpacked with one
//    v_bfi_b32 per nibble pair, made exact with one packed subtract and
//    scaled with one packed fp16 multiply — the same fp16(code-8)*scale the
//    reference's dequantize kernel produces;
//  * S^T = K Q^T per 32-key block (lane column = query, 16 key rows per lane),
//    so the softmax reduction over keys is lane-local plus one exchange
//    between the two lane halves; the probabilities are packed to fp16 in
//    register order and used directly as the B operand of O^T += V^T P^T,
//    with the V^T columns stored in the matching key order;
//  * K rows inside a 16-token chunk are stored in page pair order (row 2p =
//    token p, row 2p+1 = token p+8) and, for INT4, the dims of each 8-dim
//    group in nibble-unpack order (0,4,1,5,2,6,3,7); Q is loaded once in the
//    same dim order, so neither staging path repacks;
//  * tiles wholly inside every query's visible range skip the mask; the
//    running max is raised lazily (rescale only when exceeded by > 8 in log2
//    units).
#include "attention.hpp"
#include "page_format.hpp"

namespace memopt {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

static constexpr int kTileKeys = 64;

struct PrefillParams {
  const half_t *q;
  half_t *out;
  int32_t Lq, H;
  const uint8_t *pool;  // INT4 page buffer, or fp16 K pool (bytes)
  const uint8_t *vpool; // fp16 V pool (fp16 path only)
  int64_t nb;
  int32_t bs;           // tokens per page
  const int32_t *bt;
  int32_t M;
  const int32_t *ctx;
  int32_t W, sinks, causal;
  float qk_scale_log2;
};

// Key index of K-tile row R (pair order inside each 16-token chunk).
__device__ __forceinline__ int32_t row_key(int32_t R) {
  const int32_t w = R & 15;
  return (R & ~15) + ((w & 1) ? (w >> 1) + 8 : (w >> 1));
}

// V^T column of K-tile row R: rows 32b + 8g + 4h + q map to column
// 32b + 16(g/2) + 8h + 4(g%2) + q, the k order of the PV MFMA B operand.
__device__ __forceinline__ int32_t vt_col(int32_t R) {
  const int32_t b = R >> 5, r = R & 31, g = r >> 3, h = (r >> 2) & 1, q = r & 3;
  return 32 * b + 16 * (g >> 1) + 8 * h + 4 * (g & 1) + q;
}

__device__ __forceinline__ bool key_visible(int32_t key, int32_t qpos, int32_t ctx, int32_t W, int32_t sinks,
                                            bool causal) {
  if (key >= ctx) return false;
  if (causal) return key <= qpos && (key < sinks || key >= qpos - W + 1);
  return key >= ctx - W || key < sinks;
}

template <int D, bool INT4, int NW>
__global__ __launch_bounds__(NW * 64) void prefill_kernel(const PrefillParams p) {
  constexpr int KSTR = D * 2 + 16;          // K row stride in LDS (bytes), padded
  constexpr int VSTR = kTileKeys * 2 + 16;  // V^T row stride (bytes), padded
  constexpr int NCH = D / 16;               // 16-dim chunks of the QK contraction
  constexpr int NDB = D / 32;               // 32-dim output blocks
  constexpr int DPT = D / 8;                // dims per staging task
  __shared__ __attribute__((aligned(16))) uint8_t lds_k[kTileKeys * KSTR];
  __shared__ __attribute__((aligned(16))) uint8_t lds_v[D * VSTR];
  __shared__ int32_t s_pages[4];

  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int32_t h = blockIdx.y, b = blockIdx.z;
  const int32_t ctx = p.ctx[b];
  const int32_t kv_lim = min(ctx, p.M * p.bs);
  const int32_t q0 = blockIdx.x * 32 * NW;
  const int32_t qw0 = q0 + 32 * wave;
  const int32_t qi = qw0 + (lane & 31);
  const bool q_ok = qi < p.Lq;
  const int32_t qpos = ctx - p.Lq + qi;
  const bool causal = p.causal != 0;

  // ---- Q fragments: chunk c, lane half hl -> 8 dims (INT4: unpack order) ----
  half8_t qf[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    half8_t v = {};
    if (q_ok) {
      const uint4 u = *reinterpret_cast<const uint4 *>(p.q + (((int64_t)b * p.Lq + qi) * p.H + h) * D + 16 * c + 8 * hl);
      const half8_t n = __builtin_bit_cast(half8_t, u);
      if (INT4) {
        v[0] = n[0]; v[1] = n[4]; v[2] = n[1]; v[3] = n[5];
        v[4] = n[2]; v[5] = n[6]; v[6] = n[3]; v[7] = n[7];
      } else {
        v = n;
      }
    }
    qf[c] = v;
  }

  float16_t o[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) o[i] = (float16_t){};
  float m = -INFINITY, lsum = 0.0f;

  // ---- key tiles visited by this workgroup ----
  const int32_t qlast = min(q0 + 32 * NW, p.Lq) - 1;
  const int32_t pos_lo = ctx - p.Lq + q0, pos_hi = ctx - p.Lq + qlast;
  const int32_t hi = max(0, causal ? min(kv_lim, pos_hi + 1) : kv_lim);
  const int32_t win_lo = max(0, causal ? pos_lo - p.W + 1 : ctx - p.W);
  const int32_t sink_end = min(p.sinks, hi);  // p.sinks >= 0
  const int32_t sink_tiles = (sink_end + kTileKeys - 1) / kTileKeys;
  const int32_t t_first = max(win_lo / kTileKeys, sink_tiles);
  const int32_t t_last = (hi + kTileKeys - 1) / kTileKeys;  // exclusive
  const int32_t n_tiles = sink_tiles + max(0, t_last - t_first);
  // wave-level query span (for skipping and the unmasked fast path)
  const int32_t wq_last = min(qw0 + 31, p.Lq - 1);
  const int32_t wpos_lo = ctx - p.Lq + qw0, wpos_hi = ctx - p.Lq + wq_last;

  for (int32_t it = 0; it < n_tiles; ++it) {
    const int32_t tile = it < sink_tiles ? it : t_first + (it - sink_tiles);
    const int32_t tb = tile * kTileKeys;

    __syncthreads();  // previous tile's LDS reads are done
    if (tid < 4) {
      const int32_t key = tb + 16 * tid;
      int32_t pg = -1;
      if (key < kv_lim) {
        const int32_t e = p.bt[(int64_t)b * p.M + key / p.bs];
        pg = (e >= 0 && e < p.nb) ? e : -1;
      }
      s_pages[tid] = pg;
    }
    __syncthreads();

    // ---- stage the tile: task = (16-key chunk k, pair pp, dim slice c) ----
    for (int task = tid; task < 256; task += NW * 64) {
      const int k = task >> 6, pp = (task >> 3) & 7, c = task & 7;
      const int32_t pg = s_pages[k];
      const int R0 = 16 * k + 2 * pp;  // rows of tokens pp and pp+8 of the chunk
      uint8_t *krow0 = lds_k + R0 * KSTR + c * DPT * 2;
      uint8_t *krow1 = krow0 + KSTR;
      const int vc0 = vt_col(R0);       // V^T column of token pp; pp+8 is vc0 + 1
      if (pg < 0) {
        for (int i = 0; i < DPT / 8; ++i) {
          *reinterpret_cast<uint4 *>(krow0 + 16 * i) = make_uint4(0, 0, 0, 0);
          *reinterpret_cast<uint4 *>(krow1 + 16 * i) = make_uint4(0, 0, 0, 0);
        }
        for (int d = 0; d < DPT; ++d) *reinterpret_cast<uint32_t *>(lds_v + (c * DPT + d) * VSTR + vc0 * 2) = 0;
        continue;
      }
      if (INT4) {
        const Int4Page f(D);
        const uint8_t *blk = p.pool + ((int64_t)pg * p.H + h) * f.block;
        const int slot = 8 * pp + c;
        const int g = (c * DPT) / 64;
        const half2_t sk = *reinterpret_cast<const half2_t *>(blk + f.kscales + 2 * (g * 16 + 2 * pp));
        const half2_t sv = *reinterpret_cast<const half2_t *>(blk + f.vscales + 2 * (g * 16 + 2 * pp));
        const half2_t b1032 = {(half_t)1032.0f, (half_t)1032.0f};
        const half2_t b72 = {(half_t)72.0f, (half_t)72.0f};
        // K: token pp = first BPL/2 bytes, token pp+8 = next BPL/2 (DPT/8 words each)
        const uint32_t *kw = reinterpret_cast<const uint32_t *>(blk + f.kcodes + slot * f.BPL);
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          const half2_t s2 = t2 ? half2_t{sk.y, sk.y} : half2_t{sk.x, sk.x};
          uint8_t *dst = t2 ? krow1 : krow0;
#pragma unroll
          for (int wi = 0; wi < DPT / 8; ++wi) {
            const uint32_t w = kw[t2 * (DPT / 8) + wi], w8 = w >> 8;
            const half2_t h0 = (as_half2(bfi(0x000F000Fu, w, 0x64006400u)) - b1032) * s2;
            const half2_t h1 = (as_half2(bfi(0x00F000F0u, w, 0x54005400u)) - b72) * s2;
            const half2_t h2 = (as_half2(bfi(0x000F000Fu, w8, 0x64006400u)) - b1032) * s2;
            const half2_t h3 = (as_half2(bfi(0x00F000F0u, w8, 0x54005400u)) - b72) * s2;
            *reinterpret_cast<uint4 *>(dst + 16 * wi) = make_uint4(as_u32(h0), as_u32(h1), as_u32(h2), as_u32(h3));
          }
        }
        // V: DPT/4 words, each = 4 dims x tokens (pp, pp+8)
        const uint32_t *vw = reinterpret_cast<const uint32_t *>(blk + f.vcodes + slot * f.BPL);
#pragma unroll
        for (int wi = 0; wi < DPT / 4; ++wi) {
          const uint32_t w = vw[wi], w8 = w >> 8;
          const half2_t h0 = (as_half2(bfi(0x000F000Fu, w, 0x64006400u)) - b1032) * sv;
          const half2_t h1 = (as_half2(bfi(0x00F000F0u, w, 0x54005400u)) - b72) * sv;
          const half2_t h2 = (as_half2(bfi(0x000F000Fu, w8, 0x64006400u)) - b1032) * sv;
          const half2_t h3 = (as_half2(bfi(0x00F000F0u, w8, 0x54005400u)) - b72) * sv;
          const int d0 = c * DPT + 4 * wi;
          *reinterpret_cast<uint32_t *>(lds_v + (d0 + 0) * VSTR + vc0 * 2) = as_u32(h0);
          *reinterpret_cast<uint32_t *>(lds_v + (d0 + 1) * VSTR + vc0 * 2) = as_u32(h1);
          *reinterpret_cast<uint32_t *>(lds_v + (d0 + 2) * VSTR + vc0 * 2) = as_u32(h2);
          *reinterpret_cast<uint32_t *>(lds_v + (d0 + 3) * VSTR + vc0 * 2) = as_u32(h3);
        }
      } else {
        const int32_t key0 = tb + 16 * k + pp;  // token pp of the chunk; pp+8 is key0 + 8
        const half_t *kp = reinterpret_cast<const half_t *>(p.pool);
        const half_t *vp = reinterpret_cast<const half_t *>(p.vpool);
        const int32_t pos0 = key0 % p.bs, pos1 = (key0 + 8) % p.bs;
        // chunk k lies in one page when bs % 16 == 0
        const int64_t r0 = (((int64_t)pg * p.bs + pos0) * p.H + h) * D + c * DPT;
        const int64_t r1 = (((int64_t)pg * p.bs + pos1) * p.H + h) * D + c * DPT;
#pragma unroll
        for (int i = 0; i < DPT / 8; ++i) {
          *reinterpret_cast<uint4 *>(krow0 + 16 * i) = *reinterpret_cast<const uint4 *>(kp + r0 + 8 * i);
          *reinterpret_cast<uint4 *>(krow1 + 16 * i) = *reinterpret_cast<const uint4 *>(kp + r1 + 8 * i);
        }
#pragma unroll
        for (int i = 0; i < DPT / 8; ++i) {
          const half8_t a = __builtin_bit_cast(half8_t, *reinterpret_cast<const uint4 *>(vp + r0 + 8 * i));
          const half8_t bb = __builtin_bit_cast(half8_t, *reinterpret_cast<const uint4 *>(vp + r1 + 8 * i));
#pragma unroll
          for (int e = 0; e < 8; ++e)
            *reinterpret_cast<uint32_t *>(lds_v + (c * DPT + 8 * i + e) * VSTR + vc0 * 2) = as_u32(half2_t{a[e], bb[e]});
        }
      }
    }
    __syncthreads();

    // ---- this wave's share: skip tiles with no visible key for its queries ----
    const bool is_sink_tile = tb < sink_end;
    bool any_vis;
    if (causal)
      any_vis = tb <= wpos_hi && (is_sink_tile || tb + kTileKeys - 1 >= wpos_lo - p.W + 1) && qw0 < p.Lq;
    else
      any_vis = qw0 < p.Lq;
    if (!any_vis) continue;
    const bool pages_ok = s_pages[0] >= 0 && s_pages[1] >= 0 && s_pages[2] >= 0 && s_pages[3] >= 0;
    const bool full = pages_ok && tb + kTileKeys <= kv_lim &&
                      (causal ? (tb + kTileKeys - 1 <= wpos_lo && tb >= wpos_hi - p.W + 1)
                              : (tb >= ctx - p.W)) &&
                      wq_last == qw0 + 31;

    // S^T blocks: rows = keys (32 per block), columns = this wave's queries
    float16_t s[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      s[blk] = (float16_t){};
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const half8_t a = *reinterpret_cast<const half8_t *>(lds_k + (32 * blk + (lane & 31)) * KSTR + (16 * c + 8 * hl) * 2);
        s[blk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[c], s[blk], 0, 0, 0);
      }
    }
    // scores in log2 units; masked entries -> -inf
    float tmax = -INFINITY;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = s[blk][r] * p.qk_scale_log2;
        if (!full) {
          const int R = 32 * blk + 8 * (r >> 2) + 4 * hl + (r & 3);
          const int32_t key = tb + row_key(R);
          const bool ok = q_ok && s_pages[R >> 4] >= 0 && key < kv_lim &&
                          key_visible(key, qpos, ctx, p.W, p.sinks, causal);
          v = ok ? v : -INFINITY;
        }
        s[blk][r] = v;
        tmax = fmaxf(tmax, v);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    if (__any(tmax > m + 8.0f)) {  // lazy rescale: p stays <= 2^8 between raises
      const float mn = fmaxf(m, tmax);
      const float alpha = (mn == m) ? 1.0f : fast_exp2(m - mn);
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      m = mn;
    }
    half8_t pb[4];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
      for (int g2 = 0; g2 < 2; ++g2) {
        half8_t v;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = s[blk][8 * g2 + e];
          const float pw = (full || x != -INFINITY) ? fast_exp2(x - m) : 0.0f;
          lsum += pw;
          v[e] = (half_t)pw;
        }
        pb[2 * blk + g2] = v;
      }
    }
    // O^T += V^T P^T over the four 16-key chunks
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
        const half8_t a = *reinterpret_cast<const half8_t *>(lds_v + (32 * db + (lane & 31)) * VSTR + (16 * kc + 8 * hl) * 2);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[kc], o[db], 0, 0, 0);
      }
    }
  }

  lsum += __shfl_xor(lsum, 32, 64);
  if (!q_ok) return;
  const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
  half_t *orow = p.out + (((int64_t)b * p.Lq + qi) * p.H + h) * D;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * db + 8 * g + 4 * hl;
      const half2_t a = {(half_t)(o[db][4 * g] * inv), (half_t)(o[db][4 * g + 1] * inv)};
      const half2_t c = {(half_t)(o[db][4 * g + 2] * inv), (half_t)(o[db][4 * g + 3] * inv)};
      *reinterpret_cast<uint2 *>(orow + d0) = make_uint2(as_u32(a), as_u32(c));
    }
  }
}

bool prefill_supported(const memopt_attn_desc &d) {
  auto al16 = [](const void *x) { return ((uintptr_t)x & 15) == 0; };
  if (d.q_len < 16 || (d.head_dim != 64 && d.head_dim != 128)) return false;
  if (d.num_heads > 65535 || d.batch > 65535 || d.num_kv_blocks <= 0) return false;
  if (!al16(d.query) || !al16(d.out) || !al16(d.key_cache)) return false;
  if (d.kv_format == MEMOPT_KV_INT4) return d.block_size == 16;
  if (d.kv_format != MEMOPT_KV_FP16 || d.block_size % 16 != 0 || !al16(d.value_cache)) return false;
  // contiguous [num_blocks, block_size, H, D] pools (element strides)
  const int64_t D = d.head_dim, H = d.num_heads;
  return d.kv_head_stride == D && d.kv_token_stride == H * D && d.kv_page_stride == d.block_size * H * D;
}

int launch_prefill(const memopt_attn_desc &d, int32_t W, float qk_scale_log2, hipStream_t stream) {
  PrefillParams p;
  p.q = (const half_t *)d.query;
  p.out = (half_t *)d.out;
  p.Lq = d.q_len;
  p.H = d.num_heads;
  p.pool = (const uint8_t *)d.key_cache;
  p.vpool = (const uint8_t *)d.value_cache;
  p.nb = d.num_kv_blocks;
  p.bs = d.block_size;
  p.bt = d.block_tables;
  p.M = d.max_blocks_per_seq;
  p.ctx = d.context_lens;
  p.W = W;
  p.sinks = d.num_sink_tokens < 0 ? 0 : d.num_sink_tokens;
  p.causal = d.causal;
  p.qk_scale_log2 = qk_scale_log2;
  constexpr int NW = 4;
  const dim3 grid((unsigned)((d.q_len + 32 * NW - 1) / (32 * NW)), d.num_heads, d.batch);
  const bool int4 = d.kv_format == MEMOPT_KV_INT4;
  if (d.head_dim == 128) {
    if (int4) hipLaunchKernelGGL((prefill_kernel<128, true, NW>), grid, dim3(NW * 64), 0, stream, p);
    else hipLaunchKernelGGL((prefill_kernel<128, false, NW>), grid, dim3(NW * 64), 0, stream, p);
  } else {
    if (int4) hipLaunchKernelGGL((prefill_kernel<64, true, NW>), grid, dim3(NW * 64), 0, stream, p);
    else hipLaunchKernelGGL((prefill_kernel<64, false, NW>), grid, dim3(NW * 64), 0, stream, p);
  }
  return check_launch("paged_attention(prefill)");
}

}  // namespace memopt
