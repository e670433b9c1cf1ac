// decode_fp16.hip — single-query paged attention over fp16 page pools (the
// reference's default cache format; TheRadDani/memopt-transformer-runtime
// src/csrc/attention.cu:98-339 computes the same softmax(q K^T / sqrt(D)) V
// over the window [ctx - W, ctx) with unlinked pages skipped, :158-186).
//
// HBM-bound design for gfx950 (wave64), the fp16 counterpart of the INT4
// decode kernel:
//  * keys advance in 16-token chunks (a page of block_size tokens holds
//    block_size / 16 of them); one wave streams one chunk of one head per
//    step. Lane l = 8p + c owns tokens p and p + 8 of the chunk and, of each
//    128-byte line of a token's row (64 dims), the 16 bytes at 16c: one load
//    instruction covers 8 whole lines (8 tokens x one line), so the loads
//    can be streaming (non-temporal) without a line being fetched twice;
//  * each wave keeps U chunks in flight (double-buffered batches) and a
//    workgroup of NW waves interleaves the chunks of one (b, h); split-K
//    partials (m, l, o) are merged by the last workgroup of each (b, h) to
//    finish, in the shared decode epilogue;
//  * q . k is v_dot2_f32_f16 over the lane's dims plus 3 DPP steps across
//    the token's 8 lanes; the softmax running max is wave-uniform and raised
//    lazily (only when a score exceeds it by more than 8 in log2 units);
//  * V is accumulated in fp32 with mixed-precision FMAs (both tokens of the
//    lane into the same dims); the 8 token-pair lanes of each dim slice are
//    summed once at the end.
#include "attention.hpp"

namespace memopt {

typedef uint32_t u32x4f_t __attribute__((ext_vector_type(4)));

template <int D, int NW, int U>
__global__ __launch_bounds__(NW * 64) void decode_fp16_kernel(const DecodeParams p) {
  constexpr int NL = D / 64;   // 128-byte lines per token row
  constexpr int DPL = 8 * NL;  // dims per lane (8 of each line)
  constexpr int NLD = 2 * NL;  // 16-byte loads per lane for K (and for V): 2 tokens x NL lines
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int32_t b = blockIdx.z, h = blockIdx.y, split = blockIdx.x;
  const int pp = lane >> 3, c = lane & 7;

  __shared__ float s_acc[NW][D];
  __shared__ float s_ml[NW][2];

  const int32_t ctx = p.ctx[b];
  const KeyRange kr = key_range(ctx, ctx - 1, p.W, p.sinks, false);
  const int32_t hi_c = min((kr.hi + 15) >> 4, p.M * (p.bs >> 4));  // chunks
  const int32_t sink_c = min((kr.sink_end + 15) >> 4, hi_c);
  const int32_t win_c0 = max(kr.win_lo >> 4, sink_c);
  const int64_t n_vis = (int64_t)sink_c + max(0, hi_c - win_c0);
  const SplitRange sr = split_range((int32_t)n_vis, split, p.splits);
  const int32_t begin = sr.begin, end = sr.end;
  const int32_t cpp_shift = __builtin_ctz((uint32_t)(p.bs >> 4));  // chunks per page = 2^shift

  // q over the lane's dims: 8 per line, dims 64 n + 8 c .. 64 n + 8 c + 7.
  half2_t qh[4 * NL];
  {
    const half_t *qrow = p.q + ((int64_t)b * p.H + h) * D + 8 * c;
#pragma unroll
    for (int n = 0; n < NL; ++n) {
      const uint4 u = *reinterpret_cast<const uint4 *>(qrow + 64 * n);
      qh[4 * n + 0] = as_half2(u.x);
      qh[4 * n + 1] = as_half2(u.y);
      qh[4 * n + 2] = as_half2(u.z);
      qh[4 * n + 3] = as_half2(u.w);
    }
  }

  float m = -INFINITY, l = 0.0f;
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.0f;

  const int32_t *btrow = p.bt + (int64_t)b * p.M;
  const uint8_t *kbase = p.kc + (int64_t)h * p.kv_hs;
  const uint8_t *vbase = p.vc + (int64_t)h * p.kv_hs;
  // load k: token pp + 8 (k / NL), line k % NL
  const uint32_t loff0 = (uint32_t)(pp * p.kv_ts) + (uint32_t)(16 * c);
  const uint32_t loff8 = loff0 + (uint32_t)(8 * p.kv_ts);
  const int32_t nb32 = (int32_t)min(p.nb, (int64_t)INT32_MAX);

  // Slots past `end` (and unlinked pages) read chunk 0 of page 0 of this
  // head, which is always mapped, and are masked out.
  struct Batch {
    u32x4f_t kw[U][NLD], vw[U][NLD];
    int32_t lc[U];
    bool ok[U];
  };
  auto issue = [&](Batch &bt, int32_t base) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int32_t i = base + u;
      const int32_t lc = (i < sink_c) ? i : win_c0 + (i - sink_c);
      bt.lc[u] = lc;
      const int32_t page = lc >> cpp_shift;
      const int32_t phys = btrow[(i < end) ? page : 0];  // page < M whenever i < end
      bt.ok[u] = (i < end) && phys >= 0 && phys < nb32;
      const int64_t off = bt.ok[u] ? (int64_t)phys * p.kv_ps + (int64_t)((lc - (page << cpp_shift)) * 16) * p.kv_ts : 0;
      const __amdgpu_buffer_rsrc_t rk =
          __builtin_amdgcn_make_buffer_rsrc((void *)uniform_ptr(kbase + off), (short)0, 0x7FFFFFFF, 0x00020000);
      const __amdgpu_buffer_rsrc_t rv =
          __builtin_amdgcn_make_buffer_rsrc((void *)uniform_ptr(vbase + off), (short)0, 0x7FFFFFFF, 0x00020000);
#pragma unroll
      for (int k = 0; k < NLD; ++k)
        bt.kw[u][k] = __builtin_amdgcn_raw_buffer_load_b128(rk, (int)((k < NL ? loff0 : loff8) + 128 * (k % NL)), 0,
                                                            kStreamLoad);
#pragma unroll
      for (int k = 0; k < NLD; ++k)
        bt.vw[u][k] = __builtin_amdgcn_raw_buffer_load_b128(rv, (int)((k < NL ? loff0 : loff8) + 128 * (k % NL)), 0,
                                                            kStreamLoad);
    }
  };
  auto consume = [&](Batch &bt) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
      for (int n = 0; n < NL; ++n)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          d0 = __builtin_amdgcn_fdot2(as_half2(bt.kw[u][n][j]), qh[4 * n + j], d0, false);
          d1 = __builtin_amdgcn_fdot2(as_half2(bt.kw[u][NL + n][j]), qh[4 * n + j], d1, false);
        }
      d0 += xor1(d0);
      d1 += xor1(d1);
      d0 += xor2(d0);
      d1 += xor2(d1);
      d0 += half_mirror(d0);
      d1 += half_mirror(d1);
      const int32_t tok0 = bt.lc[u] * 16;
      const bool full = bt.ok[u] && tok0 >= kr.win_lo && tok0 + 16 <= kr.hi;
      bool vis0 = full, vis1 = full;
      if (!full) {  // wave-uniform
        const int32_t t0 = tok0 + pp, t1 = t0 + 8;
        vis0 = bt.ok[u] && t0 < kr.hi && (t0 >= kr.win_lo || t0 < kr.sink_end);
        vis1 = bt.ok[u] && t1 < kr.hi && (t1 >= kr.win_lo || t1 < kr.sink_end);
        // A masked token's V may hold any bits: it must not meet p = 0.
#pragma unroll
        for (int n = 0; n < NL; ++n) {
          bt.vw[u][n] = vis0 ? bt.vw[u][n] : (u32x4f_t){0u, 0u, 0u, 0u};
          bt.vw[u][NL + n] = vis1 ? bt.vw[u][NL + n] : (u32x4f_t){0u, 0u, 0u, 0u};
        }
      }
      const float s0 = vis0 ? d0 * p.qk_scale_log2 : -INFINITY;
      const float s1 = vis1 ? d1 * p.qk_scale_log2 : -INFINITY;
      const float smax = fmaxf(s0, s1);
      if (__any(smax > m + 8.0f)) {  // wave-uniform, rare after the first chunks
        const float mn = fmaxf(m, wave_max(smax));
        const float alpha = (mn == m) ? 1.0f : fast_exp2(m - mn);
        l *= alpha;
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] *= alpha;
        m = mn;
      }
      const float p0 = vis0 ? fast_exp2(s0 - m) : 0.0f;
      const float p1 = vis1 ? fast_exp2(s1 - m) : 0.0f;
      l += p0 + p1;
#pragma unroll
      for (int n = 0; n < NL; ++n)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const half2_t v0 = as_half2(bt.vw[u][n][j]), v1 = as_half2(bt.vw[u][NL + n][j]);
          acc[8 * n + 2 * j] = fmaf(p1, (float)v1.x, fmaf(p0, (float)v0.x, acc[8 * n + 2 * j]));
          acc[8 * n + 2 * j + 1] = fmaf(p1, (float)v1.y, fmaf(p0, (float)v0.y, acc[8 * n + 2 * j + 1]));
        }
    }
  };

  constexpr int32_t kStep = NW * U;
  Batch ba, bb;
  int32_t base = begin + wave * U;
  issue(ba, base);
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
  for (int i = 0; i < DPL; ++i) {
    float v = acc[i];
    v += dpp_f32<0x128>(v);
    v = xor16_sum(v);
    v = xor32_sum(v);
    acc[i] = v;
  }
  if (pp == 0) {
#pragma unroll
    for (int i = 0; i < DPL; ++i) s_acc[wave][64 * (i / 8) + 8 * c + (i % 8)] = acc[i];
    if (c == 0) {
      s_ml[wave][0] = m;
      s_ml[wave][1] = l;
    }
  }
  __syncthreads();
  decode_epilogue<D, NW>(p, (int64_t)b * p.H + h, split, s_acc, s_ml);
}

int launch_decode_fp16(const DecodeParams &p, int32_t batch, int32_t D, hipStream_t stream) {
  const dim3 grid(p.splits, p.H, batch);
  if (D == 128)
    hipLaunchKernelGGL((decode_fp16_kernel<128, 4, 2>), grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_fp16_kernel<64, 4, 2>), grid, dim3(256), 0, stream, p);
  return check_launch("paged_attention(decode_fp16)");
}

}  // namespace memopt
