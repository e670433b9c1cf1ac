// decode_fp16.hip — single-query paged attention over fp16 page pools (the
// reference's default cache format; TheRadDani/memopt-transformer-runtime
// src/csrc/attention.cu:98-339 computes the same softmax(q K^T / sqrt(D)) V
// over the window [ctx - W, ctx) with unlinked pages skipped, :158-186).
//
// HBM-bound design for gfx950 (wave64), the fp16 counterpart of the INT4
// decode kernel:
//  * keys advance in 16-token chunks (a page of block_size tokens holds
//    block_size / 16 of them); one wave streams one chunk of one head per
//    step: lane l owns token l / 4 of the chunk and dims
//    [(l % 4) D/4, (l % 4 + 1) D/4), read as D/32 16-byte loads for K and as
//    many for V;
//  * each wave keeps U chunks in flight (double-buffered batches) and a
//    workgroup of NW waves interleaves the chunks of one (b, h); split-K
//    partials (m, l, o) are merged by the shared combine kernel;
//  * q . k is v_dot2_f32_f16 over the lane's dims plus 2 DPP steps across the
//    token's 4 lanes; the softmax running max is wave-uniform and raised
//    lazily (only when a score exceeds it by more than 8 in log2 units);
//  * V is accumulated in fp32 with mixed-precision FMAs; the 16 token lanes
//    of each dim quarter are summed once at the end.
#include "attention.hpp"

namespace memopt {

typedef uint32_t u32x4f_t __attribute__((ext_vector_type(4)));

template <int D, int NW, int U>
__global__ __launch_bounds__(NW * 64) void decode_fp16_kernel(const DecodeParams p) {
  constexpr int DPL = D / 4;       // dims per lane
  constexpr int NLD = DPL / 8;     // 16-byte loads per lane for K (and for V)
  constexpr int NW2 = DPL / 2;     // half2 words per lane
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int32_t b = blockIdx.z, h = blockIdx.y, split = blockIdx.x;
  const int t = lane >> 2, c = lane & 3;

  __shared__ float s_acc[NW][D];
  __shared__ float s_ml[NW][2];

  const int32_t ctx = p.ctx[b];
  const KeyRange kr = key_range(ctx, ctx - 1, p.W, p.sinks, false);
  const int32_t hi_c = min((kr.hi + 15) >> 4, p.M * (p.bs >> 4));  // chunks
  const int32_t sink_c = min((kr.sink_end + 15) >> 4, hi_c);
  const int32_t win_c0 = max(kr.win_lo >> 4, sink_c);
  const int64_t n_vis = (int64_t)sink_c + max(0, hi_c - win_c0);
  const int32_t begin = (int32_t)((n_vis * split) / p.splits);
  const int32_t end = (int32_t)((n_vis * (split + 1)) / p.splits);
  const int32_t cpp_shift = __builtin_ctz((uint32_t)(p.bs >> 4));  // chunks per page = 2^shift

  half2_t qh[NW2];
  {
    const uint4 *qrow = reinterpret_cast<const uint4 *>(p.q + ((int64_t)b * p.H + h) * D + c * DPL);
#pragma unroll
    for (int k = 0; k < NLD; ++k) {
      const uint4 u = qrow[k];
      qh[4 * k + 0] = as_half2(u.x);
      qh[4 * k + 1] = as_half2(u.y);
      qh[4 * k + 2] = as_half2(u.z);
      qh[4 * k + 3] = as_half2(u.w);
    }
  }

  float m = -INFINITY, l = 0.0f;
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.0f;

  const int32_t *btrow = p.bt + (int64_t)b * p.M;
  const uint8_t *kbase = p.kc + (int64_t)h * p.kv_hs;
  const uint8_t *vbase = p.vc + (int64_t)h * p.kv_hs;
  const uint32_t loff = (uint32_t)(t * p.kv_ts) + (uint32_t)(c * DPL * 2);
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
      for (int k = 0; k < NLD; ++k) bt.kw[u][k] = __builtin_amdgcn_raw_buffer_load_b128(rk, (int)(loff + 16 * k), 0, 0);
#pragma unroll
      for (int k = 0; k < NLD; ++k) bt.vw[u][k] = __builtin_amdgcn_raw_buffer_load_b128(rv, (int)(loff + 16 * k), 0, 0);
    }
  };
  auto consume = [&](Batch &bt) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float d = 0.0f;
#pragma unroll
      for (int k = 0; k < NLD; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) d = __builtin_amdgcn_fdot2(as_half2(bt.kw[u][k][j]), qh[4 * k + j], d, false);
      d += xor1(d);
      d += xor2(d);
      const int32_t tok0 = bt.lc[u] * 16;
      const bool full = bt.ok[u] && tok0 >= kr.win_lo && tok0 + 16 <= kr.hi;
      bool vis = full;
      if (!full) {  // wave-uniform
        const int32_t tk = tok0 + t;
        vis = bt.ok[u] && tk < kr.hi && (tk >= kr.win_lo || tk < kr.sink_end);
        // A masked token's V may hold any bits: it must not meet p = 0.
#pragma unroll
        for (int k = 0; k < NLD; ++k)
          bt.vw[u][k] = vis ? bt.vw[u][k] : (u32x4f_t){0u, 0u, 0u, 0u};
      }
      const float s = vis ? d * p.qk_scale_log2 : -INFINITY;
      if (__any(s > m + 8.0f)) {  // wave-uniform, rare after the first chunks
        const float mn = fmaxf(m, wave_max(s));
        const float alpha = (mn == m) ? 1.0f : fast_exp2(m - mn);
        l *= alpha;
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] *= alpha;
        m = mn;
      }
      const float pr = vis ? fast_exp2(s - m) : 0.0f;
      l += pr;
#pragma unroll
      for (int k = 0; k < NLD; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const half2_t v2 = as_half2(bt.vw[u][k][j]);
          acc[8 * k + 2 * j] = fmaf(pr, (float)v2.x, acc[8 * k + 2 * j]);
          acc[8 * k + 2 * j + 1] = fmaf(pr, (float)v2.y, acc[8 * k + 2 * j + 1]);
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

  // Sum the 16 token lanes of each dim quarter (lanes c, c + 4, ..., c + 60):
  // row_ror 4 and 8 inside each row of 16, then across rows.
  l += dpp_f32<0x124>(l);
  l += dpp_f32<0x128>(l);
  l = xor16_sum(l);
  l = xor32_sum(l);
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    float v = acc[i];
    v += dpp_f32<0x124>(v);
    v += dpp_f32<0x128>(v);
    v = xor16_sum(v);
    v = xor32_sum(v);
    acc[i] = v;
  }
  if (t == 0) {
#pragma unroll
    for (int i = 0; i < DPL; ++i) s_acc[wave][c * DPL + i] = acc[i];
    if (c == 0) {
      s_ml[wave][0] = m;
      s_ml[wave][1] = l;
    }
  }
  __syncthreads();
  for (int dd = threadIdx.x; dd < D; dd += NW * 64) {
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) mx = fmaxf(mx, s_ml[w][0]);
    float lt = 0.0f, o = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = (s_ml[w][0] == -INFINITY) ? 0.0f : fast_exp2(s_ml[w][0] - mx);
      lt += s_ml[w][1] * f;
      o += s_acc[w][dd] * f;
    }
    const int64_t bh = (int64_t)b * p.H + h;
    if (p.splits == 1) {
      p.out[bh * D + dd] = (half_t)(lt > 0.0f ? o / lt : 0.0f);
    } else {
      const int64_t slot = bh * p.splits + split;
      p.ws_o[slot * D + dd] = o;
      if (dd == 0) {
        p.ws_ml[slot * 2] = mx;
        p.ws_ml[slot * 2 + 1] = lt;
      }
    }
  }
}

int launch_decode_fp16(const DecodeParams &p, int32_t batch, int32_t D, hipStream_t stream) {
  const dim3 grid(p.splits, p.H, batch);
  if (D == 128)
    hipLaunchKernelGGL((decode_fp16_kernel<128, 4, 2>), grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_fp16_kernel<64, 4, 2>), grid, dim3(256), 0, stream, p);
  int rc = check_launch("paged_attention(decode_fp16)");
  if (rc != MEMOPT_OK || p.splits == 1) return rc;
  return launch_decode_combine(p, batch, D, stream);
}

}  // namespace memopt
