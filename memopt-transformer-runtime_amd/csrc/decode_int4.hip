// decode_int4.hip — single-query paged attention that dequantizes INT4 pages
// just in time (the fused form of the reference's dequantize_kv_cache_int4 ->
// dynamic_sparse_attention composition; TheRadDani/memopt-transformer-runtime
// src/csrc/quantization.cu:232-270 and src/csrc/attention.cu:98-339).
//
// HBM-bound design for gfx950 (wave64):
//  * one wave streams one (page, head) block per step: 16 tokens x D/2 bytes
//    of K codes and of V codes (1 KiB each at D=128) are read with one
//    16-byte load per lane; lane l owns token l/4 and dims
//    [ (l%4)*D/4, (l%4+1)*D/4 ), i.e. half of one 64-dim scale group;
//  * nibbles become exact fp16 (code-8) with one AND-OR against an fp16
//    exponent bias (0x6400 -> 1024+n for bits 0-3, 0x5400 -> 64+n for bits
//    4-7) and one packed subtract; q.k uses v_dot2_f32_f16 (fp32 accumulate);
//  * each lane keeps its own online-softmax state (m, l, acc) for its token
//    slot, rescaling lazily only when a score exceeds the running max by more
//    than 2^8 in exp2 units, so the page loop has no cross-lane traffic
//    except a 2-step DPP sum of the 4 partial dot products of a token;
//  * waves of a workgroup interleave pages of one (b, h); workgroups split a
//    sequence's visited pages (split-K) and a small combine kernel merges the
//    (m, l, o) partials by log-sum-exp when splits > 1;
//  * only pages that intersect the sink range or the window are visited and
//    block-table entries < 0 (evicted pages) are skipped without loads.
#include "attention.hpp"

namespace memopt {

static constexpr int kDecodeWaves = 4;

template <typename ST>
__device__ __forceinline__ float load_scale(const void *p, int64_t i) {
  return (float)reinterpret_cast<const ST *>(p)[i];
}

template <int D>
struct LaneChunk;
template <>
struct LaneChunk<128> {
  uint4 w;
  static constexpr int kWords = 4;
  __device__ __forceinline__ void load(const uint8_t *p) { w = *reinterpret_cast<const uint4 *>(p); }
  __device__ __forceinline__ uint32_t word(int i) const {
    return i == 0 ? w.x : (i == 1 ? w.y : (i == 2 ? w.z : w.w));
  }
};
template <>
struct LaneChunk<64> {
  uint2 w;
  static constexpr int kWords = 2;
  __device__ __forceinline__ void load(const uint8_t *p) { w = *reinterpret_cast<const uint2 *>(p); }
  __device__ __forceinline__ uint32_t word(int i) const { return i == 0 ? w.x : w.y; }
};

// Exact (code - 8) for the 8 nibbles of a word, as 4 fp16 pairs in the order
// (e0,e4), (e1,e5), (e2,e6), (e3,e7) where e_i = bits 4i..4i+3.
__device__ __forceinline__ void unpack_word(uint32_t w, half2_t h[4]) {
  const half2_t b1024 = {(half_t)1032.0f, (half_t)1032.0f};
  const half2_t b64 = {(half_t)72.0f, (half_t)72.0f};
  const uint32_t w8 = w >> 8;
  h[0] = as_half2((w & 0x000F000Fu) | 0x64006400u) - b1024;
  h[1] = as_half2((w & 0x00F000F0u) | 0x54005400u) - b64;
  h[2] = as_half2((w8 & 0x000F000Fu) | 0x64006400u) - b1024;
  h[3] = as_half2((w8 & 0x00F000F0u) | 0x54005400u) - b64;
}

// Slot s of a lane's accumulator holds dim base + kSlotDim[s % 8] + 8*(s / 8).
__device__ __constant__ int kSlotDim[8] = {0, 4, 1, 5, 2, 6, 3, 7};

template <int D, typename ST>
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_int4_kernel(const DecodeParams p) {
  constexpr int BPL = D / 8;   // code bytes per lane per page
  constexpr int DPL = D / 4;   // dims per lane
  constexpr int NWORD = BPL / 4;
  using Chunk = LaneChunk<D>;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int32_t b = blockIdx.z, h = blockIdx.y, split = blockIdx.x;
  const int t = lane >> 2, c = lane & 3;
  const int g = (c * DPL) / 64;  // scale group of this lane's dims

  __shared__ float s_acc[kDecodeWaves][D];
  __shared__ float s_ml[kDecodeWaves][2];

  const int32_t ctx = p.ctx[b];
  const KeyRange kr = key_range(ctx, ctx - 1, p.W, p.sinks, false);

  // Visited logical pages: sink pages then window pages (deduplicated).
  const int32_t last_page = min((kr.hi + 15) >> 4, p.M);
  const int32_t sink_pages = min((kr.sink_end + 15) >> 4, last_page);
  const int32_t win_page0 = max(kr.win_lo >> 4, sink_pages);
  const int32_t n_win = max(0, last_page - win_page0);
  const int64_t n_vis = (int64_t)sink_pages + n_win;
  const int32_t begin = (int32_t)((n_vis * split) / p.splits);
  const int32_t end = (int32_t)((n_vis * (split + 1)) / p.splits);

  // q in permuted fp16 pairs: word k of this lane covers dims c*DPL + 8k + 0..7.
  half2_t qp[NWORD][4];
  {
    const half_t *qrow = p.q + ((int64_t)b * p.H + h) * D + c * DPL;
#pragma unroll
    for (int k = 0; k < NWORD; ++k) {
      const uint4 u = *reinterpret_cast<const uint4 *>(qrow + 8 * k);
      const half2_t a = as_half2(u.x), bb = as_half2(u.y), cc = as_half2(u.z), dd = as_half2(u.w);
      // elements: a=(0,1) bb=(2,3) cc=(4,5) dd=(6,7)
      qp[k][0] = half2_t{a.x, cc.x};
      qp[k][1] = half2_t{a.y, cc.y};
      qp[k][2] = half2_t{bb.x, dd.x};
      qp[k][3] = half2_t{bb.y, dd.y};
    }
  }

  float m = -INFINITY, l = 0.0f;
  float acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.0f;

  const int32_t *btrow = p.bt + (int64_t)b * p.M;
  const int64_t khead = (int64_t)h * p.kv_hs + (int64_t)t * p.kv_ts + c * BPL;
  const int64_t shead = (int64_t)h * p.sc_hs + (int64_t)t * p.sc_ts + g;

  for (int32_t i = begin + wave; i < end; i += kDecodeWaves) {
    const int32_t lp = (i < sink_pages) ? i : win_page0 + (i - sink_pages);
    const int32_t phys = __builtin_amdgcn_readfirstlane(btrow[lp]);
    if (phys < 0) continue;  // evicted / unlinked page
    Chunk kw, vw;
    kw.load(p.kc + (int64_t)phys * p.kv_ps + khead);
    vw.load(p.vc + (int64_t)phys * p.kv_ps + khead);
    const float sk = load_scale<ST>(p.ks, (int64_t)phys * p.sc_ps + shead);
    const float sv = load_scale<ST>(p.vs, (int64_t)phys * p.sc_ps + shead);

    float dot = 0.0f;
#pragma unroll
    for (int k = 0; k < NWORD; ++k) {
      half2_t hk[4];
      unpack_word(kw.word(k), hk);
#pragma unroll
      for (int j = 0; j < 4; ++j) dot = __builtin_amdgcn_fdot2(hk[j], qp[k][j], dot, false);
    }
    float s = dot * sk;
    s += xor1(s);
    s += xor2(s);
    const int32_t tok = lp * 16 + t;
    const bool valid = tok < kr.hi && (tok >= kr.win_lo || tok < kr.sink_end);
    s = valid ? s * p.qk_scale_log2 : -INFINITY;

    if (__any(s > m + 8.0f)) {
      const float mn = fmaxf(m, s);
      const float alpha = (mn == m) ? 1.0f : fast_exp2(m - mn);
      l *= alpha;
#pragma unroll
      for (int d = 0; d < DPL; ++d) acc[d] *= alpha;
      m = mn;
    }
    const float pw = (s == -INFINITY) ? 0.0f : fast_exp2(s - m);
    l += pw;
    const float wv = pw * sv;
#pragma unroll
    for (int k = 0; k < NWORD; ++k) {
      half2_t hv[4];
      unpack_word(vw.word(k), hv);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[8 * k + 2 * j] = fmaf(wv, (float)hv[j].x, acc[8 * k + 2 * j]);
        acc[8 * k + 2 * j + 1] = fmaf(wv, (float)hv[j].y, acc[8 * k + 2 * j + 1]);
      }
    }
  }

  // Merge the 16 token slots that share this lane's dims (lanes c, c+4, ...).
#pragma unroll
  for (int off = 4; off < 64; off <<= 1) {
    const float mo = shfl_xor(m, off), lo = shfl_xor(l, off);
    const float mn = fmaxf(m, mo);
    const float a = (m == mn) ? 1.0f : fast_exp2(m - mn);
    const float bsc = (mo == mn) ? 1.0f : fast_exp2(mo - mn);
    l = l * a + lo * bsc;
#pragma unroll
    for (int d = 0; d < DPL; ++d) acc[d] = acc[d] * a + shfl_xor(acc[d], off) * bsc;
    m = mn;
  }
  if (t == 0) {
#pragma unroll
    for (int s = 0; s < DPL; ++s) s_acc[wave][c * DPL + 8 * (s >> 3) + kSlotDim[s & 7]] = acc[s];
    if (c == 0) {
      s_ml[wave][0] = m;
      s_ml[wave][1] = l;
    }
  }
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += kDecodeWaves * 64) {
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) mx = fmaxf(mx, s_ml[w][0]);
    float lt = 0.0f, o = 0.0f;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
      const float f = (s_ml[w][0] == -INFINITY) ? 0.0f : fast_exp2(s_ml[w][0] - mx);
      lt += s_ml[w][1] * f;
      o += s_acc[w][d] * f;
    }
    const int64_t bh = (int64_t)b * p.H + h;
    if (p.splits == 1) {
      p.out[bh * D + d] = (half_t)(lt > 0.0f ? o / lt : 0.0f);
    } else {
      const int64_t slot = bh * p.splits + split;
      p.ws_o[slot * D + d] = o;
      if (d == 0) {
        p.ws_ml[slot * 2] = mx;
        p.ws_ml[slot * 2 + 1] = lt;
      }
    }
  }
}

// Log-sum-exp merge of split partials: one workgroup per (b, h).
__global__ __launch_bounds__(128) void decode_combine_kernel(const float *__restrict__ ws_o,
                                                             const float *__restrict__ ws_ml,
                                                             half_t *__restrict__ out, int32_t D,
                                                             int32_t splits) {
  const int64_t bh = blockIdx.x;
  const float *ml = ws_ml + bh * splits * 2;
  float mx = -INFINITY;
  for (int s = 0; s < splits; ++s) mx = fmaxf(mx, ml[2 * s]);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float lt = 0.0f, o = 0.0f;
    for (int s = 0; s < splits; ++s) {
      const float f = (ml[2 * s] == -INFINITY) ? 0.0f : fast_exp2(ml[2 * s] - mx);
      lt += ml[2 * s + 1] * f;
      o += ws_o[(bh * splits + s) * D + d] * f;
    }
    out[bh * D + d] = (half_t)(lt > 0.0f ? o / lt : 0.0f);
  }
}

static int device_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
      cus = prop.multiProcessorCount;
    if (cus <= 0) cus = 256;
  }
  return cus;
}

int decode_splits(int32_t batch, int32_t heads, int32_t max_pages_visited) {
  const int64_t units = (int64_t)batch * heads;
  if (units <= 0) return 1;
  const int64_t target_wgs = 2LL * device_cus();
  int64_t s = (target_wgs + units - 1) / units;
  // Keep at least 8 pages per wave.
  const int64_t cap = max_pages_visited / (8 * kDecodeWaves);
  if (s > cap) s = cap;
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  return (int)s;
}

int launch_decode_int4(const DecodeParams &p, int32_t batch, int32_t D, int32_t scale_dtype,
                       hipStream_t stream) {
  const dim3 grid(p.splits, p.H, batch), block(kDecodeWaves * 64);
  if (D == 128 && scale_dtype == MEMOPT_SCALE_F16)
    hipLaunchKernelGGL((decode_int4_kernel<128, half_t>), grid, block, 0, stream, p);
  else if (D == 128)
    hipLaunchKernelGGL((decode_int4_kernel<128, float>), grid, block, 0, stream, p);
  else if (scale_dtype == MEMOPT_SCALE_F16)
    hipLaunchKernelGGL((decode_int4_kernel<64, half_t>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((decode_int4_kernel<64, float>), grid, block, 0, stream, p);
  int rc = check_launch("paged_attention(decode_int4)");
  if (rc != MEMOPT_OK || p.splits == 1) return rc;
  hipLaunchKernelGGL(decode_combine_kernel, dim3((unsigned)((int64_t)batch * p.H)), dim3(128), 0, stream,
                     p.ws_o, p.ws_ml, p.out, D, p.splits);
  return check_launch("paged_attention(decode_combine)");
}

}  // namespace memopt
