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
//    running max is raised lazily (rescale only when a probability would
//    exceed 2^8); scores stay unscaled fp32 q . k and exp2 takes
//    log2(e) / sqrt(D) (score - m), so no scaled copy of Q is rounded.
#include "attention.hpp"
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include "page_format.hpp"

namespace memopt {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));


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

// Byte offset of V^T column byte `cb` in row d. 32-byte column blocks are
// XOR-swizzled by bits 4-5 of the row so the staging writes (16 rows per
// thread, 8 threads per row group) spread over the LDS banks; 16 consecutive
// rows share one swizzle, which keeps the MFMA operand reads conflict-free.
template <int SW>
__device__ __forceinline__ int vt_swz(int cb, int d) { return cb ^ (SW * ((d >> 4) & 3)); }

__device__ __forceinline__ bool key_visible(int32_t key, int32_t qpos, int32_t ctx, int32_t W, int32_t sinks,
                                            bool causal) {
  if (key >= ctx) return false;
  if (causal) return key <= qpos && (key < sinks || key >= qpos - W + 1);
  return key >= ctx - W || key < sinks;
}

// One staging task per thread: (16-key chunk k, token pair pp, dim slice c)
// of a 64-key tile; the registers below carry its raw data from the global
// load (issued one tile ahead) to the LDS write.
template <int D, bool INT4, bool SPLIT>
struct Staged {
  static constexpr int DPT = D / 8;  // dims per task
  int32_t pg;
  // INT4: K codes of tokens pp and pp+8 (DPT/8 words each) at w[KO..], V
  // codes (DPT/4 words, each 4 dims x both tokens) at w[VO..], scales
  // (token pp, token pp+8) in sc[KO] / sc[VO ? 1 : 0].
  // fp16: K and V rows of both tokens (DPT/8 16-byte vectors each), r[KO..]
  // and r[VR..]. When a thread stages only K or only V (SPLIT), both parts
  // share the same registers.
  static constexpr int NW_ = INT4 ? DPT / 4 : 1, NR_ = INT4 ? 1 : 2 * (DPT / 8);
  static constexpr int VO = SPLIT ? 0 : NW_, VR = SPLIT ? 0 : NR_, VS = SPLIT ? 0 : 1;
  uint32_t w[SPLIT ? NW_ : 2 * NW_];
  uint32_t sc[SPLIT ? 1 : 2];
  u32x4 r[SPLIT ? NR_ : 2 * NR_];
};

// Value of lane l ^ 32 combined with lane l's: both halves of the pair.
__device__ __forceinline__ float half_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int D, bool INT4, int NW, int QB, int TK>
__global__ __launch_bounds__(NW * 64, (QB == 1 && NW == 4) ? (TK == 32 ? 3 : 2) : 1) void prefill_kernel(
    const PrefillParams p) {
  // TK keys per tile = TK/16 chunks of 16 tokens; TK*4 staging tasks of
  // (chunk, token pair, dim slice). With as many threads as tasks a thread
  // stages the K and V parts of its task; with twice as many, the first half
  // of the threads stages K and the second half V.
  constexpr int NCK = TK / 16, NBLK = TK / 32, NTASK = TK * 4;
  static_assert(TK == 32 || TK == 64, "32- or 64-key tiles");
  static_assert(NW * 64 == NTASK || NW * 64 == 2 * NTASK, "one task or half a task per thread");
  constexpr bool SPLIT_KV = NW * 64 == 2 * NTASK;
  // V^T column swizzle granularity: 32-byte blocks for 128-byte rows, 16-byte
  // blocks for 64-byte rows (rows of TK fp16 keys).
  constexpr int SW = TK == 64 ? 32 : 16;
  constexpr int QW = 32 * QB;               // queries per wave
  constexpr int KSTR = D * 2 + 16;          // K row stride in LDS (bytes), padded
  constexpr int VSTR = TK * 2 + 16;  // V^T row stride (bytes), padded
  constexpr int KBUF = TK * KSTR, VBUF = D * VSTR;
  constexpr int NCH = D / 16;               // 16-dim chunks of the QK contraction
  constexpr int NDB = D / 32;               // 32-dim output blocks
  constexpr int DPT = D / 8;                // dims per staging task
  __shared__ __attribute__((aligned(16))) uint8_t lds_k[2 * KBUF];
  __shared__ __attribute__((aligned(16))) uint8_t lds_v[2 * VBUF];
  __shared__ int32_t s_pg[2][NCK];

  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroup -> (query tile, head, batch). Workgroups are dealt to the 8
  // XCDs round-robin by linear id; the remap gives each XCD a contiguous
  // range of (batch, head) so the window of a head is read into one L2, and
  // walks query tiles last-first (the longest causal tiles start first).
  const int32_t nqt = (p.Lq + QW * NW - 1) / (QW * NW);
  int32_t wg = blockIdx.x;
  const int32_t n8 = (int32_t)(gridDim.x & ~7u);
  if (wg < n8) wg = (wg & 7) * (n8 >> 3) + (wg >> 3);
  const int32_t qt = nqt - 1 - wg % nqt;
  const int32_t h = (wg / nqt) % p.H, b = wg / (nqt * p.H);
  const int32_t ctx = p.ctx[b];
  const int32_t kv_lim = min(ctx, p.M * p.bs);
  const int32_t q0 = qt * QW * NW;
  const int32_t qw0 = q0 + QW * wave;
  const bool causal = p.causal != 0;
  const float cs = p.qk_scale_log2;
  // lane column (lane & 31) of query block qb = query qw0 + 32 qb + (lane & 31)
  bool q_ok[QB];
  int32_t qpos[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int32_t qi = qw0 + 32 * qb + (lane & 31);
    q_ok[qb] = qi < p.Lq;
    qpos[qb] = ctx - p.Lq + qi;
  }

  // ---- Q fragments: chunk c, lane half hl -> 8 dims (INT4: unpack order) ----
  half8_t qf[QB][NCH];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int32_t qi = qw0 + 32 * qb + (lane & 31);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      half8_t v = {};
      if (q_ok[qb]) {
        const uint4 u =
            *reinterpret_cast<const uint4 *>(p.q + (((int64_t)b * p.Lq + qi) * p.H + h) * D + 16 * c + 8 * hl);
        const half8_t n = __builtin_bit_cast(half8_t, u);
        if (INT4) {
          v[0] = n[0]; v[1] = n[4]; v[2] = n[1]; v[3] = n[5];
          v[4] = n[2]; v[5] = n[6]; v[6] = n[3]; v[7] = n[7];
        } else {
          v = n;
        }
      }
      qf[qb][c] = v;
    }
  }

  float16_t o[QB][NDB];
  // m: running max of the raw scores q . k, -inf until the first visible
  // key. The S accumulators start from `mtile` = -m (0 while m is -inf), so
  // the MFMA returns score - m directly; exp2 takes cs (score - m) with cs =
  // log2(e) / sqrt(D) applied in fp32 (Q is not pre-scaled: a scaled fp16 Q
  // would carry a 2^-11 relative rounding into every score).
  float m[QB], lsum[QB];
  float16_t mtile[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int i = 0; i < NDB; ++i) o[qb][i] = (float16_t){};
    m[qb] = -INFINITY;
    lsum[qb] = 0.0f;
    mtile[qb] = (float16_t){};
  }

  // ---- key tiles visited by this workgroup: sink tiles, then window tiles ----
  const int32_t qlast = min(q0 + QW * NW, p.Lq) - 1;
  const int32_t pos_lo = ctx - p.Lq + q0, pos_hi = ctx - p.Lq + qlast;
  const int32_t hi = max(0, causal ? min(kv_lim, pos_hi + 1) : kv_lim);
  const int32_t win_lo = max(0, causal ? pos_lo - p.W + 1 : ctx - p.W);
  const int32_t sink_end = min(p.sinks, hi);  // p.sinks >= 0
  const int32_t sink_tiles = (sink_end + TK - 1) / TK;
  const int32_t t_first = max(win_lo / TK, sink_tiles);
  const int32_t t_last = (hi + TK - 1) / TK;  // exclusive
  const int32_t n_tiles = sink_tiles + max(0, t_last - t_first);
  auto tile_base = [&](int32_t it) { return (it < sink_tiles ? it : t_first + (it - sink_tiles)) * TK; };
  // wave-level query span (tile skipping and the unmasked fast path)
  const int32_t wq_last = min(qw0 + QW - 1, p.Lq - 1);
  const int32_t wpos_lo = ctx - p.Lq + qw0, wpos_hi = ctx - p.Lq + wq_last;

  // ---- staging task of this thread ----
  const int task = tid % NTASK;
  const bool do_k = !SPLIT_KV || tid < NTASK, do_v = !SPLIT_KV || tid >= NTASK;  // wave-uniform
  const int sk_k = task >> 6, sk_pp = (task >> 3) & 7, sk_c = task & 7;
  const int sk_R0 = 16 * sk_k + 2 * sk_pp;  // K rows of tokens pp (R0) and pp+8 (R0+1)
  const int sk_vc0 = vt_col(sk_R0);         // V^T column of token pp; pp+8 is +1
  using St = Staged<D, INT4, SPLIT_KV>;
  St st0, st1;  // two tiles in flight between global load and LDS

  // Page of this thread's 16-key chunk in tile `it` (-1: none / unlinked).
  // Looked up one tile before its data is loaded, so the dependent loads
  // never wait on the block-table read.
  auto lookup = [&](int32_t it) __attribute__((always_inline)) {
    int32_t pg = -1;
    if (it < n_tiles) {
      const int32_t key = tile_base(it) + 16 * sk_k;
      if (key < kv_lim) {
        const int32_t e = p.bt[(int64_t)b * p.M + key / p.bs];
        pg = (e >= 0 && e < p.nb) ? e : -1;
      }
    }
    return pg;
  };

  auto issue = [&](int32_t it, int32_t pg, Staged<D, INT4, SPLIT_KV> &st) __attribute__((always_inline)) {
    const int32_t key = tile_base(it) + 16 * sk_k;
    st.pg = pg;
    // Unlinked pages load page 0 (nb > 0) and stage as zeros: INT4 through a
    // zero scale, fp16 through a select.
    const bool ok = pg >= 0;
    const int64_t pgs = ok ? pg : 0;
    // V of tokens at or past the context length stages as zeros (a page's
    // unused tail may hold NaN bits, and P = 0 must not meet them in PV).
    const bool ok0 = ok && key + sk_pp < kv_lim, ok1 = ok && key + sk_pp + 8 < kv_lim;
    if constexpr (INT4) {
      const Int4Page f(D);
      const uint8_t *blk = p.pool + (pgs * p.H + h) * f.block;
      const int slot = 8 * sk_pp + sk_c, g = (sk_c * DPT) / 64;
      if (do_k) {
        if constexpr (DPT / 4 == 4) {
          const u32x4 kk = *reinterpret_cast<const u32x4 *>(blk + f.kcodes + slot * f.BPL);
          st.w[0] = kk.x; st.w[1] = kk.y; st.w[2] = kk.z; st.w[3] = kk.w;
        } else {
          const uint2 kk = *reinterpret_cast<const uint2 *>(blk + f.kcodes + slot * f.BPL);
          st.w[0] = kk.x; st.w[1] = kk.y;
        }
        const uint32_t sk = *reinterpret_cast<const uint32_t *>(blk + f.kscales + 2 * (g * 16 + 2 * sk_pp));
        st.sc[0] = ok ? sk : 0u;
      }
      if (do_v) {
        if constexpr (DPT / 4 == 4) {
          const u32x4 vv = *reinterpret_cast<const u32x4 *>(blk + f.vcodes + slot * f.BPL);
          st.w[St::VO] = vv.x; st.w[St::VO + 1] = vv.y; st.w[St::VO + 2] = vv.z; st.w[St::VO + 3] = vv.w;
        } else {
          const uint2 vv = *reinterpret_cast<const uint2 *>(blk + f.vcodes + slot * f.BPL);
          st.w[St::VO] = vv.x; st.w[St::VO + 1] = vv.y;
        }
        const uint32_t sv = *reinterpret_cast<const uint32_t *>(blk + f.vscales + 2 * (g * 16 + 2 * sk_pp));
        st.sc[St::VS] = (ok0 ? sv & 0xFFFFu : 0u) | (ok1 ? sv & 0xFFFF0000u : 0u);
      }
    } else {
      const half_t *kp = reinterpret_cast<const half_t *>(p.pool);
      const half_t *vp = reinterpret_cast<const half_t *>(p.vpool);
      const int32_t pos0 = (key + sk_pp) % p.bs;  // chunk lies in one page (bs % 16 == 0)
      const int64_t r0 = ((pgs * p.bs + pos0) * p.H + h) * D + sk_c * DPT;
      const int64_t r1 = r0 + 8LL * p.H * D;
      const u32x4 z = {0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < DPT / 8; ++i) {
        if (do_k) {
          const u32x4 k0 = *reinterpret_cast<const u32x4 *>(kp + r0 + 8 * i);
          const u32x4 k1 = *reinterpret_cast<const u32x4 *>(kp + r1 + 8 * i);
          st.r[i] = ok ? k0 : z;
          st.r[DPT / 8 + i] = ok ? k1 : z;
        }
        if (do_v) {
          const u32x4 v0 = *reinterpret_cast<const u32x4 *>(vp + r0 + 8 * i);
          const u32x4 v1 = *reinterpret_cast<const u32x4 *>(vp + r1 + 8 * i);
          st.r[St::VR + i] = ok0 ? v0 : z;
          st.r[St::VR + DPT / 8 + i] = ok1 ? v1 : z;
        }
      }
    }
  };

  auto commit = [&](int buf, const Staged<D, INT4, SPLIT_KV> &st) __attribute__((always_inline)) {
    uint8_t *krow0 = lds_k + buf * KBUF + sk_R0 * KSTR + sk_c * DPT * 2;
    uint8_t *krow1 = krow0 + KSTR;
    uint8_t *vbase = lds_v + buf * VBUF + sk_c * DPT * VSTR + vt_swz<SW>(2 * sk_vc0, sk_c * DPT);
    if (lane == 0 && do_k) s_pg[buf][sk_k] = st.pg;
    if constexpr (INT4) {
      const half2_t sk = as_half2(st.sc[0]), sv = as_half2(st.sc[St::VS]);
      const half2_t b1032 = {(half_t)1032.0f, (half_t)1032.0f};
      const half2_t b72 = {(half_t)72.0f, (half_t)72.0f};
#pragma unroll
      for (int t2 = 0; t2 < 2 && do_k; ++t2) {
        const half2_t s2 = t2 ? half2_t{sk.y, sk.y} : half2_t{sk.x, sk.x};
        uint8_t *dst = t2 ? krow1 : krow0;
#pragma unroll
        for (int wi = 0; wi < DPT / 8; ++wi) {
          const uint32_t w = st.w[t2 * (DPT / 8) + wi], w8 = w >> 8;
          const half2_t h0 = (as_half2(bfi(0x000F000Fu, w, 0x64006400u)) - b1032) * s2;
          const half2_t h1 = (as_half2(bfi(0x00F000F0u, w, 0x54005400u)) - b72) * s2;
          const half2_t h2 = (as_half2(bfi(0x000F000Fu, w8, 0x64006400u)) - b1032) * s2;
          const half2_t h3 = (as_half2(bfi(0x00F000F0u, w8, 0x54005400u)) - b72) * s2;
          *reinterpret_cast<uint4 *>(dst + 16 * wi) = make_uint4(as_u32(h0), as_u32(h1), as_u32(h2), as_u32(h3));
        }
      }
#pragma unroll
      for (int wi = 0; wi < DPT / 4 && do_v; ++wi) {
        const uint32_t w = st.w[St::VO + wi], w8 = w >> 8;
        const half2_t h0 = (as_half2(bfi(0x000F000Fu, w, 0x64006400u)) - b1032) * sv;
        const half2_t h1 = (as_half2(bfi(0x00F000F0u, w, 0x54005400u)) - b72) * sv;
        const half2_t h2 = (as_half2(bfi(0x000F000Fu, w8, 0x64006400u)) - b1032) * sv;
        const half2_t h3 = (as_half2(bfi(0x00F000F0u, w8, 0x54005400u)) - b72) * sv;
        uint8_t *vd = vbase + 4 * wi * VSTR;
        *reinterpret_cast<uint32_t *>(vd) = as_u32(h0);
        *reinterpret_cast<uint32_t *>(vd + VSTR) = as_u32(h1);
        *reinterpret_cast<uint32_t *>(vd + 2 * VSTR) = as_u32(h2);
        *reinterpret_cast<uint32_t *>(vd + 3 * VSTR) = as_u32(h3);
      }
    } else {
#pragma unroll
      for (int i = 0; i < DPT / 8; ++i) {
        if (do_k) {
          *reinterpret_cast<u32x4 *>(krow0 + 16 * i) = st.r[i];
          *reinterpret_cast<u32x4 *>(krow1 + 16 * i) = st.r[DPT / 8 + i];
        }
        if (!do_v) continue;
        const half8_t a = __builtin_bit_cast(half8_t, st.r[St::VR + i]);
        const half8_t c = __builtin_bit_cast(half8_t, st.r[St::VR + DPT / 8 + i]);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          *reinterpret_cast<uint32_t *>(vbase + (8 * i + e) * VSTR) = as_u32(half2_t{a[e], c[e]});
      }
    }
  };

  // Tiles 0, 2, 4, ... are loaded through st0 and tiles 1, 3, ... through
  // st1; loads run two tiles ahead of the LDS write, the page lookup three.
  if (n_tiles > 0) {
    issue(0, lookup(0), st0);
    commit(0, st0);
    if (n_tiles > 1) issue(1, lookup(1), st1);
    if (n_tiles > 2) issue(2, lookup(2), st0);
  }
  int32_t pg_next = lookup(3);
  __syncthreads();

  // Per-lane V^T read addresses of the 16-key chunks, swizzle included; in
  // odd 32-dim blocks the swizzle also flips chunk bit log2(SW / 16).
  int32_t va[NCK];
#pragma unroll
  for (int kc = 0; kc < NCK; ++kc)
    va[kc] = (lane & 31) * VSTR + vt_swz<SW>(32 * kc + 16 * hl, lane & 31);
  const int32_t ka = (lane & 31) * KSTR + 16 * hl;

  const half2_t ones = {(half_t)1.0f, (half_t)1.0f};
  // One tile: compute on LDS buffer it & 1 while staging tile it + 1 from
  // `sx` into the other buffer and loading tile it + 3 into `sx`.
  auto step = [&](int32_t it, Staged<D, INT4, SPLIT_KV> &sx) __attribute__((always_inline)) {
    const int buf = it & 1;
    const int32_t tb = tile_base(it);
    const uint8_t *kt = lds_k + buf * KBUF;
    const uint8_t *vt = lds_v + buf * VBUF;
    const bool is_sink_tile = tb < sink_end;
    bool any_vis = qw0 < p.Lq;
    if (causal)
      any_vis = any_vis && tb <= wpos_hi && (is_sink_tile || tb + TK - 1 >= wpos_lo - p.W + 1);
    int32_t pgs[NCK], pg_all = 0;
#pragma unroll
    for (int k = 0; k < NCK; ++k) {
      pgs[k] = s_pg[buf][k];
      pg_all |= pgs[k];
    }
    const bool full = pg_all >= 0 && tb + TK <= kv_lim &&
                      (causal ? (tb + TK - 1 <= wpos_lo && tb >= wpos_hi - p.W + 1) : (tb >= ctx - p.W)) &&
                      wq_last == qw0 + QW - 1;

    // S^T of one 32-key block (32 keys x 32 queries per query block; every K
    // fragment feeds all QB query blocks).
    auto qk = [&](int blk, float16_t (&sq)[QB]) __attribute__((always_inline)) {
      if constexpr (INT4) {  // all K-fragment reads first, then the MFMA chain
        half8_t a[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) a[c] = *reinterpret_cast<const half8_t *>(kt + 32 * blk * KSTR + ka + 32 * c);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
#pragma unroll
          for (int qb = 0; qb < QB; ++qb)
            sq[qb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[c], qf[qb][c], c == 0 ? mtile[qb] : sq[qb], 0, 0, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, NCH, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, NCH * QB, 0);
      } else {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          const half8_t a = *reinterpret_cast<const half8_t *>(kt + 32 * blk * KSTR + ka + 32 * c);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb)
            sq[qb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[qb][c], c == 0 ? mtile[qb] : sq[qb], 0, 0, 0);
        }
      }
    };
    // Masks, raises the running max lazily, and packs the probabilities of
    // one block to fp16 in PV operand order.
    auto softmax = [&](int blk, float16_t (&sq)[QB], half8_t (&pb)[QB][2]) __attribute__((always_inline)) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float16_t &s = sq[qb];
        if (!full) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int R = 32 * blk + 8 * (r >> 2) + 4 * hl + (r & 3);
            const int32_t key = tb + row_key(R);
            const bool ok = q_ok[qb] && pgs[2 * blk + (r >> 3)] >= 0 && key < kv_lim &&
                            key_visible(key, qpos[qb], ctx, p.W, p.sinks, causal);
            s[r] = ok ? s[r] : -INFINITY;
          }
        }
        float tmax = s[0];  // relative to m (absolute while m is -inf)
#pragma unroll
        for (int r = 1; r < 16; ++r) tmax = fmaxf(tmax, s[r]);
        tmax = half_max(tmax);
        // lazy rescale: p stays <= 2^8 between raises; the first visible key
        // always raises
        const bool raise = (m[qb] == -INFINITY) ? (tmax != -INFINITY) : (tmax * cs > 8.0f);
        if (__any(raise)) {
          const float base = (m[qb] == -INFINITY) ? 0.0f : m[qb];
          const float mn = fmaxf(m[qb], base + tmax);
          const float alpha = (mn == m[qb]) ? 1.0f : fast_exp2((m[qb] - mn) * cs);
          const float delta = (mn == -INFINITY) ? 0.0f : mn - base;
          lsum[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[qb][db][r] *= alpha;
#pragma unroll
          for (int r = 0; r < 16; ++r) s[r] -= delta;
          m[qb] = mn;
          const float nb = (mn == -INFINITY) ? 0.0f : -mn;
#pragma unroll
          for (int r = 0; r < 16; ++r) mtile[qb][r] = nb;
        }
#pragma unroll
        for (int g2 = 0; g2 < 2; ++g2) {
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            const half2_t pp2 = {(half_t)fast_exp2(s[8 * g2 + e] * cs), (half_t)fast_exp2(s[8 * g2 + e + 1] * cs)};
            lsum[qb] = __builtin_amdgcn_fdot2(pp2, ones, lsum[qb], false);
            pb[qb][g2][e] = pp2.x;
            pb[qb][g2][e + 1] = pp2.y;
          }
        }
      }
    };
    // O^T += V^T P^T over one block's two 16-key chunks
    auto pv = [&](int blk, half8_t (&pb)[QB][2]) __attribute__((always_inline)) {
      if constexpr (INT4) {
        // all V^T-fragment reads first, then the MFMAs (the fp16 path has no
        // registers to spare for this)
        half8_t a[NDB][2];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int g2 = 0; g2 < 2; ++g2) {
            const int kc = (2 * blk + g2) ^ ((SW / 16) * (db & 1));
            a[db][g2] = *reinterpret_cast<const half8_t *>(vt + 32 * db * VSTR + va[kc]);
          }
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int g2 = 0; g2 < 2; ++g2)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
              o[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[db][g2], pb[qb][g2], o[qb][db], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * NDB, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * NDB * QB, 0);
      } else {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
#pragma unroll
          for (int g2 = 0; g2 < 2; ++g2) {
            const int kc = (2 * blk + g2) ^ ((SW / 16) * (db & 1));
            const half8_t a = *reinterpret_cast<const half8_t *>(vt + 32 * db * VSTR + va[kc]);
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
              o[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[qb][g2], o[qb][db], 0, 0, 0);
          }
        }
      }
    };

    // Order: S(0) | staging of the next tile | softmax(0) | S(1) | PV(0) |
    // softmax(1) | PV(1): the staging VALU runs under S(0), softmax(1)
    // under PV(0). 32-key tiles have block 0 only.
    float16_t sa[QB], sc[QB];
    half8_t pa[QB][2], pc[QB][2];
    if (any_vis) qk(0, sa);
    if (it + 1 < n_tiles) commit(buf ^ 1, sx);
    if (it + 3 < n_tiles) issue(it + 3, pg_next, sx);
    pg_next = lookup(it + 4);
    if (any_vis) {
      softmax(0, sa, pa);
      if constexpr (NBLK == 2) qk(1, sc);
      pv(0, pa);
      if constexpr (NBLK == 2) {
        softmax(1, sc, pc);
        pv(1, pc);
      }
    }
    __syncthreads();
  };
  for (int32_t it = 0; it < n_tiles; it += 2) {  // unrolled by two: static register sets
    step(it, st1);
    if (it + 1 < n_tiles) step(it + 1, st0);
  }

#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float l = half_sum(lsum[qb]);
    if (!q_ok[qb]) continue;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const int32_t qi = qw0 + 32 * qb + (lane & 31);
    half_t *orow = p.out + (((int64_t)b * p.Lq + qi) * p.H + h) * D;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * db + 8 * g + 4 * hl;
        const half2_t x = {(half_t)(o[qb][db][4 * g] * inv), (half_t)(o[qb][db][4 * g + 1] * inv)};
        const half2_t y = {(half_t)(o[qb][db][4 * g + 2] * inv), (half_t)(o[qb][db][4 * g + 3] * inv)};
        *reinterpret_cast<uint2 *>(orow + d0) = make_uint2(as_u32(x), as_u32(y));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Staged variant: a pre-pass writes every 16-token chunk a call can touch in
// the exact LDS operand layout (K rows in page pair order with dims in unpack
// order, V^T columns in PV operand order), so the attention kernel fills LDS
// with global_load_lds (16 bytes per lane, no VGPRs, no VALU) and spends its
// VALU on the softmax only.
// ---------------------------------------------------------------------------

// Column of token p (p = 0..7) inside a 16-token chunk of V^T; token p + 8 is
// the next column (vt_col of K-tile row 2p).
__device__ __forceinline__ int chunk_vcol(int p) { return 8 * ((p >> 1) & 1) + 4 * (p >> 2) + 2 * (p & 1); }

// Workspace block of one (sequence, head, staged chunk): 2*16*D fp16 =
// K part [16 rows][D] then V^T part [D rows][16 columns]. Blocks are ordered
// [sequence][head][slot], so the chunks of one (sequence, head) are one
// contiguous run. After all blocks comes one int32 per (sequence, slot): 1
// if its page is linked.
//
// Only the chunks some query tile of a sequence visits are staged: the sink
// tiles [0, sc) and the window tiles [lo, hi) (64-key aligned). Chunk lc sits
// in slot lc < sc ? lc : lc - off, off = max(0, lo - sc), so a sequence uses
// hi - off slots: about (q_len + W) / 16 for causal calls, however long the
// context is.
struct StageMap {
  int32_t sc, off, hi;  // sink chunks, slot offset of the window chunks, end chunk
  __host__ __device__ int32_t slot(int32_t lc) const { return lc < sc ? lc : lc - off; }
};

__host__ __device__ inline StageMap stage_map(int32_t ctx, int32_t max_tokens, int32_t Lq, int32_t W, int32_t sinks,
                                              bool causal) {
  const int32_t kv_lim = ctx < max_tokens ? ctx : max_tokens;
  int32_t win_lo = causal ? ctx - Lq - W + 1 : ctx - W;
  win_lo = win_lo > 0 ? win_lo : 0;
  const int32_t s = sinks < kv_lim ? sinks : kv_lim;
  StageMap m;
  m.sc = 4 * (((s > 0 ? s : 0) + 63) / 64);
  m.hi = kv_lim > 0 ? 4 * ((kv_lim + 63) / 64) : 0;
  const int32_t lo = 4 * (win_lo / 64);
  m.off = lo > m.sc ? lo - m.sc : 0;
  return m;
}

template <int D>
struct StageLayout {
  static constexpr int64_t kBlock = 2 * 16 * D * 2;  // bytes
  static constexpr int64_t kVPart = 16 * D * 2;      // byte offset of V^T in a block
};

// Stages the workspace blocks of slots slot0 + i * sstride, i < n <= N, of
// (sequence, head) bh with one wave: the blocks' page lookups, then every
// block's page loads, are issued before anything waits for them, so the N
// blocks cost one chain of memory round trips. Block = bh * MC + slot;
// lane l = 8p + c owns tokens (p, p + 8) x dims [c*D/8, (c+1)*D/8), as in
// the INT4 page format. vl: the wave's 32 * D + (D / 16) * PADG bytes of
// LDS (the V^T transpose; each 16-row group PADG bytes further on, so the
// 8 lanes writing one row offset of 8 groups hit different banks).
// all_flags: write each slot's link flag from every head (else head 0's
// wave writes it).
template <int D, bool INT4, int N, int PADG = 0>
__device__ __forceinline__ void stage_blocks(const PrefillParams &p, uint8_t *__restrict__ ws, int32_t MC,
                                             int32_t units, int32_t bh, int32_t slot0, int32_t sstride, int32_t n,
                                             uint8_t *vl, bool all_flags) {
  constexpr int DPL = D / 8;
  using L = StageLayout<D>;
  const int lane = threadIdx.x & 63;
  const int pp = lane >> 3, c = lane & 7;
  bh = __builtin_amdgcn_readfirstlane(bh);
  slot0 = __builtin_amdgcn_readfirstlane(slot0);
  const int32_t b = bh / p.H, h = bh % p.H;
  const int32_t ctx = __builtin_amdgcn_readfirstlane(p.ctx[b]);
  const int32_t kvl = min(ctx, p.M * p.bs);
  const StageMap sm = stage_map(ctx, p.M * p.bs, p.Lq, p.W, p.sinks, p.causal != 0);
  int32_t key0[N], pg[N], slot[N];
  bool live[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    slot[i] = slot0 + i * sstride;
    live[i] = i < n && slot[i] < sm.hi - sm.off;  // wave-uniform: a slot past the map holds no chunk
    const int32_t lc = slot[i] < sm.sc ? slot[i] : slot[i] + sm.off;
    key0[i] = lc * 16;
    const bool in = live[i] && key0[i] < kvl;
    const int32_t e = p.bt[(int64_t)b * p.M + (in ? key0[i] / p.bs : 0)];  // loaded unconditionally
    pg[i] = (in && e >= 0 && e < p.nb) ? e : -1;
  }
  // raw page words (INT4): K codes of tokens pp, pp + 8, V codes, the scale pairs
  uint32_t kraw[INT4 ? N : 1][DPL / 4], vraw[INT4 ? N : 1][DPL / 4], skr[N], svr[N];
  if constexpr (INT4) {
    // (unconditional loads: a block with no page reads page 0, which is
    // mapped, and its values are not used)
    const Int4Page f(D);
    const int sl = 8 * pp + c, g = (c * DPL) / 64;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const uint8_t *src = p.pool + ((int64_t)(pg[i] >= 0 ? pg[i] : 0) * p.H + h) * f.block;
      const uint32_t *kc32 = reinterpret_cast<const uint32_t *>(src + f.kcodes + sl * f.BPL);
      const uint32_t *vc32 = reinterpret_cast<const uint32_t *>(src + f.vcodes + sl * f.BPL);
#pragma unroll
      for (int w = 0; w < DPL / 4; ++w) {
        kraw[i][w] = kc32[w];
        vraw[i][w] = vc32[w];
      }
      skr[i] = *reinterpret_cast<const uint32_t *>(src + f.kscales + 2 * (g * 16 + 2 * pp));
      svr[i] = *reinterpret_cast<const uint32_t *>(src + f.vscales + 2 * (g * 16 + 2 * pp));
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (!live[i]) continue;  // wave-uniform
    uint8_t *blk = ws + ((int64_t)bh * MC + slot[i]) * L::kBlock;
    uint32_t kw0[DPL / 2], kw1[DPL / 2];  // K halves of tokens pp, pp + 8 (unpack order), as packed pairs
    uint32_t vw[DPL];                     // V: dim d -> {token pp, token pp + 8}
    if (pg[i] < 0) {
#pragma unroll
      for (int k = 0; k < DPL / 2; ++k) kw0[k] = kw1[k] = 0;
#pragma unroll
      for (int k = 0; k < DPL; ++k) vw[k] = 0;
    } else if constexpr (INT4) {
      const half2_t sk = as_half2(skr[i]), sv = as_half2(svr[i]);
      const half2_t b1032 = {(half_t)1032.0f, (half_t)1032.0f}, b72 = {(half_t)72.0f, (half_t)72.0f};
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        const half2_t s2 = t2 ? half2_t{sk.y, sk.y} : half2_t{sk.x, sk.x};
        uint32_t *dst = t2 ? kw1 : kw0;
#pragma unroll
        for (int wi = 0; wi < DPL / 8; ++wi) {
          const uint32_t w = kraw[i][t2 * (DPL / 8) + wi], w8 = w >> 8;
          dst[4 * wi + 0] = as_u32((as_half2(bfi(0x000F000Fu, w, 0x64006400u)) - b1032) * s2);
          dst[4 * wi + 1] = as_u32((as_half2(bfi(0x00F000F0u, w, 0x54005400u)) - b72) * s2);
          dst[4 * wi + 2] = as_u32((as_half2(bfi(0x000F000Fu, w8, 0x64006400u)) - b1032) * s2);
          dst[4 * wi + 3] = as_u32((as_half2(bfi(0x00F000F0u, w8, 0x54005400u)) - b72) * s2);
        }
      }
#pragma unroll
      for (int wi = 0; wi < DPL / 4; ++wi) {
        const uint32_t w = vraw[i][wi], w8 = w >> 8;
        vw[4 * wi + 0] = as_u32((as_half2(bfi(0x000F000Fu, w, 0x64006400u)) - b1032) * sv);
        vw[4 * wi + 1] = as_u32((as_half2(bfi(0x00F000F0u, w, 0x54005400u)) - b72) * sv);
        vw[4 * wi + 2] = as_u32((as_half2(bfi(0x000F000Fu, w8, 0x64006400u)) - b1032) * sv);
        vw[4 * wi + 3] = as_u32((as_half2(bfi(0x00F000F0u, w8, 0x54005400u)) - b72) * sv);
      }
    } else {
      const half_t *kp = reinterpret_cast<const half_t *>(p.pool);
      const half_t *vp = reinterpret_cast<const half_t *>(p.vpool);
      const int32_t pos0 = key0[i] % p.bs;  // a 16-token chunk lies in one page (bs % 16 == 0)
      const int64_t r0 = (((int64_t)pg[i] * p.bs + pos0 + pp) * p.H + h) * D + c * DPL;
      const int64_t r1 = r0 + 8LL * p.H * D;
#pragma unroll
      for (int k = 0; k < DPL / 8; ++k) {
        const half8_t k0 = __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4 *>(kp + r0 + 8 * k));
        const half8_t k1 = __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4 *>(kp + r1 + 8 * k));
        const half8_t v0 = __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4 *>(vp + r0 + 8 * k));
        const half8_t v1 = __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4 *>(vp + r1 + 8 * k));
        // K in unpack order (0,4,1,5,2,6,3,7) within each 8-dim group
        kw0[4 * k + 0] = as_u32(half2_t{k0[0], k0[4]}); kw0[4 * k + 1] = as_u32(half2_t{k0[1], k0[5]});
        kw0[4 * k + 2] = as_u32(half2_t{k0[2], k0[6]}); kw0[4 * k + 3] = as_u32(half2_t{k0[3], k0[7]});
        kw1[4 * k + 0] = as_u32(half2_t{k1[0], k1[4]}); kw1[4 * k + 1] = as_u32(half2_t{k1[1], k1[5]});
        kw1[4 * k + 2] = as_u32(half2_t{k1[2], k1[6]}); kw1[4 * k + 3] = as_u32(half2_t{k1[3], k1[7]});
#pragma unroll
        for (int e = 0; e < 8; ++e) vw[8 * k + e] = as_u32(half2_t{v0[e], v1[e]});
      }
    }
    // Tokens at or past the context length stage as zeros: a page's unused
    // tail may hold any bits (NaN included), and P = 0 must not meet them in PV.
    if (key0[i] + pp >= kvl) {
#pragma unroll
      for (int k = 0; k < DPL / 2; ++k) kw0[k] = 0;
#pragma unroll
      for (int k = 0; k < DPL; ++k) vw[k] &= 0xFFFF0000u;
    }
    if (key0[i] + pp + 8 >= kvl) {
#pragma unroll
      for (int k = 0; k < DPL / 2; ++k) kw1[k] = 0;
#pragma unroll
      for (int k = 0; k < DPL; ++k) vw[k] &= 0x0000FFFFu;
    }
    // V dims come out of the INT4 unpack in order d, d+1, d+2, d+3 per word;
    // K words are already in unpack order for both sources.
    uint8_t *krow0 = blk + (2 * pp) * (2 * D) + c * DPL * 2;
#pragma unroll
    for (int k = 0; k < DPL / 8; ++k) {
      *reinterpret_cast<u32x4 *>(krow0 + 16 * k) = u32x4{kw0[4 * k], kw0[4 * k + 1], kw0[4 * k + 2], kw0[4 * k + 3]};
      *reinterpret_cast<u32x4 *>(krow0 + 2 * D + 16 * k) =
          u32x4{kw1[4 * k], kw1[4 * k + 1], kw1[4 * k + 2], kw1[4 * k + 3]};
    }
    // V^T goes through LDS: the 4-byte pieces of a lane (two tokens of one
    // dim) land in the block's layout there, and the wave then writes the
    // block as contiguous 16-byte stores; written directly, the scattered
    // 4-byte stores cost twice the K stores for the same bytes.
    const int vc = chunk_vcol(pp);
#pragma unroll
    for (int d = 0; d < DPL; ++d)
      *reinterpret_cast<uint32_t *>(vl + (c * DPL + d) * 32 + ((c * DPL + d) >> 4) * PADG + vc * 2) = vw[d];
    // One wave's LDS accesses complete in order; the clobber keeps the
    // compiler from moving the reads above the writes.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int k = 0; k < 32 * D / 1024; ++k)
      *reinterpret_cast<u32x4 *>(blk + L::kVPart + k * 1024 + lane * 16) =
          *reinterpret_cast<const u32x4 *>(vl + k * 1024 + lane * 16 + ((k * 1024 + lane * 16) >> 9) * PADG);
    if ((all_flags || h == 0) && lane == 0)
      reinterpret_cast<int32_t *>(ws + (int64_t)units * L::kBlock)[(int64_t)b * MC + slot[i]] = pg[i] >= 0 ? 1 : 0;
    // The LDS reads above are complete before the next block (or the
    // caller) reuses vl.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

// Four consecutive workspace blocks per wave: block q * MC + slot, q <
// nblocks / MC, of (sequence, head) q * ustride (ustride 1: every block of
// the workspace,
// head 0's writing the link flags; otherwise every head writes them, as
// the staged units need not include head 0 of each sequence). The launch
// also clears the call's `nflags` in-kernel staging flags: the attention
// pass after it compares them with the call's tag, and a stale word equal to
// that tag would let a workgroup read blocks before they are staged.
template <int D, bool INT4>
__global__ __launch_bounds__(256) void prefill_stage_kernel(const PrefillParams p, uint8_t *__restrict__ ws,
                                                            int32_t MC, int32_t units, int32_t ustride,
                                                            int32_t nblocks, uint32_t *__restrict__ flags,
                                                            int32_t nflags) {
  for (int32_t i = blockIdx.x * 256 + threadIdx.x; i < nflags; i += gridDim.x * 256) flags[i] = 0u;
  const int32_t idx = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 4;  // 4 consecutive slots per wave (MC % 4 == 0)
  if (idx >= nblocks) return;  // wave-uniform
  __shared__ __attribute__((aligned(16))) uint8_t vt_lds[4][32 * D];
  stage_blocks<D, INT4, 4>(p, ws, MC, units, (idx / MC) * ustride, idx % MC, 1, min(4, nblocks - idx),
                           vt_lds[threadIdx.x >> 6], ustride != 1);
}

template <int N>
struct IntC {
  static constexpr int value = N;
};

// Scheduling group: `n` instructions of class `mask` (0x002 VALU, 0x008
// MFMA, 0x100 LDS read, 0x400 transcendental) in this position of the order.
#define PIPE_SGB(mask, n, id) __builtin_amdgcn_sched_group_barrier(mask, n, id)

// LDS-DMA copy (buffer_load ... lds): lane i's 16 bytes at buffer offset
// voff + soff land at LDS byte m0v + 16 i. Written as inline assembly so the
// compiler does not track it: with the builtin, its wait-count pass cannot
// tell the LDS buffers apart (it waits for the next tiles' copies before
// operand reads of the current one) and the barrier's release fence turns
// the counted wait below into vmcnt(0). Callers wait for completion
// themselves (s_waitcnt vmcnt before the barrier that publishes a tile).
// m0 is an input operand ("{m0}"), so the compiler sets it and knows it is
// read; nothing is clobbered behind its back. The s_nop is the one wait
// state the hardware needs between an SALU write of m0 and an LDS DMA that
// reads it.
//
// lds_dma<C0, N> issues copies C0 .. C0 + N - 1 (N = 1 or 2) of one group
// that shares m0 and the scalar offset: copy c carries the immediate offset
// c * 1024, which the hardware adds to both the global and the LDS address
// (measured on MI355X), and the lane offset vo[c] holds the rest of its
// global address minus that immediate. So a group of copies needs one m0
// write and one wait state instead of one of each per copy.
template <int C0, int N>
__device__ __forceinline__ void lds_dma(__amdgpu_buffer_rsrc_t r, uint32_t m0v, const uint32_t *vo, uint32_t soff) {
  static_assert(N == 1 || N == 2, "one or two copies per group");
  static_assert((C0 + N) * 1024 <= 4096, "immediate offsets are 12 bits");
  if constexpr (N == 1) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen offset:%4 lds"
                 :
                 : "v"(vo[C0]), "s"(r), "s"(soff), "{m0}"(m0v), "i"(C0 * 1024)
                 : "memory");
  } else {
    asm volatile(
        "s_nop 0\n\tbuffer_load_dwordx4 %0, %2, %3 offen offset:%5 lds\n\t"
        "buffer_load_dwordx4 %1, %2, %3 offen offset:%6 lds"
        :
        : "v"(vo[C0]), "v"(vo[C0 + 1]), "s"(r), "s"(soff), "{m0}"(m0v), "i"(C0 * 1024), "i"(C0 * 1024 + 1024)
        : "memory");
  }
}

// Copies [C0, C1) of a group, two per m0 write.
template <int C0, int C1>
__device__ __forceinline__ void lds_dma_range(__amdgpu_buffer_rsrc_t r, uint32_t m0v, const uint32_t *vo,
                                              uint32_t soff) {
  if constexpr (C1 - C0 == 1) {
    lds_dma<C0, 1>(r, m0v, vo, soff);
  } else if constexpr (C1 - C0 >= 2) {
    lds_dma<C0, 2>(r, m0v, vo, soff);
    lds_dma_range<C0 + 2, C1>(r, m0v, vo, soff);
  }
}

// ds_read_b128 at LDS byte address a.
__device__ __forceinline__ half8_t lds_read16(uint32_t a) {
  return *(const __attribute__((address_space(3))) half8_t *)(uintptr_t)a;
}

__device__ __forceinline__ uint32_t lds_u32(const void *p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p);
}

// Attention over staged chunks, software-pipelined inside each wave.
//  * A workgroup of 4 waves owns 128 queries of one (batch, head); wave w
//    owns 32 of them, one query per lane column (lanes l and l+32 share
//    query l % 32). Q is held in registers as given (unscaled fp16).
//  * Keys advance in 64-key tiles (four staged 16-token chunks). Tiles are
//    copied from the workspace into LDS with buffer-to-LDS DMA: unpadded
//    rows whose 16-byte chunks are XOR-swizzled (K: chunk ^ (row & 15) for
//    256-byte rows, chunk ^ ((row >> 1) & 7) for 128-byte rows; V^T: chunk ^
//    ((row >> 1) & 7)), which keeps the MFMA operand reads conflict-free.
//  * S^T = K Q^T and O^T += V^T P^T run on v_mfma_f32_32x32x16_f16. The S^T
//    accumulator layout is the PV B-operand layout (the staged V^T columns
//    are in that key order), so probabilities go from exp2 straight into
//    the PV MFMAs. The S chains start from zero; the running max enters
//    each exp2 argument as one fma, cs s - cs m.
//  * Iteration i holds S(i) (computed by iteration i - 1) and interleaves
//      QK(i+1) block 0 MFMAs  with the running max of S(i),
//      QK(i+1) block 1 MFMAs  with exp2 / packing of S(i) block 0,
//      PV(i) block 0 MFMAs    with exp2 / packing of S(i) block 1,
//      PV(i) block 1 MFMAs,
//    so the matrix pipe has independent work while the softmax runs.
//  * K tiles are copied two tiles ahead and V tiles one tile ahead, two LDS
//    buffers each; iteration i reads K(i+1) and V(i) and refills the
//    buffers of K(i) and V(i-1), both last read in iteration i-1.
//  * A wave computes only the tiles holding keys its own queries see; it
//    still issues its share of every tile's copies and meets the barriers.
//  * Workgroup IDs are remapped so that each XCD owns whole heads (a head's
//    window stays in one L2), longest causal query tiles first.
//  * STAGE: the workspace is staged by this kernel instead of a staging
//    launch before it (StageSched), except for the first (sequence, head)
//    unit of each XCD, which a staging launch of those units only stages:
//    each XCD runs whole units one after another, and the first S
//    workgroups of a unit stage 1/S of the next unit's blocks at their
//    start, so the staging rides on memory bandwidth the MFMA-bound pass
//    leaves idle.
struct StageSched {
  uint32_t *flags;  // [sequence * H + head][64]: the call's tag once stager j's blocks are stored
  uint32_t tag;     // this call's id (nonzero)
  int32_t S;        // stagers per unit (<= 64)
  int32_t spin;     // wait bound (polls); past it a workgroup stages its unit itself (< 0: always)
};

template <int D, int NW, bool STAGE, bool INT4>
__global__ __launch_bounds__(NW * 64, NW == 4 ? 2 : 1) void prefill_pipe_kernel(const PrefillParams p,
                                                                                uint8_t *__restrict__ ws,
                                                                                int32_t MC, int32_t units,
                                                                                const StageSched ss) {
  constexpr int TK = 64, NT = NW * 64;
  constexpr int KRB = 2 * D, KC = KRB / 16, VRB = TK * 2;
  constexpr int KBUF = TK * KRB, VBUF = D * VRB;
  constexpr int NCH = D / 16, NDB = D / 32;
  constexpr int NKL = KBUF / (NT * 16), NVL = VBUF / (NT * 16);  // 16-byte copies per thread per tile
  using L = StageLayout<D>;
  constexpr uint32_t CS = (uint32_t)L::kBlock;  // bytes per staged chunk
  // Two K buffers and two V buffers: 128 KiB for the two workgroups of a CU at D = 128.
  __shared__ __attribute__((aligned(16))) uint8_t lds_k0[KBUF], lds_k1[KBUF];
  __shared__ __attribute__((aligned(16))) uint8_t lds_v0[VBUF], lds_v1[VBUF];

  auto kswz = [](int R) { return KC == 16 ? (R & 15) : ((R >> 1) & 7); };

  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int32_t nqt = (p.Lq + 32 * NW - 1) / (32 * NW);
  int32_t wg = blockIdx.x;
  const int32_t n8 = (int32_t)(gridDim.x & ~7u);
  if (wg < n8) wg = (wg & 7) * (n8 >> 3) + (wg >> 3);
  const int32_t qt = nqt - 1 - wg % nqt;
  const int32_t h = (wg / nqt) % p.H, b = wg / (nqt * p.H);
  uint32_t stage_flag = 0;
  bool stage_wait = false;
  int32_t stage_unit = 0;
  if constexpr (STAGE) {
    // Position on this XCD: unit k of its sequence of units, workgroup j of
    // that unit (the host launches this form only when every XCD owns whole
    // units: gridDim.x % 8 == 0 and (gridDim.x / 8) % nqt == 0). A stager
    // and the workgroups reading what it staged run on one XCD and share its
    // L2: the GPU places workgroup i on XCD i % (XCDs in the partition), and
    // every MI355X partition has 8, 4, 2 or 1 XCDs, so workgroups with equal
    // i % 8 share an XCD.
    const int32_t P = (int32_t)(gridDim.x >> 3), i = wg % P, k = i / nqt, j = i % nqt, U = wg / nqt;
    // (LDS scratch of the V^T transposes, free until the first tile copy)
    uint8_t *vl = (wave < 2 ? lds_k0 : lds_k1) + (wave & 1) * (32 * D + (D / 16) * 16);
    // Share j of S of unit u, slots [s0, s1): wave w takes s0 + w, s0 + w +
    // NW, ..., eight blocks per stage_blocks call (INT4; one for fp16
    // pools). Then the
    // workgroup's flag for unit u, flags[u * 64 + j] = tag, once its stores
    // are complete.
    auto stage_share = [&](int32_t u, int32_t S) {
      const int32_t s0 = (int32_t)((int64_t)j * MC / S), s1 = (int32_t)((int64_t)(j + 1) * MC / S);
      constexpr int NB = INT4 ? 8 : 1;
      for (int32_t sl = s0 + wave; sl < s1; sl += NB * NW)
        stage_blocks<D, INT4, NB, 16>(p, ws, MC, units, u, sl, NW, min(NB, (s1 - sl + NW - 1) / NW), vl, true);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's stores are complete
      __syncthreads();
      if (threadIdx.x == 0)
        __hip_atomic_store(ss.flags + (int64_t)u * 64 + j, ss.tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    if (k + 1 < P / nqt && j < ss.S) stage_share(U + 1, ss.S);
    // The first poll of this unit's stagers' flags (wave 0, lane l < S polls
    // stager l) is issued now and checked before the first read of the
    // workspace, so its round trip overlaps the setup below. The XCD's
    // first unit was staged by the launch before this one.
    if (k > 0 && wave == 0)
      stage_flag = lane < ss.S ? __hip_atomic_load(ss.flags + (int64_t)U * 64 + lane, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT)
                               : ss.tag;
    stage_wait = k > 0;
    stage_unit = U;
  }
  const int32_t ctx = p.ctx[b];
  const int32_t kv_lim = min(ctx, p.M * p.bs);
  const int32_t q0 = qt * 32 * NW;
  const int32_t qw0 = q0 + 32 * wave;
  const bool causal = p.causal != 0;
  const float cs = p.qk_scale_log2;
  const int32_t qi = qw0 + (lane & 31);
  const bool q_ok = qi < p.Lq;
  const int32_t qpos = ctx - p.Lq + qi;

  half8_t qf[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    half8_t v = {};
    if (q_ok) {
      const half8_t n = __builtin_bit_cast(
          half8_t, *reinterpret_cast<const uint4 *>(p.q + (((int64_t)b * p.Lq + qi) * p.H + h) * D + 16 * c + 8 * hl));
      v[0] = n[0]; v[1] = n[4]; v[2] = n[1]; v[3] = n[5];
      v[4] = n[2]; v[5] = n[6]; v[6] = n[3]; v[7] = n[7];
    }
    qf[c] = v;
  }
  float16_t o[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) o[i] = (float16_t){};
  // Row sums of the probabilities, one per 32-key block: two independent
  // chains of 8 dependent v_dot2 per tile instead of one chain of 16.
  // The QK chains start from zero and produce raw scores s = q.k; the block's
  // producer then turns them into exp2 arguments x = cs s + ncm with one fma
  // (ncm = -cs m for the running max m, 0 while no key of the lane is
  // visible), and the S blocks held between iterations are those x. In the
  // pipelined body the fmas run under the PV MFMAs of the iteration's last
  // segment, which has issue slots to spare, so the two segments that run
  // the exp2s carry no fma. Raising m shifts the held x by the same amount.
  float ncm = 0.0f, lsum = 0.0f, lsum1 = 0.0f;
  // Raise threshold in x units: 8 (a probability would exceed 2^8), -inf
  // until the lane's first visible key, so the per-tile test is one compare.
  float thr = -INFINITY;

  const int32_t qlast = min(q0 + 32 * NW, p.Lq) - 1;
  const int32_t pos_lo = ctx - p.Lq + q0, pos_hi = ctx - p.Lq + qlast;
  const int32_t hi = max(0, causal ? min(kv_lim, pos_hi + 1) : kv_lim);
  const int32_t win_lo = max(0, causal ? pos_lo - p.W + 1 : ctx - p.W);
  const int32_t sink_end = min(p.sinks, hi);
  const int32_t sink_tiles = (sink_end + TK - 1) / TK;
  const int32_t t_first = max(win_lo / TK, sink_tiles);
  const int32_t t_last = (hi + TK - 1) / TK;
  const int32_t n_tiles = sink_tiles + max(0, t_last - t_first);
  auto tile_base = [&](int32_t it) { return (it < sink_tiles ? it : t_first + (it - sink_tiles)) * TK; };
  const int32_t vis_hi = !q_ok ? -1 : (causal ? min(qpos, kv_lim - 1) : kv_lim - 1);
  const int32_t vis_lo = causal ? qpos - p.W + 1 : ctx - p.W;
  const int32_t wq_last = min(qw0 + 31, p.Lq - 1);
  const int32_t wpos_lo = ctx - p.Lq + qw0, wpos_hi = ctx - p.Lq + wq_last;
  // Every (key, query) slot of the tile is visible: no mask needed. The
  // position part of that test is a range of tile bases fixed per wave, so
  // each tile pays two compares instead of re-deriving it.
  const int32_t full_lo = causal ? wpos_hi - p.W + 1 : ctx - p.W;
  const int32_t full_hi = wq_last != qw0 + 31 ? INT32_MIN : min(kv_lim - TK, causal ? wpos_lo - TK + 1 : INT32_MAX);

  const int32_t *vrow = reinterpret_cast<const int32_t *>(ws + (int64_t)units * L::kBlock) + (int64_t)b * MC;
  const StageMap sm = stage_map(ctx, p.M * p.bs, p.Lq, p.W, p.sinks, causal);
  // Sink tiles sit at slots 4 it; the staged chunks of the window tiles are
  // one contiguous run, so window tile it sits at slot_w + 4 it (cheaper in
  // scalar instructions than the general chunk -> slot map, which runs for
  // every copy and flag load of every tile).
  const int32_t slot_w = n_tiles > sink_tiles ? sm.slot(4 * t_first) - 4 * sink_tiles : 0;
  auto tile_slot = [&](int32_t it) { return (uint32_t)(4 * it + (it < sink_tiles ? 0 : slot_w)); };
  // A tile skips the mask when all its (key, query) slots are visible and
  // its four chunks are linked. The fully visible tiles of this wave form
  // one run of iterations (tile bases grow with the iteration),
  // [it_full, it_full + n_full), found once here; links are checked once
  // for every chunk the workgroup visits. In a workgroup with an unlinked
  // chunk every tile takes the mask, which loads the link flags itself, so
  // the common path carries no flag loads.
  if constexpr (STAGE) {
    // Wait for this unit's stagers: workgroups dispatched a unit earlier,
    // which stage before they wait for anything. Past the bound (stagers not
    // resident) the workgroup stages its whole unit itself: the same bytes,
    // so a concurrent stager's writes agree.
    __shared__ int s_ok;
    if (stage_wait) {  // workgroup-uniform
      if (wave == 0) {
        bool ok = ss.spin >= 0 && __all(stage_flag == ss.tag);
        for (int32_t n = 0; n < ss.spin && !ok; ++n) {
          __builtin_amdgcn_s_sleep(4);
          const uint32_t v = lane < ss.S ? __hip_atomic_load(ss.flags + (int64_t)stage_unit * 64 + lane,
                                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                         : ss.tag;
          ok = __all(v == ss.tag);
        }
        if (lane == 0) s_ok = ok;
      }
      __syncthreads();
      if (!s_ok) {
        uint8_t *vl = lds_k0 + wave * 32 * D;  // free until the first tile copy
        for (int32_t sl = wave; sl < MC; sl += NW)
          stage_blocks<D, INT4, 1>(p, ws, MC, units, stage_unit, sl, NW, 1, vl, true);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
      }
    }
  }
  int32_t it_full = 0, n_full = 0;
  {
    bool first = true;
    for (int32_t base = 0; base < n_tiles; base += 64) {
      const int32_t it = base + lane, tb = tile_base(it);
      const uint64_t fm = __ballot(it < n_tiles && tb >= full_lo && tb <= full_hi);
      if (fm != 0) {
        if (first) it_full = base + __builtin_ctzll(fm);
        first = false;
        n_full = base + 63 - __builtin_clzll(fm) + 1 - it_full;
      }
    }
    int unlinked = 0;
    for (int32_t i = lane; i < 4 * n_tiles; i += 64) unlinked |= vrow[tile_slot(i >> 2) + (i & 3)] == 0;
    if (__any(unlinked)) n_full = 0;
  }
  // Tiles this wave computes: the sink tiles (when it has a query) and the
  // window iterations [it_v0, it_v1) holding keys of its queries' windows.
  // The workgroup visits the union over its four waves; a wave skips the
  // MFMAs and softmax of the tiles it sees nothing of (it still copies and
  // meets the barriers), and computes no S for the iteration after its last.
  const bool any_q = qw0 < p.Lq;
  int32_t it_v0 = sink_tiles, it_v1 = sink_tiles;
  bool win_in_tile0 = false;
  {
    const int32_t klo = max(0, causal ? wpos_lo - p.W + 1 : ctx - p.W);
    const int32_t khi = causal ? min(wpos_hi, kv_lim - 1) : kv_lim - 1;
    if (any_q && khi >= klo) {
      it_v1 = min(n_tiles, sink_tiles + max(0, khi / TK - t_first + 1));
      it_v0 = min(it_v1, sink_tiles + max(0, klo / TK - t_first));
      win_in_tile0 = klo < TK;
    }
  }
  // A sink tile whose visible keys all lie in its first 32 (16) keys: only
  // its first S block (and its first 16-key half of the PV contraction).
  const bool sink_half = any_q && sink_tiles == 1 && sink_end <= 32 && !win_in_tile0;
  const bool sink_quarter = sink_half && sink_end <= 16;
  auto wave_vis = [&](int32_t it) { return it < sink_tiles ? any_q : (it >= it_v0 && it < it_v1); };
  // Iterations [c0, c1) take the pipelined body: S(i) and S(i+1) both
  // visible, not the half sink tile. The rest (the wave's first and last
  // tiles, tiles it skips) take a plain body.
  int32_t c0 = 0, c1 = 0;
  if (any_q) {
    c0 = it_v0 == sink_tiles ? (sink_half ? 1 : 0) : it_v0;
    c1 = max(c0, it_v1 - 1);
  }
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(ws + ((int64_t)b * p.H + h) * MC * L::kBlock), (short)0, (int)(MC * CS), 0x00020000);
  // Tile copies: wave w fills NKL contiguous KiB of a K buffer (the K-tile
  // rows of chunk w) and NVL contiguous KiB of a V^T buffer (rows
  // [8 NVL w, 8 NVL (w + 1))), 1 KiB per copy, lane i writing LDS bytes
  // 16 i .. 16 i + 15 of it. Copy c of a tile reads the tile's first chunk
  // (scalar offset) + c * 1024 (immediate, also applied to the LDS address)
  // + kvo[c] / vvo[c]: the lane's row, swizzled 16-byte piece and chunk.
  constexpr int RPC = 1024 / KRB;  // K-tile rows per copy
  uint32_t kvo[NKL], vvo[NVL];
#pragma unroll
  for (int c = 0; c < NKL; ++c) {
    const int R = wave * NKL * RPC + c * RPC + lane / KC, j = (lane % KC) ^ kswz(R);
    kvo[c] = (uint32_t)((R / 16) * (int)CS + (R % 16) * KRB + 16 * j - c * 1024);
  }
#pragma unroll
  for (int c = 0; c < NVL; ++c) {
    const int d = wave * NVL * 8 + c * 8 + lane / 8, jv = (lane & 7) ^ ((d >> 1) & 7);
    vvo[c] = (uint32_t)((jv >> 1) * (int)CS + (int)L::kVPart + d * 32 + 16 * (jv & 1) - c * 1024);
  }
  const uint32_t wk = (uint32_t)wave * NKL * 1024, wv = (uint32_t)wave * NVL * 1024;
  const uint32_t mk0 = lds_u32(lds_k0) + wk, mk1 = lds_u32(lds_k1) + wk;
  const uint32_t mv0 = lds_u32(lds_v0) + wv, mv1 = lds_u32(lds_v1) + wv;
  // Copies [C0, C1) of a tile's K (V) part; a tile is split over the
  // segments of an iteration so the copies are not issued in one burst.
  auto load_k = [&](int32_t it, auto bufc, auto c0c, auto c1c) __attribute__((always_inline)) {
    constexpr int buf = decltype(bufc)::value, C0 = decltype(c0c)::value, C1 = decltype(c1c)::value;
    const uint32_t m0v = buf ? mk1 : mk0, soff = tile_slot(it) * CS;
    lds_dma_range<C0, C1>(rs, m0v, kvo, soff);
  };
  auto load_v = [&](int32_t it, auto bufc, auto c0c, auto c1c) __attribute__((always_inline)) {
    constexpr int buf = decltype(bufc)::value, C0 = decltype(c0c)::value, C1 = decltype(c1c)::value;
    const uint32_t m0v = buf ? mv1 : mv0, soff = tile_slot(it) * CS;
    lds_dma_range<C0, C1>(rs, m0v, vvo, soff);
  };
  // The same for a window tile (it >= sink_tiles), whose slot needs no select.
  auto load_kw = [&](int32_t it, auto bufc, auto c0c, auto c1c) __attribute__((always_inline)) {
    constexpr int buf = decltype(bufc)::value, C0 = decltype(c0c)::value, C1 = decltype(c1c)::value;
    const uint32_t m0v = buf ? mk1 : mk0, soff = (uint32_t)(4 * it + slot_w) * CS;
    lds_dma_range<C0, C1>(rs, m0v, kvo, soff);
  };
  auto load_vw = [&](int32_t it, auto bufc, auto c0c, auto c1c) __attribute__((always_inline)) {
    constexpr int buf = decltype(bufc)::value, C0 = decltype(c0c)::value, C1 = decltype(c1c)::value;
    const uint32_t m0v = buf ? mv1 : mv0, soff = (uint32_t)(4 * it + slot_w) * CS;
    lds_dma_range<C0, C1>(rs, m0v, vvo, soff);
  };
  // End of a tile: wait for this thread's tile copies except the newest
  // `keep` (the K prefetch, which has another tile of time) and for its LDS
  // reads (the next copies overwrite buffers read in this tile); then the
  // barrier publishes the copies of all threads.
  auto publish = [&](auto keepc) __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(decltype(keepc)::value) : "memory");
    __syncthreads();
  };

  int32_t ka[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) ka[c] = (lane & 31) * KRB + 16 * ((2 * c + hl) ^ kswz(lane & 31));
  // LDS byte addresses of this lane's V^T fragments in each V buffer, held
  // in registers (the empty asm hides their values from the compiler). The
  // second buffer lies above the 16-bit ds_read offset range: without a
  // register base per fragment the compiler rebuilds each address with a
  // v_or and the reads of that buffer lose their four-deep prefetch.
  uint32_t vb[2][4];
#pragma unroll
  for (int kc = 0; kc < 4; ++kc) {
    const uint32_t va = (uint32_t)((lane & 31) * VRB + 16 * ((2 * kc + hl) ^ (((lane & 31) >> 1) & 7)));
    vb[0][kc] = lds_u32(lds_v0) + va;
    vb[1][kc] = lds_u32(lds_v1) + va;
    asm volatile("" : "+v"(vb[0][kc]), "+v"(vb[1][kc]));
  }

  // Hidden (key, query) slots of S(i) become -inf. Slot r of block blk of
  // this lane holds key tb + 32 blk + 16(r/8) + 4((r/4)%2) + (r/2)%2 + 8(r%2) + 2 hl.
  auto apply_mask = [&](float16_t (&s)[2], int32_t tb, int32_t it) __attribute__((always_inline)) {
    int4 fl;  // link flags of the four chunks (a scalar load: the address is uniform)
    asm volatile("s_load_dwordx4 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(fl) : "s"(vrow + tile_slot(it)) : "memory");
    const int32_t kb = tb + 2 * hl;
    const int32_t rl = vis_lo - kb, rsk = p.sinks - kb;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      int32_t rh[2];
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int32_t f = (2 * blk + g) == 0 ? fl.x : (2 * blk + g) == 1 ? fl.y : (2 * blk + g) == 2 ? fl.z : fl.w;
        rh[g] = f ? vis_hi - kb : -1;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int32_t c = 32 * blk + 16 * (r >> 3) + 4 * ((r >> 2) & 1) + ((r >> 1) & 1) + 8 * (r & 1);
        const bool ok = (c <= rh[r >> 3]) & ((c >= rl) | (c < rsk));
        s[blk][r] = ok ? s[blk][r] : -INFINITY;
      }
    }
  };
  auto row_max = [&](const float16_t (&s)[2]) __attribute__((always_inline)) {
    float t = s[0][0];
#pragma unroll
    for (int r = 1; r < 16; ++r) t = fmaxf(t, s[0][r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) t = fmaxf(t, s[1][r]);
    return half_max(t);
  };
  // Raw scores of an S block to exp2 arguments.
  auto to_x = [&](float16_t &s) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = fmaf(s[r], cs, ncm);
  };
  // Lazy running max (x units, tmax = the lane's largest x of the tile):
  // rescale only when tmax exceeds 8; the lane's first visible key always
  // raises (its x becomes the reference, with o and the sums still 0; a
  // NaN or -inf tmax leaves the lane waiting). The held blocks sc shift
  // with the reference.
  auto raise_max = [&](float tmax, float16_t (&sc)[2]) __attribute__((always_inline)) {
    if (__any(tmax > thr)) {
      const bool first = thr == -INFINITY, found = tmax > -INFINITY;
      const float shift = first ? (found ? tmax : 0.0f) : fmaxf(tmax, 0.0f);
      const float alpha = first ? (found ? 0.0f : 1.0f) : (shift > 0.0f ? fast_exp2(-shift) : 1.0f);
      lsum *= alpha;
      lsum1 *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
#pragma unroll
      for (int blk = 0; blk < 2; ++blk)
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[blk][r] -= shift;
      ncm -= shift;
      thr = (first && !found) ? thr : 8.0f;
    }
  };
  const half2_t ones = {(half_t)1.0f, (half_t)1.0f};
  // exp2 of one S block (exp2 arguments), packed to fp16 in PV B-operand
  // order; adds the probabilities to the running sum from the packed words
  // themselves (the same pairs rebuilt from the half8 operands cost 12
  // conversions a tile).
  auto probs = [&](const float16_t &s, half8_t (&pb)[2], float &ls) __attribute__((always_inline)) {
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      w[i] = as_u32(half2_t{(half_t)fast_exp2(s[2 * i]), (half_t)fast_exp2(s[2 * i + 1])});
#pragma unroll
    for (int i = 0; i < 8; ++i) ls = __builtin_amdgcn_fdot2(as_half2(w[i]), ones, ls, false);
    pb[0] = __builtin_bit_cast(half8_t, make_uint4(w[0], w[1], w[2], w[3]));
    pb[1] = __builtin_bit_cast(half8_t, make_uint4(w[4], w[5], w[6], w[7]));
  };
  // Operand fragments: K chunk c of a 32-key block; V^T fragment i of a
  // 32-key block in PV order (dim block i / 2, 16-key half i % 2).
  auto kfrag = [&](const uint8_t *kt, int blk, int c) __attribute__((always_inline)) {
    return *reinterpret_cast<const half8_t *>(kt + 32 * blk * KRB + ka[c]);
  };
  auto vfrag = [&](auto vbufc, int blk, int i) __attribute__((always_inline)) {
    return lds_read16(vb[decltype(vbufc)::value][2 * blk + (i & 1)] + 32 * (i >> 1) * VRB);
  };
  // A segment's first four fragments come from `pre` when the previous
  // segment read them (PRE = 1) during its last MFMAs, so the copies and
  // bookkeeping between segments overlap their LDS latency.
  auto qk_block = [&](const uint8_t *kt, int blk, float16_t &acc, auto prec, const half8_t (&pre)[4])
                      __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16((decltype(prec)::value && c < 4) ? pre[c] : kfrag(kt, blk, c),
                                                   qf[c], c == 0 ? (float16_t){} : acc, 0, 0, 0);
  };
  auto pv_block = [&](auto vbufc, int blk, const half8_t (&pb)[2], const half8_t (&pre)[4])
                      __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2 * NDB; ++i)
      o[i >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(i < 4 ? pre[i] : vfrag(vbufc, blk, i), pb[i & 1], o[i >> 1],
                                                         0, 0, 0);
  };

  float16_t sx[2], sy[2];
  if (n_tiles > 0) {
    load_k(0, IntC<0>{}, IntC<0>{}, IntC<NKL>{});
    load_v(0, IntC<0>{}, IntC<0>{}, IntC<NVL>{});
    if (n_tiles > 1) load_k(1, IntC<1>{}, IntC<0>{}, IntC<NKL>{});
    publish(IntC<0>{});
    const half8_t none[4] = {};
    sx[1] = (float16_t){};
    if (wave_vis(0)) {
      qk_block(lds_k0, 0, sx[0], IntC<0>{}, none);
      if (!sink_half) qk_block(lds_k0, 1, sx[1], IntC<0>{}, none);
      to_x(sx[0]);
      to_x(sx[1]);
    }
    __syncthreads();  // K(0)'s buffer is refilled by the first iteration
  }

  // Iteration `it` (parity P) with S(it) in `sc` and S(it + 1) computed into
  // `sn`. K(it+1) is read from buffer P ^ 1 and K(it+2) loaded into buffer
  // P (it held K(it), last read for QK(it) in iteration it - 1); V(it) is
  // read from buffer P and V(it+1) loaded into buffer P ^ 1. Every copy an
  // iteration issues completes before its closing barrier.
  auto iter = [&](int32_t it, float16_t (&sc)[2], float16_t (&sn)[2], auto pc) __attribute__((always_inline)) {
    constexpr int P = decltype(pc)::value;
    const uint8_t *const kt = P ? lds_k0 : lds_k1;
    const int32_t tb = tile_base(it);
    const bool v_ahead = it + 1 < n_tiles, k_ahead = it + 2 < n_tiles;
    if (k_ahead) load_kw(it + 2, IntC<P>{}, IntC<0>{}, IntC<NKL / 2>{});
    // Tiles that are not fully visible go through the mask.
    if ((uint32_t)(it - it_full) >= (uint32_t)n_full) apply_mask(sc, tb, it);
    {
      // Operand fragments stream 4 ahead of the MFMA that uses them (the
      // scheduling groups below keep at most 4 in flight).
      // Seg 1: QK(i+1) block 0 | running max of S(i)
      // The four segments run at raised wave priority and the end-of-tile
      // wait at the normal one, so of the two waves sharing a SIMD the one
      // with MFMAs to issue wins the arbitration (measured ~0.7 % faster).
      __builtin_amdgcn_s_setprio(1);
      const half8_t none[4] = {};
      half8_t pre_k[4], pre_a[4], pre_b[4];
      qk_block(kt, 0, sn[0], IntC<0>{}, none);
      const float tmax = row_max(sc);
#pragma unroll
      for (int c = 0; c < 4; ++c) pre_k[c] = kfrag(kt, 1, c);
      // Each MFMA is followed by one read: this block's last four
      // fragments, then the next segment's first four.
      PIPE_SGB(0x100, 4, 0);
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        PIPE_SGB(0x008, 1, 0);
        PIPE_SGB(0x100, 1, 0);
        PIPE_SGB(0x002, 2, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      raise_max(tmax, sc);
      if (k_ahead) load_kw(it + 2, IntC<P>{}, IntC<NKL / 2>{}, IntC<NKL>{});
      // Seg 2: QK(i+1) block 1 | probabilities of S(i) block 0
      half8_t pa[2], pb[2];
      qk_block(kt, 1, sn[1], IntC<1>{}, pre_k);
      probs(sc[0], pa, lsum);
#pragma unroll
      for (int i = 0; i < 4; ++i) pre_a[i] = vfrag(IntC<P>{}, 0, i);
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        PIPE_SGB(0x008, 1, 0);
        PIPE_SGB(0x100, 1, 0);
        PIPE_SGB(0x002, 16 / NCH, 0);  // per exp2: half a pack, half a row-sum dot
        PIPE_SGB(0x400, 16 / NCH, 0);
      }
      // The probabilities must be complete here: without this use the
      // compiler sinks their exp2s past the conditional copies below into
      // segment 3, ahead of the PV MFMAs that need them.
      asm volatile("" ::"v"(pa[0]), "v"(pa[1]));
      __builtin_amdgcn_sched_barrier(0);
      if (v_ahead) load_vw(it + 1, IntC<P ^ 1>{}, IntC<0>{}, IntC<NVL / 2>{});
      // Seg 3: PV(i) block 0 | probabilities of S(i) block 1
      pv_block(IntC<P>{}, 0, pa, pre_a);
      probs(sc[1], pb, lsum1);
#pragma unroll
      for (int i = 0; i < 4; ++i) pre_b[i] = vfrag(IntC<P>{}, 1, i);
#pragma unroll
      for (int c = 0; c < 2 * NDB; ++c) {
        PIPE_SGB(0x008, 1, 0);
        PIPE_SGB(0x100, 1, 0);
        PIPE_SGB(0x002, 16 / (2 * NDB), 0);
        PIPE_SGB(0x400, 16 / (2 * NDB), 0);
      }
      asm volatile("" ::"v"(pb[0]), "v"(pb[1]));
      __builtin_amdgcn_sched_barrier(0);
      if (v_ahead) load_vw(it + 1, IntC<P ^ 1>{}, IntC<NVL / 2>{}, IntC<NVL>{});
      // Seg 4: PV(i) block 1 | S(i+1) to exp2 arguments
      pv_block(IntC<P>{}, 1, pb, pre_b);
      to_x(sn[0]);
      to_x(sn[1]);
#pragma unroll
      for (int c = 0; c < 2 * NDB; ++c) {
        PIPE_SGB(0x008, 1, 0);
        if (c < 4) PIPE_SGB(0x100, 1, 0);
        PIPE_SGB(0x002, 32 / (2 * NDB), 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
    }
    publish(IntC<0>{});
  };
  // The same iteration without the pipeline, for iterations outside
  // [c0, c1): QK(i+1) only when tile i+1 is visible to this wave, the
  // softmax and PV of S(i) only when tile i is, one S block (and one 16-key
  // half of the PV contraction) for a sink tile that needs no more. The
  // copies and the end-of-tile barrier are those of the pipelined body.
  auto iter_edge = [&](int32_t it, float16_t (&sc)[2], float16_t (&sn)[2], auto pc) __attribute__((always_inline)) {
    constexpr int P = decltype(pc)::value;
    const uint8_t *const kt = P ? lds_k0 : lds_k1;
    const int32_t tb = tile_base(it);
    const bool v_ahead = it + 1 < n_tiles, k_ahead = it + 2 < n_tiles;
    const bool cur = wave_vis(it), nxt = v_ahead && wave_vis(it + 1);
    if (k_ahead) load_k(it + 2, IntC<P>{}, IntC<0>{}, IntC<NKL>{});
    if (v_ahead) load_v(it + 1, IntC<P ^ 1>{}, IntC<0>{}, IntC<NVL>{});
    if (cur) {
      const bool one = it == 0 && sink_half;  // wave-uniform
      if ((uint32_t)(it - it_full) >= (uint32_t)n_full) apply_mask(sc, tb, it);
      float tmax;
      if (one) {
        tmax = sc[0][0];
#pragma unroll
        for (int r = 1; r < 16; ++r) tmax = fmaxf(tmax, sc[0][r]);
        tmax = half_max(tmax);
      } else {
        tmax = row_max(sc);
      }
      raise_max(tmax, sc);
      half8_t pa[2], pre[4];
      probs(sc[0], pa, lsum);
      if (one && sink_quarter) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vfrag(IntC<P>{}, 0, 2 * db), pa[0], o[db], 0, 0, 0);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) pre[i] = vfrag(IntC<P>{}, 0, i);
        pv_block(IntC<P>{}, 0, pa, pre);
      }
      if (!one) {
        half8_t pb[2];
        probs(sc[1], pb, lsum1);
#pragma unroll
        for (int i = 0; i < 4; ++i) pre[i] = vfrag(IntC<P>{}, 1, i);
        pv_block(IntC<P>{}, 1, pb, pre);
      }
    }
    // S(i+1) after S(i) is used, so the two are never live together here
    // (a skipped S(i+1) is zeroed: it is never read).
    const half8_t none[4] = {};
    if (nxt) {
      qk_block(kt, 0, sn[0], IntC<0>{}, none);
      qk_block(kt, 1, sn[1], IntC<0>{}, none);
      to_x(sn[0]);
      to_x(sn[1]);
    } else {
      sn[0] = (float16_t){};
      sn[1] = (float16_t){};
    }
    publish(IntC<0>{});
  };
  // Iterations [0, m0) and [m1, n_tiles) run the plain body, [m0, m1) the
  // pipelined one, m0 = c0 rounded up to even. Each loop takes two
  // iterations per trip, so buffer indices and score registers stay
  // compile-time constants (a parity branch per iteration instead made the
  // compiler spill).
  // (The pipelined body copies tiles it + 1 and it + 2 as window tiles, so
  // it starts no earlier than sink_tiles - 1.)
  const int32_t mp = max(c0, sink_tiles - 1);
  const int32_t m0 = min(n_tiles, mp + (mp & 1)), m1 = max(m0, c1);
  int32_t it = 0;
  for (; it < m0; it += 2) {
    iter_edge(it, sx, sy, IntC<0>{});
    if (it + 1 >= m0) {
      ++it;
      break;
    }
    iter_edge(it + 1, sy, sx, IntC<1>{});
  }
  for (; it < m1; it += 2) {
    iter(it, sx, sy, IntC<0>{});
    if (it + 1 >= m1) {
      ++it;
      break;
    }
    iter(it + 1, sy, sx, IntC<1>{});
  }
  if (it < n_tiles && (it & 1)) {
    iter_edge(it, sy, sx, IntC<1>{});
    ++it;
  }
  for (; it < n_tiles; it += 2) {
    iter_edge(it, sx, sy, IntC<0>{});
    if (it + 1 >= n_tiles) break;
    iter_edge(it + 1, sy, sx, IntC<1>{});
  }
  __builtin_amdgcn_s_waitcnt(0);

  const float l = half_sum(lsum + lsum1);
  if (!q_ok) return;
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  // The row's offset is rebuilt here from the lane id, not taken from the Q
  // load's address: that 64-bit value, live across the tile loops, spills
  // at 256 VGPRs.
  int32_t qo = qw0 + (int32_t)(__lane_id() & 31);
  asm volatile("" : "+v"(qo));
  half_t *orow = p.out + (((int64_t)b * p.Lq + qo) * p.H + h) * D;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * db + 8 * g + 4 * hl;
      const half2_t x = {(half_t)(o[db][4 * g] * inv), (half_t)(o[db][4 * g + 1] * inv)};
      const half2_t y = {(half_t)(o[db][4 * g + 2] * inv), (half_t)(o[db][4 * g + 3] * inv)};
      *reinterpret_cast<uint2 *>(orow + d0) = make_uint2(as_u32(x), as_u32(y));
    }
  }
}

bool prefill_supported(const memopt_attn_desc &d) {
  auto al16 = [](const void *x) { return ((uintptr_t)x & 15) == 0; };
  if (d.q_len < 2 || (d.head_dim != 64 && d.head_dim != 128)) return false;
  if (d.num_kv_blocks <= 0) return false;
  if (!al16(d.query) || !al16(d.out) || !al16(d.key_cache)) return false;
  if (d.kv_format == MEMOPT_KV_INT4) return d.block_size == 16;
  if (d.kv_format != MEMOPT_KV_FP16 || d.block_size % 16 != 0 || !al16(d.value_cache)) return false;
  // contiguous [num_blocks, block_size, H, D] pools (element strides)
  const int64_t D = d.head_dim, H = d.num_heads;
  return d.kv_head_stride == D && d.kv_token_stride == H * D && d.kv_page_stride == d.block_size * H * D;
}

// Staged slots per sequence: the sink tiles plus the window tiles a call can
// visit (stage_map), bounded without reading context_lens: keys
// [ctx - q_len - W + 1, ctx) for causal calls ([ctx - W, ctx) otherwise),
// plus one tile of alignment; never more than the block table's span.
static int64_t staged_chunks(const memopt_attn_desc &d) {
  const int64_t full = ((int64_t)d.max_blocks_per_seq * d.block_size / 16 + 3) / 4 * 4;
  const int64_t W = effective_window(d.window_size, d.max_seq_len);
  const int64_t span = d.causal ? (int64_t)d.q_len + W - 1 : W;
  const int64_t sinks = d.num_sink_tokens > 0 ? d.num_sink_tokens : 0;
  const int64_t bound = 4 * ((span + 63) / 64 + 1) + 4 * ((sinks + 63) / 64);
  return bound < full ? bound : full;
}

// Workspace: the staged blocks, one link flag per (sequence, slot), then
// 64 in-kernel staging flags per (sequence, head), 8-byte aligned.
static int64_t stage_counters_offset(const memopt_attn_desc &d, int64_t mc) {
  const int64_t units = (int64_t)d.batch * mc * d.num_heads;
  return (units * (64LL * d.head_dim) + (int64_t)d.batch * mc * 4 + 7) / 8 * 8;
}

int64_t prefill_workspace_bytes(const memopt_attn_desc &d) {
  const int64_t mc = staged_chunks(d);
  const int64_t units = (int64_t)d.batch * mc * d.num_heads;
  // one sequence's chunks must stay inside a 31-bit buffer range
  if (units <= 0 || units >= (1LL << 31) || mc * d.num_heads * 64LL * d.head_dim >= (1LL << 31)) return 0;
  return stage_counters_offset(d, mc) + (int64_t)d.batch * d.num_heads * 64 * 4;
}

static int prefill_device_cus() {
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

// Id of a prefill call for the in-kernel staging flags: 1 .. 2^32 - 1.
static uint32_t next_prefill_tag() {
  static std::atomic<unsigned long long> n{0};
  return (uint32_t)(n.fetch_add(1, std::memory_order_relaxed) % 0xFFFFFFFFull + 1);
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
  const int64_t need = prefill_workspace_bytes(d);
  if (need > 0 && d.workspace && d.workspace_bytes >= need) {
    // staged path: chunks in LDS operand layout, then the direct-load kernel
    const int32_t mc = (int32_t)staged_chunks(d);
    const int32_t units = d.batch * mc * d.num_heads;
    constexpr int NW = 4;  // waves (32 queries each) per workgroup
    const int64_t n_wg = (int64_t)((d.q_len + 32 * NW - 1) / (32 * NW)) * d.num_heads * d.batch;
    MEMOPT_REQUIRE(n_wg < (1LL << 31), MEMOPT_ERR_UNSUPPORTED, "paged_attention: too many query tiles");
    uint8_t *ws = (uint8_t *)d.workspace;
    const dim3 sgrid((unsigned)((units + 15) / 16)), grid((unsigned)n_wg);
    const bool int4 = d.kv_format == MEMOPT_KV_INT4;
    // In-kernel staging when every XCD owns whole (sequence, head) units of
    // at least 32 query tiles: a staging launch stages each XCD's first
    // unit, and the first S = min(nqt / 8, 16) workgroups of every unit the
    // next one (config 4: 8 to 16 stagers measured 0.5 % faster than 32,
    // 64 slower: fewer, larger shares cost less waiting in all).
    const int64_t nqt = (d.q_len + 32 * NW - 1) / (32 * NW);
    const int64_t per_xcd = n_wg / 8;
    StageSched ss{};
    ss.S = (int32_t)std::min<int64_t>(nqt / 8, 16);
    // (MEMOPT_PREFILL_STAGE_LAUNCH selects the staging launch for every
    // call, so that tests can compare the two paths.)
    const bool in_kernel = n_wg % 8 == 0 && nqt >= 32 && per_xcd % nqt == 0 &&
                           std::getenv("MEMOPT_PREFILL_STAGE_LAUNCH") == nullptr;
    if (in_kernel) {
      ss.flags = reinterpret_cast<uint32_t *>(ws + stage_counters_offset(d, mc));
      ss.tag = next_prefill_tag();
      // MEMOPT_PREFILL_STAGE_SPIN overrides the wait bound (a negative value
      // makes every waiting workgroup stage its unit itself: a test hook for
      // that path).
      const char *spin = std::getenv("MEMOPT_PREFILL_STAGE_SPIN");
      ss.spin = spin ? std::atoi(spin) : 200000;
      const int32_t upx = (int32_t)(per_xcd / nqt), first = 8 * mc;
      const int32_t nflags = d.batch * d.num_heads * 64;
      const dim3 fgrid((unsigned)((first + 15) / 16));
      if (d.head_dim == 128) {
        if (int4) {
          hipLaunchKernelGGL((prefill_stage_kernel<128, true>), fgrid, dim3(256), 0, stream, p, ws, mc, units, upx,
                             first, ss.flags, nflags);
          hipLaunchKernelGGL((prefill_pipe_kernel<128, NW, true, true>), grid, dim3(NW * 64), 0, stream, p, ws, mc,
                             units, ss);
        } else {
          hipLaunchKernelGGL((prefill_stage_kernel<128, false>), fgrid, dim3(256), 0, stream, p, ws, mc, units, upx,
                             first, ss.flags, nflags);
          hipLaunchKernelGGL((prefill_pipe_kernel<128, NW, true, false>), grid, dim3(NW * 64), 0, stream, p, ws, mc,
                             units, ss);
        }
      } else {
        if (int4) {
          hipLaunchKernelGGL((prefill_stage_kernel<64, true>), fgrid, dim3(256), 0, stream, p, ws, mc, units, upx,
                             first, ss.flags, nflags);
          hipLaunchKernelGGL((prefill_pipe_kernel<64, NW, true, true>), grid, dim3(NW * 64), 0, stream, p, ws, mc,
                             units, ss);
        } else {
          hipLaunchKernelGGL((prefill_stage_kernel<64, false>), fgrid, dim3(256), 0, stream, p, ws, mc, units, upx,
                             first, ss.flags, nflags);
          hipLaunchKernelGGL((prefill_pipe_kernel<64, NW, true, false>), grid, dim3(NW * 64), 0, stream, p, ws, mc,
                             units, ss);
        }
      }
      return check_launch("paged_attention(prefill, staged in kernel)");
    }
    if (d.head_dim == 128) {
      if (int4) hipLaunchKernelGGL((prefill_stage_kernel<128, true>), sgrid, dim3(256), 0, stream, p, ws, mc, units, 1, units,
                                   nullptr, 0);
      else hipLaunchKernelGGL((prefill_stage_kernel<128, false>), sgrid, dim3(256), 0, stream, p, ws, mc, units, 1, units,
                                   nullptr, 0);
      hipLaunchKernelGGL((prefill_pipe_kernel<128, NW, false, false>), grid, dim3(NW * 64), 0, stream, p, ws, mc,
                         units, ss);
    } else {
      if (int4) hipLaunchKernelGGL((prefill_stage_kernel<64, true>), sgrid, dim3(256), 0, stream, p, ws, mc, units, 1, units,
                                   nullptr, 0);
      else hipLaunchKernelGGL((prefill_stage_kernel<64, false>), sgrid, dim3(256), 0, stream, p, ws, mc, units, 1, units,
                                   nullptr, 0);
      hipLaunchKernelGGL((prefill_pipe_kernel<64, NW, false, false>), grid, dim3(NW * 64), 0, stream, p, ws, mc,
                         units, ss);
    }
    return check_launch("paged_attention(prefill, staged)");
  }
  // In-kernel staging (no workspace, or a workspace range beyond 31 bits):
  // 4 waves x 32 queries, 64-key tiles dequantized into LDS by the workgroup.
  const int64_t n_wg = (int64_t)((d.q_len + 127) / 128) * d.num_heads * d.batch;
  MEMOPT_REQUIRE(n_wg < (1LL << 31), MEMOPT_ERR_UNSUPPORTED, "paged_attention: too many query tiles");
  const dim3 grid((unsigned)n_wg);
  const bool int4 = d.kv_format == MEMOPT_KV_INT4;
  if (d.head_dim == 128) {
    if (int4) hipLaunchKernelGGL((prefill_kernel<128, true, 4, 1, 64>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((prefill_kernel<128, false, 4, 1, 64>), grid, dim3(256), 0, stream, p);
  } else {
    if (int4) hipLaunchKernelGGL((prefill_kernel<64, true, 4, 1, 64>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((prefill_kernel<64, false, 4, 1, 64>), grid, dim3(256), 0, stream, p);
  }
  return check_launch("paged_attention(prefill)");
}

}  // namespace memopt
