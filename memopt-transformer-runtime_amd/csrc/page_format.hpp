// page_format.hpp — byte layout of this build's INT4 KV page pool.
//
// The codes and scales are the reference's group-64 symmetric INT4 values
// (TheRadDani/memopt-transformer-runtime src/csrc/quantization.cu:104-203,
// groups = (page, token, head, 64-dim chunk) of a [nb, 16, H, D] pool); only
// their placement differs, chosen for the gfx950 decode kernel:
//
//   pool   = [num_blocks][H][block]            (one allocation, u8)
//   block  = K codes (8*D B) | V codes (8*D B) | K scales (32*G B) | V scales (32*G B)
//            with G = D/64 scale groups per token; 2176 B at D = 128.
//
// A (page, head) block is read by one wave64: lane l = 8*p + c owns the token
// pair (p, p+8) (p = 0..7) and the D/8 dims [c*D/8, (c+1)*D/8) (c = 0..7),
// i.e. BPL = D/8 bytes of K codes and BPL of V codes:
//   K: bytes [l*BPL, l*BPL + BPL/2) = token p's codes for those dims, reference
//      byte order (low nibble = even dim); the next BPL/2 bytes = token p+8.
//   V: 2-byte units interleaved: unit u (4 dims, u = 0..BPL/4-1) occupies
//      bytes [l*BPL + 4u, +2) for token p and [l*BPL + 4u + 2, +2) for p+8,
//      so one 32-bit word holds the same 4 dims of both tokens.
//   scales (fp16, RNE of the fp32 scale, except that 9360 = RNE(65504 / 7)
//      is stored as 9352 so that 7 * scale stays finite in fp16): index
//      g*16 + 2*p + h for token 8*h + p, group g — the two tokens of a lane
//      are adjacent.
// 16-token pages only. Rows never written are code 8 (0x88 bytes) with scale
// 1.0, exactly what quantizing a zero row produces. Rows removed by
// evict_tokens keep their codes and get scale 0 in every group, so they
// dequantize to +-0 like the reference's zeroed fp16 rows.
#pragma once
#include <stdint.h>

namespace memopt {

struct Int4Page {
  int32_t D, G, BPL;
  int64_t kcodes, vcodes, kscales, vscales, block;  // byte offsets / size
  __host__ __device__ explicit Int4Page(int32_t d)
      : D(d), G(d / 64), BPL(d / 8), kcodes(0), vcodes(8LL * d), kscales(16LL * d),
        vscales(16LL * d + 32LL * (d / 64)), block(16LL * d + 64LL * (d / 64)) {}
  // Byte offset inside the K (or V) code region of the nibble pair holding
  // dims (d & ~1, d | 1) of token t; the nibble is (d & 1).
  __host__ __device__ int64_t k_byte(int32_t t, int32_t d) const {
    const int32_t dpl = D / 8, c = d / dpl, r = d % dpl;
    return (int64_t)(8 * (t & 7) + c) * BPL + (t >> 3) * (BPL / 2) + r / 2;
  }
  __host__ __device__ int64_t v_byte(int32_t t, int32_t d) const {
    const int32_t dpl = D / 8, c = d / dpl, r = d % dpl;
    return (int64_t)(8 * (t & 7) + c) * BPL + (r / 4) * 4 + (t >> 3) * 2 + (r % 4) / 2;
  }
  // fp16 element index of the scale of (token t, group g) in a scale region.
  __host__ __device__ int32_t scale_idx(int32_t t, int32_t g) const { return g * 16 + 2 * (t & 7) + (t >> 3); }
};

}  // namespace memopt
