// common.hpp — shared host/device helpers for the gfx950 INT4 KV-cache
// data plane: status/error plumbing for the C ABI, the registered pool,
// fp16 bit helpers and wave64 cross-lane primitives.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>
#include <mutex>

#include "../../include/memopt_hip.h"

namespace memopt {

// ---------------------------------------------------------------------------
// Error plumbing (host)
// ---------------------------------------------------------------------------
void set_error(const std::string &msg);
void clear_error();

#define MEMOPT_REQUIRE(cond, code, msg)                                        \
  do {                                                                         \
    if (!(cond)) {                                                             \
      ::memopt::set_error(msg);                                                \
      return (code);                                                           \
    }                                                                          \
  } while (0)

// Checks the launch that was just enqueued.
int check_launch(const char *what);

// ---------------------------------------------------------------------------
// Registered pool (host state; storage is owned by the caller)
// ---------------------------------------------------------------------------
struct PoolView {
  bool initialized = false;
  int64_t num_blocks = 0;
  int32_t block_size = 0, num_heads = 0, head_dim = 0, kv_format = MEMOPT_KV_FP16;
  void *key = nullptr, *value = nullptr;  // fp16 pools; INT4: key = page buffer, value unused
  void *key_scales = nullptr, *value_scales = nullptr;  // unused (kept for the ABI)
};
// Snapshot of the live pool (taken under the pool lock).
PoolView pool_snapshot();

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_half2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// Cache-policy operand of a buffer load that streams data read once per
// launch (KV pages in decode): the nt bit (bit 1 on gfx950) marks the lines
// non-temporal, so a decode step's few hundred MB do not evict the block
// tables, q and the partials from L2, and the last-level cache is not
// refilled with pages that the next step (another page set) never touches.
// Measured on MI355X (16 x 32 heads x 4096 tokens of INT4 pages, 285 MB per
// step): 53.3 -> 48.8 us. Only for loads whose instruction covers whole
// 128-byte lines: where several instructions each read part of a line (the
// quantizer's fp16 reads, an fp16 decode layout with 16-byte row slices per
// lane), the line was fetched again and those kernels ran 1.15-1.5x slower
// with the bit.
static constexpr int kStreamLoad = 2;

// DPP lane exchange inside quads / rows of 16 (no LDS traffic).
// quad_perm xor-1 = [1,0,3,2] (0xB1), xor-2 = [2,3,0,1] (0x4E).
// All source lanes of the patterns used here are active, so bound_ctrl is
// irrelevant to the result; setting it lets the compiler fold the move into
// the consuming VALU op as a DPP source modifier.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float xor1(float v) { return dpp_f32<0xB1>(v); }
__device__ __forceinline__ float xor2(float v) { return dpp_f32<0x4E>(v); }
// row_half_mirror (0x141): lane i <-> 7-i inside each group of 8.
__device__ __forceinline__ float half_mirror(float v) { return dpp_f32<0x141>(v); }
// Generic wave64 butterfly through the LDS crossbar (ds_bpermute / swizzle).
__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

// v(lane) + v(lane ^ 16) and v(lane) + v(lane ^ 32) in registers (gfx950
// v_permlane16_swap / v_permlane32_swap: the two results of a swap of v with
// itself hold both lanes of each pair).
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// v_bfi_b32: (mask & a) | (~mask & b) in one VALU op. The compiler splits the
// equivalent C expression into AND + OR when `b` is a constant, so the
// instruction is requested directly; `mask` is a wave-uniform constant.
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(a), "v"(b));
  return r;
}

// A wave-uniform pointer rebuilt from readfirstlane'd halves: the compiler
// keeps it in SGPRs, so `p + lane_offset` becomes a scalar-base load with a
// 32-bit VGPR offset instead of 64-bit per-lane address arithmetic.
template <typename T>
__device__ __forceinline__ const T *uniform_ptr(const T *p) {
  const uint64_t a = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return (const T *)(((uint64_t)hi << 32) | lo);
}

// Wave64 max all-reduce: DPP inside rows of 16, LDS crossbar across rows.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, xor1(v));
  v = fmaxf(v, xor2(v));
  v = fmaxf(v, half_mirror(v));
  v = fmaxf(v, dpp_f32<0x140>(v));  // row_mirror
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}

// Group-64 symmetric INT4 codes, TheRadDani/memopt-transformer-runtime
// src/csrc/quantization.cu:168, :183-186: scale = absmax > 0 ? absmax / 7 : 1
// (IEEE), code = clamp((int)roundf(v / scale) + 8, 0, 15) with roundf half
// away from zero; NaN quotients give code 8, like the float->int conversion
// of the reference (v_cvt_i32_f32(NaN) = 0).

// RN(a / 7) for a >= 0 without an IEEE division (Markstein with the
// constant c7 = RN(1/7)): q0 = RN(a * c7) is within an ulp of a / 7,
// r = a - 7 * q0 is exact in one fma, and RN(q0 + r * c7) = RN(a / 7).
// Checked against the IEEE quotient for every finite fp16 absmax; a = inf
// keeps the IEEE result inf (the fma would give inf - inf).
__device__ __forceinline__ float div7(float a) {
  constexpr float c7 = 0.142857149f;  // 0x3E124925
  const float q0 = a * c7;
  const float r = fmaf(-q0, 7.0f, a);
  const float q = fmaf(r, c7, q0);
  return a == __builtin_inff() ? a : q;
}

// Group scale from the group's absmax: absmax / 7, or 1 for an all-zero group.
__device__ __forceinline__ float scale_of(float absmax) { return absmax > 0.0f ? div7(absmax) : 1.0f; }

// fp16 scale stored in an INT4 page: the RNE fp16 of the fp32 group scale,
// except 9360, which is stored as 9352. 9360 is the RNE of 65504 / 7 (the
// only fp16 absmax whose scale rounds up that far), and 7 * 9360 = 65520
// rounds to inf in fp16, so a +-65504 input would dequantize to +-inf; with
// 9352 it dequantizes to +-65464 (0.06 % low) and stays finite. Inf and NaN
// scales pass through unchanged.
__device__ __forceinline__ half_t page_scale(float s) {
  const half_t h = (half_t)s;
  return h == (half_t)9360.0f ? (half_t)9352.0f : h;
}

// Absmax of a 64-element group spread over LANES consecutive lanes (4 or 8,
// aligned): DPP max inside the lane group.
template <int LANES>
__device__ __forceinline__ float group_absmax(float a) {
  a = fmaxf(a, xor1(a));
  a = fmaxf(a, xor2(a));
  if (LANES == 8) a = fmaxf(a, half_mirror(a));
  return a;
}

template <int LANES>
__device__ __forceinline__ float group_scale(float a) {
  return scale_of(group_absmax<LANES>(a));
}

// Codes of N elements with one scale (y = RN(1 / scale)), packed 8 per word
// (element i of word k in bits 4i..4i+3, i.e. byte j = code[2j] | code[2j+1] << 4).
//  - Quotient: RN(v / scale) without a full IEEE division per element
//    (Markstein): q0 = RN(v * y) is within an ulp of v / scale,
//    r = v - q0 * scale is exact in one fma and RN(q0 + r * y) = RN(v / scale).
//    No overflow or underflow is possible (|v| <= 65504, scale in
//    [absmax / 7, 9358]); NaN/inf inputs end in a NaN quotient.
//  - Rounding: roundf(q) (half away from zero) = trunc(q + copysign(h, q))
//    with h = 0.5 - 2^-25, the float just below one half: the sum rounds up
//    to the next integer exactly when |q| reaches a half (checked for every
//    float with |q| < 16). The float->int conversion truncates and turns NaN
//    into 0 (code 8).
//  - Clamp: |q| <= 7 (1 + 2^-22) for every finite v in the group, since
//    |v| <= absmax and scale = RN(absmax / 7); the rounded value lies in
//    [-7, 7] and clamp(iq + 8, 0, 15) = iq + 8.
//  - Packing: sum over i of (iq_i + 8) << 4i = 0x88888888 + sum of iq_i << 4i
//    (mod 2^32), one shift-add per element.
template <int N>
__device__ __forceinline__ void int4_pack(const float *v, float scale, float y, uint32_t *w) {
  constexpr float h = 0.49999997f;  // 0x3EFFFFFF
#pragma unroll
  for (int k = 0; k < N / 8; ++k) {
    uint32_t acc = 0x88888888u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = v[8 * k + i];
      const float q0 = __fmul_rn(x, y);
      const float r = fmaf(-q0, scale, x);
      const float q = fmaf(r, y, q0);
      const int iq = (int)(q + __builtin_copysignf(h, q));
      acc += (uint32_t)iq << (4 * i);
    }
    w[k] = acc;
  }
}

template <int N>
__device__ __forceinline__ void int4_pack(const float *v, float scale, uint32_t *w) {
  int4_pack<N>(v, scale, 1.0f / scale, w);
}

// Quantizes 8 consecutive elements (one 16-byte lane chunk of a 64-element
// group spread over 8 lanes) into one packed word and sets `scale` to the
// group's fp32 scale. Lanes 8k..8k+7 must hold one group.
__device__ __forceinline__ uint32_t quantize8(const float v[8], float &scale) {
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) a = fmaxf(a, fabsf(v[i]));
  scale = group_scale<8>(a);
  uint32_t w;
  int4_pack<8>(v, scale, &w);
  return w;
}

__device__ __forceinline__ void unpack_half8(uint4 u, float f[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    half2_t h = as_half2(w[i]);
    f[2 * i] = (float)h.x;
    f[2 * i + 1] = (float)h.y;
  }
}

}  // namespace memopt
