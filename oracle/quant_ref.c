/*
 * quant_ref.c — C restatement of the reference INT4 quantizer, used as an
 * independent CPU check of oracle.py (TEST INFRASTRUCTURE ONLY: only tests,
 * the smoke check and the benchmark's CPU-baseline leg load it).
 *
 * Follows TheRadDani/memopt-transformer-runtime src/csrc/quantization.cu:
 *   :129-171  absmax over a 64-element group; scale = absmax > 0 ? absmax/7 : 1
 *   :183-186  code = clamp((int)roundf(v / scale) + 8, 0, 15)
 *   :198-200  byte = code[2i] | code[2i+1] << 4
 *   :254-262  dequant = float(code - 8) * scale (fp32; fp16 cast done by caller)
 * Compiled without -ffast-math so division and roundf are IEEE / C99 exact.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define GROUP 64

void oracle_quantize_int4(const float *in, int64_t num_groups, uint8_t *packed,
                          float *scales) {
  for (int64_t g = 0; g < num_groups; ++g) {
    const float *v = in + g * GROUP;
    float absmax = 0.0f;
    for (int i = 0; i < GROUP; ++i) absmax = fmaxf(absmax, fabsf(v[i]));
    const float scale = (absmax > 0.0f) ? (absmax / 7.0f) : 1.0f;
    scales[g] = scale;
    int codes[GROUP];
    for (int i = 0; i < GROUP; ++i) {
      const float r = roundf(v[i] / scale);
      int iq = isnan(r) ? 8 : (int)r + 8;
      codes[i] = iq < 0 ? 0 : (iq > 15 ? 15 : iq);
    }
    for (int i = 0; i < GROUP / 2; ++i)
      packed[g * (GROUP / 2) + i] = (uint8_t)((codes[2 * i] & 0xF) | ((codes[2 * i + 1] & 0xF) << 4));
  }
}

void oracle_dequantize_int4(const uint8_t *packed, const float *scales,
                            int64_t num_groups, float *out) {
  for (int64_t g = 0; g < num_groups; ++g) {
    const float s = scales[g];
    for (int i = 0; i < GROUP / 2; ++i) {
      const uint8_t b = packed[g * (GROUP / 2) + i];
      out[g * GROUP + 2 * i] = (float)((int)(b & 0xF) - 8) * s;
      out[g * GROUP + 2 * i + 1] = (float)((int)(b >> 4) - 8) * s;
    }
  }
}

/*
 * Checker for the division shortcut of the device quantizer (not part of the
 * reference): for each scale s[j] and every finite fp16 value v with
 * |v| <= 7 * s[j] (given as fp32 in `v`), compares the Markstein quotient
 *   y = RN(1/s); q0 = RN(v*y); r = fma(-q0, s, v); q = fma(r, y, q0)
 * with the IEEE quotient RN(v/s) by value (the shortcut turns -0 into +0;
 * both give code 8). Returns the number of mismatches (0 expected).
 */
int64_t oracle_markstein_mismatches(const float *v, int64_t nv, const float *s, int64_t ns) {
  int64_t bad = 0;
  for (int64_t j = 0; j < ns; ++j) {
    const float sc = s[j];
    const float y = 1.0f / sc;
    const float lim = 7.0f * sc * 1.0001f;
    for (int64_t i = 0; i < nv; ++i) {
      const float x = v[i];
      if (fabsf(x) > lim) continue;
      const float q0 = x * y;
      const float r = fmaf(-q0, sc, x);
      const float q = fmaf(r, y, q0);
      const float want = x / sc;
      if (q != want) ++bad;
    }
  }
  return bad;
}

/*
 * Checker for the device's group-scale shortcut (not part of the reference):
 * for each a[i] (positive), compares the Markstein quotient with the
 * constant c7 = RN(1/7)
 *   q0 = RN(a*c7); r = fma(-q0, 7, a); q = fma(r, c7, q0)
 * with the IEEE quotient RN(a/7). Returns the number of mismatches.
 */
int64_t oracle_div7_mismatches(const float *a, int64_t n) {
  const float c7 = 1.0f / 7.0f;
  int64_t bad = 0;
  for (int64_t i = 0; i < n; ++i) {
    const float x = a[i];
    const float q0 = x * c7;
    const float r = fmaf(-q0, 7.0f, x);
    const float q = fmaf(r, c7, q0);
    if (q != x / 7.0f) ++bad;
  }
  return bad;
}

/*
 * Checker for the device's rounding shortcut (not part of the reference):
 * for every float whose bit pattern lies in [lo, hi) and for its negation,
 * compares (int)(q + copysign(h, q)) with (int)roundf(q) (round half away
 * from zero); the device uses h = 0.5 - 2^-25. Patterns must encode finite
 * |q| < 2^30. Returns the number of mismatches.
 */
int64_t oracle_round_shortcut_mismatches(uint32_t lo, uint32_t hi, float h) {
  int64_t bad = 0;
  for (uint32_t b = lo; b < hi; ++b) {
    float q;
    memcpy(&q, &b, 4);
    for (int sgn = 0; sgn < 2; ++sgn, q = -q) {
      const int fast = (int)(q + copysignf(h, q));
      const int want = (int)roundf(q);
      if (fast != want) ++bad;
    }
  }
  return bad;
}
