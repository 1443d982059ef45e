/* formats.c - TEST INFRASTRUCTURE ONLY (see oracle.h).
 * Block layouts, exact dequantization and the activation quantizers of the
 * reference, restated in C from src/infer/mormot.ai.infer.tensor.pas and
 * src/infer/mormot.ai.infer.backend.cpu.pas. Compiled with
 * -ffp-contract=off: every float step rounds on its own, as the Pascal code. */
#include <math.h>
#include <string.h>
#include "oracle.h"

static inline float bits_f(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t f_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* tensor.pas:187-192 INFER_DTYPE_SIZE / INFER_DTYPE_BLOCK by TInferDType */
int orc_block_size(int t)
{
  switch (t) {
  case IHIP_F32: return 4;
  case IHIP_F16: case IHIP_BF16: return 2;
  case IHIP_Q8_0: return 34;
  case IHIP_Q4_0: return 18;
  case IHIP_Q4_K: return 144;
  case IHIP_Q6_K: return 210;
  case IHIP_Q5_0: return 22;
  case IHIP_MXFP4: return 17;
  case IHIP_Q5_1: return 24;
  default: return 0;
  }
}

int orc_block_values(int t)
{
  switch (t) {
  case IHIP_F32: case IHIP_F16: case IHIP_BF16: return 1;
  case IHIP_Q4_K: case IHIP_Q6_K: return 256;
  case IHIP_Q8_0: case IHIP_Q4_0: case IHIP_Q5_0: case IHIP_MXFP4: case IHIP_Q5_1: return 32;
  default: return 0;
  }
}

/* tensor.pas:301-326 */
uint32_t orc_half_to_single_bits(uint16_t h)
{
  uint32_t exp = (h >> 10) & 0x1f, mant = h & 0x3ff, bits;
  if (exp == 0) {
    if (mant == 0)
      bits = 0;
    else {
      exp = 127 - 15 + 1;
      while ((mant & 0x400) == 0) { mant <<= 1; exp--; }
      bits = (exp << 23) | ((mant & 0x3ff) << 13);
    }
  } else if (exp == 0x1f)
    bits = 0x7f800000u | (mant << 13);
  else
    bits = ((exp + 127 - 15) << 23) | (mant << 13);
  return bits | ((uint32_t)(h & 0x8000) << 16);
}

float orc_half_to_single(uint16_t h) { return bits_f(orc_half_to_single_bits(h)); }

/* tensor.pas:328-377 InferSingleToHalf: round to nearest even */
uint16_t orc_single_to_half(float v)
{
  uint32_t bits = f_bits(v), sign = (bits >> 16) & 0x8000, mant = bits & 0x7fffff;
  int exp = (int)((bits >> 23) & 0xff);
  uint32_t half, rest;
  if (exp == 0xff)
    return (uint16_t)(mant == 0 ? (sign | 0x7c00) : (sign | 0x7e00 | (mant >> 13)));
  exp = exp - 127 + 15;
  if (exp >= 0x1f)
    return (uint16_t)(sign | 0x7c00);
  if (exp <= 0) {
    if (exp < -10)
      return (uint16_t)sign;
    mant |= 0x800000;
    rest = (uint32_t)(14 - exp);
    half = mant >> rest;
    mant &= (1u << rest) - 1;
    if (mant > (1u << (rest - 1)) || (mant == (1u << (rest - 1)) && (half & 1)))
      half++;
    return (uint16_t)(sign | half);
  }
  half = ((uint32_t)exp << 10) | (mant >> 13);
  rest = mant & 0x1fff;
  if (rest > 0x1000 || (rest == 0x1000 && (half & 1)))
    half++;
  return (uint16_t)(sign | half);
}

/* tensor.pas:459-465 */
uint32_t orc_e8m0_half_bits(uint8_t e)
{
  return e < 2 ? (0x00200000u << e) : ((uint32_t)(e - 1) << 23);
}

/* tensor.pas:205-206 INFER_MXFP4_VALUES */
static const int8_t MXFP4_VALUES[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

/* tensor.pas:379-391 */
static void scale_min_k4(int j, const uint8_t* s, int* sc, int* m)
{
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
    *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* tensor.pas:396-416 DequantQ4K */
static void dequant_q4k(const uint8_t* b, float* y)
{
  float d = orc_half_to_single(rd16(b)), dmin = orc_half_to_single(rd16(b + 2));
  const uint8_t* sc = b + 4;
  const uint8_t* qs = b + 16;
  for (int k = 0; k < 4; k++) {
    int s, m;
    scale_min_k4(2 * k, sc, &s, &m);
    float d1 = d * (float)s, m1 = dmin * (float)m;
    for (int l = 0; l < 32; l++) {
      float t = d1 * (float)(qs[32 * k + l] & 15);
      y[64 * k + l] = t - m1;
    }
    scale_min_k4(2 * k + 1, sc, &s, &m);
    d1 = d * (float)s;
    m1 = dmin * (float)m;
    for (int l = 0; l < 32; l++) {
      float t = d1 * (float)(qs[32 * k + l] >> 4);
      y[64 * k + 32 + l] = t - m1;
    }
  }
}

/* tensor.pas:419-439 Q6KValue: ql[128], qh[64], scales[16], d */
static int q6k_value(const uint8_t* b, int i)
{
  int n = i >> 7, l, h, r;
  i &= 127;
  l = i & 31;
  h = (b[128 + 32 * n + l] >> (2 * (i >> 5))) & 3;
  switch (i >> 5) {
  case 0: r = b[64 * n + l] & 15; break;
  case 1: r = b[64 * n + l + 32] & 15; break;
  case 2: r = b[64 * n + l] >> 4; break;
  default: r = b[64 * n + l + 32] >> 4; break;
  }
  return (r | (h << 4)) - 32;
}

/* tensor.pas:441-453 DequantQ6K */
static void dequant_q6k(const uint8_t* b, float* y)
{
  float d = orc_half_to_single(rd16(b + 208));
  const int8_t* sc = (const int8_t*)(b + 192);
  for (int i = 0; i < 256; i++) {
    float t = d * (float)sc[i >> 4];
    y[i] = t * (float)q6k_value(b, i);
  }
}

/* tensor.pas:467-602 InferRowToF32 */
int orc_row_to_f32(const void* data, int t, int64_t row, int64_t cols, float* dst)
{
  const uint8_t* base = (const uint8_t*)data;
  int bv = orc_block_values(t), bs = orc_block_size(t);
  if (bv == 0 || cols % bv)
    return IHIP_E_UNSUPPORTED;
  int64_t nb = cols / bv;
  const uint8_t* r = base + row * nb * bs;
  switch (t) {
  case IHIP_F32:
    memcpy(dst, r, cols * 4);
    break;
  case IHIP_BF16:
    for (int64_t j = 0; j < cols; j++) {
      uint32_t u = (uint32_t)rd16(r + 2 * j) << 16;
      memcpy(&dst[j], &u, 4);
    }
    break;
  case IHIP_F16:
    for (int64_t j = 0; j < cols; j++)
      dst[j] = orc_half_to_single(rd16(r + 2 * j));
    break;
  case IHIP_Q8_0:
    for (int64_t b = 0; b < nb; b++, r += 34) {
      float d = orc_half_to_single(rd16(r));
      for (int j = 0; j < 32; j++)
        dst[b * 32 + j] = d * (float)(int8_t)r[2 + j];
    }
    break;
  case IHIP_Q4_K:
    for (int64_t b = 0; b < nb; b++)
      dequant_q4k(r + b * 144, dst + b * 256);
    break;
  case IHIP_Q6_K:
    for (int64_t b = 0; b < nb; b++)
      dequant_q6k(r + b * 210, dst + b * 256);
    break;
  case IHIP_Q4_0:
    for (int64_t b = 0; b < nb; b++, r += 18) {
      float d = orc_half_to_single(rd16(r));
      for (int j = 0; j < 16; j++) {
        dst[b * 32 + j] = d * (float)((int)(r[2 + j] & 15) - 8);
        dst[b * 32 + j + 16] = d * (float)((int)(r[2 + j] >> 4) - 8);
      }
    }
    break;
  case IHIP_Q5_0:
    for (int64_t b = 0; b < nb; b++, r += 22) {
      float d = orc_half_to_single(rd16(r));
      uint32_t qh = r[2] | (r[3] << 8) | ((uint32_t)r[4] << 16) | ((uint32_t)r[5] << 24);
      for (int j = 0; j < 16; j++) {
        dst[b * 32 + j] = d * (float)((int)((r[6 + j] & 15) | (((qh >> j) & 1) << 4)) - 16);
        dst[b * 32 + j + 16] =
          d * (float)((int)((r[6 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16);
      }
    }
    break;
  case IHIP_Q5_1:
    for (int64_t b = 0; b < nb; b++, r += 24) {
      float d = orc_half_to_single(rd16(r)), m = orc_half_to_single(rd16(r + 2));
      uint32_t qh = r[4] | (r[5] << 8) | ((uint32_t)r[6] << 16) | ((uint32_t)r[7] << 24);
      for (int j = 0; j < 16; j++) {
        float t0 = d * (float)((r[8 + j] & 15) | (((qh >> j) & 1) << 4));
        float t1 = d * (float)((r[8 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4));
        dst[b * 32 + j] = t0 + m;
        dst[b * 32 + j + 16] = t1 + m;
      }
    }
    break;
  case IHIP_MXFP4:
    for (int64_t b = 0; b < nb; b++, r += 17) {
      /* the IEEE product overflows to the same signed infinity the reference
       * writes for e + log2|k| >= 256 (tensor.pas:584-590) */
      float d = bits_f(orc_e8m0_half_bits(r[0]));
      for (int j = 0; j < 32; j++) {
        int q = j < 16 ? (r[1 + j] & 15) : (r[1 + j - 16] >> 4);
        dst[b * 32 + j] = d * (float)MXFP4_VALUES[q];
      }
    }
    break;
  default:
    return IHIP_E_UNSUPPORTED;
  }
  return 0;
}

static inline int nonfinite(float v) { return (f_bits(v) & 0x7f800000u) == 0x7f800000u; }

/* the rounding of backend.cpu.pas:670-684: t rounded to the nearest integer,
 * ties to even (or away from zero), spelled out on trunc */
static inline int round_q(float t, int ties_away)
{
  int f = (int)t;         /* Trunc */
  float v = t - (float)f; /* exact */
  if (v > 0.5f) f++;
  else if (v < -0.5f) f--;
  else if (v == 0.5f && (ties_away || (f & 1))) f++;
  else if (v == -0.5f && (ties_away || (f & 1))) f--;
  return f;
}

/* backend.cpu.pas:634-689 QuantizeQ8_0 */
int64_t orc_quantize_q8_0(const float* x, int64_t n, void* blocks, int ties_away)
{
  uint8_t* out = (uint8_t*)blocks;
  for (int64_t b = 0; b < n / 32; b++) {
    const float* xb = x + b * 32;
    uint8_t* o = out + b * 34;
    float amax = 0;
    for (int j = 0; j < 32; j++) {
      if (nonfinite(xb[j]))
        return b * 32 + j + 1;
      float v = fabsf(xb[j]);
      if (v > amax) amax = v;
    }
    float d = amax / 127.0f;
    uint16_t h = orc_single_to_half(d);
    o[0] = (uint8_t)h;
    o[1] = (uint8_t)(h >> 8);
    if (d < 2.9387359e-39f) {
      memset(o + 2, 0, 32);
      continue;
    }
    float id = 1.0f / d;
    for (int j = 0; j < 32; j++) {
      float t = xb[j] * id;
      o[2 + j] = (uint8_t)(int8_t)round_q(t, ties_away);
    }
  }
  return 0;
}

/* backend.cpu.pas:703-756 InferQuantizeRowQ4_0 */
int64_t orc_quantize_q4_0(const float* x, int64_t n, void* blocks)
{
  uint8_t* out = (uint8_t*)blocks;
  for (int64_t b = 0; b < n / 32; b++) {
    const float* xb = x + b * 32;
    uint8_t* o = out + b * 18;
    float amax = 0, m = 0;
    for (int j = 0; j < 32; j++) {
      if (nonfinite(xb[j]))
        return b * 32 + j + 1;
      float v = fabsf(xb[j]);
      if (amax < v) { amax = v; m = xb[j]; }
    }
    float d = m / -8.0f;
    uint16_t h = orc_single_to_half(d);
    o[0] = (uint8_t)h;
    o[1] = (uint8_t)(h >> 8);
    if (fabsf(d) < 2.9387359e-39f) {
      memset(o + 2, 0x88, 16);
      continue;
    }
    float id = 1.0f / d;
    for (int j = 0; j < 16; j++) {
      double p = (double)xb[j] * (double)id;
      float t = (float)(p + 8.5);
      int q0 = (int)t;
      if (q0 > 15) q0 = 15;
      p = (double)xb[j + 16] * (double)id;
      t = (float)(p + 8.5);
      int q1 = (int)t;
      if (q1 > 15) q1 = 15;
      o[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
  }
  return 0;
}

/* backend.cpu.pas:758-819 InferQuantizeRowQ8_K: d (single), qs[256], bsums[16] */
int64_t orc_quantize_q8_k(const float* x, int64_t n, void* blocks)
{
  uint8_t* out = (uint8_t*)blocks;
  for (int64_t b = 0; b < n / 256; b++) {
    const float* xb = x + b * 256;
    uint8_t* o = out + b * 292;
    int8_t* qs = (int8_t*)(o + 4);
    int16_t bs[16];
    float amax = 0, m = 0;
    for (int j = 0; j < 256; j++) {
      if (nonfinite(xb[j]))
        return b * 256 + j + 1;
      float v = fabsf(xb[j]);
      if (v > amax) { amax = v; m = xb[j]; }
    }
    if (amax < 3.7320437e-37f) {
      memset(o, 0, 292);
      continue;
    }
    float iscale = -127.0f / m;
    for (int j = 0; j < 256; j++) {
      float t = iscale * xb[j];
      int f = round_q(t, 0);
      if (f > 127) f = 127;
      qs[j] = (int8_t)f;
    }
    for (int g = 0; g < 16; g++) {
      int s = 0;
      for (int j = 16 * g; j < 16 * g + 16; j++) s += qs[j];
      bs[g] = (int16_t)s;
    }
    memcpy(o + 260, bs, 32);
    float d = 1.0f / iscale;
    memcpy(o, &d, 4);
  }
  return 0;
}
