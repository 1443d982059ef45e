/* fast.c - TEST INFRASTRUCTURE ONLY (see oracle.h).
 * The timed CPU baseline: TInferCpuFastBackend's default mode
 * (backend.cpu.pas:1975-2506) restated with AVX2 + FMA on a thread pool
 * (OpenMP), for the bench's cpu_baseline leg:
 *   - Linear (TInferCpuFastBackend.Linear :2409-2506): the activation rows
 *     quantized in parallel (LinearQuantizeRow :2029-2061), then work items of
 *     16 output features (TILE, LinearTileWork :2064-2397) over the pool;
 *   - K-quants (Q4_K, Q6_K): the exact super-block integer sums of
 *     InferQ4KSums / InferQ6KSums (kernels.pas:229-333; the AVX2 forms
 *     Q4KSums2Avx2Asm :2940, Q6KSums2Avx2Asm :3115) for two token rows at a
 *     time, the double arithmetic of DotK / DotK2 (backend.cpu.pas:823-927):
 *     the same bits as orc_linear;
 *   - 32-value block types: the weight rows of a tile as Q8_0, then the float
 *     lanes of Q8DotF32x4x2 (kernels.pas:1646-1653: |w| x sign(x, w) byte
 *     pairs, int16 pairs to eight exact int32 lanes, converted to float and
 *     multiply-added by dw * dx, the lanes added at the end) for four weight
 *     rows and two token rows;
 *   - F32 weights: the float lanes of InferDotsF32 (16 lanes: two 8-wide FMA
 *     chains), bias added after;
 *   - attention: CausalRows' fast branch (backend.cpu.pas:1233-1300): the
 *     scores as float dots, the softmax, the values as float axpy per tile
 *     of 128 keys, the heads over the pool.
 * Every function needs AVX2 and FMA (orc_fast_available). */
#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include "oracle.h"

#define FAST __attribute__((target("avx2,fma,f16c")))

enum { TILE = 16, CAUSAL_TILE = 128 };

int orc_fast_available(void)
{
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
         __builtin_cpu_supports("f16c");
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

FAST static inline int hsum_i32(__m256i v)
{
  __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
  return _mm_cvtsi128_si32(s);
}

FAST static inline float hsum_ps(__m256 v)
{
  __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_movehdup_ps(s));
  return _mm_cvtss_f32(s);
}

/* the 6-bit scale and min of sub-block j (InferScaleMinK4, tensor.pas:379-391) */
static inline void scale_min_k4(int j, const uint8_t* sc, int* s, int* m)
{
  if (j < 4) {
    *s = sc[j] & 63;
    *m = sc[j + 4] & 63;
  } else {
    *s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
    *m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
  }
}

/* Q4_K super-block against two Q8_K rows: isum and msum of each
 * (InferQ4KSums2): unsigned nibbles x signed codes (vpmaddubsw, exact: at
 * most 2 * 15 * 127 per int16), times the sub-block scale (vpmaddwd) */
FAST static void q4k_sums2(const uint8_t* wb, const uint8_t* x0, const uint8_t* x1, int n2,
                           int* is, int* ms)
{
  const uint8_t* sc = wb + 4;
  const uint8_t* qs = wb + 16;
  const __m256i m4 = _mm256_set1_epi8(15);
  __m256i acc0 = _mm256_setzero_si256(), acc1 = _mm256_setzero_si256();
  int scv[8], mv[8];
  for (int j = 0; j < 8; j++) scale_min_k4(j, sc, &scv[j], &mv[j]);
  for (int p = 0; p < 4; p++) {
    const __m256i q = _mm256_loadu_si256((const __m256i*)(qs + 32 * p));
    const __m256i lo = _mm256_and_si256(q, m4);
    const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
    const __m256i s_lo = _mm256_set1_epi16((short)scv[2 * p]);
    const __m256i s_hi = _mm256_set1_epi16((short)scv[2 * p + 1]);
    const __m256i a0 = _mm256_loadu_si256((const __m256i*)(x0 + 4 + 64 * p));
    const __m256i b0 = _mm256_loadu_si256((const __m256i*)(x0 + 4 + 64 * p + 32));
    acc0 = _mm256_add_epi32(acc0, _mm256_madd_epi16(_mm256_maddubs_epi16(lo, a0), s_lo));
    acc0 = _mm256_add_epi32(acc0, _mm256_madd_epi16(_mm256_maddubs_epi16(hi, b0), s_hi));
    if (n2) {
      const __m256i a1 = _mm256_loadu_si256((const __m256i*)(x1 + 4 + 64 * p));
      const __m256i b1 = _mm256_loadu_si256((const __m256i*)(x1 + 4 + 64 * p + 32));
      acc1 = _mm256_add_epi32(acc1, _mm256_madd_epi16(_mm256_maddubs_epi16(lo, a1), s_lo));
      acc1 = _mm256_add_epi32(acc1, _mm256_madd_epi16(_mm256_maddubs_epi16(hi, b1), s_hi));
    }
  }
  is[0] = hsum_i32(acc0);
  int16_t bs[16];
  memcpy(bs, x0 + 260, 32);
  int m = 0;
  for (int j = 0; j < 8; j++) m += mv[j] * (bs[2 * j] + bs[2 * j + 1]);
  ms[0] = m;
  if (n2) {
    is[1] = hsum_i32(acc1);
    memcpy(bs, x1 + 260, 32);
    m = 0;
    for (int j = 0; j < 8; j++) m += mv[j] * (bs[2 * j] + bs[2 * j + 1]);
    ms[1] = m;
  }
}

/* Q6_K super-block against two Q8_K rows (InferQ6KSums2): the 6-bit codes
 * q (unsigned) x signed codes, times the group scale, minus 32 * scale *
 * the group's activation sum (the bsums of 16) */
FAST static void q6k_sums2(const uint8_t* wb, const uint8_t* x0, const uint8_t* x1, int n2, int* is)
{
  const uint8_t* ql = wb;
  const uint8_t* qh = wb + 128;
  const int8_t* sc = (const int8_t*)(wb + 192);
  const __m256i m4 = _mm256_set1_epi8(15), m3 = _mm256_set1_epi8(3);
  __m256i acc0 = _mm256_setzero_si256(), acc1 = _mm256_setzero_si256();
  for (int n = 0; n < 2; n++) {
    const __m256i h = _mm256_loadu_si256((const __m256i*)(qh + 32 * n));
    const __m256i la = _mm256_loadu_si256((const __m256i*)(ql + 64 * n));
    const __m256i lb = _mm256_loadu_si256((const __m256i*)(ql + 64 * n + 32));
    for (int c = 0; c < 4; c++) {
      const __m256i l4 = c & 2 ? _mm256_and_si256(_mm256_srli_epi16(c & 1 ? lb : la, 4), m4)
                               : _mm256_and_si256(c & 1 ? lb : la, m4);
      __m256i h2 = h;
      if (c == 1) h2 = _mm256_srli_epi16(h, 2);
      else if (c == 2) h2 = _mm256_srli_epi16(h, 4);
      else if (c == 3) h2 = _mm256_srli_epi16(h, 6);
      const __m256i q = _mm256_or_si256(l4, _mm256_slli_epi16(_mm256_and_si256(h2, m3), 4));
      const int g = 8 * n + 2 * c;
      const __m256i s = _mm256_setr_epi16(sc[g], sc[g], sc[g], sc[g], sc[g], sc[g], sc[g], sc[g],
                                          sc[g + 1], sc[g + 1], sc[g + 1], sc[g + 1], sc[g + 1],
                                          sc[g + 1], sc[g + 1], sc[g + 1]);
      const __m256i a0 = _mm256_loadu_si256((const __m256i*)(x0 + 4 + 128 * n + 32 * c));
      acc0 = _mm256_add_epi32(acc0, _mm256_madd_epi16(_mm256_maddubs_epi16(q, a0), s));
      if (n2) {
        const __m256i a1 = _mm256_loadu_si256((const __m256i*)(x1 + 4 + 128 * n + 32 * c));
        acc1 = _mm256_add_epi32(acc1, _mm256_madd_epi16(_mm256_maddubs_epi16(q, a1), s));
      }
    }
  }
  int16_t bs[16];
  memcpy(bs, x0 + 260, 32);
  int off = 0;
  for (int g = 0; g < 16; g++) off += sc[g] * bs[g];
  is[0] = hsum_i32(acc0) - 32 * off;
  if (n2) {
    memcpy(bs, x1 + 260, 32);
    off = 0;
    for (int g = 0; g < 16; g++) off += sc[g] * bs[g];
    is[1] = hsum_i32(acc1) - 32 * off;
  }
}

/* the Q8_0 form of a 32-value block row (InferQ4ToQ8 and the others, as the
 * tile unpack of LinearTileWork :2200-2250): d and 32 signed codes */
static const int8_t MXFP4_VALUES[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

static float block_scale(const uint8_t* p, int t)
{
  if (t == IHIP_MXFP4) {
    /* the half of 2^(e-128) (MXFP4_HALF), exact in half from 104 to 143 */
    const int e = p[0];
    return (e >= 104 && e <= 143) ? ldexpf(1.0f, e - 128) : 0.0f;
  }
  return orc_half_to_single(rd16(p));
}

static void block_to_q8(const uint8_t* p, int t, float* d, float* m, int8_t* q)
{
  *m = 0;
  switch (t) {
  case IHIP_Q8_0:
    *d = block_scale(p, t);
    memcpy(q, p + 2, 32);
    break;
  case IHIP_Q4_0:
    *d = block_scale(p, t);
    for (int j = 0; j < 16; j++) {
      q[j] = (int8_t)((p[2 + j] & 15) - 8);
      q[j + 16] = (int8_t)((p[2 + j] >> 4) - 8);
    }
    break;
  case IHIP_Q5_0: {
    const uint32_t qh = p[2] | (p[3] << 8) | ((uint32_t)p[4] << 16) | ((uint32_t)p[5] << 24);
    *d = block_scale(p, t);
    for (int j = 0; j < 16; j++) {
      q[j] = (int8_t)(((p[6 + j] & 15) | (((qh >> j) & 1) << 4)) - 16);
      q[j + 16] = (int8_t)(((p[6 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16);
    }
    break;
  }
  case IHIP_Q5_1: {
    const uint32_t qh = p[4] | (p[5] << 8) | ((uint32_t)p[6] << 16) | ((uint32_t)p[7] << 24);
    *d = block_scale(p, t);
    *m = orc_half_to_single(rd16(p + 2));
    for (int j = 0; j < 16; j++) {
      q[j] = (int8_t)((p[8 + j] & 15) | (((qh >> j) & 1) << 4));
      q[j + 16] = (int8_t)((p[8 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4));
    }
    break;
  }
  case IHIP_MXFP4:
    *d = block_scale(p, t);
    for (int j = 0; j < 16; j++) {
      q[j] = MXFP4_VALUES[p[1 + j] & 15];
      q[j + 16] = MXFP4_VALUES[p[1 + j] >> 4];
    }
    break;
  }
}

/* one block of 32: eight exact int32 lanes of w . x (vpsignb, vpmaddubsw,
 * vpmaddwd) as floats */
FAST static inline __m256 q8_lanes(const int8_t* w, const int8_t* x)
{
  const __m256i wv = _mm256_loadu_si256((const __m256i*)w);
  const __m256i xv = _mm256_loadu_si256((const __m256i*)x);
  const __m256i p16 = _mm256_maddubs_epi16(_mm256_sign_epi8(wv, wv), _mm256_sign_epi8(xv, wv));
  return _mm256_cvtepi32_ps(_mm256_madd_epi16(p16, _mm256_set1_epi16(1)));
}

/* InferDotsF32: 16 float lanes (two FMA chains of 8), then one sum */
FAST static float dot_f32(const float* a, const float* b, int64_t n)
{
  __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
  int64_t i = 0;
  for (; i + 16 <= n; i += 16) {
    s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), s0);
    s1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), s1);
  }
  float r = hsum_ps(_mm256_add_ps(s0, s1));
  for (; i < n; i++) r += a[i] * b[i];
  return r;
}

FAST int orc_fast_linear(const float* x, int64_t rows, int64_t in, const void* wv, int t,
                         int64_t out, const float* bias, float* y, int threads)
{
  const uint8_t* w = (const uint8_t*)wv;
  const int bv = orc_block_values(t), bsz = orc_block_size(t);
  if (bv == 0 || in % bv) return IHIP_E_UNSUPPORTED;
  const int64_t nb = in / bv, rowbytes = nb * bsz, tiles = (out + TILE - 1) / TILE;
  if (threads <= 0) threads = 1;
  if (t == IHIP_F32 || t == IHIP_BF16 || t == IHIP_F16) {
    float* wf = NULL;
    if (t != IHIP_F32) {
      /* BF16 / F16 weights widened once (decoder.pas:2211-2221) */
      wf = (float*)malloc((size_t)out * in * 4);
#pragma omp parallel for num_threads(threads) schedule(static)
      for (int64_t o = 0; o < out; o++) orc_row_to_f32(w, t, o, in, wf + o * in);
    }
    const float* W = wf ? wf : (const float*)w;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t tl = 0; tl < tiles; tl++) {
      const int64_t o1 = tl * TILE + TILE < out ? tl * TILE + TILE : out;
      for (int64_t r = 0; r < rows; r++)
        for (int64_t o = tl * TILE; o < o1; o++) {
          float v = dot_f32(x + r * in, W + o * in, in);
          y[r * out + o] = bias ? v + bias[o] : v;
        }
    }
    free(wf);
    return 0;
  }
  if (t == IHIP_Q4_K || t == IHIP_Q6_K) {
    uint8_t* xk = (uint8_t*)malloc((size_t)rows * nb * 292);
    int bad = 0;
#pragma omp parallel for num_threads(threads) schedule(static) reduction(|: bad)
    for (int64_t r = 0; r < rows; r++)
      if (orc_quantize_q8_k(x + r * in, in, xk + r * nb * 292)) bad = 1;
    if (bad) {
      free(xk);
      return IHIP_E_NONFINITE;
    }
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t tl = 0; tl < tiles; tl++) {
      const int64_t o1 = tl * TILE + TILE < out ? tl * TILE + TILE : out;
      for (int64_t o = tl * TILE; o < o1; o++) {
        const uint8_t* wr = w + o * rowbytes;
        for (int64_t r = 0; r < rows; r += 2) {
          const int n2 = r + 1 < rows;
          const uint8_t* x0 = xk + r * nb * 292;
          const uint8_t* x1 = n2 ? x0 + nb * 292 : x0;
          double res0 = 0, res1 = 0;
          for (int64_t b = 0; b < nb; b++) {
            const uint8_t* wb = wr + b * bsz;
            const uint8_t* b0 = x0 + b * 292;
            const uint8_t* b1 = x1 + b * 292;
            float f0, f1;
            memcpy(&f0, b0, 4);
            memcpy(&f1, b1, 4);
            const double dx0 = f0, dx1 = f1;
            int is[2] = {0, 0}, ms[2] = {0, 0};
            if (t == IHIP_Q4_K) {
              q4k_sums2(wb, b0, b1, n2, is, ms);
              const double hd = orc_half_to_single(rd16(wb)), hm = orc_half_to_single(rd16(wb + 2));
              res0 = res0 + (hd * dx0) * (double)is[0];
              res0 = res0 - (hm * dx0) * (double)ms[0];
              if (n2) {
                res1 = res1 + (hd * dx1) * (double)is[1];
                res1 = res1 - (hm * dx1) * (double)ms[1];
              }
            } else {
              q6k_sums2(wb, b0, b1, n2, is);
              const double hd = orc_half_to_single(rd16(wb + 208));
              res0 = res0 + (hd * dx0) * (double)is[0];
              if (n2) res1 = res1 + (hd * dx1) * (double)is[1];
            }
          }
          double acc = bias ? bias[o] : 0.0;
          y[r * out + o] = (float)(acc + res0);
          if (n2) y[(r + 1) * out + o] = (float)(acc + res1);
        }
      }
    }
    free(xk);
    return 0;
  }
  /* 32-value block types: the rows as Q8_0 (d as float), the weight rows of
   * a tile as Q8_0, the float lanes for two token rows at a time */
  uint8_t* xq = (uint8_t*)malloc((size_t)rows * nb * 34);
  float* dxs = (float*)malloc((size_t)rows * nb * 4);
  float* sxs = (float*)malloc((size_t)rows * nb * 4);
  int bad = 0;
#pragma omp parallel for num_threads(threads) schedule(static) reduction(|: bad)
  for (int64_t r = 0; r < rows; r++) {
    if (orc_quantize_q8_0(x + r * in, in, xq + r * nb * 34, 0)) bad = 1;
    for (int64_t b = 0; b < nb; b++) {
      const uint8_t* p = xq + (r * nb + b) * 34;
      dxs[r * nb + b] = orc_half_to_single(rd16(p));
      int s = 0;
      for (int j = 0; j < 32; j++) s += (int8_t)p[2 + j];
      sxs[r * nb + b] = dxs[r * nb + b] * (float)s;
    }
  }
  if (bad) {
    free(xq); free(dxs); free(sxs);
    return IHIP_E_NONFINITE;
  }
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
  for (int64_t tl = 0; tl < tiles; tl++) {
    const int64_t o0 = tl * TILE, o1 = o0 + TILE < out ? o0 + TILE : out, n = o1 - o0;
    int8_t* wq = (int8_t*)malloc((size_t)n * nb * 32);
    float* wd = (float*)malloc((size_t)n * nb * 4);
    float* wm = (float*)malloc((size_t)n * nb * 4);
    for (int64_t i = 0; i < n; i++)
      for (int64_t b = 0; b < nb; b++)
        block_to_q8(w + (o0 + i) * rowbytes + b * bsz, t, &wd[i * nb + b], &wm[i * nb + b],
                    wq + (i * nb + b) * 32);
    for (int64_t r = 0; r < rows; r += 2) {
      const int n2 = r + 1 < rows;
      for (int64_t i = 0; i < n; i++) {
        __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
        float m0 = 0, m1 = 0;
        for (int64_t b = 0; b < nb; b++) {
          const int8_t* wb = wq + (i * nb + b) * 32;
          const float dw = wd[i * nb + b];
          a0 = _mm256_fmadd_ps(_mm256_set1_ps(dw * dxs[r * nb + b]),
                               q8_lanes(wb, (const int8_t*)(xq + (r * nb + b) * 34 + 2)), a0);
          if (t == IHIP_Q5_1) m0 += wm[i * nb + b] * sxs[r * nb + b];
          if (n2) {
            a1 = _mm256_fmadd_ps(_mm256_set1_ps(dw * dxs[(r + 1) * nb + b]),
                                 q8_lanes(wb, (const int8_t*)(xq + ((r + 1) * nb + b) * 34 + 2)), a1);
            if (t == IHIP_Q5_1) m1 += wm[i * nb + b] * sxs[(r + 1) * nb + b];
          }
        }
        const float bo = bias ? bias[o0 + i] : 0.f;
        y[r * out + o0 + i] = bo + (hsum_ps(a0) + m0);
        if (n2) y[(r + 1) * out + o0 + i] = bo + (hsum_ps(a1) + m1);
      }
    }
    free(wq); free(wd); free(wm);
  }
  free(xq); free(dxs); free(sxs);
  return 0;
}

/* CausalRows' fast branch for every head over the pool: float dots, the
 * softmax of CausalSoftmaxF32 (max, exp, sum, sinks), the values per tile of
 * 128 keys added in order */
FAST void orc_fast_attention(const float* q, int64_t rows, int64_t heads, int64_t d,
                             const float* keys, const float* values, int64_t past, int64_t kvh,
                             float* y, int64_t window, const float* sinks, int threads)
{
  const int64_t kvw = kvh * d, qw = heads * d;
  const float scale = (float)(1.0 / sqrt((double)d));
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1) collapse(2)
  for (int64_t h = 0; h < heads; h++)
    for (int64_t r = 0; r < rows; r++) {
      const int64_t g = h / (heads / kvh);
      const int64_t total = past + r + 1;
      const int64_t first = (window > 0 && total > window) ? total - window : 0, cnt = total - first;
      float* s = (float*)malloc((size_t)cnt * 4);
      float* part = (float*)malloc((size_t)d * 4);
      const float* qr = q + r * qw + h * d;
      float m = -INFINITY;
      for (int64_t j = 0; j < cnt; j++) {
        s[j] = dot_f32(qr, keys + (first + j) * kvw + g * d, d) * scale;
        if (s[j] > m) m = s[j];
      }
      if (sinks && sinks[h] > m) m = sinks[h];
      double sum = 0;
      for (int64_t j = 0; j < cnt; j++) {
        s[j] = expf(s[j] - m);
        sum += s[j];
      }
      if (sinks) sum += exp((double)sinks[h] - m);
      const float inv = (float)(1.0 / sum);
      for (int64_t j = 0; j < cnt; j++) s[j] *= inv;
      float* o = y + r * qw + h * d;
      memset(o, 0, (size_t)d * 4);
      for (int64_t j = 0; j < cnt; j += CAUSAL_TILE) {
        const int64_t tn = cnt - j < CAUSAL_TILE ? cnt - j : CAUSAL_TILE;
        memset(part, 0, (size_t)d * 4);
        for (int64_t k = 0; k < tn; k++) {
          const float* v = values + (first + j + k) * kvw + g * d;
          const __m256 a = _mm256_set1_ps(s[j + k]);
          int64_t i = 0;
          for (; i + 8 <= d; i += 8)
            _mm256_storeu_ps(part + i, _mm256_fmadd_ps(a, _mm256_loadu_ps(v + i), _mm256_loadu_ps(part + i)));
          for (; i < d; i++) part[i] += s[j + k] * v[i];
        }
        for (int64_t i = 0; i < d; i++) o[i] += part[i];
      }
      free(s);
      free(part);
    }
}
