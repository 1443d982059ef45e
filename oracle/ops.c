/* ops.c - TEST INFRASTRUCTURE ONLY (see oracle.h).
 * The non-Linear operations of TInferCpuBackend and TDecoderModel, restated
 * from src/infer/mormot.ai.infer.backend.cpu.pas, decoder.pas and
 * sampler.pas. */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include "oracle.h"

/* backend.cpu.pas:1769-1795 */
void orc_rmsnorm(const float* x, int64_t rows, int64_t cols, const float* w,
                 double eps, float* y)
{
  for (int64_t r = 0; r < rows; r++) {
    const float* xr = x + r * cols;
    float* yr = y + r * cols;
    double sum = 0;
    for (int64_t c = 0; c < cols; c++) {
      double a = xr[c];
      sum = sum + a * a;
    }
    double inv = 1.0 / sqrt(sum / (double)cols + eps);
    for (int64_t c = 0; c < cols; c++) {
      float n = (float)((double)xr[c] * inv);
      yr[c] = w[c] * n;
    }
  }
}

/* backend.cpu.pas:1797-1834 */
void orc_swiglu(float* gate, const float* up, int64_t n, float alpha, float limit)
{
  if (limit > 0) {
    for (int64_t i = 0; i < n; i++) {
      float g = gate[i], u = up[i], b;
      if (g > limit) g = limit;
      if (u > limit) u = limit;
      else if (u < -limit) u = -limit;
      b = g * alpha;
      double a = b;
      b = (float)(1.0 / (1.0 + exp(-a)));
      b = g * b;
      u = u + 1.0f;
      gate[i] = u * b;
    }
    return;
  }
  for (int64_t i = 0; i < n; i++) {
    double a = gate[i];
    float b = (float)(a / (1.0 + exp(-a)));
    gate[i] = b * up[i];
  }
}

/* backend.cpu.pas:1862-1888 */
void orc_rope(float* x, int64_t rows, int64_t heads, int64_t hd, const float* cs,
              const float* sn, int64_t rot)
{
  int64_t half = rot > 0 ? rot >> 1 : hd >> 1;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t i = 0; i < half; i++) {
      double c = cs[r * half + i], s = sn[r * half + i];
      for (int64_t h = 0; h < heads; h++) {
        float* v = x + (r * heads + h) * hd;
        double a = v[i], b = v[i + half];
        v[i] = (float)(a * c - b * s);
        v[i + half] = (float)(b * c + a * s);
      }
    }
}

/* backend.cpu.pas:1305-1354: the reference (double) rows of CausalRows */
/* One head's rows; every (head, row) is computed on its own, so splitting the
 * heads over threads changes no bit of the result. */
static void causal_head(const float* q, int64_t rows, int64_t heads, int64_t d,
                        const float* keys, const float* values, int64_t past, int64_t kvh,
                        float* y, int64_t window, const float* sinks, double scale,
                        int64_t h, double* sc, double* sums)
{
  int64_t kvw = kvh * d, qw = heads * d;
  int64_t g = h / (heads / kvh);
  for (int64_t r = 0; r < rows; r++) {
    int64_t total = past + r + 1, first = 0;
    if (window > 0 && total > window) first = total - window;
    const float* qr = q + r * qw + h * d;
    double m = 0;
    for (int64_t j = first; j < total; j++) {
      const float* k = keys + j * kvw + g * d;
      double acc = 0;
      for (int64_t t = 0; t < d; t++) acc = acc + (double)qr[t] * (double)k[t];
      acc = acc * scale;
      sc[j] = acc;
      if (j == first || acc > m) m = acc;
    }
    if (sinks && sinks[h] > m) m = sinks[h];
    double sum = 0;
    for (int64_t j = first; j < total; j++) {
      sc[j] = exp(sc[j] - m);
      sum = sum + sc[j];
    }
    if (sinks) sum = sum + exp((double)sinks[h] - m);
    for (int64_t t = 0; t < d; t++) sums[t] = 0;
    for (int64_t j = first; j < total; j++) {
      const float* v = values + j * kvw + g * d;
      double a = sc[j];
      for (int64_t t = 0; t < d; t++) sums[t] = sums[t] + a * (double)v[t];
    }
    sum = 1.0 / sum;
    float* o = y + r * qw + h * d;
    for (int64_t t = 0; t < d; t++) o[t] = (float)(sums[t] * sum);
  }
}

void orc_causal_attention_mt(const float* q, int64_t rows, int64_t heads, int64_t d,
                             const float* keys, const float* values, int64_t past,
                             int64_t kvh, float* y, int64_t window, const float* sinks,
                             double scale, int threads)
{
  int64_t total_max = past + rows;
  if (!(scale > 0)) scale = 1.0 / sqrt((double)d);
  if (threads < 1) threads = 1;
#pragma omp parallel num_threads(threads)
  {
    double* sc = (double*)malloc(total_max * sizeof(double));
    double* sums = (double*)malloc(d * sizeof(double));
#pragma omp for schedule(dynamic, 1)
    for (int64_t h = 0; h < heads; h++)
      causal_head(q, rows, heads, d, keys, values, past, kvh, y, window, sinks, scale, h, sc,
                  sums);
    free(sc);
    free(sums);
  }
}

void orc_causal_attention(const float* q, int64_t rows, int64_t heads, int64_t d,
                          const float* keys, const float* values, int64_t past,
                          int64_t kvh, float* y, int64_t window, const float* sinks,
                          double scale)
{
  orc_causal_attention_mt(q, rows, heads, d, keys, values, past, kvh, y, window, sinks, scale,
                          1);
}

/* decoder.pas:2901-2949 TDecoderModel.Route */
void orc_route(const float* lg, int64_t e, int64_t k, int norm_topk, int32_t* chosen,
               float* weights)
{
  double m = lg[0], sum = 0, picked = 0;
  for (int64_t i = 1; i < e; i++)
    if (lg[i] > m) m = lg[i];
  for (int64_t i = 0; i < e; i++) sum = sum + exp((double)lg[i] - m);
  for (int64_t j = 0; j < k; j++) {
    int64_t best = -1;
    for (int64_t i = 0; i < e; i++) {
      int taken = 0;
      for (int64_t t = 0; t < j; t++)
        if (chosen[t] == i) taken = 1;
      if (!taken && (best < 0 || lg[i] > lg[best])) best = i;
    }
    chosen[j] = (int32_t)best;
    weights[j] = (float)(exp((double)lg[best] - m) / sum);
    picked = picked + weights[j];
  }
  if (norm_topk)
    for (int64_t j = 0; j < k; j++) weights[j] = (float)(weights[j] / picked);
}

/* sampler.pas:123-160 InferArgMax */
int64_t orc_argmax(const float* v, int64_t n)
{
  int64_t res = -1;
  int32_t best = INT32_MIN;
  for (int64_t i = 0; i < n; i++) {
    uint32_t b;
    memcpy(&b, &v[i], 4);
    if ((b & 0x7fffffffu) > 0x7f800000u) continue;
    int32_t k = (int32_t)(b ^ ((b >> 31) * 0x7fffffffu));
    if (k == -1) k = 0;
    if (k > best) {
      best = k;
      res = i;
    }
  }
  return res < 0 ? 0 : res;
}

/* decoder.pas:1735-1741: 1 / theta ^ (2i / d), each step rounded to single;
 * decoder.pas:1759-1829 YarnFrequencies */
static void inv_freq(const ihip_model_desc* dsc, float* f, float* ropescale)
{
  int64_t d = dsc->rope_dims > 0 ? dsc->rope_dims : dsc->head_dim, half = d / 2;
  double lt = log(dsc->rope_theta);
  for (int64_t i = 0; i < half; i++) {
    float e = (float)((double)(2 * i) / (double)d);
    float p = (float)exp(lt * (double)e);
    f[i] = 1.0f / p;
  }
  *ropescale = 1.0f;
  if (dsc->rope_factor == 0)
    return;
  double pi2 = 2 * M_PI;
#define CORR(rotations) (((double)d * log((double)dsc->rope_original / ((rotations) * pi2))) / (2 * lt))
  double lo = CORR(dsc->rope_beta_fast), hi = CORR(dsc->rope_beta_slow);
#undef CORR
  if (dsc->rope_truncate) {
    lo = floor(lo);
    hi = ceil(hi);
  }
  if (lo < 0) lo = 0;
  if (hi > d - 1) hi = (double)(d - 1);
  if (lo == hi) hi = hi + 0.001;
  double span = hi - lo;
  float loS = (float)lo, spanS = (float)span, fct = (float)dsc->rope_factor;
  for (int64_t i = 0; i < half; i++) {
    float e = (float)((double)(2 * i) / (double)d);
    float pos = (float)exp(lt * (double)e);
    pos = fct * pos;
    float inter = 1.0f / pos, extra = f[i];
    float ramp = (float)i - loS;
    ramp = ramp / spanS;
    if (ramp < 0) ramp = 0;
    else if (ramp > 1) ramp = 1;
    float keep = 1.0f - ramp;
    ramp = 1.0f - keep;
    inter = inter * ramp;
    extra = extra * keep;
    f[i] = inter + extra;
  }
  if (dsc->rope_attention > 0)
    *ropescale = (float)dsc->rope_attention;
  else if (fct <= 1)
    *ropescale = 1.0f;
  else
    *ropescale = (float)(0.1 * log((double)fct) + 1.0);
}

/* decoder.pas:2539-2561 TDecoderModel.Rotary: [rows, rot / 2] cos, then sin,
 * rot the rotating values of a head (RopeDims) */
int orc_rotary(const ihip_model_desc* dsc, int64_t first, int64_t rows, float* cs)
{
  int64_t half = (dsc->rope_dims > 0 ? dsc->rope_dims : dsc->head_dim) / 2;
  float* f = (float*)malloc(half * sizeof(float));
  float rs;
  inv_freq(dsc, f, &rs);
  float* sn = cs + rows * half;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t i = 0; i < half; i++) {
      float angle = f[i] * (float)(first + r);
      float c = (float)cos((double)angle), s = (float)sin((double)angle);
      if (rs != 1.0f) {
        c = c * rs;
        s = s * rs;
      }
      cs[r * half + i] = c;
      sn[r * half + i] = s;
    }
  free(f);
  return 0;
}

/* decoder.pas:1742-1752 and :2524-2537 TDecoderModel.Rotary2: the second
 * rotary set over heads of hd2 values: 1 / theta2 ^ (2i / hd2), each step
 * rounded to single, for the first rope2_pairs pairs, 0 for the others (cos
 * 1, sin 0); [rows, hd2 / 2] cos, then sin */
int orc_rotary2(const ihip_model_desc* dsc, int64_t hd2, int64_t first, int64_t rows, float* cs)
{
  int64_t half = hd2 / 2;
  float* f = (float*)calloc(half > 0 ? half : 1, sizeof(float));
  double lt = log(dsc->rope2_theta);
  for (int64_t i = 0; i < half && i < dsc->rope2_pairs; i++) {
    float e = (float)((double)(2 * i) / (double)hd2);
    float p = (float)exp(lt * (double)e);
    f[i] = 1.0f / p;
  }
  float* sn = cs + rows * half;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t i = 0; i < half; i++) {
      float angle = f[i] * (float)(first + r);
      cs[r * half + i] = (float)cos((double)angle);
      sn[r * half + i] = (float)sin((double)angle);
    }
  free(f);
  return 0;
}

/* backend.cpu.pas:1836-1860 GeluTanhGlu: gelu_tanh(g) in double rounded to
 * single, then the product */
void orc_geglu(float* gate, const float* up, int64_t n)
{
  const double k = 0.7978845608028654;
  for (int64_t i = 0; i < n; i++) {
    double g = gate[i];
    double t = k * (g + 0.044715 * g * g * g);
    if (t > 20) t = 1;
    else if (t < -20) t = -1;
    else t = 1 - 2 / (exp(2 * t) + 1);
    float b = (float)(0.5 * g * (1 + t));
    gate[i] = b * up[i];
  }
}

/* decoder.pas:1293-1312 InferSoftcap: tanh(x / cap) * cap, each step single */
void orc_softcap(float* x, int64_t n, double cap)
{
  for (int64_t i = 0; i < n; i++) {
    float a = (float)(x[i] / cap);
    double d = a;
    float t;
    if (d > 20) t = 1;
    else if (d < -20) t = -1;
    else t = (float)(1 - 2 / (exp(2 * d) + 1));
    x[i] = (float)(t * cap);
  }
}
