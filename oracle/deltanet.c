/* deltanet.c - TEST INFRASTRUCTURE ONLY (see oracle.h).
 * The Gated DeltaNet mixer of Qwen3.5 and the output gate of its attention,
 * as the reference's CPU computes them: TDecoderModel.DeltaPrep
 * (decoder.pas:2755-2855), TInferCpuBackend.DeltaRule / DeltaRuleHead
 * (backend.cpu.pas:1890-1972, the double branch), GateBySigmoid and Silu
 * (decoder.pas:2594-2623). Every single-typed step rounds to single; the
 * sums are double in the order of the Pascal loops. */
#include <math.h>
#include <stdint.h>
#include "oracle.h"

/* Silu (decoder.pas:2612-2623): x / (1 + exp(-x)) in double, 0 below -100 */
static float silu(float x)
{
  double d = x;
  if (d < -100) return 0.0f;
  return (float)(d / (1 + exp(-d)));
}

/* 1 / (1 + exp(-x)) in double rounded to single, 0 below -100 */
static float sigmoid(float x)
{
  double d = x;
  if (d < -100) return 0.0f;
  return (float)(1 / (1 + exp(-d)));
}

void orc_gate_sigmoid(float* a, const float* gate, int64_t n)
{
  for (int64_t i = 0; i < n; i++) {
    float s = sigmoid(gate[i]);
    a[i] = a[i] * s;
  }
}

void orc_delta_prep(float* qkv, float* beta, float* decay, float* z, int64_t rows,
                    float* conv, const float* conv_w, const float* dt_bias, const float* neg_a,
                    int64_t kh, int64_t vh, int64_t dk, int64_t dv, int64_t kw)
{
  const int64_t vd = vh * dv, cd = 2 * kh * dk + vd, k1 = kw - 1;
  const float scale = (float)(1 / sqrt(1.0 * (double)dk));
  for (int64_t item = 0; item < 2 * kh + vh; item++) {
    const int64_t i = item - 2 * kh;
    const int64_t first = i < 0 ? item * dk : 2 * kh * dk + i * dv;
    const int64_t last = first + (i < 0 ? dk : dv) - 1;
    for (int64_t t = 0; t < rows; t++) {
      /* the causal convolution of every channel of the item, then silu */
      for (int64_t c = first; c <= last; c++) {
        float x = qkv[t * cd + c];
        double acc = conv_w[c * kw + k1];
        acc = acc * x;
        for (int64_t j = 0; j < k1; j++) {
          double e = conv_w[c * kw + j];
          acc = acc + e * conv[c * k1 + j];
        }
        for (int64_t j = 0; j + 1 < k1; j++) conv[c * k1 + j] = conv[c * k1 + j + 1];
        if (k1 > 0) conv[c * k1 + k1 - 1] = x;
        qkv[t * cd + c] = silu((float)acc);
      }
      if (i >= 0) {
        /* value head i: beta, the decay, silu of its gate */
        float x = beta[t * vh + i];
        beta[t * vh + i] = sigmoid(x);
        x = decay[t * vh + i] + dt_bias[i];
        float sp;
        if (x > 20) {
          sp = x;
        } else {
          double e = exp((double)x);
          sp = e < 1e-6 ? (float)(e - e * e / 2) : (float)log(1 + e);
        }
        sp = neg_a[i] * sp;
        decay[t * vh + i] = (float)exp((double)sp);
        float* s = z + t * vd + i * dv;
        for (int64_t j = 0; j < dv; j++) s[j] = silu(s[j]);
        continue;
      }
      /* a q or k head: L2-normed, the queries also times dk^-0.5 */
      float* s = qkv + t * cd + first;
      double acc = 0;
      for (int64_t j = 0; j < dk; j++) {
        double e = s[j];
        acc = acc + e * e;
      }
      float a = (float)(1 / sqrt(acc + 1e-6));
      for (int64_t j = 0; j < dk; j++) s[j] = s[j] * a;
      if (item < kh)
        for (int64_t j = 0; j < dk; j++) s[j] = s[j] * scale;
    }
  }
}

void orc_delta_rule(const float* qkv, int64_t rows, int64_t stride, int64_t kh, int64_t vh,
                    int64_t dk, int64_t dv, int64_t group, const float* beta, const float* decay,
                    float* state, float* y)
{
  const int64_t kd = kh * dk, vd = vh * dv;
  for (int64_t h = 0; h < vh; h++) {
    const int64_t off = ((h / group) % kh) * dk;
    float* st = state + h * dv * dk;
    for (int64_t t = 0; t < rows; t++) {
      const float* row = qkv + t * stride;
      const float* q = row + off;
      const float* k = row + kd + off;
      const float* v = row + 2 * kd + h * dv;
      float* o = y + t * vd + h * dv;
      const float g = decay[t * vh + h], b = beta[t * vh + h];
      for (int64_t j = 0; j < dv; j++) {
        /* column j of S: decayed, then what it predicts for this key */
        float* col = st + j * dk;
        double acc = 0;
        for (int64_t i = 0; i < dk; i++) {
          col[i] = col[i] * g;
          double e = col[i];
          acc = acc + e * k[i];
        }
        float a = (float)acc;
        float delta = v[j] - a;
        delta = delta * b;
        /* the correction written into the column, the column read by q */
        acc = 0;
        for (int64_t i = 0; i < dk; i++) {
          float p = k[i] * delta;
          col[i] = col[i] + p;
          double e = col[i];
          acc = acc + e * q[i];
        }
        o[j] = (float)acc;
      }
    }
  }
}
