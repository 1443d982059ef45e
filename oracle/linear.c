/* linear.c - TEST INFRASTRUCTURE ONLY (see oracle.h).
 * TInferCpuBackend.Linear restated (src/infer/mormot.ai.infer.backend.cpu.pas
 * :1409-1566, :823-967) with the integer sums of kernels.pas:190-333. */
#include <stdlib.h>
#include <string.h>
#include "oracle.h"

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static const int8_t MXFP4_VALUES[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

/* backend.cpu.pas:1135-1151 InitMxfp4Half: the FP16 scale of each E8M0
 * exponent in the exact range 104..143 (tensor.pas:212-213), else 0 */
static uint16_t mxfp4_half(uint8_t e)
{
  if (e < 104 || e > 143)
    return 0;
  uint32_t b = orc_e8m0_half_bits(e);
  float d;
  memcpy(&d, &b, 4);
  return orc_single_to_half(d);
}

/* one weight row of a 32-value block type as Q8_0 blocks (d, qs[32]) and, for
 * Q5_1, the minimum m of every block: InferQ4ToQ8 (:992), InferQ5ToQ8
 * (:1058), InferQ51ToQ8 (:1098), InferMxfp4ToQ8 (:1154) */
static void row_to_q8(const uint8_t* r, int t, int64_t nb, uint16_t* d, int8_t* qs,
                      uint16_t* mins)
{
  for (int64_t b = 0; b < nb; b++) {
    int8_t* q = qs + b * 32;
    switch (t) {
    case IHIP_Q8_0: {
      const uint8_t* p = r + b * 34;
      d[b] = rd16(p);
      memcpy(q, p + 2, 32);
      break;
    }
    case IHIP_Q4_0: {
      const uint8_t* p = r + b * 18;
      d[b] = rd16(p);
      for (int j = 0; j < 16; j++) {
        q[j] = (int8_t)((p[2 + j] & 15) - 8);
        q[j + 16] = (int8_t)((p[2 + j] >> 4) - 8);
      }
      break;
    }
    case IHIP_Q5_0: {
      const uint8_t* p = r + b * 22;
      uint32_t qh = p[2] | (p[3] << 8) | ((uint32_t)p[4] << 16) | ((uint32_t)p[5] << 24);
      d[b] = rd16(p);
      for (int j = 0; j < 16; j++) {
        q[j] = (int8_t)(((p[6 + j] & 15) | (((qh >> j) & 1) << 4)) - 16);
        q[j + 16] = (int8_t)(((p[6 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16);
      }
      break;
    }
    case IHIP_Q5_1: {
      const uint8_t* p = r + b * 24;
      uint32_t qh = p[4] | (p[5] << 8) | ((uint32_t)p[6] << 16) | ((uint32_t)p[7] << 24);
      d[b] = rd16(p);
      mins[b] = rd16(p + 2);
      for (int j = 0; j < 16; j++) {
        q[j] = (int8_t)((p[8 + j] & 15) | (((qh >> j) & 1) << 4));
        q[j + 16] = (int8_t)((p[8 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4));
      }
      break;
    }
    case IHIP_MXFP4: {
      const uint8_t* p = r + b * 17;
      d[b] = mxfp4_half(p[0]);
      for (int j = 0; j < 16; j++) {
        q[j] = MXFP4_VALUES[p[1 + j] & 15];
        q[j + 16] = MXFP4_VALUES[p[1 + j] >> 4];
      }
      break;
    }
    }
  }
}

/* kernels.pas:229-262 InferQ4KSumsPascal: isum and msum of one super-block */
static void q4k_sums(const uint8_t* wb, const uint8_t* xb, int* isum, int* msum)
{
  const uint8_t* sc = wb + 4;
  const uint8_t* qs = wb + 16;
  const int8_t* xq = (const int8_t*)(xb + 4);
  int16_t bs[16];
  memcpy(bs, xb + 260, 32);
  int is = 0, ms = 0;
  for (int j = 0; j < 8; j++) {
    int k = 32 * (j >> 1), s = 0, scv, mv;
    if (j & 1)
      for (int l = 0; l < 32; l++) s += (qs[k + l] >> 4) * xq[32 * j + l];
    else
      for (int l = 0; l < 32; l++) s += (qs[k + l] & 15) * xq[32 * j + l];
    if (j < 4) {
      scv = sc[j] & 63;
      mv = sc[j + 4] & 63;
    } else {
      scv = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
      mv = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
    is += scv * s;
    ms += mv * (bs[2 * j] + bs[2 * j + 1]);
  }
  *isum = is;
  *msum = ms;
}

/* kernels.pas:292-333 InferQ6KSumsPascal */
static int q6k_sum(const uint8_t* wb, const uint8_t* xb)
{
  const int8_t* xq = (const int8_t*)(xb + 4);
  const int8_t* sc = (const int8_t*)(wb + 192);
  int isum = 0;
  for (int g = 0; g < 16; g++) {
    int s = 0;
    for (int l = 0; l < 16; l++) {
      int i = 16 * g + l, n = i >> 7, q = (wb[128 + 32 * n + (i & 31)] >> (2 * ((i & 127) >> 5))) & 3;
      switch ((i & 127) >> 5) {
      case 0: q = (wb[64 * n + (i & 31)] & 15) | (q << 4); break;
      case 1: q = (wb[64 * n + (i & 31) + 32] & 15) | (q << 4); break;
      case 2: q = (wb[64 * n + (i & 31)] >> 4) | (q << 4); break;
      default: q = (wb[64 * n + (i & 31) + 32] >> 4) | (q << 4); break;
      }
      s += (q - 32) * xq[i];
    }
    isum += sc[g] * s;
  }
  return isum;
}

static int is_block32(int t)
{
  return t == IHIP_Q8_0 || t == IHIP_Q4_0 || t == IHIP_Q5_0 || t == IHIP_Q5_1 || t == IHIP_MXFP4;
}

int orc_linear(const float* x, int64_t rows, int64_t in, const void* wv, int t,
               int64_t out, const float* bias, float* y, int threads)
{
  const uint8_t* w = (const uint8_t*)wv;
  int bv = orc_block_values(t), bs = orc_block_size(t);
  if (bv == 0 || in % bv)
    return IHIP_E_UNSUPPORTED;
  int64_t nb = in / bv, rowbytes = nb * bs;
  if (threads <= 0) threads = 1;
  if (t == IHIP_F32 || t == IHIP_BF16 || t == IHIP_F16) {
    /* backend.cpu.pas:1548-1565: widen, then acc = bias + sum x*w in double */
    for (int64_t r = 0; r < rows; r++) {
      const float* xr = x + r * in;
#pragma omp parallel for num_threads(threads) schedule(static)
      for (int64_t o = 0; o < out; o++) {
        float* wr = (float*)malloc(in * 4);
        orc_row_to_f32(w, t, o, in, wr);
        double acc = bias ? bias[o] : 0.0;
        for (int64_t i = 0; i < in; i++) acc = acc + (double)xr[i] * (double)wr[i];
        y[r * out + o] = (float)acc;
        free(wr);
      }
    }
    return 0;
  }
  if (is_block32(t)) {
    /* LinearQ8_0, backend.cpu.pas:1409-1470 */
    uint8_t* xq = (uint8_t*)malloc(nb * 34);
    double* dxs = (double*)malloc(nb * sizeof(double));
    double* sxs = (double*)malloc(nb * sizeof(double));
    for (int64_t r = 0; r < rows; r++) {
      if (orc_quantize_q8_0(x + r * in, in, xq, 0)) {
        free(xq); free(dxs); free(sxs);
        return IHIP_E_NONFINITE;
      }
      for (int64_t b = 0; b < nb; b++) {
        dxs[b] = orc_half_to_single(rd16(xq + b * 34));
        if (t == IHIP_Q5_1) {
          int s = 0;
          for (int j = 0; j < 32; j++) s += (int8_t)xq[b * 34 + 2 + j];
          sxs[b] = dxs[b] * s;
        }
      }
#pragma omp parallel for num_threads(threads) schedule(static)
      for (int64_t o = 0; o < out; o++) {
        uint16_t* d = (uint16_t*)malloc(nb * 2 * sizeof(uint16_t));
        uint16_t* mins = d + nb;
        int8_t* qs = (int8_t*)malloc(nb * 32);
        row_to_q8(w + o * rowbytes, t, nb, d, qs, mins);
        double acc = bias ? bias[o] : 0.0;
        for (int64_t b = 0; b < nb; b++) {
          const int8_t* xb = (const int8_t*)(xq + b * 34 + 2);
          int sum = 0;
          for (int j = 0; j < 32; j++) sum += qs[b * 32 + j] * xb[j];
          double dw = orc_half_to_single(d[b]);
          acc = acc + (double)sum * (dw * dxs[b]);
        }
        if (t == IHIP_Q5_1)
          for (int64_t b = 0; b < nb; b++)
            acc = acc + (double)orc_half_to_single(mins[b]) * sxs[b];
        y[r * out + o] = (float)acc;
        free(d);
        free(qs);
      }
    }
    free(xq); free(dxs); free(sxs);
    return 0;
  }
  if (t == IHIP_Q4_K || t == IHIP_Q6_K) {
    /* LinearK, backend.cpu.pas:940-967, DotK :823-869 */
    uint8_t* xk = (uint8_t*)malloc(nb * 292);
    for (int64_t r = 0; r < rows; r++) {
      if (orc_quantize_q8_k(x + r * in, in, xk)) {
        free(xk);
        return IHIP_E_NONFINITE;
      }
#pragma omp parallel for num_threads(threads) schedule(static)
      for (int64_t o = 0; o < out; o++) {
        const uint8_t* wr = w + o * rowbytes;
        double res = 0;
        for (int64_t b = 0; b < nb; b++) {
          const uint8_t* wb = wr + b * bs;
          const uint8_t* xb = xk + b * 292;
          float dxf;
          memcpy(&dxf, xb, 4);
          double dx = dxf;
          if (t == IHIP_Q4_K) {
            int is, ms;
            q4k_sums(wb, xb, &is, &ms);
            double hd = orc_half_to_single(rd16(wb)), hm = orc_half_to_single(rd16(wb + 2));
            res = res + (hd * dx) * (double)is;
            res = res - (hm * dx) * (double)ms;
          } else {
            double hd = orc_half_to_single(rd16(wb + 208));
            res = res + (hd * dx) * (double)q6k_sum(wb, xb);
          }
        }
        double acc = bias ? bias[o] : 0.0;
        acc = acc + res;
        y[r * out + o] = (float)acc;
      }
    }
    free(xk);
    return 0;
  }
  return IHIP_E_UNSUPPORTED;
}

int orc_linear_f32(const float* x, int64_t rows, int64_t in, const void* w, int t,
                   int64_t out, const float* bias, float* y, int threads)
{
  int bv = orc_block_values(t);
  if (bv == 0 || in % bv)
    return IHIP_E_UNSUPPORTED;
  if (threads <= 0) threads = 1;
  int err = 0;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t o = 0; o < out; o++) {
    float* wr = (float*)malloc(in * 4);
    if (orc_row_to_f32(w, t, o, in, wr)) err = 1;
    for (int64_t r = 0; r < rows; r++) {
      const float* xr = x + r * in;
      double acc = bias ? bias[o] : 0.0;
      for (int64_t i = 0; i < in; i++) acc = acc + (double)xr[i] * (double)wr[i];
      y[r * out + o] = (float)acc;
    }
    free(wr);
  }
  return err ? IHIP_E_UNSUPPORTED : 0;
}
